"""GPU parity of the decode step's KV write and attention in one call
(paged_decode_append_attention / pia_paged_decode_append_attention): the reference's
_write_kv_layer of the new token at position L - 1 followed by _attn_paged over L tokens
(src/plastic_infer/exec/runner_paged.py:112-129, 251-255).

Bars: the pools after the call equal the oracle's write of the new rows at the block table's
slots bit for bit (OP.scatter_slots); the output equals the oracle's decode over the updated
pools within the bf16 attention bar (2e-2; fp32: 1e-4), and the two-launch composition
(kv_scatter, then paged_decode_attention) within 1e-2 - the two differ only in the order in
which the new token's terms enter fp32 sums. The new tokens' slots hold NaN / Inf before the
call, so an attention that read them from the pool instead of k_new / v_new would show it.
"""

from __future__ import annotations

import pytest
import torch

import oracle.paged_kv as OP
from plastic_infer.kernel import kv_scatter, paged_decode_append_attention, paged_decode_attention

pytestmark = pytest.mark.gpu

BF16_TOL = 2e-2


def _case(seed, lens, Hq, Hkv, num_pages, D=128, P=16, dtype=torch.bfloat16):
    g = torch.Generator().manual_seed(seed)
    lens_t = torch.tensor(lens, dtype=torch.int32)
    n_pages = [max(0, (L + P - 1) // P) for L in lens]
    width = max(1, max(n_pages))
    perm = torch.randperm(num_pages, generator=g).tolist()
    bt = torch.full((len(lens), width), -1, dtype=torch.int32)
    off = 0
    for b, n in enumerate(n_pages):
        bt[b, :n] = torch.tensor(perm[off:off + n], dtype=torch.int32)
        off += n
    assert off <= num_pages
    kp = torch.randn(num_pages, Hkv, D, P, generator=g).to(dtype)
    vp = torch.randn(num_pages, Hkv, D, P, generator=g).to(dtype)
    q = torch.randn(len(lens), Hq, D, generator=g).to(dtype)
    kn = torch.randn(len(lens), Hkv, D, generator=g).to(dtype)
    vn = torch.randn(len(lens), Hkv, D, generator=g).to(dtype)
    return q, kp, vp, bt, lens_t, kn, vn


def _slots(bt, lens, P, num_pages):
    """Slot of each row's new token (-1: the row writes nothing)."""
    width = bt.shape[1]
    out = []
    for b, L in enumerate(lens.tolist()):
        if L < 1 or L > width * P:
            out.append(-1)
            continue
        page = int(bt[b, (L - 1) // P])
        out.append(page * P + (L - 1) % P if 0 <= page < num_pages else -1)
    return out


def _poison(kp, vp, slots, P):
    for s in slots:
        if s >= 0:
            kp[s // P, :, :, s % P] = float("nan")
            vp[s // P, :, :, s % P] = float("inf")


def _check(dev, q, kp, vp, bt, lens, kn, vn, P, oracle_rows=None, tol=BF16_TOL):
    num_pages = kp.shape[0]
    slots = _slots(bt, lens, P, num_pages)
    _poison(kp, vp, slots, P)
    gk, gv = kp.to(dev), vp.to(dev)
    out = paged_decode_append_attention(q.to(dev), gk, gv, bt.to(dev), lens.to(dev),
                                        kn.to(dev), vn.to(dev))
    # the two-launch composition on the same inputs
    sk, sv = kp.to(dev), vp.to(dev)
    keep = [b for b, s in enumerate(slots) if s >= 0]
    if keep:
        idx = torch.tensor(keep)
        kv_scatter(kn[idx].to(dev), vn[idx].to(dev), sk, sv,
                   torch.tensor([slots[b] for b in keep], dtype=torch.int64, device=dev))
    two = paged_decode_attention(q.to(dev), sk, sv, bt.to(dev), lens.to(dev))
    assert torch.equal(gk, sk) and torch.equal(gv, sv), "pools differ from the scatter's"
    live = lens > 0
    # a bf16 output may land one step either side of a rounding boundary: 1e-2 relative
    bar = (1e-2 if q.dtype != torch.float32 else 1e-5) * two.float().abs().clamp_min(1.0)
    assert ((out.float() - two.float()).abs() <= bar).all(), \
        (out.float() - two.float()).abs().max().item()
    # the oracle: write, then decode over the updated pools
    okp, ovp = kp.clone(), vp.clone()
    OP.scatter_slots(kn[keep], vn[keep], okp, ovp, [slots[b] for b in keep])
    assert torch.equal(gk.cpu(), okp) and torch.equal(gv.cpu(), ovp)
    rows = [b for b in range(len(lens)) if live[b]] if oracle_rows is None else oracle_rows
    rows_t = torch.tensor(rows)
    ref = OP.decode_batch(q[rows_t], okp, ovp, bt[rows_t].clamp(min=0), lens[rows_t], P)
    err = (out.cpu()[rows_t].float() - ref.float()).abs().max().item()
    assert err <= tol, err
    assert not out.cpu()[~live].any()
    return out


@pytest.mark.parametrize("G", [1, 2, 4, 8])
def test_append_decode_lengths_and_groups(dev, G):
    Hkv = 8 if G < 8 else 4
    lens = [1, 15, 16, 17, 127, 128, 129, 300, 1000, 4097, 2, 64]
    q, kp, vp, bt, lens_t, kn, vn = _case(100 + G, lens, Hkv * G, Hkv, 700)
    _check(dev, q, kp, vp, bt, lens_t, kn, vn, 16)


def test_append_decode_batch_over_one_launch(dev):
    """1100 rows: two launches of the stream kernel (1024 + 76 rows) with row offsets into
    k_new / v_new; the oracle checks a sample of rows, the two-launch composition all of them."""
    g = torch.Generator().manual_seed(7)
    lens = torch.randint(1, 200, (1100,), generator=g).tolist()
    q, kp, vp, bt, lens_t, kn, vn = _case(8, lens, 8, 2, 16000)
    _check(dev, q, kp, vp, bt, lens_t, kn, vn, 16, oracle_rows=[0, 1, 511, 1023, 1024, 1099])


def test_append_decode_many_segment_ends_per_wave(dev):
    """1024 one-page rows x 64 kv heads at G = 8: 65,536 one-step segments over the launch's
    1024 waves, 64 per wave - past the 32 new-token stores a wave defers, so the rest are
    stored as they come. Pools bit-exact, outputs against the two-launch composition (all
    rows) and the oracle (a sample)."""
    g = torch.Generator().manual_seed(14)
    lens = torch.randint(1, 17, (1024,), generator=g).tolist()
    q, kp, vp, bt, lens_t, kn, vn = _case(15, lens, 512, 64, 1100)
    _check(dev, q, kp, vp, bt, lens_t, kn, vn, 16, oracle_rows=[0, 100, 1023])


@pytest.mark.parametrize("G", [4, 8])
def test_append_decode_edge_rows(dev, G):
    """Row 0: L = 0 (zeros, no write). Row 1: L = 40 > its table's 32 tokens (clamped to 32, no
    write). Row 2: the new token's page id is outside the pool (no write, that token is no key).
    Row 3: an ordinary row. G = 4 runs the vector-ALU engine, G = 8 the matrix-core one."""
    q, kp, vp, _, _, kn, vn = _case(9, [1, 1, 1, 1], 4 * G, 4, 40)
    bt = torch.tensor([[1, 2, -1], [3, 4, -1], [5, 6, 40], [7, 8, 9]], dtype=torch.int32)
    bt_w = bt[:, :2].contiguous()                               # row 1's table holds 32 tokens
    lens = torch.tensor([0, 40, 33, 35], dtype=torch.int32)
    gk, gv = kp.to(dev), vp.to(dev)
    out = paged_decode_append_attention(q.to(dev), gk, gv, bt.to(dev), lens.to(dev),
                                        kn.to(dev), vn.to(dev)).cpu()
    okp, ovp = kp.clone(), vp.clone()
    OP.scatter_slots(kn[3:4], vn[3:4], okp, ovp, [9 * 16 + 2])
    assert torch.equal(gk.cpu(), okp) and torch.equal(gv.cpu(), ovp)
    assert not out[0].any()
    ref1 = OP.paged_attention(q[1][None, None], kp, vp, [3, 4], 16, 32, causal=False)[0, 0]
    assert (out[1].float() - ref1.float()).abs().max() <= BF16_TOL   # new token's page is -1
    ref2 = OP.paged_attention(q[2][None, None], okp, ovp, [5, 6], 16, 32, causal=False)[0, 0]
    ref3 = OP.paged_attention(q[3][None, None], okp, ovp, [7, 8, 9], 16, 35, causal=False)[0, 0]
    assert (out[2].float() - ref2.float()).abs().max() <= BF16_TOL
    assert (out[3].float() - ref3.float()).abs().max() <= BF16_TOL
    # the clamped row, on a table two pages wide: the decode over its 32 tokens, nothing written
    gk2, gv2 = kp.to(dev), vp.to(dev)
    out2 = paged_decode_append_attention(q[1:2].to(dev), gk2, gv2, bt_w[1:2].to(dev),
                                         lens[1:2].to(dev), kn[1:2].to(dev), vn[1:2].to(dev))
    assert torch.equal(gk2.cpu(), kp) and torch.equal(gv2.cpu(), vp)
    assert (out2.cpu()[0].float() - ref1.float()).abs().max() <= BF16_TOL


@pytest.mark.parametrize("dtype,Hq,Hkv,D,P,tol", [
    (torch.float32, 4, 2, 64, 8, 1e-4),        # general kernel path: write kernel + decode
    (torch.float16, 6, 2, 128, 16, BF16_TOL),  # G = 3: the matrix-core kernel
    (torch.bfloat16, 8, 8, 96, 16, BF16_TOL),  # head_dim 96
])
def test_append_decode_general_shapes(dev, dtype, Hq, Hkv, D, P, tol):
    lens = [1, P, P + 1, 5 * P - 3, 100]
    q, kp, vp, bt, lens_t, kn, vn = _case(11, lens, Hq, Hkv, 64, D=D, P=P, dtype=dtype)
    _check(dev, q, kp, vp, bt, lens_t, kn, vn, P, tol=tol)


def test_append_decode_strided_new_rows(dev):
    """k_new / v_new as [B, Hkv, D] views of a wider projection output (row stride 3 * Hkv * D):
    passed in place, read at their own row stride."""
    lens = [33, 129, 7]
    q, kp, vp, bt, lens_t, kn, vn = _case(12, lens, 16, 4, 40)
    wide_k = torch.zeros(3, 12, 128, dtype=torch.bfloat16)
    wide_v = torch.zeros(3, 12, 128, dtype=torch.bfloat16)
    wide_k[:, 4:8] = kn
    wide_v[:, 4:8] = vn
    slots = _slots(bt, lens_t, 16, 40)
    _poison(kp, vp, slots, 16)
    gk, gv = kp.to(dev), vp.to(dev)
    wk, wv = wide_k.to(dev), wide_v.to(dev)
    out = paged_decode_append_attention(q.to(dev), gk, gv, bt.to(dev), lens_t.to(dev),
                                        wk[:, 4:8], wv[:, 4:8]).cpu()
    okp, ovp = kp.clone(), vp.clone()
    OP.scatter_slots(kn, vn, okp, ovp, slots)
    assert torch.equal(gk.cpu(), okp) and torch.equal(gv.cpu(), ovp)
    ref = OP.decode_batch(q, okp, ovp, bt.clamp(min=0), lens_t, 16)
    assert (out.float() - ref.float()).abs().max() <= BF16_TOL


def test_append_decode_rejects_bad_new_rows(dev):
    q, kp, vp, bt, lens_t, kn, vn = _case(13, [5, 9], 8, 2, 8)
    with pytest.raises(ValueError, match="k_new"):
        paged_decode_append_attention(q.to(dev), kp.to(dev), vp.to(dev), bt.to(dev),
                                      lens_t.to(dev), kn[:, :1].to(dev), vn.to(dev))
    with pytest.raises(ValueError, match="dtype"):
        paged_decode_append_attention(q.to(dev), kp.to(dev), vp.to(dev), bt.to(dev),
                                      lens_t.to(dev), kn.float().to(dev), vn.to(dev))


def test_append_qwen3_8b_b256_full_shape(dev):
    """The kernel the decode benchmark times, at its full size: one
    paged_decode_append_attention call on the Qwen3-8B step (B = 256, L ~ U[512, 8192], a
    160k-page pool, seed 2). The new tokens' slots hold NaN (K) / Inf (V) before the call. The
    pools afterwards equal the oracle's write of the new rows (OP.scatter_slots on a host copy
    of the poisoned pools) over the whole pool, bit for bit; all 256 rows are within 2e-2 of
    the oracle's decode over the updated pools."""
    from test_gpu_attention import oracle_max_err_all_rows, qwen3_8b_b256_inputs

    P = 16
    q, kp, vp, bt, lens, n_pages, page, offset, slots, k_new, v_new = qwen3_8b_b256_inputs(dev)
    pg, of = page.to(dev), offset.to(dev)
    kp[pg, :, :, of] = float("nan")
    vp[pg, :, :, of] = float("inf")
    kb, vb = kp.cpu(), vp.cpu()
    out = paged_decode_append_attention(q, kp, vp, bt.to(dev), lens.to(torch.int32).to(dev),
                                        k_new, v_new)
    OP.scatter_slots(k_new.cpu(), v_new.cpu(), kb, vb, slots.tolist())
    assert torch.equal(kp.cpu(), kb), "K pool differs from the oracle's write"
    assert torch.equal(vp.cpu(), vb), "V pool differs from the oracle's write"
    del kb, vb
    worst = oracle_max_err_all_rows(out.cpu(), q, kp, vp, bt, lens, n_pages, P)
    assert worst <= BF16_TOL, worst
