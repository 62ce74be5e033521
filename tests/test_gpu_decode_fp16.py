"""GPU parity of decode attention on fp16 pools. fp16 at head_dim 128 / page size 16 runs the
same kernels as bf16 (paged_decode_stream for Hq / Hkv in {1, 2, 4}, paged_decode_mfma for 8):
the scores, the online softmax and the P . V sums in fp32, the probabilities rounded to fp16
(bf16 for bf16 pools) as the operands of the P . V products, the output rounded to fp16. The
reference runs its torch path in the pools' dtype (src/plastic_infer/exec/attention.py:151-190,
src/plastic_infer/exec/runner_paged.py:112-129, 251-255).

Bars: the pools after an append call equal the oracle's write of the new rows bit for bit
(OP.scatter_slots), with the new tokens' slots holding NaN / Inf before the call; outputs are
within 5e-3 of the oracle (fp16 keeps 11 significant bits: the rounding of a probability to
fp16 moves an output of magnitude <= ~1 by at most a few 1e-4, against 2e-2 for bf16's 8).
"""

from __future__ import annotations

import pytest
import torch

import oracle.paged_kv as OP
from plastic_infer.kernel import paged_decode_append_attention, paged_decode_attention
from test_gpu_append_decode import _case, _check
from test_gpu_attention import oracle_max_err_all_rows, qwen3_8b_b256_inputs

pytestmark = pytest.mark.gpu

FP16_TOL = 5e-3


@pytest.mark.parametrize("G", [1, 2, 4, 8])
def test_fp16_append_decode_groups_and_edge_lengths(dev, G):
    """Lengths around page (16) and step (128) boundaries; the append call against the oracle
    and against kv_scatter + paged_decode_attention on the same fp16 inputs."""
    Hkv = 8 if G < 8 else 4
    lens = [1, 15, 16, 17, 127, 128, 129, 511, 512, 513, 1024, 1100]
    q, kp, vp, bt, lens_t, kn, vn = _case(60 + G, lens, Hkv * G, Hkv, 1200, dtype=torch.float16)
    _check(dev, q, kp, vp, bt, lens_t, kn, vn, 16, tol=FP16_TOL)


@pytest.mark.parametrize("G,lens", [
    (4, [8192]),                 # one segment per kv head, cut over many waves and merged
    (1, [8191, 3]),
    (2, [0, 4097, 0, 129, 0]),   # empty sequences between and around long ones
    (8, [8192]),
    (8, [0, 4097, 0, 129, 0]),
])
def test_fp16_decode_long_sequences_split_over_waves(dev, G, lens):
    Hkv = 8
    q, kp, vp, bt, lens_t, _, _ = _case(70 + G, lens, Hkv * G, Hkv, 1100, dtype=torch.float16)
    out = paged_decode_attention(q.to(dev), kp.to(dev), vp.to(dev), bt.to(dev),
                                 lens_t.to(dev)).cpu()
    assert out.dtype == torch.float16
    live = lens_t > 0
    assert not out[~live].any()
    ref = OP.decode_batch(q[live], kp, vp, bt[live].clamp(min=0), lens_t[live], 16)
    err = (out[live].float() - ref.float()).abs().max().item()
    assert err <= FP16_TOL, err


@pytest.mark.parametrize("G", [4, 8])
def test_fp16_decode_stale_tail_tokens(dev, G):
    """Tokens past a sequence's length on its last page hold NaN (K) and Inf (V): they are not
    keys, so the output stays finite and equal to the oracle's over the first L tokens."""
    Hkv = 4
    lens = [37, 200, 1000, 4093]
    q, kp, vp, bt, lens_t, _, _ = _case(80 + G, lens, Hkv * G, Hkv, 400, dtype=torch.float16)
    ref = OP.decode_batch(q, kp, vp, bt.clamp(min=0), lens_t, 16)
    for b, L in enumerate(lens):
        page = int(bt[b, (L - 1) // 16])
        kp[page, :, :, L % 16:] = float("nan")
        vp[page, :, :, L % 16:] = float("inf")
    out = paged_decode_attention(q.to(dev), kp.to(dev), vp.to(dev), bt.to(dev),
                                 lens_t.to(dev)).cpu()
    assert torch.isfinite(out.float()).all()
    err = (out.float() - ref.float()).abs().max().item()
    assert err <= FP16_TOL, err


def test_fp16_append_qwen3_8b_b256_full_shape(dev):
    """The decode step of the benchmark at full size on fp16 pools: one
    paged_decode_append_attention call (B = 256, L ~ U[512, 8192], a 160k-page pool, seed 2),
    the new tokens' slots poisoned first; the pools bit-exact against the oracle's write over
    the whole pool and all 256 rows against the oracle's decode."""
    P = 16
    q, kp, vp, bt, lens, n_pages, page, offset, slots, k_new, v_new = qwen3_8b_b256_inputs(
        dev, torch.float16)
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
    assert worst <= FP16_TOL, worst
