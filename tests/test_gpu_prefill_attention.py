"""GPU parity of multi-row paged attention on the matrix cores (pia_paged_attention's prefill
kernel: bf16 or fp16, head_dim 128, page size 16, G in {1, 2, 4, 8}, at least 4 query rows per
sequence on average) against the oracle's paged attention (the reference's gather + SDPA, and the
explicit offset mask of src/plastic_infer/exec/runner_paged.py:61-95, oracle/paged_kv.py).

Bar: 2e-2 absolute on bf16 outputs (the bf16 attention bar of the decode tests: the kernel
rounds the probabilities to bf16 for the P.V products, the oracle's CPU SDPA rounds its own
intermediates); 5e-3 on fp16 outputs (the same with fp16's 11 significant bits). Invalid block-table ids inside a context and rows without any admissible key are
checked against fp64 brute force with those keys removed.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle.paged_kv as OP
from plastic_infer.kernel import paged_attention

pytestmark = pytest.mark.gpu

BF16_TOL = 2e-2
FP16_TOL = 5e-3
P, D = 16, 128


def _pools(seed, n_pages, Hkv, dtype=torch.bfloat16):
    g = torch.Generator().manual_seed(seed)
    kp = torch.randn(n_pages, Hkv, D, P, generator=g).to(dtype)
    vp = torch.randn(n_pages, Hkv, D, P, generator=g).to(dtype)
    return kp, vp, g


def _tables(kv_lens, n_pages, g):
    width = max(1, max((L + P - 1) // P for L in kv_lens))
    perm = torch.randperm(n_pages, generator=g).tolist()
    bt = torch.full((len(kv_lens), width), -1, dtype=torch.int32)
    tables, off = [], 0
    for b, L in enumerate(kv_lens):
        n = (L + P - 1) // P
        tables.append(perm[off:off + n])
        bt[b, :n] = torch.tensor(tables[-1], dtype=torch.int32)
        off += n
    assert off <= n_pages
    return bt, tables


def _run(dev, q, kp, vp, bt, kv_lens, q_rows, offsets):
    cu = torch.tensor(np.concatenate([[0], np.cumsum(q_rows)]), dtype=torch.int32)
    offs = None if offsets is None else torch.tensor(offsets, dtype=torch.int32, device=dev)
    out = paged_attention(q.to(dev), kp.to(dev), vp.to(dev), bt.to(dev),
                          torch.tensor(kv_lens, dtype=torch.int32, device=dev),
                          cu_q=cu.to(dev), q_pos_offsets=offs)
    return out.cpu(), cu


@pytest.mark.parametrize("G", [1, 2, 4, 8])
def test_prefill_causal_chunks(dev, G):
    """Three sequences: a chunk at the end of a longer context (offset = kv - rows), a fresh
    causal prefill (offset 0), a short chunk after a long context; partial last pages."""
    Hkv = 2
    q_rows = [100, 64, 37]
    kv_lens = [300, 64, 1000]
    offsets = [kv - n for kv, n in zip(kv_lens, q_rows)]
    offsets[1] = 0
    kp, vp, g = _pools(20 + G, 120, Hkv)
    bt, tables = _tables(kv_lens, 120, g)
    q = torch.randn(sum(q_rows), Hkv * G, D, generator=g).to(torch.bfloat16)
    out, cu = _run(dev, q, kp, vp, bt, kv_lens, q_rows, offsets)
    for b in range(3):
        rows = q[cu[b]:cu[b + 1]][None]
        ref = OP.paged_attention(rows, kp, vp, tables[b], P, kv_lens[b], causal=True,
                                 q_start_pos=offsets[b])[0]
        err = (out[cu[b]:cu[b + 1]].float() - ref.float()).abs().max().item()
        assert err <= BF16_TOL, (b, err)


@pytest.mark.parametrize("G", [1, 8])
def test_prefill_nonfinite_stale_tail_tokens(dev, G):
    """Slots past kv_len on a sequence's last page hold NaN (K) and Inf (V), as stale pool memory
    may: they are no keys, so the outputs stay finite and match the oracle, which never reads
    them. Causal chunks end at kv_len, so the last tile of every row crosses the tail."""
    Hkv = 2
    q_rows, kv_lens = [40, 9, 70], [300, 9, 1000]
    offsets = [kv - n for kv, n in zip(kv_lens, q_rows)]
    kp, vp, g = _pools(40 + G, 100, Hkv)
    bt, tables = _tables(kv_lens, 100, g)
    for t, L in zip(tables, kv_lens):
        kp[t[-1], :, :, L % P:] = float("nan")
        vp[t[-1], :, :, L % P:] = float("inf")
    q = torch.randn(sum(q_rows), Hkv * G, D, generator=g).to(torch.bfloat16)
    out, cu = _run(dev, q, kp, vp, bt, kv_lens, q_rows, offsets)
    assert torch.isfinite(out.float()).all()
    for b in range(3):
        rows = q[cu[b]:cu[b + 1]][None]
        ref = OP.paged_attention(rows, kp, vp, tables[b], P, kv_lens[b], causal=True,
                                 q_start_pos=offsets[b])[0]
        assert (out[cu[b]:cu[b + 1]].float() - ref.float()).abs().max() <= BF16_TOL, b


def test_prefill_no_causal_limit(dev):
    """q_pos_offsets absent: every row attends all kv_len keys (SDPA without a mask)."""
    G, Hkv = 4, 2
    q_rows, kv_lens = [20, 70], [500, 129]
    kp, vp, g = _pools(31, 60, Hkv)
    bt, tables = _tables(kv_lens, 60, g)
    q = torch.randn(sum(q_rows), Hkv * G, D, generator=g).to(torch.bfloat16)
    out, cu = _run(dev, q, kp, vp, bt, kv_lens, q_rows, None)
    for b in range(2):
        rows = q[cu[b]:cu[b + 1]][None]
        ref = OP.paged_attention(rows, kp, vp, tables[b], P, kv_lens[b], causal=False)[0]
        assert (out[cu[b]:cu[b + 1]].float() - ref.float()).abs().max() <= BF16_TOL


def test_prefill_long_chunk_qwen3_8b_heads(dev):
    """One 1024-row chunk at the end of a 4096-token context with Qwen3-8B heads (32 q / 8 kv),
    plus a second sequence with an empty context (its rows are zeros)."""
    G, Hkv = 4, 8
    q_rows, kv_lens = [1024, 16], [4096, 0]
    offsets = [4096 - 1024, 0]
    kp, vp, g = _pools(41, 300, Hkv)
    bt, tables = _tables(kv_lens, 300, g)
    q = torch.randn(sum(q_rows), Hkv * G, D, generator=g).to(torch.bfloat16)
    out, cu = _run(dev, q, kp, vp, bt, kv_lens, q_rows, offsets)
    ref = OP.paged_attention(q[:1024][None], kp, vp, tables[0], P, 4096, causal=True,
                             q_start_pos=offsets[0])[0]
    assert (out[:1024].float() - ref.float()).abs().max() <= BF16_TOL
    assert not out[1024:].any()


def _brute_masked(q, kp, vp, table, kv_len, offset, num_pages):
    """fp64: row i over keys j < kv_len (and j <= offset + i) whose page id is in the pool;
    no key -> zeros."""
    q, kp, vp = (np.asarray(x, dtype=np.float64) for x in (q, kp, vp))
    Sq, H, _ = q.shape
    G = H // kp.shape[1]
    out = np.zeros((Sq, H, D))
    for i in range(Sq):
        lim = kv_len if offset is None else min(kv_len, offset + i + 1)
        js = [j for j in range(lim) if 0 <= table[j // P] < num_pages]
        if not js:
            continue
        ks = np.stack([kp[table[j // P], :, :, j % P] for j in js])   # [J, Hkv, D]
        vs = np.stack([vp[table[j // P], :, :, j % P] for j in js])
        for h in range(H):
            s = ks[:, h // G] @ q[i, h] / np.sqrt(D)
            w = np.exp(s - s.max())
            out[i, h] = (w / w.sum()) @ vs[:, h // G]
    return out


def test_prefill_invalid_ids_and_rows_without_keys(dev):
    """Block-table ids -1 and num_pages inside the context (their keys are skipped; page 0,
    which no table uses, holds NaN); offset -20 leaves the first 20 rows without any key."""
    G, Hkv, n = 2, 2, 12
    kp, vp, g = _pools(51, n, Hkv)
    kp[0] = float("nan")
    vp[0] = float("nan")
    table = [3, -1, 7, n, 5, 9]
    kv_len, Sq = 90, 40
    q = torch.randn(Sq, Hkv * G, D, generator=g).to(torch.bfloat16)
    bt = torch.tensor([table], dtype=torch.int32)
    for offset in (None, 60, -20):
        out, _ = _run(dev, q, kp, vp, bt, [kv_len], [Sq], None if offset is None else [offset])
        ref = _brute_masked(q.float().numpy(), kp.float().numpy(), vp.float().numpy(), table,
                            kv_len, offset, n)
        assert np.isfinite(out.float().numpy()).all()
        err = np.abs(out.double().numpy() - ref).max()
        assert err <= BF16_TOL, (offset, err)


def test_prefill_many_ragged_sequences(dev):
    """40 sequences with ragged chunks (4..150 rows) after ragged contexts (0..300 tokens): the
    work list is cut into per-XCD runs at arbitrary points inside sequences and kv heads; every
    row must still be written exactly once."""
    G, Hkv = 2, 4
    g0 = torch.Generator().manual_seed(61)
    q_rows = torch.randint(4, 151, (40,), generator=g0).tolist()
    kv_lens = [n + int(c) for n, c in zip(q_rows, torch.randint(0, 301, (40,), generator=g0))]
    offsets = [kv - n for kv, n in zip(kv_lens, q_rows)]
    n_pages = sum((L + P - 1) // P for L in kv_lens) + 8
    kp, vp, g = _pools(62, n_pages, Hkv)
    bt, tables = _tables(kv_lens, n_pages, g)
    q = torch.randn(sum(q_rows), Hkv * G, D, generator=g).to(torch.bfloat16)
    out, cu = _run(dev, q, kp, vp, bt, kv_lens, q_rows, offsets)
    for b in range(40):
        rows = q[cu[b]:cu[b + 1]][None]
        ref = OP.paged_attention(rows, kp, vp, tables[b], P, kv_lens[b], causal=True,
                                 q_start_pos=offsets[b])[0]
        err = (out[cu[b]:cu[b + 1]].float() - ref.float()).abs().max().item()
        assert err <= BF16_TOL, (b, err)


@pytest.mark.parametrize("G", [1, 4])
def test_prefill_nan_key_reaches_exactly_the_rows_that_see_it(dev, G):
    """A NaN in a K token inside the context: exactly the rows allowed to attend that token get
    NaN, in the q heads of that kv head (their softmax has a NaN score); every other output is
    finite and within the bf16 bar of the oracle on the pool without the NaN. (The reference's
    explicit offset mask is additive, so there a NaN score stays NaN in masked positions too and
    the whole head becomes NaN; the kernel replaces keys a row may not see by -inf.) Pins the
    kernel's NaN behaviour: its row max is the NaN-propagating IEEE 754-2019 maximum."""
    Hkv = 2
    q_rows = [80, 40]
    kv_lens = [200, 150]
    offsets = [kv - n for kv, n in zip(kv_lens, q_rows)]
    kp, vp, g = _pools(40 + G, 40, Hkv)
    bt, tables = _tables(kv_lens, 40, g)
    q = torch.randn(sum(q_rows), Hkv * G, D, generator=g).to(torch.bfloat16)
    tok = 150                                     # a key of sequence 0, kv head 1
    page, off = tables[0][tok // P], tok % P
    kp_nan = kp.clone()
    kp_nan[page, 1, 7, off] = float("nan")
    out, cu = _run(dev, q, kp_nan, vp, bt, kv_lens, q_rows, offsets)
    for b in range(2):
        rows = q[cu[b]:cu[b + 1]][None]
        ref = OP.paged_attention(rows, kp, vp, tables[b], P, kv_lens[b], causal=True,
                                 q_start_pos=offsets[b])[0].float()
        got = out[cu[b]:cu[b + 1]].float()
        want = torch.zeros(got.shape, dtype=torch.bool)
        if b == 0:
            sees = torch.arange(q_rows[0]) + offsets[0] >= tok
            assert bool(sees.any()) and bool((~sees).any())
            want[sees, G:2 * G, :] = True
        assert torch.equal(torch.isnan(got), want), b
        err = (got[~want] - ref[~want]).abs().max().item()
        assert err <= BF16_TOL, (b, err)


@pytest.mark.parametrize("G", [1, 2, 4, 8])
def test_prefill_fp16_causal_chunks(dev, G):
    """The chunk layouts of test_prefill_causal_chunks on fp16 pools and queries."""
    Hkv = 2
    q_rows = [100, 64, 37]
    kv_lens = [300, 64, 1000]
    offsets = [kv - n for kv, n in zip(kv_lens, q_rows)]
    offsets[1] = 0
    kp, vp, g = _pools(120 + G, 120, Hkv, torch.float16)
    bt, tables = _tables(kv_lens, 120, g)
    q = torch.randn(sum(q_rows), Hkv * G, D, generator=g).to(torch.float16)
    out, cu = _run(dev, q, kp, vp, bt, kv_lens, q_rows, offsets)
    assert out.dtype == torch.float16
    for b in range(3):
        rows = q[cu[b]:cu[b + 1]][None]
        ref = OP.paged_attention(rows, kp, vp, tables[b], P, kv_lens[b], causal=True,
                                 q_start_pos=offsets[b])[0]
        err = (out[cu[b]:cu[b + 1]].float() - ref.float()).abs().max().item()
        assert err <= FP16_TOL, (b, err)


def test_prefill_fp16_stale_tail_and_long_chunk(dev):
    """fp16: a 1024-row chunk at the end of a 4096-token context with Qwen3-8B heads, and a
    short chunk whose last page holds NaN (K) / Inf (V) past its length."""
    G, Hkv = 4, 8
    q_rows, kv_lens = [1024, 40], [4096, 300]
    offsets = [kv - n for kv, n in zip(kv_lens, q_rows)]
    kp, vp, g = _pools(141, 300, Hkv, torch.float16)
    bt, tables = _tables(kv_lens, 300, g)
    kp[tables[1][-1], :, :, 300 % P:] = float("nan")
    vp[tables[1][-1], :, :, 300 % P:] = float("inf")
    q = torch.randn(sum(q_rows), Hkv * G, D, generator=g).to(torch.float16)
    out, cu = _run(dev, q, kp, vp, bt, kv_lens, q_rows, offsets)
    assert torch.isfinite(out.float()).all()
    for b in range(2):
        rows = q[cu[b]:cu[b + 1]][None]
        ref = OP.paged_attention(rows, kp, vp, tables[b], P, kv_lens[b], causal=True,
                                 q_start_pos=offsets[b])[0]
        err = (out[cu[b]:cu[b + 1]].float() - ref.float()).abs().max().item()
        assert err <= FP16_TOL, (b, err)
