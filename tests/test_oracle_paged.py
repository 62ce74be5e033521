"""Pins the paged-KV oracle (CPU, no GPU).

Checks, chosen so a plausible mistake fails at least one of them:
  * the reference tests' known answers (reference tests/test_ops.py:102-147 gather KATs,
    :186-266 paged == contiguous SDPA, tests/test_kv_store.py:63-74 write placement);
  * an fp64 brute-force attention that reads pages token by token through the block table
    (independent of index_select / permute / repeat_interleave / SDPA);
  * closed forms: one key -> its value; identical keys -> mean of the values;
  * planted mistakes in the oracle (transposed page layout, wrong GQA head map, wrong causal
    offset) must be caught by those checks.
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

import oracle.paged_kv as OP


def brute_attention(q, k_pages, v_pages, table, page_size, kv_len, causal_offset=None):
    """fp64 loops: q [Sq, H, D] numpy; returns [Sq, H, D]. Key j of the request is
    k_pages[table[j // P], h_kv, :, j % P]; row i sees j < kv_len and, with an offset,
    j <= causal_offset + i."""
    q = np.asarray(q, dtype=np.float64)
    kp = np.asarray(k_pages, dtype=np.float64)
    vp = np.asarray(v_pages, dtype=np.float64)
    Sq, H, D = q.shape
    Hkv = kp.shape[1]
    G = H // Hkv
    out = np.zeros((Sq, H, D))
    for i in range(Sq):
        lim = kv_len if causal_offset is None else min(kv_len, causal_offset + i + 1)
        for h in range(H):
            hk = h // G
            scores = []
            vals = []
            for j in range(lim):
                page = table[j // page_size]
                kj = kp[page, hk, :, j % page_size]
                scores.append(float(q[i, h] @ kj) / math.sqrt(D))
                vals.append(vp[page, hk, :, j % page_size])
            s = np.array(scores)
            w = np.exp(s - s.max())
            w /= w.sum()
            out[i, h] = (w[:, None] * np.array(vals)).sum(0)
    return out


def _pages(seed, n, H, D, P, dtype=torch.float32):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(n, H, D, P, generator=g, dtype=dtype),
            torch.randn(n, H, D, P, generator=g, dtype=dtype))


# ---- reference known answers ------------------------------------------------------------------

class TestGatherKATs:
    def test_single_page(self):
        k, v = _pages(0, 10, 2, 8, 16)
        kg, vg = OP.gather_paged_kv(k, v, [3], 16)
        assert kg.shape == (1, 16, 2, 8)
        assert torch.equal(kg[0, 0], k[3, :, :, 0])
        assert torch.equal(vg[0, 5], v[3, :, :, 5])

    def test_multiple_pages_in_order(self):
        k, v = _pages(1, 5, 2, 4, 8)
        kg, _ = OP.gather_paged_kv(k, v, [0, 2, 4], 8)
        assert kg.shape == (1, 24, 2, 4)
        for t, (p, o) in {0: (0, 0), 8: (2, 0), 16: (4, 0), 23: (4, 7)}.items():
            assert torch.equal(kg[0, t], k[p, :, :, o])

    def test_partial_last_page_and_empty(self):
        k, v = _pages(2, 4, 2, 4, 16)
        kg, _ = OP.gather_paged_kv(k, v, [0, 1], 16, num_tokens=20)
        assert kg.shape == (1, 20, 2, 4)
        assert torch.equal(kg[0, 19], k[1, :, :, 3])
        ke, ve = OP.gather_paged_kv(k, v, [], 16)
        assert ke.shape == (1, 0, 2, 4) and ve.shape == (1, 0, 2, 4)


class TestScatterKATs:
    def test_write_placement(self):
        k_pages = torch.zeros(8, 2, 4, 4)
        v_pages = torch.zeros(8, 2, 4, 4)
        g = torch.Generator().manual_seed(42)
        kt, vt = torch.randn(1, 2, 4, generator=g), torch.randn(1, 2, 4, generator=g)
        OP.scatter_slots(kt, vt, k_pages, v_pages, [5 * 4 + 2])
        assert torch.equal(k_pages[5, :, :, 2], kt[0])
        assert torch.equal(v_pages[5, :, :, 2], vt[0])
        assert int((k_pages != 0).sum()) == 8   # nothing else touched

    def test_scatter_gather_round_trip(self):
        P, H, D = 4, 2, 3
        table = [6, 1, 4]
        k_pages = torch.zeros(8, H, D, P)
        v_pages = torch.zeros(8, H, D, P)
        g = torch.Generator().manual_seed(7)
        k = torch.randn(10, H, D, generator=g)
        v = torch.randn(10, H, D, generator=g)
        slots = [table[t // P] * P + t % P for t in range(10)]
        OP.scatter_slots(k, v, k_pages, v_pages, slots)
        kg, vg = OP.gather_paged_kv(k_pages, v_pages, table, P, num_tokens=10)
        assert torch.equal(kg[0], k) and torch.equal(vg[0], v)

    def test_write_kv_layer_equals_slots(self):
        P, H, D = 4, 2, 3
        table = [3, 0, 5]
        g = torch.Generator().manual_seed(9)
        k = torch.randn(7, H, D, generator=g)
        v = torch.randn(7, H, D, generator=g)
        a = [torch.zeros(6, H, D, P) for _ in range(2)]
        b = [torch.zeros(6, H, D, P) for _ in range(2)]
        OP.write_kv_layer(table, P, 2, k, v, a[0], a[1])
        slots = [table[(2 + t) // P] * P + (2 + t) % P for t in range(7)]
        OP.scatter_slots(k, v, b[0], b[1], slots)
        assert torch.equal(a[0], b[0]) and torch.equal(a[1], b[1])


class TestAttentionKATs:
    def test_matches_contiguous_sdpa_gqa(self):
        # reference tests/test_ops.py:186-228
        torch.manual_seed(7)
        Sq, H, D, P, n_pages, Hkv = 8, 4, 16, 4, 3, 2
        q = torch.randn(1, Sq, H, D) * 0.1
        kc = torch.randn(1, n_pages * P, Hkv, D) * 0.1
        vc = torch.randn(1, n_pages * P, Hkv, D) * 0.1
        kp = torch.zeros(n_pages, Hkv, D, P)
        vp = torch.zeros(n_pages, Hkv, D, P)
        for p in range(n_pages):
            for t in range(P):
                kp[p, :, :, t] = kc[0, p * P + t]
                vp[p, :, :, t] = vc[0, p * P + t]
        out = OP.paged_attention(q, kp, vp, list(range(n_pages)), P, n_pages * P, causal=True)
        ref = F.scaled_dot_product_attention(
            q.transpose(1, 2), kc.transpose(1, 2).repeat_interleave(2, 1),
            vc.transpose(1, 2).repeat_interleave(2, 1), is_causal=True).transpose(1, 2)
        assert torch.allclose(out, ref, atol=1e-4)

    def test_noncontiguous_pages(self):
        # reference tests/test_ops.py:230-266
        torch.manual_seed(11)
        q = torch.randn(1, 6, 2, 8) * 0.1
        kp = torch.randn(5, 2, 8, 3) * 0.1
        vp = torch.randn(5, 2, 8, 3) * 0.1
        out = OP.paged_attention(q, kp, vp, [4, 1, 3], 3, 9, causal=True)
        kc = torch.cat([kp[p].permute(2, 0, 1) for p in [4, 1, 3]]).unsqueeze(0)
        vc = torch.cat([vp[p].permute(2, 0, 1) for p in [4, 1, 3]]).unsqueeze(0)
        ref = F.scaled_dot_product_attention(q.transpose(1, 2), kc.transpose(1, 2),
                                             vc.transpose(1, 2), is_causal=True).transpose(1, 2)
        assert torch.allclose(out, ref, atol=1e-4)


# ---- independent brute force ------------------------------------------------------------------

CASES = [  # (seed, n_pages, Hkv, G, D, P, table, kv_len, Sq, mode)
    (0, 6, 2, 2, 8, 4, [5, 0, 3], 11, 1, "none"),
    (1, 7, 1, 4, 16, 3, [2, 6, 1, 4], 12, 3, "top_left"),
    (2, 9, 2, 1, 8, 16, [8, 3], 20, 4, "offset"),
    (3, 5, 2, 4, 32, 16, [1], 1, 1, "none"),
    (4, 8, 4, 2, 8, 2, [7, 0, 6, 1, 5], 9, 2, "offset"),
]


@pytest.mark.parametrize("case", CASES)
def test_oracle_vs_fp64_brute_force(case):
    seed, n, Hkv, G, D, P, table, kv_len, Sq, mode = case
    kp, vp = _pages(seed, n, Hkv, D, P, torch.float64)
    q = torch.randn(1, Sq, Hkv * G, D, generator=torch.Generator().manual_seed(seed + 100),
                    dtype=torch.float64)
    q_start = kv_len - Sq if mode == "offset" else 0
    out = OP.paged_attention(q, kp, vp, table, P, kv_len, causal=(mode != "none"),
                             q_start_pos=q_start)
    offset = None if mode == "none" else q_start
    ref = brute_attention(q[0].numpy(), kp.numpy(), vp.numpy(), table, P, kv_len, offset)
    np.testing.assert_allclose(out[0].numpy(), ref, atol=1e-10)


def test_decode_batch_vs_brute_force():
    kp, vp = _pages(5, 12, 2, 8, 4, torch.float64)
    bt = torch.tensor([[3, 7, 1, 0], [11, 2, 0, 0], [5, 6, 8, 9]], dtype=torch.int32)
    lens = [13, 5, 16]
    q = torch.randn(3, 4, 8, generator=torch.Generator().manual_seed(55), dtype=torch.float64)
    out = OP.decode_batch(q, kp, vp, bt, lens, 4)
    for b in range(3):
        ref = brute_attention(q[b][None].numpy(), kp.numpy(), vp.numpy(), bt[b].tolist(), 4, lens[b])
        np.testing.assert_allclose(out[b].numpy(), ref[0], atol=1e-10)


def test_closed_forms():
    kp, vp = _pages(6, 4, 1, 8, 4, torch.float64)
    q = torch.randn(1, 1, 2, 8, dtype=torch.float64)
    one = OP.paged_attention(q, kp, vp, [2], 4, kv_num_tokens=1, causal=False)
    assert torch.allclose(one[0, 0, 0], vp[2, 0, :, 0]) and torch.allclose(one[0, 0, 1], vp[2, 0, :, 0])
    kp_same = kp.clone()
    kp_same[:] = kp[0, :, :, :1]          # every key equal -> uniform weights
    out = OP.paged_attention(q, kp_same, vp, [0, 3], 4, kv_num_tokens=7, causal=False)
    mean = torch.stack([vp[[0, 3][t // 4], 0, :, t % 4] for t in range(7)]).mean(0)
    assert torch.allclose(out[0, 0, 0], mean)


# ---- planted mistakes: the checks above must catch each of them --------------------------------

def _wrong_gather_transposed(k_pages, v_pages, block_table, page_size, num_tokens=None):
    ids = torch.tensor(block_table, dtype=torch.long)
    kg, vg = k_pages.index_select(0, ids), v_pages.index_select(0, ids)
    n, H, D, P = kg.shape
    k = kg.permute(0, 2, 1, 3).reshape(n * P, H, D)   # wrong: D and P axes swapped
    v = vg.permute(0, 2, 1, 3).reshape(n * P, H, D)
    if num_tokens is not None:
        k, v = k[:num_tokens], v[:num_tokens]
    return k.unsqueeze(0), v.unsqueeze(0)


def test_planted_transposed_gather_is_caught(monkeypatch):
    monkeypatch.setattr(OP, "gather_paged_kv", _wrong_gather_transposed)
    seed, n, Hkv, G, D, P, table, kv_len, Sq, mode = CASES[0]
    kp, vp = _pages(seed, n, Hkv, D, P, torch.float64)
    q = torch.randn(1, Sq, Hkv * G, D, dtype=torch.float64)
    out = OP.paged_attention(q, kp, vp, table, P, kv_len, causal=False)
    ref = brute_attention(q[0].numpy(), kp.numpy(), vp.numpy(), table, P, kv_len)
    assert not np.allclose(out[0].numpy(), ref, atol=1e-6)


def test_planted_gqa_head_map_is_caught(monkeypatch):
    real = torch.Tensor.repeat_interleave

    def wrong(self, repeats, dim=None, **kw):  # h % Hkv instead of h // G
        if dim == 1 and isinstance(repeats, int):
            return self.repeat(1, repeats, 1, 1)
        return real(self, repeats, dim=dim, **kw)

    monkeypatch.setattr(torch.Tensor, "repeat_interleave", wrong)
    kp, vp = _pages(1, 7, 2, 8, 3, torch.float64)
    q = torch.randn(1, 1, 8, 8, dtype=torch.float64)
    out = OP.paged_attention(q, kp, vp, [2, 6, 1], 3, 8, causal=False)
    monkeypatch.undo()
    ref = brute_attention(q[0].numpy(), kp.numpy(), vp.numpy(), [2, 6, 1], 3, 8)
    assert not np.allclose(out[0].numpy(), ref, atol=1e-6)


def test_planted_causal_offset_is_caught():
    kp, vp = _pages(2, 9, 2, 8, 16, torch.float64)
    q = torch.randn(1, 4, 2, 8, dtype=torch.float64)
    wrong = OP.paged_attention(q, kp, vp, [8, 3], 16, 20, causal=True, q_start_pos=15)  # off by one
    ref = brute_attention(q[0].numpy(), kp.numpy(), vp.numpy(), [8, 3], 16, 20, 16)
    assert not np.allclose(wrong[0].numpy(), ref, atol=1e-6)


# ---- page -> chunk copy ------------------------------------------------------------------------

def _chunk_by_token_map(pages, ids, L, ppc):
    """The relation the reference's sink round-trip test checks (tests/test_kv_store.py:133-161):
    chunk[layer, :, :, t] == pages[page of token t in that layer, :, :, t % P]."""
    _, H, D, P = pages.shape
    out = torch.zeros(L, H, D, ppc * P, dtype=pages.dtype)
    for layer in range(L):
        for t in range(ppc * P):
            pid = ids[layer * ppc + t // P]
            if pid >= 0:
                out[layer, :, :, t] = pages[pid, :, :, t % P]
    return out


def test_pages_to_chunk_matches_the_token_map():
    g = torch.Generator().manual_seed(8)
    pages = torch.randn(12, 2, 3, 4, generator=g)
    ids = [5, 0, 7, 11, -1, 2]               # 2 layers x 3 pages, one absent
    assert torch.equal(OP.pages_to_chunk(pages, ids, 2, 3), _chunk_by_token_map(pages, ids, 2, 3))
    # planted: page-major instead of layer-major ids
    wrong = [ids[(i % 2) * 3 + i // 2] for i in range(6)]
    assert not torch.equal(OP.pages_to_chunk(pages, wrong, 2, 3),
                           _chunk_by_token_map(pages, ids, 2, 3))


# ---- host-stream attention ---------------------------------------------------------------------

HS_CASES = [  # (seed, total, host_len, chunk, q_len, q_start, causal); the first four are the
              # reference's tests/test_ops.py:488-545 scenarios
    (1, 10, 6, 3, 2, 10, True), (2, 8, 5, 4, 1, 8, True), (3, 8, 4, 2, 2, 5, True),
    (4, 6, 6, 3, 6, 0, True), (5, 9, 7, 3, 2, 4, False), (6, 12, 12, 5, 3, 9, True)]


def _hs_inputs(seed, total, host_len, chunk, q_len, Hkv=2, G=2, D=16):
    g = torch.Generator().manual_seed(seed)
    kf = torch.randn(1, total, Hkv, D, generator=g, dtype=torch.float64)
    vf = torch.randn(1, total, Hkv, D, generator=g, dtype=torch.float64)
    q = torch.randn(1, q_len, Hkv * G, D, generator=g, dtype=torch.float64)
    chunks = [(kf[0, s:min(s + chunk, host_len)].permute(1, 2, 0).contiguous(),
               vf[0, s:min(s + chunk, host_len)].permute(1, 2, 0).contiguous())
              for s in range(0, host_len, chunk)]
    return q, kf, vf, chunks


def _hs_brute(q, kf, vf, q_start, causal):
    """fp64 loops over the contiguous KV as one-token pages."""
    T = kf.shape[1]
    return brute_attention(q[0].numpy(), kf[0].unsqueeze(-1).numpy(), vf[0].unsqueeze(-1).numpy(),
                           list(range(T)), 1, T, q_start if causal else None)


@pytest.mark.parametrize("case", HS_CASES)
def test_host_stream_oracle_vs_brute_force(case):
    seed, total, host_len, chunk, q_len, q_start, causal = case
    q, kf, vf, chunks = _hs_inputs(seed, total, host_len, chunk, q_len)
    out = OP.host_stream_attention(q, chunks, kf[:, host_len:], vf[:, host_len:],
                                   q_start_pos=q_start, causal=causal)
    np.testing.assert_allclose(out[0].numpy(), _hs_brute(q, kf, vf, q_start, causal), atol=1e-10)


def test_planted_host_stream_mistakes_are_caught():
    # the mask cuts inside the host chunks, so their order matters (a softmax over all keys
    # would not see it)
    seed, total, host_len, chunk, q_len, q_start, causal = 7, 10, 8, 3, 2, 2, True
    q, kf, vf, chunks = _hs_inputs(seed, total, host_len, chunk, q_len)
    ref = _hs_brute(q, kf, vf, q_start, causal)
    rk, rv = kf[:, host_len:], vf[:, host_len:]
    newest_first = OP.host_stream_attention(q, chunks[::-1], rk, rv, q_start_pos=q_start)
    assert not np.allclose(newest_first[0].numpy(), ref, atol=1e-6)
    off_by_one = OP.host_stream_attention(q, chunks, rk, rv, q_start_pos=q_start - 1)
    assert not np.allclose(off_by_one[0].numpy(), ref, atol=1e-6)
    # [H, D, C] chunks read as if token-major
    flat = [(k.reshape(k.shape[2], k.shape[0], k.shape[1]).permute(1, 2, 0),
             v.reshape(v.shape[2], v.shape[0], v.shape[1]).permute(1, 2, 0)) for k, v in chunks]
    wrong_layout = OP.host_stream_attention(q, flat, rk, rv, q_start_pos=q_start)
    assert not np.allclose(wrong_layout[0].numpy(), ref, atol=1e-6)
