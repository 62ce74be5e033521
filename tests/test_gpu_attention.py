"""GPU parity of paged attention against the oracle.

Tolerances: bf16 inputs with fp32 accumulation -> max |err| <= 2e-2 against the oracle (the
reference's torch path on the same bf16 inputs); fp32 inputs -> 1e-4 (the reference tests'
tolerance) and 1e-5 against the fp64 brute force.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch
import torch.nn.functional as F

import oracle.paged_kv as OP
import oracle.workloads as W
from plastic_infer.exec.attention import (
    gather_paged_kv,
    host_stream_attention_v1,
    paged_attention_v1,
)
from plastic_infer.kernel import (
    decode_workspace_bytes,
    kv_scatter,
    paged_attention,
    paged_decode_attention,
)
from test_oracle_paged import brute_attention

pytestmark = pytest.mark.gpu

BF16_TOL = 2e-2


def _run_decode_step(wl: W.DecodeWorkload, dev):
    gk, gv = wl.k_pages.to(dev), wl.v_pages.to(dev)
    kv_scatter(wl.k_new.to(dev), wl.v_new.to(dev), gk, gv, wl.slot_mapping.to(dev))
    out = paged_decode_attention(wl.q.to(dev), gk, gv, wl.block_tables.to(dev),
                                 wl.context_lens.to(dev))
    return out.cpu()


def _oracle_decode_step(wl: W.DecodeWorkload, seqs=None):
    kp, vp = wl.k_pages.clone(), wl.v_pages.clone()
    OP.scatter_slots(wl.k_new, wl.v_new, kp, vp, wl.slot_mapping.tolist())
    idx = list(range(wl.q.shape[0])) if seqs is None else seqs
    return OP.decode_batch(wl.q[idx], kp, vp, wl.block_tables[idx], wl.context_lens[idx],
                           wl.page_size)


def test_decode_b32_fast_path(dev):
    wl = W.decode_b32_small()
    got = _run_decode_step(wl, dev)
    ref = _oracle_decode_step(wl)
    err = (got.float() - ref.float()).abs().max().item()
    assert err <= BF16_TOL, err


@pytest.mark.parametrize("G", [1, 2, 4, 8])
def test_decode_group_sizes_and_lengths(dev, G):
    Hkv = 8 if G < 8 else 4
    wl = W.decode_workload(20 + G, 900, 12, 1, 1100, Hkv * G, Hkv, max_len=1200)
    lens = torch.tensor([1, 15, 16, 17, 127, 128, 129, 511, 512, 513, 1024, 1100], dtype=torch.int32)
    wl.context_lens = lens          # edge lengths around page and partition boundaries
    n_pages = (lens + 15) // 16
    perm = torch.randperm(900, generator=torch.Generator().manual_seed(G))
    off = 0
    bt = torch.zeros_like(wl.block_tables)
    for b in range(12):
        bt[b, :n_pages[b]] = perm[off:off + n_pages[b]].to(torch.int32)
        off += int(n_pages[b])
    wl.block_tables = bt
    last = lens.long() - 1
    wl.slot_mapping = bt[torch.arange(12), last // 16].long() * 16 + last % 16
    got = _run_decode_step(wl, dev)
    ref = _oracle_decode_step(wl)
    err = (got.float() - ref.float()).abs().max().item()
    assert err <= BF16_TOL, err


def _decode_case(seed: int, lens: list[int], Hq: int, Hkv: int, num_pages: int):
    """Random pools and tables for the given context lengths (pages drawn without reuse)."""
    g = torch.Generator().manual_seed(seed)
    lens_t = torch.tensor(lens, dtype=torch.int32)
    n_pages = (lens_t + 15) // 16
    max_pages = max(1, int(n_pages.max()))
    perm = torch.randperm(num_pages, generator=g)
    bt = torch.full((len(lens), max_pages), -1, dtype=torch.int32)  # unused entries invalid
    off = 0
    for b, n in enumerate(n_pages.tolist()):
        bt[b, :n] = perm[off:off + n].to(torch.int32)
        off += n
    kp = torch.randn(num_pages, Hkv, 128, 16, generator=g).to(torch.bfloat16)
    vp = torch.randn(num_pages, Hkv, 128, 16, generator=g).to(torch.bfloat16)
    q = torch.randn(len(lens), Hq, 128, generator=g).to(torch.bfloat16)
    return q, kp, vp, bt, lens_t


@pytest.mark.parametrize("G,lens", [
    (4, [8192]),                 # one segment per kv head, cut into one-step wave ranges
    (1, [8191, 3]),
    (2, [0, 4097, 0, 129, 0]),   # empty sequences between and around long ones
    (8, [8192]),                 # GQA 8: one wave per SIMD, eight q rows per partial
    (8, [0, 4097, 0, 129, 0]),
])
def test_decode_stream_few_long_sequences(dev, G, lens):
    """Few long sequences: every segment is split across many waves and merged from partials."""
    Hkv = 8
    q, kp, vp, bt, lens_t = _decode_case(40 + G, lens, Hkv * G, Hkv, 1100)
    out = paged_decode_attention(q.to(dev), kp.to(dev), vp.to(dev), bt.to(dev),
                                 lens_t.to(dev)).cpu()
    live = lens_t > 0
    assert not out[~live].any()
    ref = OP.decode_batch(q[live], kp, vp, bt[live].clamp(min=0), lens_t[live], 16)
    err = (out[live].float() - ref.float()).abs().max().item()
    assert err <= BF16_TOL, err


@pytest.mark.parametrize("Hq", [8, 16])
def test_decode_stream_batch_over_one_launch(dev, Hq):
    """1100 sequences (more than one launch's 1024), a third of them empty, short lengths;
    GQA 4 and 8 over two kv heads."""
    g = torch.Generator().manual_seed(44)
    lens = torch.randint(1, 300, (1100,), generator=g)
    lens[torch.randperm(1100, generator=g)[:370]] = 0
    q, kp, vp, bt, lens_t = _decode_case(45, lens.tolist(), Hq, 2, 14000)
    ws_dev = torch.empty(decode_workspace_bytes(1100, Hq, 2, 128, 16, bt.shape[1]),
                         dtype=torch.uint8, device=dev)
    outs = []
    for _ in range(2):   # the same workspace twice in a row
        outs.append(paged_decode_attention(q.to(dev), kp.to(dev), vp.to(dev), bt.to(dev),
                                           lens_t.to(dev), workspace=ws_dev).cpu())
    assert torch.equal(outs[0], outs[1])
    live = lens_t > 0
    assert not outs[0][~live].any()
    ref = OP.decode_batch(q[live], kp, vp, bt[live].clamp(min=0), lens_t[live], 16)
    err = (outs[0][live].float() - ref.float()).abs().max().item()
    assert err <= BF16_TOL, err


def test_decode_stream_workspace_any_contents(dev):
    """The workspace needs no initialisation: filled with 0xFF bytes or random bytes (so the
    chunk counter holds a value of no launch), the result equals that of a fresh workspace,
    bit for bit, and the oracle's."""
    g = torch.Generator().manual_seed(47)
    lens = torch.randint(1, 2000, (96,), generator=g)
    q, kp, vp, bt, lens_t = _decode_case(48, lens.tolist(), 32, 8, 12000)
    args = (q.to(dev), kp.to(dev), vp.to(dev), bt.to(dev), lens_t.to(dev))
    need = decode_workspace_bytes(96, 32, 8, 128, 16, bt.shape[1])
    base = paged_decode_attention(*args).cpu()
    filled = torch.full((need,), 255, dtype=torch.uint8, device=dev)
    rnd = torch.randint(0, 256, (need,), generator=g, dtype=torch.uint8).to(dev)
    for ws in (filled, rnd, rnd):   # random bytes, then the same buffer again
        assert torch.equal(paged_decode_attention(*args, workspace=ws).cpu(), base)
    ref = OP.decode_batch(q, kp, vp, bt, lens_t, 16)
    err = (base.float() - ref.float()).abs().max().item()
    assert err <= BF16_TOL, err


def test_decode_stream_graph_replays(dev):
    """One decode call captured in a HIP graph (one epoch for every replay): each of several
    replays, with eager calls on the same workspace in between, equals the eager result."""
    g = torch.Generator().manual_seed(49)
    lens = torch.randint(1, 2500, (64,), generator=g)
    q, kp, vp, bt, lens_t = _decode_case(50, lens.tolist(), 32, 8, 12000)
    qd, kd, vd, btd, ld = q.to(dev), kp.to(dev), vp.to(dev), bt.to(dev), lens_t.to(dev)
    ws = torch.empty(decode_workspace_bytes(64, 32, 8, 128, 16, bt.shape[1]), dtype=torch.uint8,
                     device=dev)
    out = torch.empty(64, 32, 128, dtype=torch.bfloat16, device=dev)
    eager = paged_decode_attention(qd, kd, vd, btd, ld, workspace=ws).cpu()
    side = torch.cuda.Stream(dev)
    side.wait_stream(torch.cuda.current_stream(dev))
    with torch.cuda.stream(side):   # warm-up off the capture
        paged_decode_attention(qd, kd, vd, btd, ld, out=out, workspace=ws)
    torch.cuda.current_stream(dev).wait_stream(side)
    torch.cuda.synchronize(dev)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        paged_decode_attention(qd, kd, vd, btd, ld, out=out, workspace=ws)
    for i in range(4):
        out.zero_()
        graph.replay()
        torch.cuda.synchronize(dev)
        assert torch.equal(out.cpu(), eager), f"replay {i}"
        assert torch.equal(paged_decode_attention(qd, kd, vd, btd, ld, workspace=ws).cpu(), eager)


def qwen3_8b_b256_inputs(dev, dtype=torch.bfloat16):
    """The Qwen3-8B decode step at full size: B = 256, L ~ U[512, 8192] including the new token,
    a 160k-page pool, block tables from one seeded permutation (host generator, seed 2), pools,
    new rows and q drawn on the device in `dtype`. Returns (q, kp, vp, bt, lens, n_pages, page,
    offset, slots, k_new, v_new); bt / lens / n_pages / page / offset / slots on the host."""
    B, Hq, Hkv, D, P, N_ = 256, 32, 8, 128, 16, 160_000
    g = torch.Generator().manual_seed(2)
    lens = torch.randint(512, 8193, (B,), generator=g)
    perm = torch.randperm(N_, generator=g)
    n_pages = (lens + P - 1) // P
    bt = torch.zeros(B, 512, dtype=torch.int32)
    off = 0
    for b in range(B):
        bt[b, :n_pages[b]] = perm[off:off + n_pages[b]].to(torch.int32)
        off += int(n_pages[b])
    last = lens - 1
    page = bt[torch.arange(B), last // P].long()
    slots = page * P + last % P
    gd = torch.Generator(device=dev).manual_seed(2)
    kp = torch.empty(N_, Hkv, D, P, dtype=dtype, device=dev)
    vp = torch.empty_like(kp)
    for pool in (kp, vp):
        for s in range(0, N_, 20_000):
            pool[s:s + 20_000] = torch.randn(pool[s:s + 20_000].shape, generator=gd,
                                             device=dev).to(dtype)
    k_new = torch.randn(B, Hkv, D, generator=gd, device=dev).to(dtype)
    v_new = torch.randn(B, Hkv, D, generator=gd, device=dev).to(dtype)
    q = torch.randn(B, Hq, D, generator=gd, device=dev).to(dtype)
    return q, kp, vp, bt, lens, n_pages, page, last % P, slots, k_new, v_new


def oracle_max_err_all_rows(out, q, kp, vp, bt, lens, n_pages, P=16, chunk=64):
    """max |out - oracle| over every row: the oracle's decode over each sequence's own pages
    (gathered from the device pools), `chunk` sequences at a time."""
    dev = kp.device
    B = q.shape[0]
    worst = 0.0
    for b0 in range(0, B, chunk):
        seqs = list(range(b0, min(B, b0 + chunk)))
        ids, tables = [], []
        for b in seqs:
            n = int(n_pages[b])
            tables.append(list(range(len(ids), len(ids) + n)))
            ids += bt[b, :n].tolist()
        sel = torch.tensor(ids, device=dev)
        kl, vl = kp.index_select(0, sel).cpu(), vp.index_select(0, sel).cpu()
        btl = torch.zeros(len(seqs), bt.shape[1], dtype=torch.int32)
        for i, t in enumerate(tables):
            btl[i, :len(t)] = torch.tensor(t, dtype=torch.int32)
        ref = OP.decode_batch(q[seqs].cpu(), kl, vl, btl, lens[seqs], P)
        err = (out[seqs].float() - ref.float()).abs().max().item()
        worst = max(worst, err)
    return worst


def test_decode_qwen3_8b_b256_full_shape(dev):
    """The Qwen3-8B decode step at full size through the two-launch path: the 256-row scatter
    is checked bit for bit over the whole pool (the new rows at their slots, every other
    element unchanged), then the attention of all 256 sequences against the oracle over their
    own pages (2e-2), 64 sequences at a time."""
    q, kp, vp, bt, lens, n_pages, page, offset, slots, k_new, v_new = qwen3_8b_b256_inputs(dev)
    kb, vb = kp.clone(), vp.clone()
    kv_scatter(k_new, v_new, kp, vp, slots.to(dev))
    pg, of = page.to(dev), offset.to(dev)
    kb[pg, :, :, of] = k_new
    vb[pg, :, :, of] = v_new
    assert torch.equal(kp, kb) and torch.equal(vp, vb)
    del kb, vb
    out = paged_decode_attention(q, kp, vp, bt.to(dev), lens.to(torch.int32).to(dev)).cpu()
    worst = oracle_max_err_all_rows(out, q, kp, vp, bt, lens, n_pages)
    assert worst <= BF16_TOL, worst


def test_decode_empty_and_clamped_lengths(dev):
    g = torch.Generator().manual_seed(31)
    kp = torch.randn(8, 2, 128, 16, generator=g).to(torch.bfloat16)
    vp = torch.randn(8, 2, 128, 16, generator=g).to(torch.bfloat16)
    q = torch.randn(3, 4, 128, generator=g).to(torch.bfloat16)
    bt = torch.tensor([[1, 2], [3, 4], [5, 6]], dtype=torch.int32)
    lens = torch.tensor([0, 40, 32], dtype=torch.int32)    # 40 > table capacity 32: clamped
    out = paged_decode_attention(q.to(dev), kp.to(dev), vp.to(dev), bt.to(dev), lens.to(dev)).cpu()
    assert not out[0].any()
    for b in (1, 2):
        ref = OP.paged_attention(q[b][None, None], kp, vp, bt[b].tolist(), 16, 32, causal=False)
        assert (out[b].float() - ref[0, 0].float()).abs().max() <= BF16_TOL


@pytest.mark.parametrize("G", [2, 8])
def test_decode_nonfinite_stale_tokens_are_ignored(dev, G):
    """Tokens past L in the last page may hold NaN/Inf (stale memory): output stays finite.
    G = 2 runs the vector-ALU engine, G = 8 the matrix-core one."""
    g = torch.Generator().manual_seed(32)
    kp = torch.randn(4, 1, 128, 16, generator=g).to(torch.bfloat16)
    vp = torch.randn(4, 1, 128, 16, generator=g).to(torch.bfloat16)
    kp[2, :, :, 5:] = float("nan")
    vp[2, :, :, 5:] = float("inf")
    q = torch.randn(1, G, 128, generator=g).to(torch.bfloat16)
    bt = torch.tensor([[0, 2]], dtype=torch.int32)
    out = paged_decode_attention(q.to(dev), kp.to(dev), vp.to(dev), bt.to(dev),
                                 torch.tensor([21], dtype=torch.int32, device=dev)).cpu()
    ref = OP.paged_attention(q[0][None, None], kp, vp, [0, 2], 16, 21, causal=False)
    assert torch.isfinite(out).all()
    assert (out[0].float() - ref[0, 0].float()).abs().max() <= BF16_TOL


@pytest.mark.parametrize("G", [1, 2, 4, 8])
def test_decode_invalid_table_ids_inside_context(dev, G):
    """Block-table ids outside [0, num_pages) inside a context (-1, num_pages, INT32_MAX, -7):
    those pages' tokens are not keys. Page 0 holds NaN/Inf, so a kernel that read a substitute
    page there would show it. Decode attention is invariant under key order, so the expected
    rows are the oracle's over the table with the invalid pages removed (the partial last page
    stays last, or every kept page is whole). A row with every page invalid is zeros."""
    Hkv, num_pages = 4, 600
    lens = [300, 21, 130, 1000, 16, 64, 257]
    q, kp, vp, bt, lens_t = _decode_case(60 + G, lens, Hkv * G, Hkv, num_pages)
    kp[0] = float("nan")
    vp[0] = float("inf")
    used = set(bt[bt >= 0].tolist())
    bt[bt == 0] = next(p for p in range(1, num_pages) if p not in used)   # no table uses page 0
    bad_vals = [-1, num_pages, 2**31 - 1, -7]
    g = torch.Generator().manual_seed(70 + G)
    n_pages = [(L + 15) // 16 for L in lens]
    for b, n in enumerate(n_pages):
        if b == 4:
            bt[b, :n] = -1                       # every page invalid
            continue
        for i in torch.randperm(n, generator=g)[: max(1, n // 5)].tolist():
            bt[b, i] = bad_vals[(b + i) % len(bad_vals)]
    bt[6, n_pages[6] - 1] = num_pages            # the partial last page (1 token) invalid
    out = paged_decode_attention(q.to(dev), kp.to(dev), vp.to(dev), bt.to(dev),
                                 lens_t.to(dev)).cpu()
    assert torch.isfinite(out.float()).all()
    assert not out[4].any()
    for b, L in enumerate(lens):
        if b == 4:
            continue
        row = bt[b, :n_pages[b]].tolist()
        keep = [(i, p) for i, p in enumerate(row) if 0 <= p < num_pages]
        toks = sum(min(16, L - 16 * i) for i, _ in keep)
        ref = OP.paged_attention(q[b][None, None], kp, vp, [p for _, p in keep], 16, toks,
                                 causal=False)[0, 0]
        err = (out[b].float() - ref.float()).abs().max().item()
        assert err <= BF16_TOL, (b, err)


def _brute_masked(q, kp, vp, table, P, kv_len, offset, num_pages):
    """fp64: row i of q [Sq, H, D] over keys j < kv_len (and j <= offset + i) whose page id is
    inside the pool; no key -> zeros."""
    q, kp, vp = (np.asarray(x, dtype=np.float64) for x in (q, kp, vp))
    Sq, H, D = q.shape
    G = H // kp.shape[1]
    out = np.zeros((Sq, H, D))
    for i in range(Sq):
        lim = kv_len if offset is None else min(kv_len, offset + i + 1)
        js = [j for j in range(lim) if 0 <= table[j // P] < num_pages]
        if not js:
            continue
        for h in range(H):
            ks = np.stack([kp[table[j // P], h // G, :, j % P] for j in js])
            vs = np.stack([vp[table[j // P], h // G, :, j % P] for j in js])
            s = ks @ q[i, h] / np.sqrt(D)
            w = np.exp(s - s.max())
            out[i, h] = (w / w.sum()) @ vs
    return out


@pytest.mark.parametrize("offset", [None, 5])
def test_general_kernel_invalid_table_ids(dev, offset):
    """The general kernel (fp32, head_dim 64, 4-token pages) with ids -1 and num_pages inside
    the context: those keys are skipped, never read through a substitute page (page 0 is
    NaN). The first row under the causal offset sees only an invalid page: zeros."""
    g = torch.Generator().manual_seed(81)
    n, Hkv, G, D, P = 9, 2, 2, 64, 4
    kp = torch.randn(n, Hkv, D, P, generator=g)
    vp = torch.randn(n, Hkv, D, P, generator=g)
    kp[0] = float("nan")
    vp[0] = float("nan")
    table = [-1, 3, 9, 5, -1, 7, 2]
    kv_len, Sq = 26, 4
    q = torch.randn(Sq, Hkv * G, D, generator=g)
    offs = None if offset is None else torch.tensor([offset - 5], dtype=torch.int32, device=dev)
    out = paged_attention(q.to(dev), kp.to(dev), vp.to(dev),
                          torch.tensor([table], dtype=torch.int32, device=dev),
                          torch.tensor([kv_len], dtype=torch.int32, device=dev),
                          cu_q=torch.tensor([0, Sq], dtype=torch.int32, device=dev),
                          q_pos_offsets=offs).cpu()
    ref = _brute_masked(q.numpy(), kp.numpy(), vp.numpy(), table, P, kv_len,
                        None if offset is None else offset - 5, n)
    assert np.isfinite(out.numpy()).all()
    np.testing.assert_allclose(out.double().numpy(), ref, atol=1e-5)


def test_dropin_tables_with_out_of_range_ids_raise(dev):
    """The drop-in wrappers take host lists and raise IndexError for an id outside the pool,
    as the reference's index_select does."""
    kp = torch.zeros(4, 2, 8, 4, device=dev)
    q = torch.zeros(1, 1, 2, 8, device=dev)
    for bad in ([0, 4], [-1], [1, 2, 7]):
        with pytest.raises(IndexError):
            gather_paged_kv(kp, kp, bad, 4)
        with pytest.raises(IndexError):
            paged_attention_v1(q, kp, kp, bad, 4, causal=False)


# ---- general kernel ---------------------------------------------------------------------------

GEN_CASES = [  # (seed, n_pages, Hkv, G, D, P, table, kv_len, Sq, mode)
    (0, 6, 2, 2, 8, 4, [5, 0, 3], 11, 1, "none"),
    (1, 7, 1, 4, 16, 3, [2, 6, 1, 4], 12, 3, "top_left"),
    (2, 9, 2, 1, 64, 16, [8, 3], 20, 4, "offset"),
    (3, 5, 2, 4, 256, 16, [1], 1, 1, "none"),
    (4, 8, 4, 2, 96, 2, [7, 0, 6, 1, 5], 9, 2, "offset"),
    (5, 40, 2, 3, 128, 8, list(range(39, 0, -1)), 300, 5, "offset"),
    # G * head_dim 2304: 16 accumulator pairs per thread, 16-key chunks
    (6, 14, 1, 9, 256, 16, [13, 2, 7, 0, 11, 4, 9, 1, 12, 5], 150, 3, "offset"),
    # head_dim 202 (zero pad columns to 204), 5-token pages: element loads
    (7, 9, 2, 2, 202, 5, [8, 1, 6, 3, 0, 4, 7], 33, 2, "top_left"),
    # G * head_dim 10240, above the tiled kernel's limit: one wave per (row, q head)
    (8, 4, 1, 20, 512, 4, [3, 1, 2], 10, 1, "none"),
]


@pytest.mark.parametrize("case", GEN_CASES)
def test_general_kernel_fp32_vs_brute_force(dev, case):
    seed, n, Hkv, G, D, P, table, kv_len, Sq, mode = case
    g = torch.Generator().manual_seed(seed)
    kp = torch.randn(n, Hkv, D, P, generator=g)
    vp = torch.randn(n, Hkv, D, P, generator=g)
    q = torch.randn(Sq, Hkv * G, D, generator=g)
    q_start = kv_len - Sq if mode == "offset" else 0
    offs = None if mode == "none" else torch.tensor([q_start], dtype=torch.int32, device=dev)
    out = paged_attention(q.to(dev), kp.to(dev), vp.to(dev),
                          torch.tensor([table], dtype=torch.int32, device=dev),
                          torch.tensor([kv_len], dtype=torch.int32, device=dev),
                          cu_q=torch.tensor([0, Sq], dtype=torch.int32, device=dev),
                          q_pos_offsets=offs).cpu()
    ref = brute_attention(q.double().numpy(), kp.double().numpy(), vp.double().numpy(), table, P,
                          kv_len, None if mode == "none" else q_start)
    np.testing.assert_allclose(out.double().numpy(), ref, atol=1e-5)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_general_kernel_half_types_batched(dev, dtype):
    g = torch.Generator().manual_seed(7)
    kp = torch.randn(30, 2, 64, 8, generator=g).to(dtype)
    vp = torch.randn(30, 2, 64, 8, generator=g).to(dtype)
    tables = [[3, 9, 27, 1], [0], [12, 13, 14, 15, 16, 17]]
    kv = [29, 8, 41]
    qlen = [3, 1, 4]
    bt = torch.zeros(3, 6, dtype=torch.int32)
    for b, t in enumerate(tables):
        bt[b, :len(t)] = torch.tensor(t)
    q = torch.randn(sum(qlen), 4, 64, generator=g).to(dtype)
    cu = torch.tensor([0, 3, 4, 8], dtype=torch.int32)
    offs = torch.tensor([kv[b] - qlen[b] for b in range(3)], dtype=torch.int32)
    out = paged_attention(q.to(dev), kp.to(dev), vp.to(dev), bt.to(dev),
                          torch.tensor(kv, dtype=torch.int32, device=dev), cu_q=cu.to(dev),
                          q_pos_offsets=offs.to(dev)).cpu()
    for b in range(3):
        rows = q[cu[b]:cu[b + 1]]
        ref = OP.paged_attention(rows[None], kp, vp, tables[b], 8, kv[b], causal=True,
                                 q_start_pos=int(offs[b]))
        assert (out[cu[b]:cu[b + 1]].float() - ref[0].float()).abs().max() <= BF16_TOL


# ---- drop-in API (the reference's tests/test_ops.py scenarios on the device) -----------------

def test_dropin_gather_paged_kv(dev):
    torch.manual_seed(1)
    kp = torch.randn(5, 2, 4, 8)
    vp = torch.randn(5, 2, 4, 8)
    k, v = gather_paged_kv(kp.to(dev), vp.to(dev), [0, 2, 4], 8)
    rk, rv = OP.gather_paged_kv(kp, vp, [0, 2, 4], 8)
    assert torch.equal(k.cpu(), rk) and torch.equal(v.cpu(), rv)
    k, _ = gather_paged_kv(kp.to(dev), vp.to(dev), [0, 1], 8, num_tokens=11)
    assert k.shape == (1, 11, 2, 4)
    k, v = gather_paged_kv(kp.to(dev), vp.to(dev), [], 8)
    assert k.shape == (1, 0, 2, 4) and v.shape == (1, 0, 2, 4)


def test_dropin_paged_attention_v1(dev):
    torch.manual_seed(7)
    q = torch.randn(1, 8, 4, 16) * 0.1
    kc = torch.randn(1, 12, 2, 16) * 0.1
    vc = torch.randn(1, 12, 2, 16) * 0.1
    kp = kc[0].view(3, 4, 2, 16).permute(0, 2, 3, 1).contiguous()
    vp = vc[0].view(3, 4, 2, 16).permute(0, 2, 3, 1).contiguous()
    out = paged_attention_v1(q.to(dev), kp.to(dev), vp.to(dev), [0, 1, 2], 4, 12, causal=True)
    ref = F.scaled_dot_product_attention(
        q.transpose(1, 2), kc.transpose(1, 2).repeat_interleave(2, 1),
        vc.transpose(1, 2).repeat_interleave(2, 1), is_causal=True).transpose(1, 2)
    assert torch.allclose(out.cpu(), ref, atol=1e-4)
    one = paged_attention_v1(q[:, :1].to(dev), kp.to(dev), vp.to(dev), [0, 1, 2], 4, 12,
                             causal=True)
    assert one.shape == (1, 1, 4, 16) and torch.isfinite(one).all()
    dec = paged_attention_v1(q[:, :1].to(dev), kp.to(dev), vp.to(dev), [2, 0], 4, 7,
                             causal=False)
    refd = OP.paged_attention(q[:, :1], kp, vp, [2, 0], 4, 7, causal=False)
    assert torch.allclose(dec.cpu(), refd, atol=1e-5)


@pytest.mark.parametrize("seed,total,host_len,chunk,q_len,q_start", [
    (1, 10, 6, 3, 2, 10), (2, 8, 5, 4, 1, 8), (3, 8, 4, 2, 2, 5), (4, 6, 6, 3, 6, 0)])
def test_dropin_host_stream_attention(dev, seed, total, host_len, chunk, q_len, q_start):
    torch.manual_seed(seed)
    kf = torch.randn(1, total, 2, 16) * 0.1
    vf = torch.randn(1, total, 2, 16) * 0.1
    chunks = []
    for s in range(0, host_len, chunk):
        e = min(s + chunk, host_len)
        chunks.append((kf[0, s:e].permute(1, 2, 0).contiguous(), vf[0, s:e].permute(1, 2, 0).contiguous()))
    rk, rv = kf[:, host_len:], vf[:, host_len:]
    if host_len == total:
        chunks, rk, rv = [], kf, vf
    q = torch.randn(1, q_len, 4, 16) * 0.1
    out = host_stream_attention_v1(q.to(dev), chunks, rk.to(dev), rv.to(dev), q_start_pos=q_start)
    ref = OP.host_stream_attention(q, chunks, rk, rv, q_start_pos=q_start)
    assert torch.allclose(out.cpu(), ref, atol=1e-4)


def test_rejects_host_tensors():
    with pytest.raises(ValueError):
        paged_decode_attention(torch.zeros(1, 2, 128), torch.zeros(2, 1, 128, 16),
                               torch.zeros(2, 1, 128, 16), torch.zeros(1, 1, dtype=torch.int32),
                               torch.ones(1, dtype=torch.int32))


def _hs_split(total, host_len, chunk, Hkv, D, dtype, seed, where):
    g = torch.Generator().manual_seed(seed)
    kf = (torch.randn(1, total, Hkv, D, generator=g) * 0.5).to(dtype)
    vf = torch.randn(1, total, Hkv, D, generator=g).to(dtype)
    chunks = []
    for s in range(0, host_len, chunk):
        e = min(s + chunk, host_len)
        k_c = kf[0, s:e].permute(1, 2, 0).contiguous()
        v_c = vf[0, s:e].permute(1, 2, 0).contiguous()
        if where == "pinned":
            k_c, v_c = k_c.pin_memory(), v_c.pin_memory()
        elif where == "device":
            k_c, v_c = k_c.cuda(), v_c.cuda()
        chunks.append((k_c, v_c))
    return kf, vf, chunks


@pytest.mark.parametrize("where", ["pinned", "device", "pageable"])
@pytest.mark.parametrize("dtype,Hq,Hkv,D", [(torch.bfloat16, 32, 8, 128),
                                            (torch.float16, 8, 2, 256),
                                            (torch.float32, 16, 4, 64),
                                            (torch.float32, 8, 2, 256),
                                            (torch.float32, 4, 4, 160)])
@pytest.mark.parametrize("q_len,causal", [(1, True), (4, True), (3, False), (20, True)])
def test_host_stream_attention_shapes(dev, where, dtype, Hq, Hkv, D, q_len, causal):
    """Chunks of 256 tokens with a ragged 100-token last chunk and a 37-token device tail;
    q rows at the end of the KV (decode / a few appended tokens), in the middle (non-causal), and
    enough rows (20 x G) that the chunks are staged to HBM instead of streamed."""
    host_len, chunk, tail = 5 * 256 + 100, 256, 37
    total = host_len + tail
    kf, vf, chunks = _hs_split(total, host_len, chunk, Hkv, D, dtype, 31 + q_len, where)
    g = torch.Generator().manual_seed(7)
    q = torch.randn(1, q_len, Hq, D, generator=g).to(dtype)
    q_start = total - q_len if causal else 500
    rk, rv = kf[:, host_len:].to(dev), vf[:, host_len:].to(dev)
    out = host_stream_attention_v1(q.to(dev), chunks, rk, rv, q_start_pos=q_start,
                                   causal=causal)
    f32 = [(k.float().cpu(), v.float().cpu()) for k, v in chunks]
    ref = OP.host_stream_attention(q.float(), f32, kf[:, host_len:].float(),
                                   vf[:, host_len:].float(), q_start_pos=q_start, causal=causal)
    tol = 1e-4 if dtype == torch.float32 else 2e-2
    err = (out.float().cpu() - ref).abs().max().item()
    assert err <= tol, err


def test_host_stream_attention_long_pinned_decode(dev):
    """8192 host tokens (32 pinned chunks) + 300 resident: several tiles per split."""
    Hq, Hkv, D = 32, 8, 128
    host_len, tail = 8192, 300
    kf, vf, chunks = _hs_split(host_len + tail, host_len, 256, Hkv, D, torch.bfloat16, 5,
                               "pinned")
    q = torch.randn(1, 1, Hq, D).to(torch.bfloat16)
    rk, rv = kf[:, host_len:].to(dev), vf[:, host_len:].to(dev)
    out = host_stream_attention_v1(q.to(dev), chunks, rk, rv, q_start_pos=host_len + tail)
    f32 = [(k.float(), v.float()) for k, v in chunks]
    ref = OP.host_stream_attention(q.float(), f32, kf[:, host_len:].float(),
                                   vf[:, host_len:].float(), q_start_pos=host_len + tail)
    assert (out.float().cpu() - ref).abs().max().item() <= 2e-2


def test_host_stream_attention_edge_cases(dev):
    Hq, Hkv, D = 4, 2, 16
    kf, vf, chunks = _hs_split(30, 20, 8, Hkv, D, torch.float32, 9, "pinned")
    q = torch.randn(1, 2, Hq, D)
    # resident tail given as a strided view: rows of a wider [T, 2*Hkv, D] buffer
    wide_k = torch.zeros(10, 2 * Hkv, D)
    wide_v = torch.zeros(10, 2 * Hkv, D)
    wide_k[:, :Hkv] = kf[0, 20:]
    wide_v[:, :Hkv] = vf[0, 20:]
    rk = wide_k.to(dev)[:, :Hkv].unsqueeze(0)
    rv = wide_v.to(dev)[:, :Hkv].unsqueeze(0)
    out = host_stream_attention_v1(q.to(dev), chunks, rk, rv, q_start_pos=28)
    ref = OP.host_stream_attention(q, chunks, kf[:, 20:], vf[:, 20:], q_start_pos=28)
    assert torch.allclose(out.cpu(), ref, atol=1e-4)
    # chunks of unequal lengths (not C, ..., C, last <= C): laid out as a device tail
    odd = [(kf[0, 0:5].permute(1, 2, 0).contiguous(), vf[0, 0:5].permute(1, 2, 0).contiguous()),
           (kf[0, 5:20].permute(1, 2, 0).contiguous(), vf[0, 5:20].permute(1, 2, 0).contiguous())]
    out = host_stream_attention_v1(q.to(dev), odd, kf[:, 20:].to(dev), vf[:, 20:].to(dev),
                                   q_start_pos=28)
    assert torch.allclose(out.cpu(), ref, atol=1e-4)
    # causal rows that see only a prefix of the host chunks (keys past q_start + q_len dropped)
    out = host_stream_attention_v1(q.to(dev), chunks, kf[:, 20:].to(dev), vf[:, 20:].to(dev),
                                   q_start_pos=3)
    ref = OP.host_stream_attention(q, chunks, kf[:, 20:], vf[:, 20:], q_start_pos=3)
    assert torch.allclose(out.cpu(), ref, atol=1e-4)
    # no keys at all: zeros (the reference's SDPA over an empty KV has no defined output)
    empty = torch.zeros(1, 0, Hkv, D, device=dev)
    out = host_stream_attention_v1(q.to(dev), [], empty, empty, q_start_pos=0)
    assert out.shape == (1, 2, Hq, D) and not out.any()
    # mismatched dtypes are rejected
    with pytest.raises(ValueError):
        host_stream_attention_v1(q.to(dev), [(c[0].half(), c[1].half()) for c in chunks],
                                 kf[:, 20:].to(dev), vf[:, 20:].to(dev), q_start_pos=28)
