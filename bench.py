#!/usr/bin/env python3
"""Benchmark of the paged-KV decode hot path on one MI355X.

Workload (Qwen3-8B-shaped decode, one layer): 32 query heads, 8 KV heads, head_dim 128, bf16,
page size 16; batch 256 with context lengths ~ U[512, 8192] (including the new token); block
tables are consecutive slices of one seeded permutation of a 160,000-page pool; K, V, q and the
new K/V rows ~ N(0,1). One step = the write of the 256 new K/V rows into their slots + paged
GQA decode attention over every sequence (new token included), as one call
(paged_decode_append_attention: the attention kernel takes each new token from k_new / v_new
and stores it into its slot). --separate-write runs the same step as two calls (kv_scatter,
then paged_decode_attention). Inputs are resident in HBM before timing starts.

Prints ONE JSON line with the whole-job throughput (algorithmic GB/s of a step), tokens/s,
the roofline of the dominant kernel (attention: algorithmic bytes / average duration measured
with HIP events on the launch stream) and the CPU baseline (the oracle's restatement of the
reference torch path on this host's cores, on a bounded sample of the same inputs).

  python bench.py [--steps K] [--warmup W] [--gpus 1] [--cpu-sample-seqs S] [--no-cpu-baseline]
                  [--separate-write] [--dtype bf16|fp16|fp32]
                  # fp16: the same step on fp16 pools (the same kernel); fp32: on fp32 pools,
                  # which the general tiled kernel serves (write and attention as two calls)
  python bench.py --calibrate-copy     # 1 GiB read + 1 GiB write elementwise copy, three times:
                                       # the known-size reference for HBM byte counters
  python bench.py --workload decode-gqa8     # Qwen3-30B-A3B attention layer: 64 x 4096 tokens,
                                             # 32 q / 4 kv heads (GQA 8)
  python bench.py --workload prefill-write   # ragged chunked-prefill KV write + gather back
                                             # (8 sequences, S ~ U[256, 4096], seed 3)
  python bench.py --workload moe-permute     # Qwen3-30B-A3B routing: top-8 of 128 experts,
                                             # permute, identity expert, weighted unpermute
                                             # (4096 tokens, hidden 2048, seed 4)
  python bench.py --workload expert-stream   # Qwen3-30B-A3B routed experts of a decode step:
                                             # 48 layers of pinned banks (54 GiB), 3072 HBM
                                             # slots, LRU, expert FFN on the slots
  python bench.py --workload moe-experts     # Qwen3-30B-A3B routed expert FFN, one layer,
                                             # 64 decode tokens, 128 resident experts top-8
  python bench.py --workload moe-experts-prefill   # the same FFN over 4096 prefill tokens
  python bench.py --workload prefill-stream  # Qwen3-30B-A3B prefill of 4096 tokens through the
                                             # expert double buffer, 48 layers of pinned banks
  python bench.py --workload prefill-attn    # chunked-prefill paged attention (matrix cores):
                                             # 8 x 1024-token chunks after 3072 context tokens
  python bench.py --workload hbm-read        # the streaming-read rate of the box (fixed cost +
                                             # rate over 26 MB .. 3.4 GB): the practical ceiling
The default workload (decode) is the headline; the others print their own JSON line.
"""

from __future__ import annotations

import argparse
import json
import os
import pathlib
import statistics
import sys
import time

ROOT = pathlib.Path(__file__).resolve().parent
for _p in (ROOT, ROOT / "plastic-infer_amd"):
    if str(_p) not in sys.path:
        sys.path.insert(0, str(_p))

HBM_PEAK_GBPS = 8000.0
B, HQ, HKV, D, P, NUM_PAGES = 256, 32, 8, 128, 16, 160_000
LEN_LO, LEN_HI, SEED = 512, 8192, 2
MAX_PAGES = LEN_HI // P
WORKLOAD = "qwen3-8b paged decode: kv scatter + gqa paged attention, 1 layer"
PMC_FILE = ROOT / "profiles" / "paged_decode_qwen3_8b_b256_pmc.json"
PMC_FP16_FILE = ROOT / "profiles" / "paged_decode_qwen3_8b_b256_fp16_pmc.json"
PMC_FP32_FILE = ROOT / "profiles" / "paged_attention_tiled_qwen3_8b_b256_fp32_pmc.json"
GQA8_PMC_FILE = ROOT / "profiles" / "paged_decode_gqa8_qwen3_30b_b64_pmc.json"


def build_inputs(torch, dev, dtype=None):
    dtype = dtype or torch.bfloat16
    g = torch.Generator().manual_seed(SEED)
    lens = torch.randint(LEN_LO, LEN_HI + 1, (B,), generator=g)
    perm = torch.randperm(NUM_PAGES, generator=g)
    n_pages = (lens + P - 1) // P
    bt = torch.zeros(B, MAX_PAGES, dtype=torch.int32)
    off = 0
    for b in range(B):
        n = int(n_pages[b])
        bt[b, :n] = perm[off:off + n].to(torch.int32)
        off += n
    last = lens - 1
    slots = bt[torch.arange(B), last // P].to(torch.int64) * P + last % P
    gd = torch.Generator(device=dev).manual_seed(SEED)
    kp = torch.empty(NUM_PAGES, HKV, D, P, dtype=dtype, device=dev)
    vp = torch.empty_like(kp)
    step = 20_000
    for pool in (kp, vp):
        for s in range(0, NUM_PAGES, step):
            pool[s:s + step] = torch.randn(pool[s:s + step].shape, generator=gd,
                                           device=dev).to(dtype)
    k_new = torch.randn(B, HKV, D, generator=gd, device=dev).to(dtype)
    v_new = torch.randn(B, HKV, D, generator=gd, device=dev).to(dtype)
    q = torch.randn(B, HQ, D, generator=gd, device=dev).to(dtype)
    return dict(lens=lens, n_pages=n_pages, bt=bt, slots=slots, kp=kp, vp=vp, k_new=k_new,
                v_new=v_new, q=q, bt_d=bt.to(dev), lens_d=lens.to(torch.int32).to(dev),
                slots_d=slots.to(dev))


def algorithmic_bytes(lens, n_pages, seqs=None, elem=2):
    """Bytes a step must move at minimum: K+V of every context token, q in, out, the block
    table entries and lengths read, and the scatter (new rows read + written, slots); elem is
    the storage type's size in bytes."""
    idx = range(len(lens)) if seqs is None else seqs
    tok = sum(int(lens[b]) for b in idx)
    pages = sum(int(n_pages[b]) for b in idx)
    nb = len(list(idx))
    kv_row = 2 * HKV * D * elem                    # K + V bytes of one token, one layer
    attn = tok * kv_row + nb * HQ * D * elem * 2 + pages * 4 + nb * 4
    scatter = nb * kv_row * 2 + nb * 8
    return attn, scatter


def cpu_info():
    model, phys = "unknown", set()
    try:
        cur = {}
        for line in open("/proc/cpuinfo"):
            if ":" not in line:
                if "physical id" in cur and "core id" in cur:
                    phys.add((cur["physical id"], cur["core id"]))
                cur = {}
                continue
            k, v = (s.strip() for s in line.split(":", 1))
            cur[k] = v
            if k == "model name":
                model = v
    except OSError:
        pass
    return model, len(phys) or None


def cpu_baseline(torch, inp, n_seqs, gpu_out):
    """The oracle (CPU restatement of the reference torch path: per-token index store, then per
    sequence index_select gather + repeat_interleave + SDPA) on the first n_seqs sequences of
    the same inputs, copied from the device. 1 warm-up, median of 3. The warm-up's output is
    also the parity check of the timed GPU step: gpu_out [B, Hq, D] (the attention output after
    the same scatter) must agree on the sampled sequences within 2e-2 (the bf16 bar)."""
    import oracle.paged_kv as OP

    threads = len(os.sched_getaffinity(0))
    torch.set_num_threads(threads)
    seqs = list(range(min(n_seqs, B)))
    # compact host pool holding only the sample's pages, renumbered 0..n-1
    tables, ids = [], []
    for b in seqs:
        n = int(inp["n_pages"][b])
        tables.append(list(range(len(ids), len(ids) + n)))
        ids.extend(inp["bt"][b, :n].tolist())
    dev_ids = torch.tensor(ids, device=inp["kp"].device)
    kp = inp["kp"].index_select(0, dev_ids).cpu()
    vp = inp["vp"].index_select(0, dev_ids).cpu()
    bt = torch.zeros(len(seqs), MAX_PAGES, dtype=torch.int32)
    for i, t in enumerate(tables):
        bt[i, :len(t)] = torch.tensor(t, dtype=torch.int32)
    lens = inp["lens"][seqs].to(torch.int32)
    last = lens.long() - 1
    slots = bt[torch.arange(len(seqs)), last // P].long() * P + last % P
    k_new, v_new = inp["k_new"][seqs].cpu(), inp["v_new"][seqs].cpu()
    q = inp["q"][seqs].cpu()

    def step():
        OP.scatter_slots(k_new, v_new, kp, vp, slots.tolist())
        return OP.decode_batch(q, kp, vp, bt, lens, P)

    ref = step()
    max_err = (gpu_out[seqs].float().cpu() - ref.float()).abs().max().item()
    if not max_err <= 2e-2:
        raise AssertionError(f"bench parity: GPU decode output differs from the oracle on the "
                             f"sampled sequences, max |err| {max_err:.3e} > 2e-2")
    times = []
    for _ in range(3):
        t0 = time.perf_counter()
        step()
        times.append(time.perf_counter() - t0)
    t = statistics.median(times)
    attn, sc = algorithmic_bytes(inp["lens"], inp["n_pages"], seqs, inp["kp"].element_size())
    model, phys = cpu_info()
    return {
        "value": round((attn + sc) / t / 1e9, 3), "unit": "GB/s", "cores": threads,
        "kind": "port",
        "sample": f"first {len(seqs)} of {B} sequences of the same step (same input bits), "
                  f"1 warm-up + median of 3, {t * 1e3:.1f} ms per sample step",
        "tokens_per_s": round(len(seqs) / t, 2), "cpu_model": model, "physical_cores": phys,
        "parity_max_abs_err": max_err, "parity_seqs": len(seqs),
    }


def _phase_timer(torch, dev, step, n_phases, steps, warmup):
    """Runs step(events) warmup + steps + steps times. The first timed region records no event
    inside it (event records are queue packets that cost a few microseconds each, as much as a
    short kernel's gaps); the second records n_phases + 1 events per step on the launch stream
    for the split. Returns (ms per step over the first region, mean ms of each phase over the
    second, wall s of the first)."""
    stream = torch.cuda.current_stream(dev)
    for _ in range(warmup):
        step(None)
    torch.cuda.synchronize(dev)
    t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    wall0 = time.perf_counter()
    t0.record(stream)
    for _ in range(steps):
        step(None)
    t1.record(stream)
    torch.cuda.synchronize(dev)
    wall = time.perf_counter() - wall0
    evs = [[torch.cuda.Event(enable_timing=True) for _ in range(n_phases + 1)]
           for _ in range(steps)]
    for i in range(steps):
        step(evs[i])
    torch.cuda.synchronize(dev)
    phases = [statistics.mean(e[j].elapsed_time(e[j + 1]) for e in evs) for j in range(n_phases)]
    return t0.elapsed_time(t1) / steps, phases, wall


def _result(metric, value, unit, args, ms, dtype, config, extra, roofline, cpu=None):
    r = {"metric": metric, "value": round(value, 2), "unit": unit, "n_gpus": 1,
         "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms, 4),
         "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": dtype,
         "data": "synthetic (seeded)", "config": config}
    r.update(extra)
    r["roofline"] = roofline
    if cpu is not None:
        r["cpu_baseline"] = cpu
    return r


PF_B, PF_LO, PF_HI, PF_SEED, PF_SPARE = 8, 256, 4096, 3, 1024


def bench_prefill_write(torch, dev, args) -> dict:
    """Ragged chunked-prefill KV write: packed [sum S, 8, 128] bf16 rows of 8 sequences with
    S ~ U[256, 4096] scattered into a seeded random page allocation (partial last pages), then
    gathered back. One step = kv_scatter + kv_gather; both bit-exact (checked once here)."""
    from plastic_infer.kernel import kv_gather, kv_scatter

    g = torch.Generator().manual_seed(PF_SEED)
    lens = torch.randint(PF_LO, PF_HI + 1, (PF_B,), generator=g)
    n_pages = (lens + P - 1) // P
    num_pages = int(n_pages.sum()) + PF_SPARE
    perm = torch.randperm(num_pages, generator=g)
    max_pages = (PF_HI + P - 1) // P
    bt = torch.zeros(PF_B, max_pages, dtype=torch.int32)
    slots, off = [], 0
    for b in range(PF_B):
        n = int(n_pages[b])
        bt[b, :n] = perm[off:off + n].to(torch.int32)
        off += n
        pos = torch.arange(int(lens[b]))
        slots.append(bt[b, pos // P].to(torch.int64) * P + pos % P)
    total = int(lens.sum())
    k = torch.randn(total, HKV, D, generator=g).to(torch.bfloat16).to(dev)
    v = torch.randn(total, HKV, D, generator=g).to(torch.bfloat16).to(dev)
    cu = torch.zeros(PF_B + 1, dtype=torch.int64)
    cu[1:] = torch.cumsum(lens, 0)
    slots_d, bt_d, cu_d = torch.cat(slots).to(dev), bt.to(dev), cu.to(dev)
    kp = torch.zeros(num_pages, HKV, D, P, dtype=torch.bfloat16, device=dev)
    vp = torch.zeros_like(kp)
    kb, vb = torch.empty_like(k), torch.empty_like(v)

    def step(ev):
        if ev:
            ev[0].record()
        kv_scatter(k, v, kp, vp, slots_d)
        if ev:
            ev[1].record()
        kv_gather(kp, vp, bt_d, cu_d, PF_HI, out=(kb, vb))
        if ev:
            ev[2].record()

    ms, (sc_ms, ga_ms), wall = _phase_timer(torch, dev, step, 2, args.steps, args.warmup)
    if not (torch.equal(kb, k) and torch.equal(vb, v)):
        raise RuntimeError("prefill write: gather-back differs from the written rows")
    row = HKV * D * 2                                   # one token's K (or V) bytes
    scatter_bytes = total * row * 2 * 2 + total * 8     # K+V read and written, slots
    gather_bytes = total * row * 2 * 2 + int(n_pages.sum()) * 4 + (PF_B + 1) * 8
    step_bytes = scatter_bytes + gather_bytes
    dom, dom_bytes, dom_ms = (("kv_scatter16_kernel", scatter_bytes, sc_ms) if sc_ms >= ga_ms
                              else ("kv_gather16_kernel", gather_bytes, ga_ms))
    cpu = None
    if not args.no_cpu_baseline:
        cpu = _cpu_prefill_write(torch, k, v, slots, num_pages, total, scatter_bytes)
    gbps = step_bytes / (ms / 1e3) / 1e9
    return _result(
        "ragged prefill KV write + gather-back GB/s", gbps, "GB/s", args, ms, "bf16",
        {"workload": "ragged chunked-prefill kv write (8 seqs, S~U[256,4096], 8 kv heads x "
                     "128, page 16) + gather back", "tokens": total, "pool_pages": num_pages},
        {"tokens_per_s": round(total / (ms / 1e3), 1), "hbm_frac": round(gbps / HBM_PEAK_GBPS, 4),
         "bytes_per_step": step_bytes, "scatter_ms": round(sc_ms, 4), "gather_ms": round(ga_ms, 4),
         "wall_s_timed": round(wall, 4)},
        {"kernel": dom, "bound": "hbm", "achieved": round(dom_bytes / (dom_ms / 1e3) / 1e9, 2),
         "peak": HBM_PEAK_GBPS, "unit": "GB/s",
         "frac": round(dom_bytes / (dom_ms / 1e3) / 1e9 / HBM_PEAK_GBPS, 4), "traffic": None,
         "algorithmic_bytes_per_launch": dom_bytes, "avg_launch_ms": round(dom_ms, 4)},
        cpu)


def _cpu_prefill_write(torch, k, v, slots, num_pages, total, scatter_bytes) -> dict:
    """The oracle's per-token advanced-index store (the reference's _write_kv_layer loop) on
    the first 2048 tokens of the same rows, 1 warm-up + median of 3; scaled per byte."""
    import oracle.paged_kv as OP

    threads = len(os.sched_getaffinity(0))
    torch.set_num_threads(threads)
    n = min(2048, total)
    kc, vc = k[:n].cpu(), v[:n].cpu()
    sl = torch.cat(slots)[:n].tolist()
    kp = torch.zeros(num_pages, HKV, D, P, dtype=torch.bfloat16)
    vp = torch.zeros_like(kp)
    OP.scatter_slots(kc, vc, kp, vp, sl)
    times = []
    for _ in range(3):
        t0 = time.perf_counter()
        OP.scatter_slots(kc, vc, kp, vp, sl)
        times.append(time.perf_counter() - t0)
    t = statistics.median(times)
    model, phys = cpu_info()
    return {"value": round(scatter_bytes * n / total / t / 1e9, 3), "unit": "GB/s",
            "cores": threads, "kind": "port",
            "sample": f"scatter of the first {n} of {total} tokens (same rows and slots), "
                      f"1 warm-up + median of 3, {t * 1e3:.1f} ms",
            "cpu_model": model, "physical_cores": phys}


MOE_T, MOE_H, MOE_E, MOE_K, MOE_BS, MOE_SEED = 4096, 2048, 128, 8, 64, 4


def bench_moe_permute(torch, dev, args) -> dict:
    """Qwen3-30B-A3B MoE routing and permutation: router logits [4096, 128] fp32 N(0,1) ->
    softmax top-8 renormalised -> align (block 64) -> permute hidden [4096, 2048] bf16 into
    expert-contiguous rows -> identity expert -> weighted unpermute."""
    from plastic_infer.kernel import moe_permute, moe_topk_align, moe_unpermute

    g = torch.Generator().manual_seed(MOE_SEED)
    hidden = torch.randn(MOE_T, MOE_H, generator=g).to(torch.bfloat16).to(dev)
    logits = torch.randn(MOE_T, MOE_E, generator=g, dtype=torch.float32).to(dev)
    state = {}

    def step(ev):
        if ev:
            ev[0].record()
        w, ids, s, e, npp, pos = moe_topk_align(logits, MOE_K, MOE_BS)
        if ev:
            ev[1].record()
        xp = moe_permute(hidden, s, npp, MOE_K, route_pos=pos)
        if ev:
            ev[2].record()
        out = moe_unpermute(xp, pos, w, MOE_T, MOE_K)
        if ev:
            ev[3].record()
        state["out"], state["w"] = out, w

    ms, (route_ms, perm_ms, comb_ms), wall = _phase_timer(torch, dev, step, 3, args.steps,
                                                          args.warmup)
    closed = (hidden.double() * state["w"].double().sum(1, keepdim=True)).to(torch.bfloat16)
    if (state["out"].float() - closed.float()).abs().max().item() > 2e-2:
        raise RuntimeError("moe permute: identity-expert round trip is off")
    T, H, K, E = MOE_T, MOE_H, MOE_K, MOE_E
    route_bytes = T * E * 4 + T * K * 8
    perm_bytes = T * H * 2 + T * K * H * 2 + T * K * 4
    comb_bytes = T * K * H * 2 + T * H * 2 + T * K * 4 + T * K * 4
    step_bytes = route_bytes + perm_bytes + comb_bytes
    phases = [("moe_topk_hist + moe_align_place", route_bytes, route_ms),
              ("moe_permute_tokens_kernel", perm_bytes, perm_ms),
              ("moe_combine_kernel", comb_bytes, comb_ms)]
    dom, dom_bytes, dom_ms = max(phases, key=lambda x: x[2])
    cpu = None
    if not args.no_cpu_baseline:
        cpu = _cpu_moe(torch, hidden, logits, perm_bytes + comb_bytes + route_bytes)
    gbps = step_bytes / (ms / 1e3) / 1e9
    return _result(
        "MoE route + permute + unpermute GB/s", gbps, "GB/s", args, ms, "bf16",
        {"workload": "qwen3-30b-a3b moe routing/permute (4096 tokens, hidden 2048, 128 experts "
                     "top-8, identity expert)", "tokens": T, "hidden": H, "experts": E, "topk": K},
        {"tokens_per_s": round(T / (ms / 1e3), 1), "hbm_frac": round(gbps / HBM_PEAK_GBPS, 4),
         "bytes_per_step": step_bytes, "route_ms": round(route_ms, 4),
         "permute_ms": round(perm_ms, 4), "combine_ms": round(comb_ms, 4),
         "wall_s_timed": round(wall, 4)},
        {"kernel": dom, "bound": "hbm", "achieved": round(dom_bytes / (dom_ms / 1e3) / 1e9, 2),
         "peak": HBM_PEAK_GBPS, "unit": "GB/s",
         "frac": round(dom_bytes / (dom_ms / 1e3) / 1e9 / HBM_PEAK_GBPS, 4), "traffic": None,
         "algorithmic_bytes_per_launch": dom_bytes, "avg_launch_ms": round(dom_ms, 4)},
        cpu)


def _cpu_moe(torch, hidden, logits, step_bytes) -> dict:
    """The oracle's restatement (softmax top-k, stable align, row gather, sequential fp32
    combine) on the first 512 of the 4096 tokens, 1 warm-up + median of 3; scaled per token."""
    import oracle.moe_route as OM

    threads = len(os.sched_getaffinity(0))
    torch.set_num_threads(threads)
    n = 512
    h, lg = hidden[:n].cpu(), logits[:n].cpu()

    def run():
        w, ids = OM.fused_topk(lg, MOE_K, True)
        s, _, npp, pos = OM.moe_align_block_size(ids.numpy(), MOE_BS, MOE_E)
        xp = OM.permute(h, s, npp, MOE_K)
        OM.unpermute(xp, pos, w.numpy(), n, MOE_K, torch.bfloat16)

    run()
    times = []
    for _ in range(3):
        t0 = time.perf_counter()
        run()
        times.append(time.perf_counter() - t0)
    t = statistics.median(times)
    model, phys = cpu_info()
    return {"value": round(step_bytes * n / MOE_T / t / 1e9, 3), "unit": "GB/s",
            "cores": threads, "kind": "port",
            "sample": f"first {n} of {MOE_T} tokens (same inputs), 1 warm-up + median of 3, "
                      f"{t * 1e3:.1f} ms", "cpu_model": model, "physical_cores": phys}


def bench_decode_gqa8(torch, dev, args) -> dict:
    """Qwen3-30B-A3B attention layer at its decode shape: 32 q heads over 4 kv heads (GQA 8),
    head_dim 128, bf16, page 16; 64 sequences of 4096 tokens in a seeded random page
    permutation of a 20,000-page pool. One step = the decode step's write of the 64 new rows
    and the paged decode attention, as one paged_decode_append_attention call (the call the
    paged MoE decoder makes per layer; --separate-write: kv_scatter, then
    paged_decode_attention)."""
    from plastic_infer.kernel import (decode_workspace_bytes, kv_scatter,
                                      paged_decode_append_attention, paged_decode_attention)

    b, hq, hkv, L, npool = 64, 32, 4, 4096, 20_000
    g = torch.Generator().manual_seed(6)
    lens = torch.full((b,), L, dtype=torch.int64)
    n_pages = (lens + P - 1) // P
    perm = torch.randperm(npool, generator=g)
    bt = perm[: b * int(n_pages[0])].view(b, -1).to(torch.int32)
    last = lens - 1
    slots = bt[torch.arange(b), last // P].to(torch.int64) * P + last % P
    gd = torch.Generator(device=dev).manual_seed(6)
    kp = torch.randn(npool, hkv, D, P, generator=gd, device=dev).to(torch.bfloat16)
    vp = torch.randn(npool, hkv, D, P, generator=gd, device=dev).to(torch.bfloat16)
    kn = torch.randn(b, hkv, D, generator=gd, device=dev).to(torch.bfloat16)
    vn = torch.randn(b, hkv, D, generator=gd, device=dev).to(torch.bfloat16)
    q = torch.randn(b, hq, D, generator=gd, device=dev).to(torch.bfloat16)
    out = torch.empty(b, hq, D, dtype=torch.bfloat16, device=dev)
    ws = torch.empty(max(1, decode_workspace_bytes(b, hq, hkv, D, P, bt.shape[1])),
                     dtype=torch.uint8, device=dev)
    bt_d, lens_d, slots_d = bt.to(dev), lens.to(torch.int32).to(dev), slots.to(dev)
    separate = args.separate_write

    def step(ev):
        if ev:
            ev[0].record()
        if separate:
            kv_scatter(kn, vn, kp, vp, slots_d)
        if ev:
            ev[1].record()
        if separate:
            paged_decode_attention(q, kp, vp, bt_d, lens_d, out=out, workspace=ws)
        else:
            paged_decode_append_attention(q, kp, vp, bt_d, lens_d, kn, vn, out=out, workspace=ws)
        if ev:
            ev[2].record()

    ms, (sc_ms, at_ms), wall = _phase_timer(torch, dev, step, 2, args.steps, args.warmup)
    if not separate:
        at_ms = ms  # the step is the one launch: its time over the region with no events inside
    kv_row = 2 * hkv * D * 2
    attn_bytes = b * L * kv_row + b * hq * D * 2 * 2 + int(n_pages.sum()) * 4 + b * 4
    sc_bytes = b * kv_row * 2 + b * 8
    gbps = (attn_bytes + sc_bytes) / (ms / 1e3) / 1e9
    launch_bytes = attn_bytes if separate else attn_bytes + sc_bytes
    a_gbps = launch_bytes / (at_ms / 1e3) / 1e9
    kernel = ("paged_decode_mfma<8, false> (attention call after a kv_scatter launch)" if separate
              else "paged_decode_mfma<8, true> (one write + attention launch)")
    traffic = None
    if not separate and GQA8_PMC_FILE.exists():
        try:
            traffic = json.loads(GQA8_PMC_FILE.read_text()).get("hbm_bytes_per_launch")
        except (OSError, ValueError):
            traffic = None
    return _result(
        "KV scatter + paged decode-attn GB/s (GQA 8)", gbps, "GB/s", args, ms, "bf16",
        {"workload": "qwen3-30b-a3b attention layer decode: 64 seqs x 4096 tokens, 32 q / 4 kv "
                     "heads, head_dim 128, page 16", "batch": b, "context_len": L},
        {"tokens_per_s": round(b / (ms / 1e3), 1), "hbm_frac": round(gbps / HBM_PEAK_GBPS, 4),
         "bytes_per_step": attn_bytes + sc_bytes,
         "step": "kv_scatter, then paged_decode_attention" if separate
                 else "paged_decode_append_attention (write + attention, one call)",
         "scatter_ms": round(sc_ms, 4) if separate else None,
         "attention_ms": round(at_ms, 4), "wall_s_timed": round(wall, 4)},
        {"kernel": kernel, "bound": "hbm", "achieved": round(a_gbps, 2), "peak": HBM_PEAK_GBPS,
         "unit": "GB/s", "frac": round(a_gbps / HBM_PEAK_GBPS, 4), "traffic": traffic,
         "algorithmic_bytes_per_launch": launch_bytes, "avg_launch_ms": round(at_ms, 4)})


PA_B, PA_CTX, PA_CHUNK, PA_SEED = 8, 4096, 1024, 9


def bench_prefill_attn(torch, dev, args) -> dict:
    """Chunked-prefill attention over the paged pool with Qwen3-8B heads (32 q / 8 kv,
    head_dim 128, bf16, page 16): 8 sequences, each a 1024-token chunk whose rows attend
    causally to the 3072 earlier tokens of the context and to the chunk itself (kv 4096,
    q_pos_offset 3072), block tables a seeded permutation of the pool. One step = one
    paged_attention call (the matrix-core prefill kernel). FLOPs: 4 * head_dim per (row, q head,
    visible key) - the QK dot and the PV accumulation."""
    from plastic_infer.kernel import paged_attention

    b, ctx, chunk = PA_B, PA_CTX, PA_CHUNK
    g = torch.Generator().manual_seed(PA_SEED)
    per = ctx // P
    npool = b * per + 64
    bt = torch.randperm(npool, generator=g)[: b * per].view(b, per).to(torch.int32)
    gd = torch.Generator(device=dev).manual_seed(PA_SEED)
    kp = torch.randn(npool, HKV, D, P, generator=gd, device=dev).to(torch.bfloat16)
    vp = torch.randn(npool, HKV, D, P, generator=gd, device=dev).to(torch.bfloat16)
    q = torch.randn(b * chunk, HQ, D, generator=gd, device=dev).to(torch.bfloat16)
    cu = torch.arange(0, (b + 1) * chunk, chunk, dtype=torch.int32).to(dev)
    lens = torch.full((b,), ctx, dtype=torch.int32, device=dev)
    offs = torch.full((b,), ctx - chunk, dtype=torch.int32, device=dev)
    bt_d = bt.to(dev)
    res = {}

    def step(ev):
        if ev:
            ev[0].record()
        res["out"] = paged_attention(q, kp, vp, bt_d, lens, cu_q=cu, q_pos_offsets=offs)
        if ev:
            ev[1].record()

    ms, (k_ms,), wall = _phase_timer(torch, dev, step, 1, args.steps, args.warmup)
    keys = chunk * (ctx - chunk) + chunk * (chunk + 1) // 2      # visible keys per (seq, head)
    flops = b * HQ * keys * 4 * D
    hbm = b * ctx * HKV * D * 2 * 2 + 2 * b * chunk * HQ * D * 2 + b * per * 4
    tflops = flops / (k_ms / 1e3) / 1e12           # the launch, by its events
    step_tflops = flops / (ms / 1e3) / 1e12        # the timed region (the chip's clocks ramp
    #                                                up over the first ~50 calls: --warmup 50)
    cpu = None if args.no_cpu_baseline else _cpu_prefill_attn(torch, q, kp, vp, bt, res["out"])
    return _result(
        "paged chunked-prefill attention TFLOP/s (bf16 matrix cores)", step_tflops, "TFLOP/s",
        args, ms, "bf16",
        {"workload": "qwen3-8b chunked prefill attention: 8 seqs x 1024-token chunks after 3072 "
                     "context tokens, 32 q / 8 kv heads, head_dim 128, page 16, causal",
         "batch": b, "chunk": chunk, "context_len": ctx},
        {"flops_per_step": flops, "hbm_bytes_per_step": hbm,
         "hbm_gbps": round(hbm / (k_ms / 1e3) / 1e9, 2), "wall_s_timed": round(wall, 4)},
        {"kernel": "paged_prefill_mfma<4, 8 waves, bf16>", "bound": "mfma",
         "achieved": round(tflops, 2), "peak": 2500.0, "unit": "TFLOP/s",
         "frac": round(tflops / 2500.0, 4), "traffic": None,
         "algorithmic_flops_per_launch": flops, "avg_launch_ms": round(k_ms, 4)},
        cpu)


def _cpu_prefill_attn(torch, q, kp, vp, bt, gpu_out) -> dict:
    """The oracle (gather + GQA repeat + SDPA with the offset mask, on this host's cores) on the
    last 128 rows of sequence 0 (the rows with the most keys), 1 warm-up + median of 3; its output
    is also the parity check of the GPU's rows (2e-2)."""
    import oracle.paged_kv as OP

    threads = len(os.sched_getaffinity(0))
    torch.set_num_threads(threads)
    n = 128
    pages = bt[0].tolist()
    ids = torch.tensor(pages, device=kp.device)
    kc, vc = kp.index_select(0, ids).cpu(), vp.index_select(0, ids).cpu()
    table = list(range(len(pages)))
    rows = q[PA_CHUNK - n:PA_CHUNK].cpu()[None]
    start = PA_CTX - n

    def run():
        return OP.paged_attention(rows, kc, vc, table, P, PA_CTX, causal=True, q_start_pos=start)

    ref = run()[0]
    err = (gpu_out[PA_CHUNK - n:PA_CHUNK].float().cpu() - ref.float()).abs().max().item()
    if not err <= 2e-2:
        raise AssertionError(f"bench parity: prefill attention differs from the oracle, {err:.3e}")
    times = []
    for _ in range(3):
        t0 = time.perf_counter()
        run()
        times.append(time.perf_counter() - t0)
    t = statistics.median(times)
    keys = sum(start + i + 1 for i in range(n))
    flops = HQ * keys * 4 * D
    return {"value": round(flops / t / 1e12, 4), "unit": "TFLOP/s", "cores": threads,
            "kind": "port", "sample": f"last {n} rows of sequence 0 (kv up to {PA_CTX}), "
            f"1 warm-up + median of 3, {t * 1e3:.1f} ms", "parity_max_abs_err": err}


XS_L, XS_E, XS_H, XS_I, XS_B, XS_K, XS_SLOTS, XS_SEED = 48, 128, 2048, 768, 64, 8, 3072, 5
def _pinned_exact(torch, shape):
    """A bf16 host tensor in page-locked memory of exactly its size."""
    from plastic_infer.kernel.pinned import alloc_pinned_exact

    return alloc_pinned_exact(shape, torch.bfloat16)


def _pin_expert_banks(torch, markers: bool):
    """48 layers of pinned gate_up [128, 1536, 2048] / down [128, 2048, 768] bf16 banks.
    markers: layer l holds l / -l with row markers (expert index at [e, 0, 0]) for slot checks;
    else layer l holds (l + 1) / 64 and -(l + 1) / 64 everywhere (exact in bf16), which gives the
    expert FFN a closed form."""
    L, E, H, I = XS_L, XS_E, XS_H, XS_I
    row_bytes = 2 * I * H * 2 + H * I * 2
    print(f"bench: pinning {L * E * row_bytes / 2**30:.1f} GiB of expert banks", file=sys.stderr,
          flush=True)
    banks = {"gate_up": [], "down": []}
    for l in range(L):
        gu = _pinned_exact(torch, (E, 2 * I, H))
        dn = _pinned_exact(torch, (E, H, I))
        if markers:
            gu.fill_(float(l))
            dn.fill_(float(-l))
            gu[:, 0, 0] = torch.arange(E, dtype=torch.bfloat16)
            dn[:, 0, 0] = torch.arange(E, dtype=torch.bfloat16)
        else:
            gu.fill_((l + 1) / 64.0)
            dn.fill_(-(l + 1) / 64.0)
        banks["gate_up"].append(gu)
        banks["down"].append(dn)
        if l % 8 == 7:
            print(f"bench: {l + 1}/{L} layers pinned", file=sys.stderr, flush=True)
    return banks


def bench_hbm_read(torch, dev, args) -> dict:
    """The box's streaming-read rate (pia_hbm_read_probe) for two access patterns: `flat` (the
    buffer front to back) and `tiles` (distinct 4 KiB tiles drawn at random from a 12 GiB
    buffer, the paged-KV access of the decode kernels). Reads of X bytes, X = 25 MiB .. 3.2 GiB
    in doublings, each from a region that the reads before it did not touch for at least 10 GB
    (the 256 MB last-level cache holds none of it) or from fresh random tiles, timed by events
    around each launch: one untimed launch, then the mean of `steps` (at least 6). Per pattern
    t(X) = fixed + X / rate, fitted by least squares over X >= 200 MB. `value` is the tiles
    rate: the ceiling the paged decode kernels are compared with. `row_shapes`: 3 GiB read as
    16-row blocks (the weight tiles of the expert GEMMs) with every load instruction covering
    R rows x 1024 / R bytes, R = 16 (the MFMA operand layout) .. 1 (1 KiB contiguous)."""
    from plastic_infer import _native as N

    pool_bytes = 12 << 30
    pool_tiles = pool_bytes // 4096
    pool = torch.zeros(pool_bytes, dtype=torch.uint8, device=dev)
    sink = torch.zeros(1, dtype=torch.int32, device=dev)
    stream = torch.cuda.current_stream(dev)
    sizes = [(25 << 20) << i for i in range(8)]
    reps = max(6, args.steps)
    out = {}
    for pattern in ("flat", "tiles"):
        rows, off = [], 0
        for X in sizes:
            times = []
            for r in range(reps + 1):
                ids, n = None, 0
                if pattern == "tiles":
                    n = X // 4096
                    ids = torch.randperm(pool_tiles, device=dev)[:n].to(torch.int32)
                elif off + X > pool_bytes:
                    off = 0
                a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                a.record(stream)
                N.call("pia_hbm_read_probe", pool.data_ptr() + (off if ids is None else 0),
                       X if ids is None else pool_bytes, None if ids is None else ids.data_ptr(),
                       n, sink.data_ptr(), N.stream_of(dev))
                b.record(stream)
                b.synchronize()
                if r > 0:
                    times.append(a.elapsed_time(b) / 1e3)
                if ids is None:
                    off += (X + (4 << 20)) & ~((2 << 20) - 1)
            t = statistics.mean(times)
            rows.append({"bytes": X, "mean_us": round(t * 1e6, 2),
                         "min_us": round(min(times) * 1e6, 2), "gbps": round(X / t / 1e9, 1)})
        fit = [r for r in rows if r["bytes"] >= 200e6]
        xs = [r["bytes"] for r in fit]
        ts = [r["mean_us"] / 1e6 for r in fit]
        mx, mt = statistics.mean(xs), statistics.mean(ts)
        slope = sum((x - mx) * (t - mt) for x, t in zip(xs, ts)) / sum((x - mx) ** 2 for x in xs)
        out[pattern] = {"fixed_us": round((mt - slope * mx) * 1e6, 2),
                        "rate_gbps": round(1.0 / slope / 1e9, 1),
                        "rate_frac_of_8tbps": round(1.0 / slope / 1e9 / HBM_PEAK_GBPS, 4),
                        "per_size": rows}
    # the load shape of a GEMM weight tile (pia_hbm_read_rows_probe): 3 GiB of 16-row blocks,
    # R rows x 1024 / R bytes per load instruction, regions rotated through the buffer as above
    shapes, off, X = [], 0, 3 << 30
    for row_bytes in (1536, 4096):
        for r_per in (16, 8, 4, 2, 1):
            times = []
            for r in range(reps + 1):
                if off + X > pool_bytes:
                    off = 0
                a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                a.record(stream)
                N.call("pia_hbm_read_rows_probe", pool.data_ptr() + off, X, row_bytes, r_per,
                       sink.data_ptr(), N.stream_of(dev))
                b.record(stream)
                b.synchronize()
                if r > 0:
                    times.append(a.elapsed_time(b) / 1e3)
                off += (X + (4 << 20)) & ~((2 << 20) - 1)
            read = X // (16 * row_bytes) * 16 * row_bytes
            t = statistics.mean(times)
            shapes.append({"row_bytes": row_bytes, "rows_per_load": r_per,
                           "mean_us": round(t * 1e6, 2), "gbps": round(read / t / 1e9, 1)})
    rate = out["tiles"]["rate_gbps"]
    return {"metric": "HBM streaming-read GB/s, random 4 KiB tiles (fit: fixed cost + bytes / "
                      "rate)",
            "value": rate, "unit": "GB/s", "n_gpus": 1, "steps": reps,
            "higher_is_better": True, "vs_baseline": None, "dtype": "u8",
            "data": "zero-filled 12 GiB buffer; flat regions never re-read within 10 GB, tiles "
                    "drawn without repeats per launch",
            "config": {"workload": "pia_hbm_read_probe: 16-byte loads, 4 x 256-thread "
                                   "workgroups per CU", "sizes_bytes": sizes},
            "hbm_frac": round(rate / HBM_PEAK_GBPS, 4), "patterns": out,
            "row_shapes": {"bytes": X, "per_shape": shapes,
                           "what": "16-row blocks of row_bytes, rows_per_load rows x 1024 / "
                                   "rows_per_load bytes per load instruction (16: the MFMA "
                                   "operand layout; 1: 1 KiB of the block)"}}


def bench_expert_stream(torch, dev, args) -> dict:
    """Qwen3-30B-A3B expert streaming through the GPU slot cache: 48 layers x 128 experts,
    gate_up [1536, 2048] + down [2048, 768] bf16 = 9 MiB per expert (54 GiB of pinned host
    banks), 3072 HBM slots (50% of the experts), global LRU admission (the reference's
    OffloadMoeCache policy). One step = for every layer in order: ensure_experts on a seeded
    uniform top-8 routing of 64 decode tokens, then copy_missing of the admitted experts (one
    multi-bank launch reading the pinned banks over the host link)."""
    from plastic_infer.kernel import copy_rows_async
    from plastic_infer.moe.fused import fused_experts_decode_impl
    from plastic_infer.moe.offload_cache import OffloadMoeCache

    L, E, H, I, B, K = XS_L, XS_E, XS_H, XS_I, XS_B, XS_K
    row_bytes = 2 * I * H * 2 + H * I * 2
    banks = _pin_expert_banks(torch, markers=True)
    cache = OffloadMoeCache(num_layers=L, num_experts=E, cache_size=XS_SLOTS, device=dev)
    cache.collect_stats = True
    cache.set_bank_sources(banks)

    # host-link rates of the two copy engines on one whole layer (1.18 GB)
    rows = list(range(E))
    scratch = torch.empty(E, 2 * I, H, dtype=torch.bfloat16, device=dev)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    copy_rows_async(scratch, rows, banks["gate_up"][0], rows)          # warm
    e0.record()
    copy_rows_async(scratch, rows, banks["gate_up"][0], rows)
    e1.record()
    torch.cuda.synchronize(dev)
    dma_gbps = E * 2 * I * H * 2 / (e0.elapsed_time(e1) / 1e3) / 1e9
    cache.materialize_layer(1)
    cache.copy_missing()
    cache.materialize_layer(0)
    e0.record()
    cache.copy_missing()
    e1.record()
    torch.cuda.synchronize(dev)
    kern_gbps = E * row_bytes / (e0.elapsed_time(e1) / 1e3) / 1e9
    del scratch
    cache.reset()
    cache.reset_stats()

    steps, warmup = args.steps, args.warmup
    g = torch.Generator(device=dev).manual_seed(XS_SEED)
    routing = torch.rand(steps + warmup, L, B, E, generator=g, device=dev).argsort(dim=3)[..., :K]
    routing = routing.to(torch.int32).contiguous()
    rw = torch.rand(L, B, K, generator=g, device=dev)
    rw = (rw / rw.sum(-1, keepdim=True)).contiguous()
    x = torch.randn(B, H, generator=g, device=dev).to(torch.bfloat16)
    gu_cache, dn_cache = cache.bank_caches["gate_up"], cache.bank_caches["down"]
    ffn_ev = []

    def step(i, timed=False):
        for l in range(L):
            ids = routing[i, l].clone()
            cache.ensure_experts(l, ids)          # ids become slot ids, in place
            cache.copy_missing()
            if timed:
                a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                a.record()
            fused_experts_decode_impl(x, gu_cache, dn_cache, rw[l], ids)
            if timed:
                b.record()
                ffn_ev.append((a, b))

    for i in range(warmup):
        step(i)
        print(f"bench: warm-up step {i + 1}/{warmup}", file=sys.stderr, flush=True)
    torch.cuda.synchronize(dev)
    cache.reset_stats()
    t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    wall0 = time.perf_counter()
    t0.record()
    for i in range(steps):
        step(warmup + i, timed=True)
        print(f"bench: step {i + 1}/{steps}", file=sys.stderr, flush=True)
    t1.record()
    torch.cuda.synchronize(dev)
    wall = time.perf_counter() - wall0
    ms = t0.elapsed_time(t1) / steps
    ffn_ms = sum(a.elapsed_time(b) for a, b in ffn_ev) / steps
    active, missing, calls = (int(v) for v in cache.lru_stats.sum(0))
    streamed = missing * row_bytes / steps
    # spot check: the last step's slots hold the right layer's rows
    gu_cache = cache.bank_caches["gate_up"]
    last = routing[warmup + steps - 1, L - 1].reshape(-1)
    slots = cache.slot_for_id[L - 1, last.long()]
    got = gu_cache[slots.long(), 0, :2].float().cpu()
    exp = torch.stack([last.float().cpu(), torch.full((last.numel(),), float(L - 1))], 1)
    if not torch.equal(got, exp):
        raise RuntimeError("expert stream: slot contents differ from the host banks")
    gbps = streamed / (ms / 1e3) / 1e9
    return _result(
        "MoE expert streaming GB/s over the host link; decode tokens/s", gbps, "GB/s", args, ms,
        "bf16",
        {"workload": "qwen3-30b-a3b routed experts of a decode step over the slot cache (48 layers "
                     "x 128 experts, 9 MiB each, 3072 HBM slots, global LRU, 64 decode tokens "
                     "top-8): admission, streaming of the misses, expert FFN on the slots",
         "layers": L, "experts": E, "slots": XS_SLOTS, "batch": B, "topk": K},
        {"tokens_per_s": round(B / (ms / 1e3), 2), "ffn_ms_per_step": round(ffn_ms, 3),
         "hit_rate": round(1 - missing / max(active, 1), 4),
         "experts_per_layer_step": round(active / max(calls, 1), 2),
         "streamed_bytes_per_step": int(streamed), "dma_copy_gbps": round(dma_gbps, 2),
         "kernel_copy_gbps": round(kern_gbps, 2), "wall_s_timed": round(wall, 3),
         "overlap_fraction": 0.0,
         "overlap_note": "decode: a layer's routing needs its attention output and its expert "
                         "GEMM needs the copied rows, so the copies are serial with compute"},
        {"kernel": "index_copy_rows_multi_kernel (copy_missing)", "bound": "host-link",
         "achieved": round(gbps, 2), "peak": 64.0, "unit": "GB/s",
         "frac": round(gbps / 64.0, 4), "traffic": None,
         "algorithmic_bytes_per_launch": int(streamed / L), "avg_launch_ms": round(ms / L, 4)})


DS_B, DS_CTX, DS_SEED = 64, 4096, 5


def _decode_step_policy(torch, dev, args, cfg, w, banks, kp, vp, batch, tokens, policy):
    """Warm-up + timed steps of MoePagedDecoder under one expert residency policy. Returns the
    per-policy report (timings, streaming, overlap) and the last step's layer-(L-1) tensors."""
    from plastic_infer.exec.runner_moe_paged import MoePagedDecoder
    from plastic_infer.moe.offload_cache import OffloadMoeCache

    L, E = cfg.n_layers, cfg.n_experts
    if policy == "static":
        cache = OffloadMoeCache(L, E, L * E // 2 + E // 2, dev, cache_policy="static")
    else:
        cache = OffloadMoeCache(L, E, XS_SLOTS, dev)
    cache.collect_stats = True
    t0 = time.perf_counter()
    cache.set_bank_sources(banks)
    setup_s = time.perf_counter() - t0
    dec = MoePagedDecoder(w, cfg, cache, kp, vp, max_batch=DS_B, overlap=True)
    layer_ev = []
    last = {}

    def hook(l, d):
        ev = d.get("events") or {}
        r = d.get("routes")
        if r is not None and r.issued is not None and ev:
            layer_ev.append((r.issued, r.ready, ev["a0"], ev["a1"], r.copied_bytes))
        if l == L - 1:
            last.clear()
            last.update({k: d[k] for k in ("q", "attn", "moe_in", "topk_weights", "topk_ids",
                                           "routed")})

    dec.layer_hook = hook
    for i in range(args.warmup):
        dec.step(tokens, batch)
        print(f"bench: {policy}: warm-up step {i + 1}/{args.warmup}", file=sys.stderr, flush=True)
    torch.cuda.synchronize(dev)
    cache.reset_stats()
    cache.record_copy_start = True
    layer_ev.clear()
    compute = torch.cuda.current_stream(dev)
    s0, s1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    wall0 = time.perf_counter()
    s0.record(compute)
    for i in range(args.steps):
        logits = dec.step(tokens, batch)
        print(f"bench: {policy}: step {i + 1}/{args.steps}", file=sys.stderr, flush=True)
    s1.record(compute)
    torch.cuda.synchronize(dev)
    wall = time.perf_counter() - wall0
    ms = s0.elapsed_time(s1) / args.steps
    copy_ms = overlap_ms = pass_a_ms = 0.0
    copied = 0
    for issued, ready, a0, a1, nbytes in layer_ev:
        c0, c1 = s0.elapsed_time(issued), s0.elapsed_time(ready)
        p0, p1 = s0.elapsed_time(a0), s0.elapsed_time(a1)
        copy_ms += max(0.0, c1 - c0)
        pass_a_ms += max(0.0, p1 - p0)
        overlap_ms += max(0.0, min(c1, p1) - max(c0, p0))
        copied += nbytes
    st = cache.decode_miss_stats()
    n = max(args.steps, 1)
    rep = {
        "ms_per_step": round(ms, 3), "tokens_per_s": round(DS_B / (ms / 1e3), 2),
        "slots": cache.cache_size, "resident_per_layer": cache.resident_per_layer,
        "hit_rate": round(st["hit_rate"], 4), "experts_per_layer_step":
            round(st["active_per_layer"], 2),
        "streamed_bytes_per_step": int(copied / n),
        "host_link_gbps": round(copied / n / (copy_ms / n / 1e3) / 1e9, 2) if copy_ms else None,
        "copy_ms_per_step": round(copy_ms / n, 3),
        "overlap_fraction": round(overlap_ms / copy_ms, 4) if copy_ms else 0.0,
        "compute_hidden_fraction": round(overlap_ms / pass_a_ms, 4) if pass_a_ms else None,
        "in_hbm_ffn_ms_per_step": round(pass_a_ms / n, 3),
        "bank_setup_s": round(setup_s, 2), "wall_s_timed": round(wall, 3),
    }
    del cache, dec
    return rep, last, logits


def bench_decode_step(torch, dev, args) -> dict:
    """A full Qwen3-30B-A3B decode step for 64 sequences at 4096 context through the package's
    batched MoE-paged decoder (plastic_infer.exec.runner_moe_paged.MoePagedDecoder): for each of
    48 layers, RMSNorm, q / k / v projections, q / k norm, RoPE, KV scatter, GQA-8 paged decode
    attention over the layer's share of a 25.8 GB KV pool, o projection, router top-8 of 128,
    the routed experts over the expert slot cache (54 GiB of pinned banks, half of the experts'
    worth of HBM slots) with the misses copied by the DMA engines on the cache's copy stream
    while the routes of experts already in HBM compute; then the final norm and the LM head.
    Random-init weights. Both residency policies run: "static" (64 experts of every layer
    resident for good, the other half streamed through a 64-slot staging area) and "lru" (one
    global LRU over 3072 slots, the reference's policy). value = tokens/s of the better one."""
    from plastic_infer.exec.runner_moe_paged import (DecodeBatch, qwen3_30b_a3b_config,
                                                     random_dense_weights, random_expert_banks)

    cfg = qwen3_30b_a3b_config(n_layers=XS_L, max_seq_len=DS_CTX)
    L, b, ctx = cfg.n_layers, DS_B, DS_CTX
    npl = b * ctx // P                           # pages per layer
    g = torch.Generator().manual_seed(DS_SEED)
    perm = torch.cat([torch.randperm(npl, generator=g) + l * npl for l in range(L)])
    bt = perm.view(L, b, ctx // P).to(torch.int32)
    lens = torch.full((b,), ctx, dtype=torch.int32)
    pos = lens.long() - 1
    slots = (bt[:, :, -1].to(torch.int64) * P + pos % P).contiguous()
    batch = DecodeBatch(bt.to(dev), lens.to(dev), slots.to(dev), pos.to(dev))
    print(f"bench: filling {2 * L * npl * cfg.n_kv_heads * D * P * 2 / 1e9:.1f} GB of KV pool",
          file=sys.stderr, flush=True)
    gd = torch.Generator(device=dev).manual_seed(DS_SEED)
    kp = torch.empty(L * npl, cfg.n_kv_heads, D, P, dtype=torch.bfloat16, device=dev)
    vp = torch.empty_like(kp)
    for l in range(L):
        for pool in (kp, vp):
            pool[l * npl:(l + 1) * npl] = torch.randn(npl, cfg.n_kv_heads, D, P, generator=gd,
                                                      device=dev)
    w = random_dense_weights(cfg, dev, seed=DS_SEED)
    print(f"bench: drawing {L * cfg.n_experts * 9 / 1024:.1f} GiB of random expert banks into "
          "pinned host memory", file=sys.stderr, flush=True)
    banks = random_expert_banks(cfg, dev, seed=DS_SEED + 1,
                                pin=lambda shape: _pinned_exact(torch, shape))
    tokens = torch.randint(0, cfg.vocab_size, (b,), generator=g).to(dev)
    reports, last = {}, {}
    logits = {}
    for policy in ("static", "lru"):
        reports[policy], last[policy], logits[policy] = _decode_step_policy(
            torch, dev, args, cfg, w, banks, kp, vp, batch, tokens, policy)
    same = bool(torch.equal(logits["static"], logits["lru"]))
    if not same:
        raise RuntimeError("decode step: the two residency policies gave different logits")
    best = max(reports, key=lambda k: reports[k]["tokens_per_s"])
    rb = reports[best]
    cpu = None if args.no_cpu_baseline else _cpu_decode_step(torch, cfg, w, banks, kp, vp, bt,
                                                             last[best])
    kv_row = 2 * cfg.n_kv_heads * D * 2
    return _result(
        "Qwen3-30B-A3B decode step tokens/s (48 layers through the paged MoE decoder, experts "
        "streamed over the host link)", rb["tokens_per_s"], "tokens/s", args, rb["ms_per_step"],
        "bf16",
        {"workload": "qwen3-30b-a3b decode step, 64 seqs x 4096 context, 48 layers: norms, "
                     "projections, rope, kv scatter, gqa-8 paged attention, router top-8 of 128, "
                     "routed experts over the slot cache (half the experts' worth of hbm "
                     "slots, misses streamed from 54 GiB of pinned banks by dma on a side "
                     "stream, overlapped with the in-hbm experts' ffn), lm head",
         "layers": L, "batch": b, "context_len": ctx, "experts": cfg.n_experts, "topk": 8,
         "policy": best},
        {"policies": reports, "policies_bit_identical": same,
         "kv_bytes_per_step": L * b * ctx * kv_row,
         "overlap_definition": "overlap_fraction = copy time during which the in-HBM experts' "
                               "FFN ran / total copy time (1 - exposed copy / total copy); "
                               "compute_hidden_fraction = that time / the in-HBM FFN's time"},
        {"kernel": "hipMemcpyAsync expert rows (DMA, copy stream)", "bound": "host-link",
         "achieved": rb["host_link_gbps"], "peak": 64.0, "unit": "GB/s",
         "frac": round(rb["host_link_gbps"] / 64.0, 4) if rb["host_link_gbps"] else None,
         "traffic": None, "algorithmic_bytes_per_launch": rb["streamed_bytes_per_step"] // L,
         "avg_launch_ms": round(rb["copy_ms_per_step"] / L, 4)}, cpu)


def _cpu_decode_step(torch, cfg, w, banks, kp, vp, bt, last) -> dict:
    """The oracle's pieces of one layer of the step on the host cores, for the last layer of the
    timed steps: attention of 8 rows over their 4096 tokens, the dense projections and router of
    all 64 rows, the routed FFN of 8 tokens; each scaled to 64 rows, then x48 layers. The
    attention and FFN results also check the GPU's (2e-2 and 1e-2 of the largest magnitude)."""
    import torch.nn.functional as F

    import oracle.fused_experts as OF
    import oracle.paged_kv as OP

    threads = len(os.sched_getaffinity(0))
    torch.set_num_threads(threads)
    L, B = cfg.n_layers, DS_B
    l = L - 1
    picks = list(range(0, B, B // 8))
    rows = bt[l][picks]
    pages = torch.unique(rows.reshape(-1))
    remap = torch.full((int(bt.max()) + 1,), -1, dtype=torch.int64)
    remap[pages] = torch.arange(pages.numel())
    kl = kp.index_select(0, pages.to(kp.device)).cpu()
    vl = vp.index_select(0, pages.to(vp.device)).cpu()
    btl = remap[rows.long()].to(torch.int32)
    q = last["q"][picks].cpu()
    t0 = time.perf_counter()
    ref = OP.decode_batch(q, kl, vl, btl, [DS_CTX] * len(picks), P)
    t_attn = (time.perf_counter() - t0) * B / len(picks)
    err_attn = (last["attn"][picks].float().cpu() - ref.float()).abs().max().item()
    if err_attn > 2e-2:
        raise RuntimeError(f"decode step: attention differs from the oracle ({err_attn})")
    p = f"layers.{l}."
    wc = {k: w[p + k].cpu() for k in ("self_attn.q_proj.weight", "self_attn.k_proj.weight",
                                      "self_attn.v_proj.weight", "self_attn.o_proj.weight",
                                      "mlp.router.weight")}
    h = last["moe_in"].cpu()
    t0 = time.perf_counter()
    for name in ("self_attn.q_proj.weight", "self_attn.k_proj.weight", "self_attn.v_proj.weight",
                 "mlp.router.weight"):
        F.linear(h, wc[name])
    F.linear(last["attn"].cpu().view(B, -1), wc["self_attn.o_proj.weight"])
    t_dense = time.perf_counter() - t0
    tw, ti = last["topk_weights"][picks].cpu(), last["topk_ids"][picks].cpu()
    used = torch.unique(ti)
    re = torch.full((cfg.n_experts,), -1, dtype=torch.int64)
    re[used] = torch.arange(used.numel())
    w1, w2 = banks["gate_up"][l][used], banks["down"][l][used]
    t0 = time.perf_counter()
    ffn = OF.fused_experts(h[picks], w1, w2, tw, re[ti.long()].to(torch.int32))
    t_ffn = (time.perf_counter() - t0) * B / len(picks)
    got = last["routed"][picks].float().cpu()
    err_ffn = (got - ffn.float()).abs().max().item() / ffn.float().abs().max().item()
    if err_ffn > 1e-2:
        raise RuntimeError(f"decode step: routed FFN differs from the oracle ({err_ffn})")
    per_layer = t_attn + t_dense + t_ffn
    model, phys = cpu_info()
    return {"value": round(B / (per_layer * L), 4), "unit": "tokens/s", "cores": threads,
            "kind": "port",
            "sample": f"layer {l}: attention of {len(picks)} rows x {DS_CTX} tokens "
                      f"{t_attn * 1e3 * len(picks) / B:.0f} ms, dense projections + router of "
                      f"{B} rows {t_dense * 1e3:.0f} ms, routed FFN of {len(picks)} tokens "
                      f"{t_ffn * 1e3 * len(picks) / B:.0f} ms; scaled to {B} rows, x{L} layers "
                      f"(host banks need no copy)",
            "parity": {"attention_max_abs_err": err_attn, "ffn_rel_err": err_ffn},
            "cpu_model": model, "physical_cores": phys}


PS_T, PS_SEED = 4096, 7


def bench_prefill_stream(torch, dev, args) -> dict:
    """Qwen3-30B-A3B prefill through the expert double buffer (the reference's OffloadMoeCache
    prefill overlap): 48 layers of pinned banks (54 GiB), one 4096-token prefill chunk. Layer
    l's experts stream host -> one of two HBM layer buffers on the cache's copy stream while
    layer l - 1's routed expert FFN (fused_experts_impl over the buffer views, position ==
    expert id) runs on the compute stream; a buffer is refilled once the FFN that read it has
    finished. One step = the 48 layers (router logits fp32 N(0,1), top-8 renormalised,
    computed before timing)."""
    from plastic_infer.kernel import copy_rows_async, moe_topk
    from plastic_infer.moe.fused import fused_experts_impl
    from plastic_infer.moe.offload_cache import OffloadMoeCache

    L, E, H, I, K, T = XS_L, XS_E, XS_H, XS_I, XS_K, PS_T
    row_bytes = 2 * I * H * 2 + H * I * 2
    banks = _pin_expert_banks(torch, markers=False)
    cache = OffloadMoeCache(num_layers=L, num_experts=E, cache_size=XS_SLOTS, device=dev,
                            prefill_overlap=True)
    cache.set_bank_sources(banks)
    g = torch.Generator(device=dev).manual_seed(PS_SEED)
    x = torch.randn(T, H, generator=g, device=dev).to(torch.bfloat16)
    routes = [moe_topk(torch.randn(T, E, generator=g, device=dev), K, True) for _ in range(L)]
    work = torch.empty_like(x)

    # host-link rate of the DMA engines on one whole layer (both banks), alone
    scratch = [torch.empty(E, 2 * I, H, dtype=torch.bfloat16, device=dev),
               torch.empty(E, H, I, dtype=torch.bfloat16, device=dev)]
    rows = list(range(E))
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    for rep in range(2):
        e0.record()
        copy_rows_async(scratch[0], rows, banks["gate_up"][1], rows)
        copy_rows_async(scratch[1], rows, banks["down"][1], rows)
        e1.record()
        torch.cuda.synchronize(dev)
    dma_gbps = E * row_bytes / (e0.elapsed_time(e1) / 1e3) / 1e9
    del scratch
    ffn_ev = []

    def step(timed):
        for l in range(L):
            if l == 0:
                cache.begin_prefill()
            cache.prefetch_prefill_layer(l)
            cache.prefetch_prefill_layer(l + 1)
            gu, dn = cache.wait_prefill_layer(l)
            work.copy_(x)
            tw, ids = routes[l]
            if timed:
                a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                a.record()
            fused_experts_impl(work, gu, dn, tw, ids)
            if timed:
                b.record()
                ffn_ev.append((a, b))
            cache.release_prefill_layer(l)

    for i in range(args.warmup):
        step(False)
        print(f"bench: warm-up step {i + 1}/{args.warmup}", file=sys.stderr, flush=True)
    torch.cuda.synchronize(dev)
    t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    wall0 = time.perf_counter()
    t0.record()
    for i in range(args.steps):
        step(True)
        print(f"bench: step {i + 1}/{args.steps}", file=sys.stderr, flush=True)
    t1.record()
    torch.cuda.synchronize(dev)
    wall = time.perf_counter() - wall0
    ms = t0.elapsed_time(t1) / args.steps
    ffn_ms = sum(a.elapsed_time(b) for a, b in ffn_ev) / args.steps
    # closed form of the last layer (all gate/up weights c, all down weights d): every gate and
    # up value of token t is R(c * sum(x_t)), the activation a = R(silu(g) * g) is the same in
    # all I columns, route j's output is R(I * a * d * w_j), the FFN output R(sum_j of those)
    c, d = L / 64.0, -L / 64.0
    n = 4
    xs = x[:n].double().sum(1).cpu()
    bf = lambda v: v.to(torch.bfloat16).double()
    gsum = bf((c * xs).float())
    act = bf((gsum / (1 + torch.exp(-gsum)) * gsum).float())
    tw, _ = routes[L - 1]
    c3 = bf(((I * act * d).float()[:, None] * tw[:n].cpu()).float())
    exp = bf(c3.float().sum(1))
    got = work[:n].double().cpu()
    err = (got - exp[:, None]).abs().max().item()
    if not err <= 2e-2 * max(exp.abs().max().item(), 1e-6):
        raise RuntimeError(f"prefill stream: last layer's output is off its closed form ({err})")
    layer_bytes = E * row_bytes
    copy_ms = L * layer_bytes / (dma_gbps * 1e9) * 1e3
    exposed_ms = max(0.0, ms - ffn_ms)
    overlap = max(0.0, 1.0 - exposed_ms / copy_ms)
    gbps = L * layer_bytes / (ms / 1e3) / 1e9
    return _result(
        "prefill expert streaming GB/s over the host link (double buffer); prefill tokens/s",
        gbps, "GB/s", args, ms, "bf16",
        {"workload": "qwen3-30b-a3b prefill, 48 layers of pinned expert banks (54 GiB) through "
                     "the two-buffer overlap, 4096 tokens, 128 experts top-8",
         "layers": L, "experts": E, "tokens": T, "topk": K},
        {"tokens_per_s": round(T / (ms / 1e3), 1), "ffn_ms_per_step": round(ffn_ms, 3),
         "dma_copy_gbps": round(dma_gbps, 2), "copy_ms_per_step_at_dma_rate": round(copy_ms, 2),
         "exposed_copy_ms": round(exposed_ms, 2), "overlap_fraction": round(overlap, 4),
         "ffn_hidden_fraction": round(min(1.0, max(0.0, (copy_ms + ffn_ms - ms) / ffn_ms)), 4),
         "overlap_note": "1 - (step time - expert FFN time) / (the step's bytes at the measured "
                         "DMA rate); the FFN of a layer hides under the next layer's copy",
         "streamed_bytes_per_step": L * layer_bytes, "wall_s_timed": round(wall, 3)},
        {"kernel": "hipMemcpyAsync runs (copy_rows_async) on the copy stream", "bound": "host-link",
         "achieved": round(gbps, 2), "peak": 64.0, "unit": "GB/s", "frac": round(gbps / 64.0, 4),
         "traffic": None, "algorithmic_bytes_per_launch": layer_bytes,
         "avg_launch_ms": round(ms / L, 4)})


EXP_H, EXP_I, EXP_E, EXP_K, EXP_BM, EXP_SEED = 2048, 768, 128, 8, 16, 6
MFMA_BF16_PEAK_TFLOPS = 2500.0


def bench_moe_experts(torch, dev, args, tokens: int) -> dict:
    """Qwen3-30B-A3B routed expert FFN, one layer, experts resident in HBM: gate_up
    [128, 1536, 2048] and down [128, 2048, 768] bf16 ~ N(0, 0.02); hidden [tokens, 2048] bf16
    ~ N(0,1); router logits fp32 N(0,1) -> softmax top-8 renormalised (outside the step). One
    step = moe_align_block_size (block 16) + first expert GEMM with SiLU-and-mul fused +
    second expert GEMM with the routing weight + sum over the 8 routes (fused_experts)."""
    from plastic_infer import _native as N
    from plastic_infer.kernel import moe_align_block_size, moe_expert_gemm, moe_sum_reduce, moe_topk

    H, I, E, K = EXP_H, EXP_I, EXP_E, EXP_K
    g = torch.Generator(device=dev).manual_seed(EXP_SEED)
    x = torch.randn(tokens, H, generator=g, device=dev).to(torch.bfloat16)
    w1 = (torch.randn(E, 2 * I, H, generator=g, device=dev) * 0.02).to(torch.bfloat16)
    w2 = (torch.randn(E, H, I, generator=g, device=dev) * 0.02).to(torch.bfloat16)
    logits = torch.randn(tokens, E, generator=g, device=dev)
    tw, ids = moe_topk(logits, K, True)
    numel = tokens * K
    mpad = numel + (E + 1) * (EXP_BM - 1) if numel >= E + 1 else numel * EXP_BM
    ws = torch.empty(N.query("pia_moe_expert_gemm_workspace_bytes", mpad, EXP_BM),
                     dtype=torch.uint8, device=dev)
    c2 = torch.empty(numel, I, dtype=torch.bfloat16, device=dev)
    c3 = torch.empty(tokens, K, H, dtype=torch.bfloat16, device=dev)
    out = torch.empty(tokens, H, dtype=torch.bfloat16, device=dev)

    def step(ev):
        if ev:
            ev[0].record()
        s, e, npp = moe_align_block_size(ids, EXP_BM, E)
        if ev:
            ev[1].record()
        moe_expert_gemm(x, w1, tw, s, e, npp, EXP_BM, numel, K, activation="silu", out=c2,
                        workspace=ws)
        if ev:
            ev[2].record()
        moe_expert_gemm(c2, w2, tw, s, e, npp, EXP_BM, numel, 1, mul_routed_weight=True,
                        out=c3.view(numel, H), workspace=ws)
        if ev:
            ev[3].record()
        moe_sum_reduce(c3, out)
        if ev:
            ev[4].record()

    ms, (align_ms, g1_ms, g2_ms, sum_ms), wall = _phase_timer(torch, dev, step, 4, args.steps,
                                                              args.warmup)
    distinct = int(torch.unique(ids).numel())
    w1_bytes, w2_bytes = distinct * 2 * I * H * 2, distinct * H * I * 2
    g1_bytes = w1_bytes + tokens * H * 2 + numel * I * 2
    g2_bytes = w2_bytes + numel * I * 2 + numel * H * 2 + numel * 4
    sum_bytes = numel * H * 2 + tokens * H * 2
    g1_flops, g2_flops = numel * 2 * I * H * 2, numel * H * I * 2
    step_bytes = g1_bytes + g2_bytes + sum_bytes
    step_flops = g1_flops + g2_flops
    # the dominant kernel's bound: the larger of its HBM time and its MFMA time at peak
    dom_name = "moe_gemm_stream_fused" if numel < 2048 else "moe_gemm_wide"
    dom_name += "<bf16, silu> (first expert GEMM)"
    t_hbm = g1_bytes / (HBM_PEAK_GBPS * 1e9)
    t_mfma = g1_flops / (MFMA_BF16_PEAK_TFLOPS * 1e12)
    if t_hbm >= t_mfma:
        achieved, peak, unit, bound = g1_bytes / (g1_ms / 1e3) / 1e9, HBM_PEAK_GBPS, "GB/s", "hbm"
    else:
        achieved, peak, unit, bound = (g1_flops / (g1_ms / 1e3) / 1e12, MFMA_BF16_PEAK_TFLOPS,
                                       "TFLOP/s", "mfma")
    traffic = None
    pmc = ROOT / "profiles" / f"moe_experts_t{tokens}_pmc.json"
    if pmc.exists():
        try:
            traffic = json.loads(pmc.read_text()).get("hbm_bytes_per_launch")
        except (OSError, ValueError):
            traffic = None
    decode = tokens < 512
    cpu = None
    if not args.no_cpu_baseline:
        cpu = _cpu_experts(torch, x, w1, w2, tw, ids, out, decode)
    if decode:
        value, unit_v, metric = step_bytes / (ms / 1e3) / 1e9, "GB/s", \
            "routed expert FFN GB/s (weights of the experts hit + activations); tokens/s"
    else:
        value, unit_v, metric = step_flops / (ms / 1e3) / 1e12, "TFLOP/s", \
            "routed expert FFN TFLOP/s; tokens/s"
    return _result(
        metric, value, unit_v, args, ms, "bf16",
        {"workload": f"qwen3-30b-a3b routed expert FFN, one layer, experts resident "
                     f"({tokens} tokens, hidden 2048, moe_intermediate 768, 128 experts top-8)",
         "tokens": tokens, "hidden": H, "intermediate": I, "experts": E, "topk": K},
        {"tokens_per_s": round(tokens / (ms / 1e3), 1), "distinct_experts": distinct,
         "bytes_per_step": step_bytes, "flops_per_step": step_flops,
         "hbm_frac": round(step_bytes / (ms / 1e3) / 1e9 / HBM_PEAK_GBPS, 4),
         "align_ms": round(align_ms, 4), "gemm1_ms": round(g1_ms, 4),
         "gemm2_ms": round(g2_ms, 4), "sum_ms": round(sum_ms, 4),
         "wall_s_timed": round(wall, 4)},
        {"kernel": dom_name, "bound": bound, "achieved": round(achieved, 2), "peak": peak,
         "unit": unit, "frac": round(achieved / peak, 4), "traffic": traffic,
         "algorithmic_bytes_per_launch": g1_bytes, "flops_per_launch": g1_flops,
         "avg_launch_ms": round(g1_ms, 4)},
        cpu)


def _cpu_experts(torch, x, w1, w2, tw, ids, out, decode: bool) -> dict:
    """The oracle's fused experts (float64 dot products, the reference's rounding points) on the
    first 8 tokens, with only the experts they route to; 1 warm-up + median of 3. Scaled to
    the workload's unit (weight + activation bytes per second for decode, FLOP/s for
    prefill). Its result also checks the GPU output of those tokens (1e-2 of the largest
    magnitude, the parity bar of the expert GEMM tests)."""
    import oracle.fused_experts as OF

    threads = len(os.sched_getaffinity(0))
    torch.set_num_threads(threads)
    n = 8
    sub = ids[:n]
    used = torch.unique(sub)
    remap = torch.full((w1.shape[0],), -1, dtype=torch.int32, device=ids.device)
    remap[used.long()] = torch.arange(used.numel(), dtype=torch.int32, device=ids.device)
    xs, a, b = x[:n].cpu(), w1[used.long()].cpu(), w2[used.long()].cpu()
    ws, rs = tw[:n].cpu(), remap[sub.long()].cpu()
    ref = OF.fused_experts(xs, a, b, ws, rs)
    err = (out[:n].float().cpu() - ref.float()).abs().max().item()
    if err > 1e-2 * max(ref.float().abs().max().item(), 1e-6):
        raise RuntimeError(f"moe experts: GPU output differs from the oracle ({err})")
    times = []
    for _ in range(3):
        t0 = time.perf_counter()
        OF.fused_experts(xs, a, b, ws, rs)
        times.append(time.perf_counter() - t0)
    t = statistics.median(times)
    H, I, K = EXP_H, EXP_I, EXP_K
    nb = used.numel() * 3 * I * H * 2 + n * H * 2 * 2 + n * K * (I + H) * 2 * 2
    fl = n * K * 3 * I * H * 2
    model, phys = cpu_info()
    value, unit = (nb / t / 1e9, "GB/s") if decode else (fl / t / 1e12, "TFLOP/s")
    return {"value": round(value, 4), "unit": unit, "cores": threads, "kind": "port",
            "sample": f"first {n} of the step's tokens with their {used.numel()} experts (same "
                      f"inputs), 1 warm-up + median of 3, {t * 1e3:.1f} ms",
            "cpu_model": model, "physical_cores": phys}


KS_L, KS_H, KS_D, KS_P, KS_PPC, KS_T, KS_SEED = 36, 8, 128, 16, 16, 16384, 9


def bench_kv_sink(torch, dev, args) -> dict:
    """KV chunk sink and prefix load of the reference's KVStore on a Qwen3-8B KV cache (36
    layers x 8 KV heads x 128 dims, bf16, 16-token pages, 256-token chunks = 37.7 MB of K+V per
    chunk). One step = a finished 16384-token request sinks its 64 chunks to the host cache
    (evicting the previous step's 64, LRU) and is freed, then a new request with the same
    tokens loads the 64-chunk prefix back into fresh pages. Each direction is one page<->chunk
    launch per pool over device-mapped pinned host chunks."""
    from plastic_infer.kernel import pages_chunks_copy
    from plastic_infer.kv.kv_store import KVConfig, KVStore

    L, H, D, P, ppc, T = KS_L, KS_H, KS_D, KS_P, KS_PPC, KS_T
    C = P * ppc
    n_chunks = T // C
    cfg = KVConfig(n_layers=L, n_kv_heads=H, head_dim=D, page_size=P, pages_per_chunk=ppc,
                   max_pages=T // P * L + 1024, max_host_chunks=n_chunks, dtype=torch.bfloat16,
                   device=dev)
    store = KVStore(cfg)
    g = torch.Generator(device=dev).manual_seed(KS_SEED)
    for pool in (store.gpu.k_pages, store.gpu.v_pages):
        pool.copy_(torch.randn(pool.shape, generator=g, device=dev).to(torch.bfloat16))
    chunk_bytes = 2 * L * H * D * C * 2
    dir_bytes = n_chunks * chunk_bytes

    # kernel-only and DMA rates of one direction's bytes (K pool, all chunks)
    host = [torch.empty(L, H, D, C, dtype=torch.bfloat16, pin_memory=True) for _ in range(n_chunks)]
    ids = torch.randperm(cfg.max_pages, generator=g, device=dev)[:n_chunks * L * ppc]
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    rates = {}
    for name, to_chunk in (("d2h", True), ("h2d", False)):
        pages_chunks_copy(host, store.gpu.k_pages, ids, to_chunk=to_chunk)
        e0.record()
        pages_chunks_copy(host, store.gpu.k_pages, ids, to_chunk=to_chunk)
        e1.record()
        torch.cuda.synchronize(dev)
        rates[f"kernel_{name}_gbps"] = round(dir_bytes / 2 / (e0.elapsed_time(e1) / 1e3) / 1e9, 2)
    flat = torch.empty(n_chunks * L * H * D * C, dtype=torch.bfloat16, pin_memory=True)
    dflat = torch.empty(flat.shape, dtype=torch.bfloat16, device=dev)
    for name, (dst, src) in (("d2h", (flat, dflat)), ("h2d", (dflat, flat))):
        dst.copy_(src, non_blocking=True)
        e0.record()
        dst.copy_(src, non_blocking=True)
        e1.record()
        torch.cuda.synchronize(dev)
        rates[f"dma_{name}_gbps"] = round(dir_bytes / 2 / (e0.elapsed_time(e1) / 1e3) / 1e9, 2)
    del host, flat, dflat

    def step(i, snapshot=False):
        toks = list(range(i * T, (i + 1) * T))
        a = store.new_request()
        a._ensure_pages(T)
        a._length = T
        a.set_token_ids(toks)
        t0 = time.perf_counter()
        sunk = store.sink_completed_chunks(a)
        t1 = time.perf_counter()
        if sunk != n_chunks:
            raise RuntimeError(f"kv sink: {sunk} chunks sunk, expected {n_chunks}")
        old = [list(a.block_table.pages[l]) for l in range(L)]
        snap = (store.gpu.k_pages.clone(), store.gpu.v_pages.clone()) if snapshot else None
        store.free_request(a)
        b = store.new_request()
        t2 = time.perf_counter()
        matched, _ = store.load_prefix(b, toks)
        torch.cuda.synchronize(dev)
        t3 = time.perf_counter()
        if matched != T:
            raise RuntimeError(f"kv load: {matched} tokens matched, expected {T}")
        new = [list(b.block_table.pages[l]) for l in range(L)]
        store.free_request(b)
        return t1 - t0, t3 - t2, old, new, snap

    for i in range(args.warmup):
        step(i)
        print(f"bench: warm-up step {i + 1}/{args.warmup}", file=sys.stderr, flush=True)
    sink_s, load_s = [], []
    wall0 = time.perf_counter()
    for i in range(args.steps):
        last = i == args.steps - 1
        s_t, l_t, old, new, snap = step(args.warmup + i, snapshot=last)
        sink_s.append(s_t)
        load_s.append(l_t)
        print(f"bench: step {i + 1}/{args.steps}", file=sys.stderr, flush=True)
    wall = time.perf_counter() - wall0
    # round trip: every page of the loaded request equals the page it was sunk from
    old_t = torch.tensor(old, dtype=torch.int64, device=dev).reshape(-1)
    new_t = torch.tensor(new, dtype=torch.int64, device=dev).reshape(-1)
    for pool, ref in zip((store.gpu.k_pages, store.gpu.v_pages), snap):
        if not torch.equal(pool[new_t], ref[old_t]):
            raise RuntimeError("kv sink/load: loaded pages differ from the sunk pages")
    sink_ms = statistics.mean(sink_s) * 1e3
    load_ms = statistics.mean(load_s) * 1e3
    ms = sink_ms + load_ms
    gbps = 2 * dir_bytes / (ms / 1e3) / 1e9
    sink_gbps = dir_bytes / (sink_ms / 1e3) / 1e9
    cpu = None
    if not args.no_cpu_baseline:
        cpu = _cpu_kv_sink(torch, store, snap, old)
    return _result(
        "KV chunk sink + prefix load GB/s over the host link", gbps, "GB/s", args, ms, "bf16",
        {"workload": "qwen3-8b kv cache (36 layers x 8 kv heads x 128, bf16, 16-token pages, "
                     "256-token chunks): sink a 16384-token request's 64 chunks to pinned host "
                     "memory, then load them back as a prefix",
         "layers": L, "kv_heads": H, "head_dim": D, "page_size": P, "pages_per_chunk": ppc,
         "tokens": T},
        {"sink_ms": round(sink_ms, 3), "load_ms": round(load_ms, 3),
         "sink_gbps": round(sink_gbps, 2), "load_gbps": round(dir_bytes / (load_ms / 1e3) / 1e9, 2),
         "bytes_per_direction": dir_bytes, **rates, "wall_s_timed": round(wall, 3)},
        {"kernel": "kv_chunks_copy_kernel<uint4> (sink, pages -> pinned host chunks)",
         "bound": "host-link", "achieved": round(sink_gbps, 2), "peak": 64.0, "unit": "GB/s",
         "frac": round(sink_gbps / 64.0, 4), "traffic": None,
         "algorithmic_bytes_per_launch": dir_bytes // 2,
         "avg_launch_ms": round(sink_ms / 2, 4)}, cpu)


def _cpu_kv_sink(torch, store, snap, old) -> dict:
    """The oracle's page -> chunk copy (the reference's per-page slice copies) on the host
    cores over the K side of all chunks of the last step, from a host copy of the pool; its
    result also checks those chunks' host tensors bit for bit."""
    import oracle.paged_kv as OP

    threads = len(os.sched_getaffinity(0))
    torch.set_num_threads(threads)
    cfg = store.config
    n = len(store._host_cache)
    kp = snap[0].cpu()
    ppc = cfg.pages_per_chunk
    ids = [[old[l][c * ppc + p] for l in range(cfg.n_layers) for p in range(ppc)]
           for c in range(n)]
    t0 = time.perf_counter()
    chunks = [OP.pages_to_chunk(kp, ids[c], cfg.n_layers, ppc) for c in range(n)]
    t = time.perf_counter() - t0
    keys = list(store._host_cache)
    for c in range(n):
        if not torch.equal(store._host_cache[keys[c]][0], chunks[c]):
            raise RuntimeError("kv sink: host chunk differs from the oracle's page -> chunk copy")
    nbytes = n * chunks[0].numel() * 2
    model, phys = cpu_info()
    return {"value": round(nbytes / t / 1e9, 3), "unit": "GB/s", "cores": threads,
            "kind": "port", "sample": f"K of all {n} chunks of the last step "
                                      f"({nbytes / 1e6:.1f} MB), {t * 1e3:.1f} ms",
            "cpu_model": model, "physical_cores": phys}


HS_HQ, HS_HKV, HS_D, HS_C, HS_CHUNKS, HS_TAIL, HS_SEED = 32, 8, 128, 256, 512, 512, 11


def bench_host_stream(torch, dev, args) -> dict:
    """Long-context decode over host-resident KV (the reference's host_stream_attention_v1):
    one Qwen3-8B attention layer (32 q / 8 kv heads, D 128, bf16), 131072 context tokens in 512
    pinned host chunks of 256 tokens ([8, 128, 256] K and V each, 537 MB) plus a 512-token
    device tail; one step = one decode query row over all of it. The kernel streams the chunks
    over the host link in place (no device copy of the KV)."""
    from plastic_infer.exec.attention import host_stream_attention_v1

    Hq, Hkv, D, C, n, tail = HS_HQ, HS_HKV, HS_D, HS_C, HS_CHUNKS, HS_TAIL
    host_len = n * C
    g = torch.Generator().manual_seed(HS_SEED)
    print(f"bench: pinning {2 * host_len * Hkv * D * 2 / 1e6:.0f} MB of host chunks",
          file=sys.stderr, flush=True)
    kh = torch.empty(n, Hkv, D, C, dtype=torch.bfloat16, pin_memory=True)
    vh = torch.empty(n, Hkv, D, C, dtype=torch.bfloat16, pin_memory=True)
    kh.copy_((torch.randn(n, Hkv, D, C, generator=g) * 0.5).to(torch.bfloat16))
    vh.copy_(torch.randn(n, Hkv, D, C, generator=g).to(torch.bfloat16))
    chunks = [(kh[i], vh[i]) for i in range(n)]
    rk = (torch.randn(1, tail, Hkv, D, generator=g) * 0.5).to(torch.bfloat16)
    rv = torch.randn(1, tail, Hkv, D, generator=g).to(torch.bfloat16)
    q = torch.randn(1, 1, Hq, D, generator=g).to(torch.bfloat16)
    rk_d, rv_d, q_d = rk.to(dev), rv.to(dev), q.to(dev)
    pos = host_len + tail
    host_bytes = 2 * host_len * Hkv * D * 2
    step_bytes = host_bytes + 2 * tail * Hkv * D * 2 + 2 * Hq * D * 2

    def step():
        return host_stream_attention_v1(q_d, chunks, rk_d, rv_d, q_start_pos=pos)

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize(dev)
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
          for _ in range(args.steps)]
    stream = torch.cuda.current_stream(dev)
    wall0 = time.perf_counter()
    for a, b in ev:
        a.record(stream)
        out = step()
        b.record(stream)
    torch.cuda.synchronize(dev)
    wall = time.perf_counter() - wall0
    ms = statistics.mean(a.elapsed_time(b) for a, b in ev)
    gbps = host_bytes / (ms / 1e3) / 1e9

    # the DMA engines moving the same host bytes to HBM: the transfer a materialising
    # implementation pays before its attention even starts
    kd = torch.empty(kh.shape, dtype=kh.dtype, device=dev)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    kd.copy_(kh, non_blocking=True)
    e0.record()
    kd.copy_(kh, non_blocking=True)
    kd.copy_(vh, non_blocking=True)
    e1.record()
    torch.cuda.synchronize(dev)
    dma_ms = e0.elapsed_time(e1)
    del kd
    cpu = None
    if not args.no_cpu_baseline:
        cpu = _cpu_host_stream(torch, q, chunks, rk, rv, pos, out)
    return _result(
        "host-stream decode attention GB/s over the host link", gbps, "GB/s", args, ms, "bf16",
        {"workload": "qwen3-8b attention layer, 1 decode row over 131072 host tokens (512 pinned "
                     "chunks of 256) + 512 device tokens, 32 q / 8 kv heads, head_dim 128",
         "heads": Hq, "kv_heads": Hkv, "head_dim": D, "chunk_tokens": C, "host_chunks": n,
         "resident_tokens": tail},
        {"host_bytes_per_step": host_bytes, "bytes_per_step": step_bytes,
         "dma_same_bytes_ms": round(dma_ms, 3),
         "dma_gbps": round(host_bytes / (dma_ms / 1e3) / 1e9, 2),
         "wall_s_timed": round(wall, 3)},
        {"kernel": "hs_attn_partial<bf16, 2> + hs_attn_merge (one call)", "bound": "host-link",
         "achieved": round(gbps, 2), "peak": 64.0, "unit": "GB/s", "frac": round(gbps / 64.0, 4),
         "traffic": None, "algorithmic_bytes_per_launch": host_bytes,
         "avg_launch_ms": round(ms, 4)}, cpu)


def _cpu_host_stream(torch, q, chunks, rk, rv, pos, out) -> dict:
    """The oracle (concatenate + GQA expand + SDPA, fp32) on the host cores over the whole
    workload; its result also checks the GPU output (2e-2, the bf16 attention bar)."""
    import oracle.paged_kv as OP

    threads = len(os.sched_getaffinity(0))
    torch.set_num_threads(threads)
    f32 = [(k.float(), v.float()) for k, v in chunks]
    rkf, rvf, qf = rk.float(), rv.float(), q.float()
    t0 = time.perf_counter()
    ref = OP.host_stream_attention(qf, f32, rkf, rvf, q_start_pos=pos)
    t = time.perf_counter() - t0
    err = (out.float().cpu() - ref).abs().max().item()
    if err > 2e-2:
        raise RuntimeError(f"host stream: GPU output differs from the oracle ({err})")
    nbytes = sum(k.numel() + v.numel() for k, v in chunks) * 2
    model, phys = cpu_info()
    return {"value": round(nbytes / t / 1e9, 3), "unit": "GB/s", "cores": threads, "kind": "port",
            "sample": f"the whole step (fp32 copies of the bf16 KV), {t * 1e3:.0f} ms; max "
                      f"|GPU - oracle| {err:.2e}",
            "cpu_model": model, "physical_cores": phys}


def calibrate_copy(torch, dev) -> int:
    """A plain elementwise copy of known size (2^30 bytes read, 2^30 written per launch) for
    scaling FETCH_SIZE / WRITE_SIZE readings of the attention kernel to bytes."""
    n = (1 << 30) // 2
    src = torch.ones(n, dtype=torch.bfloat16, device=dev)
    dst = torch.empty_like(src)
    for _ in range(3):
        torch.mul(src, 1.0, out=dst)
    torch.cuda.synchronize(dev)
    print(json.dumps({"calibration": "elementwise copy", "bytes_read": 1 << 30,
                      "bytes_written": 1 << 30, "launches": 3}), flush=True)
    return 0


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--cpu-sample-seqs", type=int, default=128)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--calibrate-copy", action="store_true")
    ap.add_argument("--separate-write", action="store_true",
                    help="decode: write the new rows with kv_scatter, then attend (two calls)")
    ap.add_argument("--dtype", choices=("bf16", "fp16", "fp32"), default="bf16",
                    help="decode: storage dtype of the pools, q and the new rows (fp32: the "
                         "general tiled kernel, write and attention as two calls)")
    ap.add_argument("--workload", choices=("decode", "decode-gqa8", "prefill-write",
                                           "moe-permute", "expert-stream", "moe-experts",
                                           "moe-experts-prefill", "prefill-stream", "kv-sink",
                                           "host-stream", "decode-step", "prefill-attn",
                                           "hbm-read"),
                    default="decode")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures the paged decode path on ONE GPU (per-GPU shard of a "
              "sequence-sharded deployment); multi-GPU runs are not part of this build.",
              file=sys.stderr)
        return 2

    import torch

    from plastic_infer.kernel import (
        decode_workspace_bytes,
        kv_scatter,
        paged_decode_append_attention,
        paged_decode_attention,
    )

    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    if args.calibrate_copy:
        return calibrate_copy(torch, dev)
    if args.workload != "decode":
        run = {"decode-gqa8": bench_decode_gqa8, "prefill-write": bench_prefill_write,
               "moe-permute": bench_moe_permute, "expert-stream": bench_expert_stream,
               "moe-experts": lambda t, d, a: bench_moe_experts(t, d, a, 64),
               "moe-experts-prefill": lambda t, d, a: bench_moe_experts(t, d, a, 4096),
               "prefill-stream": bench_prefill_stream, "kv-sink": bench_kv_sink,
               "host-stream": bench_host_stream, "decode-step": bench_decode_step,
               "prefill-attn": bench_prefill_attn, "hbm-read": bench_hbm_read,
               }[args.workload]
        print(f"bench: workload {args.workload}", file=sys.stderr, flush=True)
        print(json.dumps(run(torch, dev, args)), flush=True)
        return 0
    print(f"bench: generating inputs (B={B}, pool={NUM_PAGES} pages)", file=sys.stderr, flush=True)
    kv_dtype = {"bf16": torch.bfloat16, "fp16": torch.float16, "fp32": torch.float32}[args.dtype]
    inp = build_inputs(torch, dev, kv_dtype)
    out = torch.empty(B, HQ, D, dtype=kv_dtype, device=dev)
    ws = torch.empty(decode_workspace_bytes(B, HQ, HKV, D, P, MAX_PAGES), dtype=torch.uint8, device=dev)
    stream = torch.cuda.current_stream(dev)

    # fp32 pools: the append entry point runs its write kernel and then the general kernel, so
    # the step is timed as the two calls and the attention call alone carries the roofline
    separate = args.separate_write or args.dtype == "fp32"

    def step(ev_a=None, ev_b=None):
        if separate:
            kv_scatter(inp["k_new"], inp["v_new"], inp["kp"], inp["vp"], inp["slots_d"])
        if ev_a is not None:
            ev_a.record(stream)
        if separate:
            paged_decode_attention(inp["q"], inp["kp"], inp["vp"], inp["bt_d"], inp["lens_d"],
                                   out=out, workspace=ws)
        else:
            paged_decode_append_attention(inp["q"], inp["kp"], inp["vp"], inp["bt_d"],
                                          inp["lens_d"], inp["k_new"], inp["v_new"], out=out,
                                          workspace=ws)
        if ev_b is not None:
            ev_b.record(stream)

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize(dev)
    print(f"bench: warmup done, timing {args.steps} steps", file=sys.stderr, flush=True)

    # the timed region records no event inside it; a second pass brackets each attention call
    t_start, t_end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize(dev)
    wall0 = time.perf_counter()
    t_start.record(stream)
    for _ in range(args.steps):
        step()
    t_end.record(stream)
    torch.cuda.synchronize(dev)
    wall = time.perf_counter() - wall0
    ms_step = t_start.elapsed_time(t_end) / args.steps
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
          for _ in range(args.steps)]
    for i in range(args.steps):
        step(*ev[i])
    torch.cuda.synchronize(dev)
    # the step is one launch unless the write is separate: then the attention call's events
    attn_ms = statistics.mean(a.elapsed_time(b) for a, b in ev) if separate else ms_step

    attn_bytes, scatter_bytes = algorithmic_bytes(inp["lens"], inp["n_pages"],
                                                  elem=inp["kp"].element_size())
    step_bytes = attn_bytes + scatter_bytes
    gbps = step_bytes / (ms_step / 1e3) / 1e9
    # the dominant launch: the attention call alone (separate write) or the one call that also
    # writes the new rows
    launch_bytes = attn_bytes if separate else step_bytes
    attn_gbps = launch_bytes / (attn_ms / 1e3) / 1e9
    traffic = None
    # the counter files hold the dominant launch: the one write + attention launch (bf16, fp16)
    # or the attention call alone (fp32)
    pmc_file = {"bf16": PMC_FILE, "fp16": PMC_FP16_FILE, "fp32": PMC_FP32_FILE}[args.dtype]
    if pmc_file.exists() and (args.dtype == "fp32" or not separate):
        try:
            traffic = json.loads(pmc_file.read_text()).get("hbm_bytes_per_launch")
        except (OSError, ValueError):
            traffic = None
    result = {
        "metric": "KV scatter + paged decode-attn GB/s (% of HBM peak); decode tokens/s",
        "value": round(gbps, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": args.dtype,
        "data": "synthetic (seeded N(0,1) K/V/q, seeded lengths and block tables)",
        "config": {"workload": WORKLOAD, "batch": B, "q_heads": HQ, "kv_heads": HKV,
                   "head_dim": D, "page_size": P, "context_len": f"U[{LEN_LO},{LEN_HI}]",
                   "pool_pages": NUM_PAGES, "tokens_in_context": int(inp["lens"].sum())},
        "tokens_per_s": round(B / (ms_step / 1e3), 1),
        "hbm_frac": round(gbps / HBM_PEAK_GBPS, 4),
        "bytes_per_step": step_bytes,
        "wall_s_timed": round(wall, 4),
        "step": "kv_scatter + paged_decode_attention" if separate
                else "paged_decode_append_attention (write + attention, one call)",
        "roofline": {
            "kernel": ("paged_attention_tiled<fp32, 32-key chunks, 16-byte loads> "
                       "(one attention call)" if args.dtype == "fp32" else
                       f"paged_decode_stream<4, {args.dtype}> (one attention call)"
                       if separate else f"paged_decode_stream<4, append, {args.dtype}> "
                       "(one write + attention launch)"),
            "bound": "hbm", "achieved": round(attn_gbps, 2), "peak": HBM_PEAK_GBPS,
            "unit": "GB/s", "frac": round(attn_gbps / HBM_PEAK_GBPS, 4), "traffic": traffic,
            "algorithmic_bytes_per_launch": launch_bytes, "avg_launch_ms": round(attn_ms, 4),
        },
    }
    if not args.no_cpu_baseline:
        print(f"bench: cpu baseline on {args.cpu_sample_seqs} sequences", file=sys.stderr, flush=True)
        result["cpu_baseline"] = cpu_baseline(torch, inp, args.cpu_sample_seqs, out)
        result["parity"] = {"max_abs_err": result["cpu_baseline"]["parity_max_abs_err"],
                            "tol": 2e-2, "seqs_checked": result["cpu_baseline"]["parity_seqs"],
                            "against": "oracle (reference torch path restated) on the same "
                                       "input bits, after the same scatter"}
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
