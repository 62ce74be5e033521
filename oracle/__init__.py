"""ORACLE — test infrastructure only.

A CPU restatement of the reference's algorithm for the paged-KV / expert-cache data path
(zuver-lab/plastic-infer), written from the reference's semantics, each function citing the
reference file:line it follows. It exists to CHECK the HIP library, and is imported only by
tests/, by __graft_entry__.smoke() and by the cpu_baseline leg of bench.py. Nothing in the
product package (plastic-infer_amd/plastic_infer) imports it, and the product never falls
back to it.

Modules:
  paged_kv     slot scatter, block-table gather, gather+GQA+SDPA paged attention (torch CPU)
  moe_route    router top-k, moe_align_block_size permute plan, permute / unpermute (numpy)
  expert_copy  row index copy and the ExpertSlotPool LRU policy (numpy / pure Python)
  workloads    the seeded synthetic inputs of the benchmark configurations

Pinning status (what checks each function; see tests/test_oracle_*.py):
  paged_kv.scatter_slots / write_kv_layer  pinned: placement KATs of the reference tests,
                                           scatter->gather round trip, planted-mistake checks
  paged_kv.gather_paged_kv                 pinned: page-order / partial-page / empty KATs
  paged_kv.paged_attention / decode_batch  pinned: fp64 brute-force loops, contiguous-SDPA KAT,
                                           GQA head mapping, single-key and uniform-value
                                           closed forms
  moe_route.fused_topk / topk_route        pinned: reference KAT logits, closed forms
  moe_route.moe_align_block_size           pinned: the reference docstring's worked example,
                                           invariants (counts, padding, sortedness, bijection)
  moe_route.permute / unpermute            pinned: closed forms (identity expert => sum of weights
                                           times hidden), brute-force loops
  expert_copy.index_copy_rows              pinned: brute force
  expert_copy.SlotPoolPolicy               pinned: the reference's ExpertSlotPool test sequences
"""
