"""plastic_infer (MI355X build): the paged-KV and expert-cache data path of plastic-infer,
re-implemented as hand-written HIP kernels for gfx950 behind the reference's Python API.

Subpackages mirror the reference's import paths:
  kv        page allocator, block tables, chunk keys, the HBM KV store
  exec      paged attention / MoE routing ops and the runner's KV call sites
  moe       fused-MoE routing front end
  store     LRU residency and the expert slot pool
  planning  storage tiers
  kernel    batched entry points over libplastic_infer_amd.so
Every tensor op runs on a HIP device through the library; there is no host execution path.
"""

__version__ = "0.1.0"
