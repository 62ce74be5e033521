// HBM streaming-read probe (a measurement aid; no counterpart in the reference): the read rate
// the machine sustains for two access patterns, which puts every "fraction of the 8 TB/s peak"
// of the path's kernels in context. A persistent grid of four 256-thread workgroups per CU
// reads with 16-byte non-temporal loads and folds what it read with XOR so the loads are not elided; the
// fold is stored only if it equals a pattern the caller's data never produces in practice (the
// store keeps the loads alive for the compiler).
//   flat:  the buffer front to back, grid-stride, four loads in flight per thread;
//   tiles: 4 KiB tiles at the given tile indices (the paged-KV access: a page of one kv head is
//          a 4 KiB tile at bf16 / head_dim 128 / page 16), one wave per tile, two tiles in
//          flight per wave (each lane 4 x 16 bytes of each).
//   rows:  16-row blocks (16 x row_bytes, contiguous; a weight tile of the expert GEMMs), one
//          wave per block, four loads in flight per lane, each load instruction shaped as R
//          rows x 1024 / R bytes: R = 16 is the MFMA operand layout (lane l reads a 16-byte
//          vector of row l % 16), R = 1 reads 1 KiB of the block contiguously. Same bytes and
//          the same grid for every R, so the rates compare the load shape alone.
#include <algorithm>

#include "pia_internal.h"

namespace pia {
namespace {

constexpr int HP_THREADS = 256;
constexpr int HP_WGS_PER_CU = 4;
constexpr int HP_UNROLL = 4;

typedef uint32_t hp_u32x4 __attribute__((ext_vector_type(4)));

// 16-byte load with the non-temporal hint (data read once), as the path's streaming kernels do.
__device__ __forceinline__ uint4 hp_load(const uint4* p) {
  const hp_u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const hp_u32x4*>(p));
  return make_uint4(v.x, v.y, v.z, v.w);
}

__global__ __launch_bounds__(HP_THREADS) void hbm_read_probe_kernel(const uint4* __restrict__ p,
                                                                    int64_t n16,
                                                                    uint32_t* __restrict__ sink) {
  uint32_t acc = 0;
  const int64_t step = int64_t(gridDim.x) * HP_THREADS;
  for (int64_t i = int64_t(blockIdx.x) * HP_THREADS + threadIdx.x; i < n16;
       i += step * HP_UNROLL) {
    uint4 v[HP_UNROLL];
#pragma unroll
    for (int u = 0; u < HP_UNROLL; ++u) {
      const int64_t j = i + u * step;
      v[u] = j < n16 ? hp_load(p + j) : make_uint4(0u, 0u, 0u, 0u);
    }
#pragma unroll
    for (int u = 0; u < HP_UNROLL; ++u) acc ^= v[u].x ^ v[u].y ^ v[u].z ^ v[u].w;
  }
  if (acc == 0x9e3779b9u) sink[0] = acc;
}

__global__ __launch_bounds__(HP_THREADS) void hbm_read_tiles_kernel(
    const uint4* __restrict__ p, int64_t n_pool_tiles, const int32_t* __restrict__ ids,
    int64_t n_tiles, uint32_t* __restrict__ sink) {
  constexpr int WAVES = HP_THREADS / 64;
  const int lane = threadIdx.x & 63;
  const int64_t nw = int64_t(gridDim.x) * WAVES;
  uint32_t acc = 0;
  for (int64_t t = int64_t(blockIdx.x) * WAVES + (threadIdx.x >> 6); t < n_tiles; t += 2 * nw) {
    const int64_t t2 = t + nw;
    const int32_t a = ids[t], b = t2 < n_tiles ? ids[t2] : -1;
    const bool a_ok = a >= 0 && a < n_pool_tiles, b_ok = b >= 0 && b < n_pool_tiles;
    const uint4* pa = p + int64_t(a_ok ? a : 0) * 256;
    const uint4* pb = p + int64_t(b_ok ? b : 0) * 256;
    uint4 v[8];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      v[u] = a_ok ? hp_load(pa + lane + 64 * u) : make_uint4(0u, 0u, 0u, 0u);
      v[4 + u] = b_ok ? hp_load(pb + lane + 64 * u) : make_uint4(0u, 0u, 0u, 0u);
    }
#pragma unroll
    for (int u = 0; u < 8; ++u) acc ^= v[u].x ^ v[u].w;
  }
  if (acc == 0x9e3779b9u) sink[0] = acc;
}

// 16-row blocks, R rows per load instruction (64 / R lanes, 1024 / R contiguous bytes per row);
// R = 1: 1 KiB of the block per instruction. row16 = row_bytes / 16, a multiple of 64 / R (and
// of 4). The block's loads go group by group (R rows each; R = 1: one group, the whole block),
// HP_UNROLL in flight per lane; the per-lane offset is fixed, so every shape costs the same
// address arithmetic per load.
template <int R>
__global__ __launch_bounds__(HP_THREADS) void hbm_read_rows_kernel(const uint4* __restrict__ p,
                                                                   int64_t n_blocks, int row16,
                                                                   uint32_t* __restrict__ sink) {
  constexpr int WAVES = HP_THREADS / 64, LPR = 64 / R, NG = R == 1 ? 1 : 16 / R;
  const int lane = threadIdx.x & 63;
  const int block16 = 16 * row16, per_group = row16 / 4 / NG;  // instructions per group
  const int lane_off = R == 1 ? lane : (lane / LPR) * row16 + lane % LPR;
  const int group16 = R == 1 ? 0 : R * row16;
  uint32_t acc = 0;
  for (int64_t b = int64_t(blockIdx.x) * WAVES + (threadIdx.x >> 6); b < n_blocks;
       b += int64_t(gridDim.x) * WAVES) {
    for (int g = 0; g < NG; ++g) {
      const uint4* base = p + b * block16 + g * group16 + lane_off;
      for (int c = 0; c < per_group; c += HP_UNROLL) {
        uint4 v[HP_UNROLL];
#pragma unroll
        for (int u = 0; u < HP_UNROLL; ++u)
          v[u] = hp_load(base + (c + u < per_group ? c + u : per_group - 1) * LPR);
#pragma unroll
        for (int u = 0; u < HP_UNROLL; ++u) acc ^= v[u].x ^ v[u].w;
      }
    }
  }
  if (acc == 0x9e3779b9u) sink[0] = acc;
}

}  // namespace
}  // namespace pia

using namespace pia;

extern "C" int pia_hbm_read_probe(const void* src, int64_t bytes, const int32_t* tile_ids,
                                  int64_t n_tiles, uint32_t* sink, void* stream) {
  if (!src || !sink) return fail(PIA_EINVAL, "hbm_read_probe: null pointer");
  if (bytes <= 0 || bytes % 16)
    return fail(PIA_EINVAL, "hbm_read_probe: bytes must be a positive multiple of 16");
  if (!aligned(src, 16) || !aligned(sink, 4))
    return fail(PIA_EINVAL, "hbm_read_probe: src must be 16-byte aligned, sink 4-byte aligned");
  const unsigned full_grid = unsigned(int64_t(device_cus()) * HP_WGS_PER_CU);
  if (tile_ids) {  // 4 KiB tiles of the buffer; ids outside it are skipped
    if (n_tiles < 0) return fail(PIA_EINVAL, "hbm_read_probe: n_tiles < 0");
    if (n_tiles == 0) return 0;
    const int64_t waves = ceil_div(n_tiles, 2);
    const unsigned grid =
        unsigned(std::min<int64_t>(ceil_div(waves, HP_THREADS / 64), int64_t(full_grid)));
    hipLaunchKernelGGL(hbm_read_tiles_kernel, dim3(grid), dim3(HP_THREADS), 0, as_stream(stream),
                       reinterpret_cast<const uint4*>(src), bytes / 4096, tile_ids, n_tiles,
                       sink);
    return check_launch("hbm_read_probe");
  }
  const int64_t n16 = bytes / 16;
  const int64_t need = ceil_div(n16, HP_THREADS);
  const unsigned grid = unsigned(std::min<int64_t>(need, int64_t(full_grid)));
  hipLaunchKernelGGL(hbm_read_probe_kernel, dim3(grid), dim3(HP_THREADS), 0, as_stream(stream),
                     reinterpret_cast<const uint4*>(src), n16, sink);
  return check_launch("hbm_read_probe");
}

extern "C" int pia_hbm_read_rows_probe(const void* src, int64_t bytes, int row_bytes,
                                       int rows_per_load, uint32_t* sink, void* stream) {
  if (!src || !sink) return fail(PIA_EINVAL, "hbm_read_rows_probe: null pointer");
  const int R = rows_per_load;
  if (R != 1 && R != 2 && R != 4 && R != 8 && R != 16)
    return fail(PIA_EINVAL, "hbm_read_rows_probe: rows_per_load must be 1, 2, 4, 8 or 16");
  if (row_bytes <= 0 || row_bytes % 64 || (R > 1 && row_bytes % (1024 / R)))
    return fail(PIA_EINVAL, "hbm_read_rows_probe: row_bytes must be a positive multiple of 64 "
                            "and of 1024 / rows_per_load");
  if (bytes < 16 * int64_t(row_bytes))
    return fail(PIA_EINVAL, "hbm_read_rows_probe: bytes must hold one 16-row block");
  if (!aligned(src, 16) || !aligned(sink, 4))
    return fail(PIA_EINVAL, "hbm_read_rows_probe: src must be 16-byte aligned, sink 4-byte aligned");
  const int64_t n_blocks = bytes / (16 * int64_t(row_bytes));
  const int64_t waves_per_wg = HP_THREADS / 64;
  const unsigned grid = unsigned(std::min<int64_t>(ceil_div(n_blocks, waves_per_wg),
                                                   int64_t(device_cus()) * 2));
  const uint4* p = reinterpret_cast<const uint4*>(src);
  const int row16 = row_bytes / 16;
  hipStream_t s = as_stream(stream);
  switch (R) {
    case 1: hipLaunchKernelGGL(hbm_read_rows_kernel<1>, dim3(grid), dim3(HP_THREADS), 0, s, p, n_blocks, row16, sink); break;
    case 2: hipLaunchKernelGGL(hbm_read_rows_kernel<2>, dim3(grid), dim3(HP_THREADS), 0, s, p, n_blocks, row16, sink); break;
    case 4: hipLaunchKernelGGL(hbm_read_rows_kernel<4>, dim3(grid), dim3(HP_THREADS), 0, s, p, n_blocks, row16, sink); break;
    case 8: hipLaunchKernelGGL(hbm_read_rows_kernel<8>, dim3(grid), dim3(HP_THREADS), 0, s, p, n_blocks, row16, sink); break;
    default: hipLaunchKernelGGL(hbm_read_rows_kernel<16>, dim3(grid), dim3(HP_THREADS), 0, s, p, n_blocks, row16, sink); break;
  }
  return check_launch("hbm_read_rows_probe");
}
