// Attention of a few query rows over KV that is split between host chunks and a device tail,
// without materialising it (reference src/plastic_infer/exec/attention.py:193-250, which
// concatenates the chunks and the tail on the device and calls SDPA).
//
// KV positions: chunk c covers [c*C, c*C + len_c) with len_c = C except the last chunk, which may
// be shorter; the resident tail follows at host_len. Chunks are [Hkv, D, len_c] (token innermost,
// the layout of a pool page with page_size len_c) at any device-readable address: HBM or pinned
// host memory through its device mapping, which the kernel then reads over the host link in
// place. The tail is token-major: row t at resident + t * token_stride holds [Hkv, D].
//
// hs_attn_partial<DT, DPL, RT>: grid (split, kv head, row tile). The KV of one kv head is cut
// into 64-token tiles (a tile never crosses a chunk); split s takes a contiguous run of tiles. A
// 256-thread workgroup stages each tile's K as [D][64] and V as [64][D] in LDS (16-byte loads,
// fetched into registers one tile ahead, where the layout allows), then its 4 waves each carry
// RT/4 of the row tile's RT query rows (row r = query i * G + g, head hk * G + g): lane = token
// for QK^T, an fp32 base-2 online softmax per row, lane = head-dim element for PV. It writes one
// (max, sum, unnormalised acc) partial per (split, query, head).
// hs_attn_merge<DT>: one 64-lane wave per (query, head) folds the splits' partials.
//
// With one row tile (decode: q_len * G <= 32) every KV byte crosses the host link once; the
// host-side wrapper stages host chunks into HBM first when several row tiles would re-read them.
#include <algorithm>

#include "pia_internal.h"

namespace pia {
namespace {

constexpr float kLog2eHs = 1.4426950408889634f;
constexpr float kNegBigHs = -1.0e30f;
constexpr int HS_SUB = 64;      // tokens per compute step (one per lane)

// Tokens per staged tile: 256-byte stored rows (128 bf16 / fp16 tokens, 64 fp32) for
// head_dim <= 128, half that above. Host reads in 128-byte pieces run at about 3/4 of the rate of
// 256-byte and longer ones, so a chunk's [d][t] rows are fetched 256 bytes at a time.
__host__ __device__ constexpr int hs_tile_tokens(int dm, int elem_bytes) {
  return (dm <= 128 ? 256 : 128) / elem_bytes;
}

struct HsGeom {
  const void* const* chunk_k;
  const void* const* chunk_v;
  const void* res_k;
  const void* res_v;
  int64_t chunk_tokens;   // C
  int64_t host_len;
  int64_t res_len;
  int64_t res_stride;     // elements between tail rows
  int64_t q_start;
  int64_t last_row;       // row length (tokens) of the last chunk as stored
  int num_chunks;         // chunks holding visible keys (a prefix of the stored ones)
  int stored_chunks;
  int tpc;                // tiles per full chunk
  int full_tiles;         // tiles of chunks 0..n-2
  int host_tiles;         // tiles of all chunks
  int total_tiles;
  int tiles_per_split;
  int chunk_vec;          // 16-byte loads valid for full chunks
  int last_vec;           // ... for the last chunk
  int res_vec;            // ... for the tail
};

template <typename T>
struct HsTile {
  const T* kb;
  const T* vb;
  int64_t pos0;     // global position of the tile's token 0
  int64_t rowlen;   // layout 0: tokens per stored (h, d) row; layout 1: elements per token row
  int tl;           // tokens in the tile
  int layout;       // 0: chunk [Hkv, D, len] (token innermost); 1: tail rows [len][Hkv, D]
  int vec;          // 16-byte loads are aligned and stay inside the stored rows
};

template <typename T, int TT>
__device__ __forceinline__ HsTile<T> hs_locate(const HsGeom& g, int tile, int hk, int D) {
  HsTile<T> f;
  if (tile < g.host_tiles) {
    int c, j;
    if (tile < g.full_tiles) {
      c = tile / g.tpc;
      j = tile - c * g.tpc;
    } else {
      c = g.num_chunks - 1;
      j = tile - g.full_tiles;
    }
    // visible tokens of chunk c vs the row length it is stored with
    const int64_t vis = c == g.num_chunks - 1 ? g.host_len - int64_t(c) * g.chunk_tokens
                                              : g.chunk_tokens;
    const bool last = c == g.stored_chunks - 1;
    const int64_t clen = last ? g.last_row : g.chunk_tokens;
    const int64_t t0 = int64_t(j) * TT;
    f.tl = int(min<int64_t>(TT, vis - t0));
    f.kb = reinterpret_cast<const T*>(g.chunk_k[c]) + int64_t(hk) * D * clen + t0;
    f.vb = reinterpret_cast<const T*>(g.chunk_v[c]) + int64_t(hk) * D * clen + t0;
    f.pos0 = int64_t(c) * g.chunk_tokens + t0;
    f.rowlen = clen;
    f.layout = 0;
    f.vec = last ? g.last_vec : g.chunk_vec;
  } else {
    const int64_t t0 = int64_t(tile - g.host_tiles) * TT;
    f.tl = int(min<int64_t>(TT, g.res_len - t0));
    f.kb = reinterpret_cast<const T*>(g.res_k) + t0 * g.res_stride + int64_t(hk) * D;
    f.vb = reinterpret_cast<const T*>(g.res_v) + t0 * g.res_stride + int64_t(hk) * D;
    f.pos0 = g.host_len + t0;
    f.rowlen = g.res_stride;
    f.layout = 1;
    f.vec = g.res_vec;
  }
  return f;
}

// 16-byte group n of a thread: layout 0 -> (d, t..t+VW), layout 1 -> (t, d..d+VW).
template <int VW, int TT>
__device__ __forceinline__ bool hs_group(int layout, int e, int D, int tl, int& d, int& t) {
  if (layout == 0) {
    constexpr int GPR = TT / VW;
    d = e / GPR;
    t = (e - d * GPR) * VW;
    return d < D && t < tl;
  }
  const int gpr = D / VW;
  t = e / gpr;
  d = (e - t * gpr) * VW;
  return t < tl;
}

template <int DT, int DPL, int RT>
__global__ __launch_bounds__(256, 2) void hs_attn_partial(
    HsGeom g, const void* __restrict__ q_, int64_t q_len, int Hq, int Hkv, int D, int causal,
    float scale_log2, float* __restrict__ part) {
  using E = Elem<DT>;
  using T = typename E::T;
  constexpr int DM = 64 * DPL;
  constexpr int VW = 16 / int(sizeof(T));
  constexpr int TT = hs_tile_tokens(DM, int(sizeof(T)));
  constexpr int NV = DM * TT / VW / 256;   // 16-byte groups per thread per tile (K or V)
  constexpr int RPW = RT / 4;                   // query rows per wave
  // tokens per compute step: one per lane, or all of a narrower tile (fp32 at head_dim > 128
  // stages 32-token tiles; lanes SUB..63 then hold no token)
  constexpr int SUB = TT < HS_SUB ? TT : HS_SUB;
  __shared__ __align__(16) T k_s[DM * TT];     // [d][t]
  __shared__ __align__(16) T v_s[TT * DM];     // [t][d]
  __shared__ float q_s[RT * DM];
  __shared__ float p_s[RT * HS_SUB];

  const T* q = reinterpret_cast<const T*>(q_);
  const int split = blockIdx.x, hk = blockIdx.y, rt = blockIdx.z;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int G = Hq / Hkv;
  const int64_t R = q_len * G;
  const int64_t r0 = int64_t(rt) * RT;

  for (int e = tid; e < RT * DM; e += 256) {
    const int r = e / DM, d = e - r * DM;
    const int64_t row = r0 + r;
    float v = 0.f;
    if (row < R && d < D) {
      const int64_t i = row / G;
      const int hq = hk * G + int(row - i * G);
      v = E::load(q, (i * Hq + hq) * D + d);
    }
    q_s[e] = v;
  }

  // rows of this wave: r0 + wave + 4k
  int64_t qpos[RPW];
  bool live[RPW];
  float m[RPW], l[RPW], acc[RPW][DPL];
#pragma unroll
  for (int k = 0; k < RPW; ++k) {
    const int64_t row = r0 + wave + 4 * k;
    live[k] = row < R;
    qpos[k] = g.q_start + (live[k] ? row / G : 0);
    m[k] = kNegBigHs;
    l[k] = 0.f;
#pragma unroll
    for (int i = 0; i < DPL; ++i) acc[k][i] = 0.f;
  }

  const int tile_lo = split * g.tiles_per_split;
  const int tile_hi = min(g.total_tiles, tile_lo + g.tiles_per_split);
  // 16-byte tiles are fetched into registers one tile ahead, so the host-link (or HBM) reads
  // of tile n+1 are in flight while tile n is computed from LDS.
  uint4 kr[NV], vr[NV];
  auto fetch = [&](const HsTile<T>& f) {
#pragma unroll
    for (int n = 0; n < NV; ++n) {
      int d, t;
      const bool ok = hs_group<VW, TT>(f.layout, tid + 256 * n, D, f.tl, d, t);
      const int64_t off = f.layout == 0 ? int64_t(d) * f.rowlen + t : int64_t(t) * f.rowlen + d;
      kr[n] = ok ? *reinterpret_cast<const uint4*>(f.kb + off) : uint4{0, 0, 0, 0};
      vr[n] = ok ? *reinterpret_cast<const uint4*>(f.vb + off) : uint4{0, 0, 0, 0};
    }
  };
  HsTile<T> cur{};
  if (tile_lo < tile_hi) {
    cur = hs_locate<T, TT>(g, tile_lo, hk, D);
    if (cur.vec) fetch(cur);
  }
  for (int tile = tile_lo; tile < tile_hi; ++tile) {
    __syncthreads();   // the previous tile's LDS reads are done
    if (cur.vec) {
#pragma unroll
      for (int n = 0; n < NV; ++n) {
        int d, t;
        if (!hs_group<VW, TT>(cur.layout, tid + 256 * n, D, cur.tl, d, t)) continue;
        const T* ke = reinterpret_cast<const T*>(&kr[n]);
        const T* ve = reinterpret_cast<const T*>(&vr[n]);
        if (cur.layout == 0) {
          *reinterpret_cast<uint4*>(&k_s[d * TT + t]) = kr[n];
#pragma unroll
          for (int x = 0; x < VW; ++x) v_s[(t + x) * DM + d] = ve[x];
        } else {
          *reinterpret_cast<uint4*>(&v_s[t * DM + d]) = vr[n];
#pragma unroll
          for (int x = 0; x < VW; ++x) k_s[(d + x) * TT + t] = ke[x];
        }
      }
    } else if (cur.layout == 0) {
      for (int e = tid; e < D * TT; e += 256) {
        const int d = e / TT, t = e - d * TT;
        if (t < cur.tl) {
          k_s[d * TT + t] = cur.kb[int64_t(d) * cur.rowlen + t];
          v_s[t * DM + d] = cur.vb[int64_t(d) * cur.rowlen + t];
        }
      }
    } else {
      for (int e = tid; e < TT * D; e += 256) {
        const int t = e / D, d = e - t * D;
        if (t < cur.tl) {
          k_s[d * TT + t] = cur.kb[int64_t(t) * cur.rowlen + d];
          v_s[t * DM + d] = cur.vb[int64_t(t) * cur.rowlen + d];
        }
      }
    }
    __syncthreads();
    const int64_t pos0 = cur.pos0;
    const int tl = cur.tl;
    if (tile + 1 < tile_hi) {
      cur = hs_locate<T, TT>(g, tile + 1, hk, D);
      if (cur.vec) fetch(cur);
    }

    // lanes past SUB read token 0 of the step (in bounds) and are masked below
    const int tok = lane < SUB ? lane : 0;
    for (int sub = 0; sub * SUB < tl; ++sub) {
      const int tls = min(SUB, tl - sub * SUB);
      // QK^T: lane = token
      float s[RPW];
#pragma unroll
      for (int k = 0; k < RPW; ++k) s[k] = 0.f;
#pragma unroll 4
      for (int d = 0; d < D; ++d) {
        const float kv = E::load(k_s, d * TT + sub * SUB + tok);
#pragma unroll
        for (int k = 0; k < RPW; ++k) s[k] = fmaf(q_s[(wave + 4 * k) * DM + d], kv, s[k]);
      }
      const int64_t pos = pos0 + sub * SUB + lane;
#pragma unroll
      for (int k = 0; k < RPW; ++k) {
        const bool valid = live[k] && lane < tls && (!causal || pos <= qpos[k]);
        const float x = valid ? s[k] * scale_log2 : -INFINITY;
        const float mnew = fmaxf(m[k], wave_max(x));
        const float alpha = __builtin_amdgcn_exp2f(m[k] - mnew);
        const float p = __builtin_amdgcn_exp2f(x - mnew);
        l[k] = l[k] * alpha + wave_sum(p);
#pragma unroll
        for (int i = 0; i < DPL; ++i) acc[k][i] *= alpha;
        m[k] = mnew;
        p_s[(wave + 4 * k) * HS_SUB + lane] = p;
      }
      // p_s rows belong to this wave alone: LDS operations of one wave complete in order
      __builtin_amdgcn_wave_barrier();
      // PV: lane = head-dim element
#pragma unroll 4
      for (int t = 0; t < tls; ++t) {
        float vv[DPL];
#pragma unroll
        for (int i = 0; i < DPL; ++i) {
          const int d = lane + 64 * i;
          vv[i] = d < D ? E::load(v_s, (sub * SUB + t) * DM + d) : 0.f;
        }
#pragma unroll
        for (int k = 0; k < RPW; ++k) {
          const float pk = p_s[(wave + 4 * k) * HS_SUB + t];
#pragma unroll
          for (int i = 0; i < DPL; ++i) acc[k][i] = fmaf(pk, vv[i], acc[k][i]);
        }
      }
      __builtin_amdgcn_wave_barrier();
    }
  }

#pragma unroll
  for (int k = 0; k < RPW; ++k) {
    if (!live[k]) continue;
    const int64_t row = r0 + wave + 4 * k;
    const int64_t i = row / G;
    const int hq = hk * G + int(row - i * G);
    float* o = part + ((int64_t(split) * q_len + i) * Hq + hq) * (D + 2);
    if (lane == 0) {
      o[0] = m[k];
      o[1] = l[k];
    }
#pragma unroll
    for (int x = 0; x < DPL; ++x) {
      const int d = lane + 64 * x;
      if (d < D) o[2 + d] = acc[k][x];
    }
  }
}

// One wave per (query, head): out = sum_s acc_s 2^(m_s - M) / sum_s l_s 2^(m_s - M).
template <int DT, int DPL>
__global__ __launch_bounds__(64) void hs_attn_merge(void* __restrict__ out_,
                                                    const float* __restrict__ part, int splits,
                                                    int64_t q_len, int Hq, int D) {
  using E = Elem<DT>;
  using T = typename E::T;
  const int64_t row = blockIdx.x;   // i * Hq + hq
  const int lane = threadIdx.x;
  const int64_t stride = q_len * Hq * int64_t(D + 2);
  const float* p = part + row * (D + 2);
  float M = kNegBigHs;
  for (int s = 0; s < splits; ++s) M = fmaxf(M, p[s * stride]);
  float L = 0.f, acc[DPL];
#pragma unroll
  for (int i = 0; i < DPL; ++i) acc[i] = 0.f;
  for (int s = 0; s < splits; ++s) {
    const float* ps = p + s * stride;
    const float w = __builtin_amdgcn_exp2f(ps[0] - M);
    L = fmaf(ps[1], w, L);
#pragma unroll
    for (int i = 0; i < DPL; ++i) {
      const int d = lane + 64 * i;
      if (d < D) acc[i] = fmaf(ps[2 + d], w, acc[i]);
    }
  }
  T* out = reinterpret_cast<T*>(out_);
#pragma unroll
  for (int i = 0; i < DPL; ++i) {
    const int d = lane + 64 * i;
    if (d < D) E::store(out, row * D + d, L > 0.f ? acc[i] / L : 0.f);
  }
}

struct HsPlan {
  int64_t kv_len, tiles, row_tiles, want;
  int tt, rt, splits, tiles_per_split;
};

// Row tile: 8 rows (2 per wave) when the kv head's rows fit, else 32. Splits: as many
// workgroups as fit on the chip at once, never more than one per tile, and balanced so every
// split takes the same number of tiles. elem_bytes 0 gives an upper bound on the split count of
// any dtype (the workspace size).
HsPlan hs_plan(int64_t q_len, int num_heads, int num_kv_heads, int head_dim, int elem_bytes,
               int num_chunks, int64_t chunk_tokens, int64_t host_len, int64_t resident_len) {
  HsPlan p{};
  p.kv_len = host_len + resident_len;
  const int dm = head_dim <= 64 ? 64 : head_dim <= 128 ? 128 : 256;
  // the smallest tile of any dtype (the widest element, fp32) when sizing the workspace
  p.tt = hs_tile_tokens(dm, elem_bytes > 0 ? elem_bytes : 4);
  const int64_t tpc = ceil_div(chunk_tokens, p.tt);
  const int64_t last = num_chunks > 0 ? host_len - int64_t(num_chunks - 1) * chunk_tokens : 0;
  p.tiles = (num_chunks > 0 ? int64_t(num_chunks - 1) * tpc + ceil_div(last, p.tt) : 0) +
            ceil_div(resident_len, p.tt);
  const int G = num_heads / num_kv_heads;
  p.rt = q_len * G <= 8 ? 8 : 32;
  p.row_tiles = ceil_div(q_len * G, p.rt);
  // workgroups per CU: the launch bounds (2) or the LDS, whichever
  // is smaller
  int occ = 4;
  if (elem_bytes > 0) {
    const int lds = 2 * dm * p.tt * elem_bytes + p.rt * dm * 4 + p.rt * HS_SUB * 4;
    occ = std::max(1, std::min(2, 160 * 1024 / lds));
  }
  p.want = ceil_div(int64_t(device_cus()) * occ, int64_t(num_kv_heads) * p.row_tiles);
  const int64_t splits = std::max<int64_t>(1, std::min<int64_t>(p.want, p.tiles));
  p.tiles_per_split = int(ceil_div(std::max<int64_t>(p.tiles, 1), splits));
  p.splits = int(ceil_div(std::max<int64_t>(p.tiles, 1), p.tiles_per_split));
  return p;
}

int hs_check(int64_t q_len, int num_heads, int num_kv_heads, int head_dim, int num_chunks,
             int64_t chunk_tokens, int64_t host_len, int64_t resident_len) {
  if (q_len < 0 || num_chunks < 0 || host_len < 0 || resident_len < 0)
    return fail(PIA_EINVAL, "host_stream_attention: negative size");
  if (num_heads <= 0 || num_kv_heads <= 0 || num_heads % num_kv_heads)
    return fail(PIA_EINVAL, "host_stream_attention: num_heads must be a positive multiple of "
                            "num_kv_heads");
  if (head_dim <= 0 || head_dim > 256)
    return fail(PIA_EUNSUPPORTED, "host_stream_attention: head_dim must be in [1, 256]");
  if (num_chunks > 0) {
    if (chunk_tokens <= 0) return fail(PIA_EINVAL, "host_stream_attention: chunk_tokens <= 0");
    const int64_t last = host_len - int64_t(num_chunks - 1) * chunk_tokens;
    if (last <= 0 || last > chunk_tokens)
      return fail(PIA_EINVAL, "host_stream_attention: host_len must put 1..chunk_tokens tokens "
                              "in the last chunk");
  } else if (host_len != 0) {
    return fail(PIA_EINVAL, "host_stream_attention: host_len > 0 without chunks");
  }
  if (ceil_div(host_len + resident_len, HS_SUB) + num_chunks > 0x7fffffff)
    return fail(PIA_EINVAL, "host_stream_attention: KV too long");
  return 0;
}

// tiles == 0 (no visible key): only the merge runs, over zero splits, and writes zeros.
template <int DT>
int hs_launch(const HsGeom& g, const HsPlan& p, void* out, const void* q, int64_t q_len, int Hq,
              int Hkv, int D, int causal, float scale_log2, float* part, hipStream_t s) {
  const dim3 grid(unsigned(p.splits), unsigned(Hkv), unsigned(p.row_tiles));
  const unsigned rows = unsigned(q_len * Hq);
  const int splits = p.tiles > 0 ? p.splits : 0;
#define PIA_HS(DPL)                                                                           \
  do {                                                                                        \
    if (splits > 0) {                                                                         \
      if (p.rt == 8)                                                                          \
        hipLaunchKernelGGL((hs_attn_partial<DT, DPL, 8>), grid, dim3(256), 0, s, g, q, q_len, \
                           Hq, Hkv, D, causal, scale_log2, part);                             \
      else                                                                                    \
        hipLaunchKernelGGL((hs_attn_partial<DT, DPL, 32>), grid, dim3(256), 0, s, g, q,       \
                           q_len, Hq, Hkv, D, causal, scale_log2, part);                      \
      if (int rc = check_launch("hs_attn_partial")) return rc;                                \
    }                                                                                         \
    hipLaunchKernelGGL((hs_attn_merge<DT, DPL>), dim3(rows), dim3(64), 0, s, out, part,       \
                       splits, q_len, Hq, D);                                                 \
  } while (0)
  if (D <= 64) PIA_HS(1);
  else if (D <= 128) PIA_HS(2);
  else PIA_HS(4);
#undef PIA_HS
  return check_launch("hs_attn_merge");
}

}  // namespace
}  // namespace pia

using namespace pia;

extern "C" int64_t pia_host_stream_attention_workspace_bytes(int64_t q_len, int num_heads,
                                                             int num_kv_heads, int head_dim,
                                                             int num_chunks, int64_t chunk_tokens,
                                                             int64_t host_len,
                                                             int64_t resident_len) {
  if (hs_check(q_len, num_heads, num_kv_heads, head_dim, num_chunks, chunk_tokens, host_len,
               resident_len))
    return -1;
  // Causal clipping in the call only removes tiles; min(want, tiles) bounds the splits of any
  // clipped plan.
  const HsPlan p = hs_plan(q_len, num_heads, num_kv_heads, head_dim, 0, num_chunks,
                           chunk_tokens, host_len, resident_len);
  const int64_t bound = std::max<int64_t>(1, std::min<int64_t>(p.want, p.tiles));
  return bound * q_len * num_heads * (head_dim + 2) * int64_t(sizeof(float));
}

extern "C" int pia_host_stream_attention(
    void* out, const void* q, int64_t q_len, int num_heads, const void* const* chunk_k,
    const void* const* chunk_v, int num_chunks, int64_t chunk_tokens, int64_t host_len,
    const void* resident_k, const void* resident_v, int64_t resident_len,
    int64_t resident_token_stride, int num_kv_heads, int head_dim, int64_t q_start_pos,
    int causal, float scale, int dtype, void* workspace, int64_t workspace_bytes, void* stream) {
  if (int rc = hs_check(q_len, num_heads, num_kv_heads, head_dim, num_chunks, chunk_tokens,
                        host_len, resident_len))
    return rc;
  if (dtype != PIA_DTYPE_F32 && dtype != PIA_DTYPE_F16 && dtype != PIA_DTYPE_BF16)
    return fail(PIA_EINVAL, "host_stream_attention: unknown dtype");
  if (q_len == 0) return 0;
  if (!out || !q) return fail(PIA_EINVAL, "host_stream_attention: null q / out");
  if (num_chunks > 0 && (!chunk_k || !chunk_v))
    return fail(PIA_EINVAL, "host_stream_attention: null chunk table");
  if (resident_len > 0) {
    if (!resident_k || !resident_v)
      return fail(PIA_EINVAL, "host_stream_attention: null resident tail");
    if (resident_token_stride < int64_t(num_kv_heads) * head_dim)
      return fail(PIA_EINVAL, "host_stream_attention: resident_token_stride < num_kv_heads * "
                              "head_dim");
  }
  const int stored_chunks = num_chunks;
  const int64_t last_row =
      num_chunks > 0 ? host_len - int64_t(num_chunks - 1) * chunk_tokens : 0;
  if (causal) {
    // keys at positions >= q_start_pos + q_len are visible to no row: drop them
    const int64_t visible = std::max<int64_t>(0, q_start_pos + q_len);
    if (visible <= host_len) {
      num_chunks = int(ceil_div(visible, std::max<int64_t>(chunk_tokens, 1)));
      host_len = visible;
      resident_len = 0;
    } else {
      resident_len = std::min(resident_len, visible - host_len);
    }
  }
  const int eb = dtype == PIA_DTYPE_F32 ? 4 : 2;
  const HsPlan p = hs_plan(q_len, num_heads, num_kv_heads, head_dim, eb, num_chunks,
                           chunk_tokens, host_len, resident_len);
  const int64_t need = int64_t(p.splits) * q_len * num_heads * (head_dim + 2) * 4;
  if (!workspace || workspace_bytes < need || !aligned(workspace, 4))
    return fail(PIA_EINVAL, "host_stream_attention: workspace too small or misaligned");
  if (p.row_tiles > 65535) return fail(PIA_EINVAL, "host_stream_attention: too many query rows");
  if (q_len * num_heads > 0x7fffffff)
    return fail(PIA_EINVAL, "host_stream_attention: too many query rows");

  HsGeom g{};
  g.chunk_k = chunk_k;
  g.chunk_v = chunk_v;
  g.res_k = resident_k;
  g.res_v = resident_v;
  g.chunk_tokens = chunk_tokens;
  g.host_len = host_len;
  g.res_len = resident_len;
  g.res_stride = resident_token_stride;
  g.q_start = q_start_pos;
  g.last_row = last_row;
  g.num_chunks = num_chunks;
  g.stored_chunks = stored_chunks;
  g.tpc = num_chunks > 0 ? int(ceil_div(chunk_tokens, p.tt)) : 0;
  g.full_tiles = num_chunks > 0 ? (num_chunks - 1) * g.tpc : 0;
  g.host_tiles = num_chunks > 0
                     ? g.full_tiles + int(ceil_div(host_len - int64_t(num_chunks - 1) *
                                                              chunk_tokens, p.tt))
                     : 0;
  g.total_tiles = int(p.tiles);
  g.tiles_per_split = p.tiles_per_split;
  // Chunk bases must be 16-byte aligned (documented); rows of a chunk then are whenever the row
  // length in bytes is a multiple of 16.
  g.chunk_vec = (chunk_tokens * eb) % 16 == 0;
  g.last_vec = (last_row * eb) % 16 == 0;
  g.res_vec = resident_len > 0 && (resident_token_stride * eb) % 16 == 0 &&
              (int64_t(head_dim) * eb) % 16 == 0 && aligned(resident_k, 16) &&
              aligned(resident_v, 16);
  const float sl2 = scale * kLog2eHs;
  float* part = reinterpret_cast<float*>(workspace);
  hipStream_t s = as_stream(stream);
  switch (dtype) {
    case PIA_DTYPE_F32:
      return hs_launch<PIA_DTYPE_F32>(g, p, out, q, q_len, num_heads, num_kv_heads, head_dim,
                                      causal, sl2, part, s);
    case PIA_DTYPE_F16:
      return hs_launch<PIA_DTYPE_F16>(g, p, out, q, q_len, num_heads, num_kv_heads, head_dim,
                                      causal, sl2, part, s);
    default:
      return hs_launch<PIA_DTYPE_BF16>(g, p, out, q, q_len, num_heads, num_kv_heads, head_dim,
                                       causal, sl2, part, s);
  }
}
