// Paged GQA attention over the KV pool layout [num_pages, Hkv, D, P] (token innermost).
//
// 1. paged_decode_stream<G> (G = Hq/Hkv in {1,2,4}): the decode hot path for bf16 and fp16,
//    D = 128, P = 16 (described where it is defined): the batch's 128-token steps split over persistent
//    single waves (a fixed, XCD-aware split), two per SIMD. Per 8-page (128-token) step:
//      K tile loads: lane l reads page l/8, rows d = 4i + (l&3), token half (l>>2)&1, so load i
//        of the wave covers one whole 128-byte line of each of the 8 pages (32 loads / 8 pages).
//      QK^T: pairs of rows (d, d+4) are packed per token with v_perm, then v_dot2_f32_bf16
//        against (q[d], q[d+4]); partial sums over the 4 row subsets are folded by two DPP
//        quad exchanges, after which lane l owns the scores of tokens 2l and 2l+1.
//      Softmax: fp32, base-2 with the scale folded in; wave max by DPP/shuffles.
//      PV: lane l reads V rows d = 32j + l/2, token half l&1 (1 KiB contiguous per load); the
//        probabilities of its 8 tokens come from LDS as bf16 pairs, v_dot2 accumulates in fp32.
//    Segments cut by a wave-range boundary leave (max, sum, unnormalised acc) partials; the
//    wave that writes a segment's last partial merges them in the same launch.
//    Block-table ids outside [0, num_pages) inside a context are not dereferenced: their tokens
//    are not keys (score -inf, V zeroed); a row with no key at all is written as zeros.
// 2. paged_decode_mfma<G> (G = 3, 5..8, 16): the same split, cursor, partials and merge, with
//    the tile work of a step on the matrix cores (QK^T and PV as 16x16x32 MFMAs, K through a
//    swizzled LDS tile and transposing reads, V straight into the MFMA operand registers).
// 3. paged_attention_tiled<DT, C, VEC, R>: everything else up to head_dim 512 and G * head_dim
//    8192 (any dtype and page size, several query rows per sequence with optional causal
//    offsets). One workgroup per (query row, kv head) serves its G q heads from K / V chunks of
//    C keys staged once in LDS (described where it is defined).
// 4. paged_attention_generic<DT, DPL>: what the tiled kernel's LDS or register budget does not
//    take (G * head_dim above 8192). One wave per (query row, head); keys are processed 64 at a
//    time (lane = key for QK, lane = head-dim element for PV).
#include <algorithm>
#include <atomic>
#include <mutex>
#include <random>
#include <type_traits>

#include "attn_tiles.h"
#include "pia_internal.h"

namespace pia {
namespace {

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kNegBig = -1.0e30f;  // finite "no key yet" running max (avoids inf - inf)

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

// 16-byte streaming load (KV tiles are read once per launch: non-temporal hint).
__device__ __forceinline__ uint4 load16_nt(const uint16_t* p) {
  const u32x4_t v = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(p));
  return uint4{v.x, v.y, v.z, v.w};
}

__device__ __forceinline__ float dot2_bf16(uint32_t a, uint32_t b, float c) {
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, a),
                                         __builtin_bit_cast(bf16x2_t, b), c, false);
}

// DPP lane exchanges within a quad (row_mask/bank_mask all lanes, every source lane valid).
template <int CTRL>
__device__ __forceinline__ float dpp_f32(float x) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), CTRL, 0xF, 0xF, false));
}
constexpr int kDppQuadXor1 = 0xB1;  // quad_perm [1,0,3,2]
constexpr int kDppQuadXor2 = 0x4E;  // quad_perm [2,3,0,1]
constexpr int kDppRowRor4 = 0x124;  // row_ror:4
constexpr int kDppRowRor8 = 0x128;  // row_ror:8

// Max over all 64 lanes: quad xor by DPP, rows of 16 by DPP rotations, then across rows.
__device__ __forceinline__ float wave_max_dpp(float v) {
  v = fmaxf(v, dpp_f32<kDppQuadXor1>(v));
  v = fmaxf(v, dpp_f32<kDppQuadXor2>(v));
  v = fmaxf(v, dpp_f32<kDppRowRor4>(v));
  v = fmaxf(v, dpp_f32<kDppRowRor8>(v));
  v = fmaxf(v, __shfl_xor(v, 16, 64));
  v = fmaxf(v, __shfl_xor(v, 32, 64));
  return v;
}
__device__ __forceinline__ float wave_sum_dpp(float v) {
  v += dpp_f32<kDppQuadXor1>(v);
  v += dpp_f32<kDppQuadXor2>(v);
  v += dpp_f32<kDppRowRor4>(v);
  v += dpp_f32<kDppRowRor8>(v);
  v += __shfl_xor(v, 16, 64);
  v += __shfl_xor(v, 32, 64);
  return v;
}

// (lo16(a), lo16(c)) and (hi16(a), hi16(c)) — v_perm_b32 byte selects over {S0 = c, S1 = a}.
__device__ __forceinline__ uint32_t pack_lo(uint32_t a, uint32_t c) {
  return __builtin_amdgcn_perm(c, a, 0x05040100u);
}
__device__ __forceinline__ uint32_t pack_hi(uint32_t a, uint32_t c) {
  return __builtin_amdgcn_perm(c, a, 0x07060302u);
}

// Two f32 -> one bf16x2 word, round to nearest even (one v_cvt_pk_bf16_f32 on gfx950).
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  const bf16x2_t p = {static_cast<__bf16>(lo), static_cast<__bf16>(hi)};
  return __builtin_bit_cast(uint32_t, p);
}

// The fast kernels' two 16-bit storage types, DT = PIA_DTYPE_BF16 or PIA_DTYPE_F16: a dot
// product of two element pairs accumulated in fp32, two fp32 packed into a pair and one fp32
// rounded (both to nearest even), and one element (the low 16 bits) widened to fp32.
typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));
template <int DT>
__device__ __forceinline__ float dot2(uint32_t a, uint32_t b, float c) {
  if constexpr (DT == PIA_DTYPE_F16)
    return __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2_t, a), __builtin_bit_cast(f16x2_t, b),
                                  c, false);
  else
    return dot2_bf16(a, b, c);
}
template <int DT>
__device__ __forceinline__ uint32_t pack2(float lo, float hi) {
  return tile::pack16x2<DT>(lo, hi);
}
template <int DT>
__device__ __forceinline__ uint16_t to16(float v) {
  if constexpr (DT == PIA_DTYPE_F16) return f32_to_half(v);
  else return f32_to_bf16(v);
}
template <int DT>
__device__ __forceinline__ float from16(uint32_t x) {
  if constexpr (DT == PIA_DTYPE_F16) return half_to_f32(uint16_t(x & 0xffffu));
  else return __uint_as_float((x & 0xffffu) << 16);
}

// 2^x with the hardware v_exp_f32 (no denormal-range fix-up branches): softmax arguments are
// <= 0, results below 2^-126 flush to 0 and exp2(-inf) = 0.
__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// Branch-free per-lane select: (a & m) | (b & ~m), one v_bfi_b32.
__device__ __forceinline__ float bsel(uint32_t m, float a, float b) {
  return __uint_as_float((__float_as_uint(a) & m) | (__float_as_uint(b) & ~m));
}

// Reduce-scatter of per-lane partial scores over a quad of lanes. On entry lane l of a quad
// holds partial sums s[t][g] for the quad's 8 tokens t (each lane a different subset of the
// head dimension); on exit r[0][g], r[1][g] are the quad-wide sums for tokens 2q and 2q + 1,
// q = l & 3 (lanes exchange the half they do not keep: xor 2, then xor 1).
template <int G>
__device__ __forceinline__ void quad_reduce_scatter(const float (&s)[8][G], float (&r)[2][G],
                                                    int lane) {
  const uint32_t m2 = 0u - uint32_t((lane >> 1) & 1);  // keep tokens 4..7
  const uint32_t m1 = 0u - uint32_t(lane & 1);         // keep the upper pair of the four
#pragma unroll
  for (int g = 0; g < G; ++g) {
    float h[4];
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      const float keep = bsel(m2, s[4 + t][g], s[t][g]);
      const float send = bsel(m2, s[t][g], s[4 + t][g]);
      h[t] = keep + dpp_f32<kDppQuadXor2>(send);
    }
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      const float keep = bsel(m1, h[2 + t], h[t]);
      const float send = bsel(m1, h[t], h[2 + t]);
      r[t][g] = keep + dpp_f32<kDppQuadXor1>(send);
    }
  }
}

using tile::mask_pair;

constexpr int FD_D = 128;
constexpr int FD_P = 16;
constexpr int FD_PAGES_PER_WAVE = 8;  // pages of one 128-token step

__device__ __forceinline__ int clamp_len(int L, int64_t bt_stride, int P) {
  const int64_t cap = bt_stride * P;
  if (L < 0) return 0;
  return int64_t(L) > cap ? int(cap) : L;
}

// ---------------------------------------------------------------------------------------------
// Stream decode kernel: persistent single waves over an even split of the batch.
//
// The work of a launch is the ordered list of 128-token steps of every (sequence, kv head)
// segment, sequence-major then head then step: T = Hkv * sum_b ceil(L_b / 128) steps. Wave w of
// the NW launched (every CU full at two single-wave workgroups per SIMD) walks one contiguous
// range of the list, so every wave streams about the same number of KV bytes whatever the mix
// of context lengths. Two measured effects shape the split:
//   - Waves are dispatched to XCD w % 8, and the odd XCDs finish the same work about 8 % later
//     than the even ones (the last ~50 us of an even split ran on odd XCDs only, at ~4.8 TB/s).
//     So waves pair up as (2p, 2p + 1), one on an even and one on an odd XCD: the pair takes
//     Dp = ceil(2T / NW) steps, the even wave the first Ce = 51.5 % of them, the odd one the rest.
//   - The older of the two waves of a SIMD wins issue arbitration. Each wave sets its priority
//     from its progress (quartiles of its range: 3 down to 0), so a wave that has fallen behind
//     gets the issue slots first.
// Both only move the point where the waves finish; results do not depend on them beyond the
// fixed split. Only the first step of a wave waits on a prologue: the next step's block-table row (and its q, when it opens a segment) is fetched one
// step ahead and its K tiles are prefetched during the current step's PV, across segment
// boundaries. Per step the tile work uses the lane mappings above in four 16 KiB load groups,
// K rows 0..63 (ka), K rows 64..127 (kb), V of pages 0..3 (va), V of pages 4..7 (vb):
//     QK(ka) | issue va | QK(kb) | softmax | issue vb | PV(va) | issue ka' | PV(vb) | issue kb'
// so about 32 KiB stay in flight per wave through the compute, with 128 VGPRs of tile data.
// A segment that lies inside one wave's range is finished there (output written directly); a
// segment cut by a range boundary leaves (max, sum, unnormalised acc) partials, at most two per
// wave: slot 0 for the segment that began before the wave's range, slot 1 for the one that
// began inside it and continues after. The wave that writes a segment's last partial merges
// them (see sd_arrive), in the same launch: no second kernel, no launch gap.
//
// Range of wave w (steps): pair p = w / 2 covers [p*Dp, (p+1)*Dp); the even wave [p*Dp, p*Dp+Ce),
// the odd wave [p*Dp+Ce, (p+1)*Dp); both clipped to T. stream_range_of() is the inverse.
// ---------------------------------------------------------------------------------------------
constexpr int SD_MAX_SEQS = 1024;   // sequences per launch (step-prefix table in LDS)
constexpr int SD_MAX_WAVES = 4096;  // partial slots are sized for this many waves
constexpr int SD_WAVES_PER_CU = 8;  // two single-wave workgroups per SIMD
constexpr int SD_STEP_TOKENS = FD_PAGES_PER_WAVE * FD_P;  // 128 tokens per step

// The decode scratch (a caller's workspace, or the no-alloc entry point's static array), laid
// out for `waves` waves; every entry point takes its layout from here and nowhere else:
//   [0, part_offset)           one 64-bit arrival counter per wave w (for the cut segment whose
//                              first step lies in w's range), starting at the first 8-byte
//                              boundary (the buffer need only be 4-byte aligned), padded to
//                              256 bytes;
//   [part_offset, total_bytes) two partial slots per wave, each G rows of D + 2 fp32.
struct DecodeScratchLayout {
  int64_t part_offset;
  int64_t total_bytes;
};
constexpr DecodeScratchLayout decode_scratch_layout(int G, int waves) {
  return {(int64_t(waves) * 8 + 8 + 255) / 256 * 256,
          (int64_t(waves) * 8 + 8 + 255) / 256 * 256 +
              int64_t(waves) * 2 * G * (FD_D + 2) * int64_t(sizeof(float))};
}
// Group sizes of the fast kernels: 1, 2, 4 on the vector ALU (paged_decode_stream), 3, 5..8 and 16
// on the matrix cores (paged_decode_mfma, whose 16-row MFMA blocks hold up to 16 q rows).
constexpr bool stream_group_ok(int G) { return (G >= 1 && G <= 8) || G == 16; }
constexpr int SD_EVEN_SHARE_PERMILLE = 515;                // even-XCD wave's share of a pair

// Steps of a wave pair and the even wave's share of them, for T steps over NW waves.
__device__ __forceinline__ int stream_pair_steps(int T, int NW) {
  return int((2 * int64_t(T) + NW - 1) / NW);
}
__device__ __forceinline__ int stream_even_share(int Dp) {
  return (Dp * SD_EVEN_SHARE_PERMILLE + 500) / 1000;
}
// The wave whose range holds step st.
__device__ __forceinline__ int stream_range_of(int st, int Dp, int Ce) {
  const int p = st / Dp;
  return 2 * p + (st - p * Dp >= Ce ? 1 : 0);
}

// All members are ints: with a bool the struct has three bytes of tail padding, and copies of
// the cursor through selects then went via private memory, a scratch load and store per step
// whose wait held the step behind every load issued before it.
struct StreamCursor {
  int b, h, ls, ns, L;  // sequence, kv head, step in the segment, steps in it, its tokens
  int app;              // append mode: position L - 1 is the new token given in k_new / v_new
};

// seq_len LDS word: the clamped context length, bit 30 set when (append mode) the row's raw
// length does not fit its block table, so it has no new token to take from k_new / v_new.
constexpr int SD_NO_APPEND = 1 << 30;
constexpr int SD_APP_REC = 32;  // new-token slots a wave defers to the end of its range

__device__ __forceinline__ int wave_inclusive_scan(int v, int lane) {
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const int t = __shfl_up(v, o, 64);
    if (lane >= o) v += t;
  }
  return v;
}

__device__ __forceinline__ int uniform(int v) { return __builtin_amdgcn_readfirstlane(v); }

// Pool pointers of the stream kernel: restrict-qualified when the launch only reads the pools,
// plain when it also writes the new tokens into them (append mode).
template <bool APPEND>
using PoolIn = std::conditional_t<APPEND, const uint16_t*, const uint16_t* __restrict__>;

// Append mode (APPEND): every row's position L - 1 is its new token, given in k_new / v_new
// ([B, Hkv, D] rows new_seq_stride elements apart). The wave that runs a segment's last step
// scores the new key against the staged q (one v_dot2 per lane over the (d, d + 4) pairs, a
// wave sum), puts that score in place of the pool slot's, zeroes the slot's V words and adds
// p * v_new itself; the slot's old contents are never used and no other segment reads it.
// The stores of k_new / v_new into the slot wait until the wave has run its last step: vector
// memory counters retire in issue order, so a store issued between a step's loads would hold
// every later wait on a load behind its write acknowledgment (a measured 9 % of the launch).
// The wave keeps up to SD_APP_REC pending slots in LDS and stores any further ones at once.
// The stores are non-temporal (streamed through the cache): the next step reads these lines
// from another XCD, and that read was measured 0.4 % faster than after ordinary stores.
// A wave's arrival on the counter of a cut segment with n partials: the counter holds
// (token << 16 | count) where token identifies the launch (the upper 48 bits, from the host, a
// fresh value per launch); a count under another token is stale (an earlier launch, or a
// workspace never used before) and reads as 0. Returns true for the n-th arrival, which also
// leaves the count at 0 under this token, so a replay of the same launch (a graph) starts from
// zero again. Workspace contents collide with a token with probability 2^-48.
// Device-coherent partial stores and loads (sc1: through the XCD's L2 to memory).
__device__ __forceinline__ void sd_store(float* p, float v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float sd_load(const float* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ bool sd_arrive(uint64_t* ctr, uint64_t token, int n) {
  uint64_t old = __hip_atomic_load(ctr, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  for (;;) {  // retried only when another wave updated the counter in between
    const uint64_t cnt = (old >> 16) == (token >> 16) ? (old & 0xffffu) : 0u;
    const bool last = int(cnt) + 1 >= n;
    const uint64_t nv = token | (last ? 0u : cnt + 1);
    uint64_t expect = old;
    if (__hip_atomic_compare_exchange_strong(ctr, &expect, nv, __ATOMIC_RELAXED,
                                             __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT))
      return last;
    old = expect;
  }
}

// Step prefix of the batch, built by every wave in its own LDS copy: seq_q[b] = steps of the
// sequences before b (seq_q[B] = all of them), seq_len[b] = b's clamped context length (with
// SD_NO_APPEND in append mode when its raw length does not fit its block table). Returns the
// steps per kv head, sum_b ceil(L_b / 128).
template <bool APPEND>
__device__ __forceinline__ int sd_build_prefix(const int32_t* __restrict__ context_lens, int B,
                                               int64_t bt_stride, int* seq_q, int* seq_len,
                                               int lane) {
  constexpr int NCH = SD_MAX_SEQS / 64;
  int lv[NCH], lflag[NCH];
#pragma unroll
  for (int c = 0; c < NCH; ++c) {
    const int i = c * 64 + lane;
    const int raw = (c * 64 < B && i < B) ? context_lens[i] : 0;
    lv[c] = clamp_len(raw, bt_stride, FD_P);
    lflag[c] = (APPEND && raw != lv[c]) ? SD_NO_APPEND : 0;
  }
  int carry = 0;
#pragma unroll
  for (int c = 0; c < NCH; ++c) {
    if (c * 64 >= B) break;
    const int incl = wave_inclusive_scan((lv[c] + SD_STEP_TOKENS - 1) / SD_STEP_TOKENS, lane);
    const int i = c * 64 + lane;
    if (i < B) {
      seq_q[i + 1] = carry + incl;
      seq_len[i] = lv[c] | lflag[c];
    }
    carry = uniform(carry + __shfl(incl, 63, 64));
  }
  if (lane == 0) seq_q[0] = 0;
  __syncthreads();
  return carry;
}

// Rows of sequences with no steps are written as zeros: wave w takes sequences w, w + NW, ...
__device__ __forceinline__ void sd_zero_empty_rows(uint16_t* out, const int* seq_len, int B,
                                                   int Hq, int w, int NW, int lane) {
  for (int b = w; b < B; b += NW) {
    if ((uniform(seq_len[b]) & ~SD_NO_APPEND) == 0) {
      uint16_t* o = out + int64_t(b) * Hq * FD_D;
      for (int i = lane; i < Hq * FD_D; i += 64) o[i] = 0;
    }
  }
}

// Walks the ordered step list (sequence-major, then kv head, then step) over the LDS prefix.
struct StreamPlan {
  const int* seq_q;
  const int* seq_len;
  int B, Hkv;
  bool append;

  __device__ __forceinline__ void set_len(StreamCursor& c) const {
    const int sl = uniform(seq_len[c.b]);
    c.L = sl & ~SD_NO_APPEND;
    c.app = append && !(sl & SD_NO_APPEND);
  }
  // cursor of global step gs: the last sequence b with Hkv * seq_q[b] <= gs (it has steps)
  __device__ __forceinline__ StreamCursor seg_of(int gs) const {
    int lo = 0, hi = B - 1;
    while (lo < hi) {
      const int mid = (lo + hi + 1) >> 1;
      if (Hkv * uniform(seq_q[mid]) <= gs) lo = mid; else hi = mid - 1;
    }
    StreamCursor c;
    c.b = lo;
    const int q0 = uniform(seq_q[lo]);
    c.ns = uniform(seq_q[lo + 1]) - q0;
    const int r = gs - Hkv * q0;
    c.h = r / c.ns;
    c.ls = r - c.h * c.ns;
    set_len(c);
    return c;
  }
  // the step after c (only asked for when one exists inside the range)
  __device__ __forceinline__ StreamCursor next_of(StreamCursor c) const {
    if (++c.ls == c.ns) {
      c.ls = 0;
      if (++c.h == Hkv) {
        c.h = 0;
        do { ++c.b; } while (c.b < B - 1 && uniform(seq_q[c.b + 1]) == uniform(seq_q[c.b]));
        c.ns = uniform(seq_q[c.b + 1]) - uniform(seq_q[c.b]);
        set_len(c);
      }
    }
    return c;
  }
};

// Append mode: k_new / v_new rows of one new token into its pool slot (element offset `slot` of
// its (page, kv head) tile plus its token), non-temporally; src = the rows' element offset.
__device__ __forceinline__ void sd_store_new_token(const uint16_t* __restrict__ k_new,
                                                   const uint16_t* __restrict__ v_new,
                                                   uint16_t* kpool_w, uint16_t* vpool_w,
                                                   int64_t slot, int64_t src, int lane) {
  const int d0 = 8 * (lane >> 2) + (lane & 3);
  __builtin_nontemporal_store(k_new[src + d0], kpool_w + slot + d0 * FD_P);
  __builtin_nontemporal_store(k_new[src + d0 + 4], kpool_w + slot + (d0 + 4) * FD_P);
  if ((lane & 1) == 0) {
#pragma unroll
    for (int j = 0; j < 4; ++j)
      __builtin_nontemporal_store(v_new[src + 32 * j + (lane >> 1)],
                                  vpool_w + slot + (32 * j + (lane >> 1)) * FD_P);
  }
}

// Append mode: the deferred new-token stores of a wave's range (k_new / v_new rows reread: they
// are small and cached). rec[r] = {pool element offset of the slot, k_new / v_new offset}.
__device__ __forceinline__ void sd_flush_appends(const int64_t (*rec)[2], int n_rec,
                                                 const uint16_t* __restrict__ k_new,
                                                 const uint16_t* __restrict__ v_new,
                                                 uint16_t* kpool_w, uint16_t* vpool_w, int lane) {
  __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
  __builtin_amdgcn_wave_barrier();
  for (int r = 0; r < n_rec; ++r)
    sd_store_new_token(k_new, v_new, kpool_w, vpool_w, rec[r][0], rec[r][1], lane);
}

// Arrivals at the end of a wave's range: its partials (slot 0 / 1: arr_first = the segment's
// first global step or -1, arr_ns its steps, arr_row = b * Hkv + h) are written; count them in
// on their segments' counters and merge every segment whose last partial this is. Partial
// layout per slot: G rows of [D unnormalised output, running max (log2 units), row sum].
template <int G, int DT>
__device__ __forceinline__ void sd_arrive_and_merge(const int (&arr_first)[2],
                                                    const int (&arr_ns)[2],
                                                    const int (&arr_row)[2], int Dp, int Ce,
                                                    const float* ws_part, int32_t* ws_meta,
                                                    uint64_t token, uint16_t* out, int Hkv,
                                                    int lane) {
  constexpr int D = FD_D;
  if (arr_first[0] < 0 && arr_first[1] < 0) return;
  uint64_t* ctr = reinterpret_cast<uint64_t*>(
      (reinterpret_cast<uintptr_t>(ws_meta) + 7) & ~uintptr_t(7));
  const int inc = Ce < Dp ? 1 : 2;  // odd waves hold no steps when pairs have one step
  __builtin_amdgcn_s_waitcnt(0);  // this wave's partial stores have completed before its count
  bool merge[2] = {false, false};
#pragma unroll
  for (int k = 0; k < 2; ++k) {
    if (arr_first[k] < 0) continue;
    const int c0 = stream_range_of(arr_first[k], Dp, Ce);
    const int c1 = stream_range_of(arr_first[k] + arr_ns[k] - 1, Dp, Ce);
    int last = 0;
    if (lane == 0) last = sd_arrive(ctr + c0, token, (c1 - c0) / inc + 1) ? 1 : 0;
    merge[k] = __builtin_amdgcn_readfirstlane(last) != 0;
  }
  if (!merge[0] && !merge[1]) return;
#pragma unroll
  for (int k = 0; k < 2; ++k) {
    if (!merge[k]) continue;
    // one online pass over the pieces in wave order (slot 1 of the first wave, slot 0 of the
    // rest); lane l: elements l and l + 64 of every row
    const int c0 = stream_range_of(arr_first[k], Dp, Ce);
    const int c1 = stream_range_of(arr_first[k] + arr_ns[k] - 1, Dp, Ce);
    float M[G], o0[G], o1[G], lt[G];
#pragma unroll
    for (int g = 0; g < G; ++g) {
      M[g] = kNegBig;
      o0[g] = o1[g] = lt[g] = 0.f;
    }
    // pieces four at a time: all their loads in flight together, then folded in order
    constexpr int PB = 4;
    for (int cb = c0; cb <= c1; cb += PB * inc) {
      float mc[PB][G], lc[PB][G], a0[PB][G], a1[PB][G];
#pragma unroll
      for (int u = 0; u < PB; ++u) {
        const int c = cb + u * inc;
        if (c > c1) continue;
        const float* pp = ws_part + (int64_t(c) * 2 + (c == c0 ? 1 : 0)) * G * (D + 2);
#pragma unroll
        for (int g = 0; g < G; ++g) {
          mc[u][g] = sd_load(pp + g * (D + 2) + D);
          lc[u][g] = sd_load(pp + g * (D + 2) + D + 1);
          a0[u][g] = sd_load(pp + g * (D + 2) + lane);
          a1[u][g] = sd_load(pp + g * (D + 2) + 64 + lane);
        }
      }
#pragma unroll
      for (int u = 0; u < PB; ++u) {
        if (cb + u * inc > c1) continue;
#pragma unroll
        for (int g = 0; g < G; ++g) {
          const float mn = fmaxf(M[g], mc[u][g]);
          const float fo = fast_exp2(M[g] - mn), fc = fast_exp2(mc[u][g] - mn);
          lt[g] = lt[g] * fo + lc[u][g] * fc;
          o0[g] = o0[g] * fo + a0[u][g] * fc;
          o1[g] = o1[g] * fo + a1[u][g] * fc;
          M[g] = mn;
        }
      }
    }
    const int b = arr_row[k] / Hkv, h = arr_row[k] - b * Hkv;
    uint16_t* orow = out + (int64_t(b) * Hkv * G + int64_t(h) * G) * D;
#pragma unroll
    for (int g = 0; g < G; ++g) {
      orow[g * D + lane] = to16<DT>(lt[g] > 0.f ? o0[g] / lt[g] : 0.f);
      orow[g * D + 64 + lane] = to16<DT>(lt[g] > 0.f ? o1[g] / lt[g] : 0.f);
    }
  }
}

template <int G, bool APPEND, int DT>
__global__ __launch_bounds__(64, 2) void paged_decode_stream(
    uint16_t* __restrict__ out, const uint16_t* __restrict__ q, int64_t q_seq_stride,
    PoolIn<APPEND> kpool, PoolIn<APPEND> vpool,
    const int32_t* __restrict__ block_tables, int64_t bt_stride,
    const int32_t* __restrict__ context_lens, int B, int Hkv, int64_t num_pages,
    float* __restrict__ ws_part, int32_t* __restrict__ ws_meta, float scale_log2,
    uint16_t* kpool_w, uint16_t* vpool_w, const uint16_t* __restrict__ k_new,
    const uint16_t* __restrict__ v_new, int64_t new_seq_stride, uint64_t token) {
  static_assert(G == 1 || G == 2 || G == 4, "G = 8 runs paged_decode_mfma");
  constexpr int D = FD_D, P = FD_P, TILE = D * P, STEP = FD_PAGES_PER_WAVE;
  const int lane = threadIdx.x, w = blockIdx.x, NW = gridDim.x;
  const int Hq = Hkv * G;
  extern __shared__ int sd_lds[];
  int* seq_q = sd_lds;            // [B + 1]: steps of the sequences before b
  int* seq_len = sd_lds + B + 1;  // [B]: clamped context length
  __shared__ uint32_t q_lds[4][16][G];
  __shared__ uint32_t p_lds[64][G];
  // append mode: deferred new-token stores, {pool element offset of the slot, k_new offset}
  __shared__ int64_t app_rec[APPEND ? SD_APP_REC : 1][2];
  int n_rec = 0;

  const int T = Hkv * sd_build_prefix<APPEND>(context_lens, B, bt_stride, seq_q, seq_len, lane);
  const int Dp = stream_pair_steps(T, NW), Ce = stream_even_share(Dp);
  sd_zero_empty_rows(out, seq_len, B, Hq, w, NW, lane);
  const int start = (w >> 1) * Dp + ((w & 1) ? Ce : 0);
  const int end = min((w >> 1) * Dp + ((w & 1) ? Dp : Ce), T);
  if (start >= end) return;
  const int span = end - start;

  const StreamPlan plan{seq_q, seq_len, B, Hkv, APPEND};
  // lane l: block-table entry of page l/8 of the step (entries past the sequence repeat its
  // last page; ids are range-checked where they are used)
  auto load_bt = [&](const StreamCursor& c) -> int {
    const int npg = (c.L + P - 1) / P;
    const int i = min(c.ls * STEP + (lane >> 3), npg - 1);
    return block_tables[int64_t(c.b) * bt_stride + i];
  };
  auto page_ok = [&](int p) -> int64_t {
    return (p < 0 || int64_t(p) >= num_pages) ? 0 : int64_t(p);
  };
  // q rows of a segment: lane l < 16G holds q[g][8pp .. 8pp+7], g = l/16, pp = l%16 (four dword
  // loads: q is only 4-byte aligned); staged as the (d, d+4) pairs of row-pair pp.
  constexpr int QW = 1;
  using QRows = uint4[QW];
  auto load_q = [&](const StreamCursor& c, QRows& r) {
#pragma unroll
    for (int k = 0; k < QW; ++k) {
      r[k] = make_uint4(0u, 0u, 0u, 0u);
      const int g = (lane >> 4) + 4 * k;
      if (g < G) {
        const uint32_t* qw = reinterpret_cast<const uint32_t*>(
            q + int64_t(c.b) * q_seq_stride + int64_t(c.h) * G * D + g * D + 8 * (lane & 15));
        r[k] = make_uint4(qw[0], qw[1], qw[2], qw[3]);
      }
    }
  };
  auto stage_q = [&](const QRows& wr) {
#pragma unroll
    for (int k = 0; k < QW; ++k) {
      const int g = (lane >> 4) + 4 * k, pp = lane & 15;
      if (g < G) {
        const uint4 wq = wr[k];
        q_lds[0][pp][g] = pack_lo(wq.x, wq.z);
        q_lds[1][pp][g] = pack_hi(wq.x, wq.z);
        q_lds[2][pp][g] = pack_lo(wq.y, wq.w);
        q_lds[3][pp][g] = pack_hi(wq.y, wq.w);
      }
    }
  };

  const int dsub = lane & 3, vhalf = lane & 1;
  const int64_t page_stride = int64_t(Hkv) * TILE;
  const uint16_t* kbase = kpool + dsub * P + ((lane >> 2) & 1) * 8;
  const uint16_t* vbase = vpool + lane * 8;

  float m[G], lsum[G], acc[4][G];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    m[g] = kNegBig;
    lsum[g] = 0.f;
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[j][g] = 0.f;
  }

  int gs = start;
  StreamCursor cur = plan.seg_of(gs);
  // partials this wave writes (slot 0, slot 1): the first global step, step count and row of
  // their segments, for the arrivals after the range (arr_first -1: no partial in that slot)
  int arr_first[2] = {-1, -1}, arr_ns[2] = {0, 0}, arr_row[2] = {0, 0};
  int bt_cur;
  // Two 16 KiB register buffers whose role rotates through a step:
  //   A: K rows 0..63 -> V pages 0..3 -> next step's K rows 0..63
  //   B: K rows 64..127 -> V pages 4..7 -> next step's K rows 64..127
  uint4 bufA[16], bufB[16];
  {
    QRows q0;
    load_q(cur, q0);
    bt_cur = load_bt(cur);
    const uint16_t* kp = kbase + int64_t(cur.h) * TILE + page_ok(bt_cur) * page_stride;
#pragma unroll
    for (int i = 0; i < 16; ++i) bufA[i] = load16_nt(kp + 64 * i);
#pragma unroll
    for (int i = 0; i < 16; ++i) bufB[i] = load16_nt(kp + 64 * (16 + i));
    stage_q(q0);
    __syncthreads();
  }

  auto qk_rows = [&](const uint4 (&kr)[16], int pp0, float (&sacc)[8][G]) {
#pragma unroll
    for (int pp = 0; pp < 8; ++pp) {
      const uint4 a = kr[2 * pp], c = kr[2 * pp + 1];  // rows d = 8(pp0+pp) + dsub and d + 4
      uint32_t kk[8];
      kk[0] = pack_lo(a.x, c.x); kk[1] = pack_hi(a.x, c.x);
      kk[2] = pack_lo(a.y, c.y); kk[3] = pack_hi(a.y, c.y);
      kk[4] = pack_lo(a.z, c.z); kk[5] = pack_hi(a.z, c.z);
      kk[6] = pack_lo(a.w, c.w); kk[7] = pack_hi(a.w, c.w);
      uint32_t qq[G];
#pragma unroll
      for (int g = 0; g < G; ++g) qq[g] = q_lds[dsub][pp0 + pp][g];
#pragma unroll
      for (int t = 0; t < 8; ++t)
#pragma unroll
        for (int g = 0; g < G; ++g) sacc[t][g] = dot2<DT>(kk[t], qq[g], sacc[t][g]);
    }
  };

  // V of pages pg0..pg0+3 of the step; vr[4*pg + j] holds rows d = 32j + lane/2 of page pg.
  auto load_v = [&](uint4 (&vr)[16], const uint16_t* head_v, int bt, int pg0) {
#pragma unroll
    for (int pg = 0; pg < 4; ++pg) {
      const int64_t vphys = page_ok(__builtin_amdgcn_readlane(bt, 8 * (pg0 + pg)));
      const uint16_t* vp = head_v + vphys * page_stride;
#pragma unroll
      for (int j = 0; j < 4; ++j) vr[4 * pg + j] = load16_nt(vp + 512 * j);
    }
  };

  // Tokens at or past the step's valid count (partial last page, re-read pages after it) and
  // tokens of pages whose block-table id is out of the pool carry P = 0, but their V words
  // (stale or another page's) may be non-finite: zero them before the PV products.
  // bad: bit 8 * pg set when page pg of the step has an invalid id.
  auto mask_tail = [&](uint4 (&vr)[16], int pg0, int valid, uint64_t bad) {
#pragma unroll
    for (int pgi = 0; pgi < 4; ++pgi) {
      const bool pg_bad = (bad >> (8 * (pg0 + pgi))) & 1ull;
      const int nvalid = pg_bad ? 0 : valid - ((pg0 + pgi) * P + vhalf * 8);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        uint4& wv = vr[4 * pgi + j];
        wv.x = mask_pair(wv.x, 0, nvalid);
        wv.y = mask_pair(wv.y, 2, nvalid);
        wv.z = mask_pair(wv.z, 4, nvalid);
        wv.w = mask_pair(wv.w, 6, nvalid);
      }
    }
  };

  auto pv_pages = [&](const uint4 (&vr)[16], int pg0) {
#pragma unroll
    for (int pgi = 0; pgi < 4; ++pgi) {
      __builtin_amdgcn_sched_barrier(0);  // one page's probability reads at a time (4*G VGPRs)
      const int pg = pg0 + pgi;
      const uint32_t* prow = &p_lds[pg * 8 + vhalf * 4][0];
      uint32_t pr[4][G];
#pragma unroll
      for (int mm = 0; mm < 4; ++mm)
#pragma unroll
        for (int g = 0; g < G; ++g) pr[mm][g] = prow[mm * G + g];
#pragma unroll
      for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int g = 0; g < G; ++g) {
          const uint4 wv = vr[4 * pgi + j];
          float a = acc[j][g];
          a = dot2<DT>(wv.x, pr[0][g], a);
          a = dot2<DT>(wv.y, pr[1][g], a);
          a = dot2<DT>(wv.z, pr[2][g], a);
          a = dot2<DT>(wv.w, pr[3][g], a);
          acc[j][g] = a;
        }
    }
  };

  for (;;) {
    {  // issue priority from progress: quartile 0 of the range -> 3, quartile 3 -> 0
      const int quarter = (4 * (gs - start)) / span;
      if (quarter <= 0) __builtin_amdgcn_s_setprio(3);
      else if (quarter == 1) __builtin_amdgcn_s_setprio(2);
      else if (quarter == 2) __builtin_amdgcn_s_setprio(1);
      else __builtin_amdgcn_s_setprio(0);
    }
    const bool has_next = gs + 1 < end;
    // The next step's block-table row and (when it opens a segment) q go out first, ahead of
    // this step's V loads, so they have landed by the time they are consumed. At the end of
    // the range the "next" step repeats the current one (its K is not prefetched).
    const StreamCursor nxt = has_next ? plan.next_of(cur) : cur;
    const bool nxt_opens = has_next && nxt.ls == 0;
    const int bt_nxt = load_bt(nxt);
    QRows q_nxt;
#pragma unroll
    for (int k = 0; k < QW; ++k) q_nxt[k] = make_uint4(0u, 0u, 0u, 0u);
    if (nxt_opens) load_q(nxt, q_nxt);
    const int valid = min(SD_STEP_TOKENS, cur.L - cur.ls * SD_STEP_TOKENS);
    const uint16_t* head_v = vbase + int64_t(cur.h) * TILE;

    // append mode, the segment's last step: token tn of the step is the new one. Lane l takes
    // k_new[d], k_new[d + 4] with d = 8 (l / 4) + l % 4 (the q pair q_lds[l % 4][l / 4]) and
    // v_new[32 j + l / 2], j < 4 (the V rows of its PV accumulators).
    const bool app_step = APPEND && cur.app && cur.ls == cur.ns - 1;
    const int tn = valid - 1;
    uint32_t kn = 0;
    uint32_t vn[4] = {0u, 0u, 0u, 0u};
    if (app_step) {
      const uint16_t* kr = k_new + int64_t(cur.b) * new_seq_stride + int64_t(cur.h) * D;
      const uint16_t* vr = v_new + int64_t(cur.b) * new_seq_stride + int64_t(cur.h) * D;
      const int d0 = 8 * (lane >> 2) + (lane & 3);
      kn = uint32_t(kr[d0]) | (uint32_t(kr[d0 + 4]) << 16);
#pragma unroll
      for (int j = 0; j < 4; ++j) vn[j] = vr[32 * j + (lane >> 1)];
    }

    // pages of this step whose id is outside the pool: their tokens are not keys (lane l holds
    // the id of page l / 8, the page of its scores' tokens 2l and 2l + 1)
    const bool pg_ok = bt_cur >= 0 && int64_t(bt_cur) < num_pages;
    const uint64_t bad = __ballot(!pg_ok);
    const bool masked_step = valid < SD_STEP_TOKENS || bad != 0 || app_step;
    // V words of tokens at or past v_valid are zeroed (the new token's slot in append mode)
    const int v_valid = app_step ? tn : valid;

    float sacc[8][G];
#pragma unroll
    for (int t = 0; t < 8; ++t)
#pragma unroll
      for (int g = 0; g < G; ++g) sacc[t][g] = 0.f;
    // sched_barrier(0) pins every load group between the compute phases it overlaps, so at
    // most two groups (128 VGPRs) of tile data are live at any point.
    qk_rows(bufA, 0, sacc);
    __builtin_amdgcn_sched_barrier(0);
    load_v(bufA, head_v, bt_cur, 0);
    __builtin_amdgcn_sched_barrier(0);
    qk_rows(bufB, 8, sacc);
    // quad reduce-scatter: lane l ends with the scores of tokens 2l, 2l+1 of the step
    float sc[2][G];
    quad_reduce_scatter<G>(sacc, sc, lane);
    const int tok0 = 2 * lane;
    if (app_step) {  // the new token's score from k_new, in place of its pool slot's
      const bool own0 = tok0 == tn, own1 = tok0 + 1 == tn;
#pragma unroll
      for (int g = 0; g < G; ++g) {
        const float sn = wave_sum_dpp(dot2<DT>(kn, q_lds[lane & 3][lane >> 2][g], 0.f));
        sc[0][g] = own0 ? sn : sc[0][g];
        sc[1][g] = own1 ? sn : sc[1][g];
      }
    }
    uint32_t pw[G];
#pragma unroll
    for (int g = 0; g < G; ++g) {
      const float x0 = (tok0 < valid && pg_ok) ? sc[0][g] * scale_log2 : -INFINITY;
      const float x1 = (tok0 + 1 < valid && pg_ok) ? sc[1][g] * scale_log2 : -INFINITY;
      const float mnew = fmaxf(m[g], wave_max_dpp(fmaxf(x0, x1)));
      const float alpha = fast_exp2(m[g] - mnew);
      const float p0 = fast_exp2(x0 - mnew), p1 = fast_exp2(x1 - mnew);
      lsum[g] = lsum[g] * alpha + (p0 + p1);
      m[g] = mnew;
      pw[g] = pack2<DT>(p0, p1);
#pragma unroll
      for (int j = 0; j < 4; ++j) acc[j][g] *= alpha;
    }
#pragma unroll
    for (int g = 0; g < G; ++g) p_lds[lane][g] = pw[g];
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
    __builtin_amdgcn_wave_barrier();
    if (app_step) {
      // p of the new token (the 16-bit value the pool tokens' products use) times v_new, on the
      // even lanes (the odd lane of a pair accumulates the other token half); then k_new /
      // v_new go into the slot, unless its page id is outside the pool (then it is no key)
      const uint32_t half_sh = (tn & 1) ? 16u : 0u;
#pragma unroll
      for (int g = 0; g < G; ++g) {
        const float pn = from16<DT>(p_lds[tn >> 1][g] >> half_sh);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const float v = (lane & 1) ? 0.f : from16<DT>(vn[j]);
          acc[j][g] = pn > 0.f ? fmaf(pn, v, acc[j][g]) : acc[j][g];
        }
      }
      const int idn = __builtin_amdgcn_readlane(bt_cur, 8 * (tn >> 4));
      if (idn >= 0 && int64_t(idn) < num_pages) {
        const int64_t slot = int64_t(idn) * page_stride + int64_t(cur.h) * TILE + (tn & 15);
        if (n_rec < SD_APP_REC) {
          if (lane == 0) {
            app_rec[n_rec][0] = slot;
            app_rec[n_rec][1] = int64_t(cur.b) * new_seq_stride + int64_t(cur.h) * D;
          }
          ++n_rec;
        } else {
          const int d0 = 8 * (lane >> 2) + (lane & 3);
          __builtin_nontemporal_store(uint16_t(kn & 0xffffu), kpool_w + slot + d0 * P);
          __builtin_nontemporal_store(uint16_t(kn >> 16), kpool_w + slot + (d0 + 4) * P);
          if ((lane & 1) == 0) {
#pragma unroll
            for (int j = 0; j < 4; ++j)
              __builtin_nontemporal_store(uint16_t(vn[j]),
                                          vpool_w + slot + (32 * j + (lane >> 1)) * P);
          }
        }
      }
    }
    __builtin_amdgcn_sched_barrier(0);
    load_v(bufB, head_v, bt_cur, 4);
    __builtin_amdgcn_sched_barrier(0);
    if (masked_step) {
      mask_tail(bufA, 0, v_valid, bad);
      pv_pages(bufA, 0);
    } else {
      pv_pages(bufA, 0);
    }
    __builtin_amdgcn_sched_barrier(0);
    // the next step's K (none after the range's last step: the wave's end waits for its
    // outstanding loads before it counts its partials in)
    const uint16_t* kp = kbase + int64_t(nxt.h) * TILE + page_ok(bt_nxt) * page_stride;
    if (has_next) {
#pragma unroll
      for (int i = 0; i < 16; ++i) bufA[i] = load16_nt(kp + 64 * i);
    }
    __builtin_amdgcn_sched_barrier(0);
    if (masked_step) {
      mask_tail(bufB, 4, v_valid, bad);
      pv_pages(bufB, 4);
    } else {
      pv_pages(bufB, 4);
    }
    __builtin_amdgcn_sched_barrier(0);
    if (has_next) {
#pragma unroll
      for (int i = 0; i < 16; ++i) bufB[i] = load16_nt(kp + 64 * (16 + i));
    }
    // the next step overwrites p_lds (and maybe q_lds): keep this step's reads ahead of them
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
    __builtin_amdgcn_wave_barrier();

    const bool seg_last = cur.ls == cur.ns - 1;
    if (seg_last || !has_next) {
#pragma unroll
      for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int g = 0; g < G; ++g) acc[j][g] += dpp_f32<kDppQuadXor1>(acc[j][g]);
#pragma unroll
      for (int g = 0; g < G; ++g) lsum[g] = wave_sum_dpp(lsum[g]);
      const int seg_first = gs - cur.ls;  // global index of the segment's first step
      const int64_t row0 = int64_t(cur.b) * Hq + int64_t(cur.h) * G;
      if (seg_last && seg_first >= start) {
        if ((lane & 1) == 0) {
#pragma unroll
          for (int g = 0; g < G; ++g)
#pragma unroll
            for (int j = 0; j < 4; ++j)
              out[(row0 + g) * D + 32 * j + (lane >> 1)] =
                  to16<DT>(lsum[g] > 0.f ? acc[j][g] / lsum[g] : 0.f);
        }
      } else {
        const int slot = seg_first < start ? 0 : 1;
        arr_first[slot] = seg_first;
        arr_ns[slot] = cur.ns;
        arr_row[slot] = cur.b * Hkv + cur.h;
        // partials go out as device-coherent stores (through this XCD's L2 to memory): the
        // merging wave may run on another XCD and reads them with device-coherent loads, so
        // neither side needs a cache-wide write-back or invalidate
        float* part = ws_part + (int64_t(w) * 2 + slot) * G * (D + 2);
        if ((lane & 1) == 0) {
#pragma unroll
          for (int g = 0; g < G; ++g)
#pragma unroll
            for (int j = 0; j < 4; ++j)
              sd_store(part + g * (D + 2) + 32 * j + (lane >> 1), acc[j][g]);
        }
        if (lane == 0) {
#pragma unroll
          for (int g = 0; g < G; ++g) {
            sd_store(part + g * (D + 2) + D, m[g]);
            sd_store(part + g * (D + 2) + D + 1, lsum[g]);
          }
        }
      }
#pragma unroll
      for (int g = 0; g < G; ++g) {
        m[g] = kNegBig;
        lsum[g] = 0.f;
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[j][g] = 0.f;
      }
    }
    if (!has_next) break;
    if (nxt_opens) stage_q(q_nxt);
    cur = nxt;
    bt_cur = bt_nxt;
    ++gs;
  }
  if constexpr (APPEND) sd_flush_appends(app_rec, n_rec, k_new, v_new, kpool_w, vpool_w, lane);
  // All arrivals at the end of the range, so no fence drains a step's prefetch.
  sd_arrive_and_merge<G, DT>(arr_first, arr_ns, arr_row, Dp, Ce, ws_part, ws_meta, token, out, Hkv,
                         lane);
}

// ---------------------------------------------------------------------------------------------
// Stream decode kernel on the matrix cores (bf16 or fp16, D = 128, P = 16), launched for G = 3,
// 5..8 and 16 (q rows G..15 of its 16-row MFMA blocks are zero).
//
// The same work split, cursor, partial slots, arrivals and merge as paged_decode_stream, one wave
// per SIMD; only the tile work of a step differs. Eight q rows against 128 keys cost 2048
// v_dot2 per lane and step on the vector ALU (a third of the step's share of HBM time, issued
// by the one wave that must also keep its loads in flight); on the matrix cores they are 32 +
// 32 MFMAs and the vector ALU keeps only the softmax. A 128-token step is two 64-token tiles
// (pages 0..3 and 4..7 of the step), each:
//   K: sixteen 16-byte loads per lane (load 4 p + r: page p of the tile, rows 32 r + l / 2,
//      token half l % 2; 1 KiB contiguous per load), stored into the wave's swizzled
//      [d][64 tokens] LDS tile (tile::swz64).
//   S^T = K . Q^T: 16 MFMAs (4 token blocks x 4 d chunks); A = K^T built by transposing LDS
//      reads, B = the segment's q rows in registers (operand rows G..15 are zero). Lane l then
//      holds the scores of q row l % 16 for tokens 16 mb + 4 (l / 16) + j.
//   V: thirty-two 8-byte loads per lane straight into the B operands of P . V: for 32-token
//      chunk c and d block nb, lane l reads row d = 16 nb + l % 16 at tokens 4 (l / 16) .. + 3
//      of pages 2c (k slots 8 (l / 16) .. + 3) and 2c + 1 (k slots + 4 .. + 7): the tokens
//      whose probabilities lane l already holds, in the same k order.
//   O += P . V: 16 MFMAs, and 2 more against a column of ones for the row sums.
// Softmax per q row in fp32, base 2 with the scale folded in; the reference point of a row's
// exponentials moves only when a step's max exceeds it by more than SD_RESCALE (probabilities
// stay <= 2^8; the final division is exact either way). Pipeline per step, two rotating 16 KiB
// register buffers (A: K tile 0 -> V tile 0 -> next K tile 0; B likewise for tile 1):
//   stage K0 | issue V0 | QK0 | stage K1 | issue V1 | QK1 | softmax | PV0 | issue K0' | PV1 |
//   issue K1'
// Append mode: the new token's key goes into the LDS tile and its value into the V operand
// registers in place of the slot's, so it is scored and summed like every other token; the
// stores into the slot are deferred to the end of the range as in paged_decode_stream.
// ---------------------------------------------------------------------------------------------
constexpr float SD_RESCALE = 8.0f;

template <int G, bool APPEND, int DT>
__global__ __launch_bounds__(64, 1) void paged_decode_mfma(
    uint16_t* __restrict__ out, const uint16_t* __restrict__ q, int64_t q_seq_stride,
    PoolIn<APPEND> kpool, PoolIn<APPEND> vpool,
    const int32_t* __restrict__ block_tables, int64_t bt_stride,
    const int32_t* __restrict__ context_lens, int B, int Hkv, int64_t num_pages,
    float* __restrict__ ws_part, int32_t* __restrict__ ws_meta, float scale_log2,
    uint16_t* kpool_w, uint16_t* vpool_w, const uint16_t* __restrict__ k_new,
    const uint16_t* __restrict__ v_new, int64_t new_seq_stride, uint64_t token) {
  using tile::f32x4_t;
  typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));
  constexpr int D = FD_D, P = FD_P, TILE = D * P, STEP = FD_PAGES_PER_WAVE;
  constexpr int KT = tile::kTileTokens;
  const int lane = threadIdx.x, w = blockIdx.x, NW = gridDim.x;
  const int Hq = Hkv * G;
  extern __shared__ int sd_lds[];
  int* seq_q = sd_lds;            // [B + 1]: steps of the sequences before b
  int* seq_len = sd_lds + B + 1;  // [B]: clamped context length
  __shared__ __align__(16) uint16_t ks[D * KT];
  // append mode: deferred new-token stores, {pool element offset of the slot, k_new offset}
  __shared__ int64_t app_rec[APPEND ? SD_APP_REC : 1][2];
  int n_rec = 0;

  const int T = Hkv * sd_build_prefix<APPEND>(context_lens, B, bt_stride, seq_q, seq_len, lane);
  const int Dp = stream_pair_steps(T, NW), Ce = stream_even_share(Dp);
  sd_zero_empty_rows(out, seq_len, B, Hq, w, NW, lane);
  const int start = (w >> 1) * Dp + ((w & 1) ? Ce : 0);
  const int end = min((w >> 1) * Dp + ((w & 1) ? Dp : Ce), T);
  if (start >= end) return;
  const int span = end - start;
  const StreamPlan plan{seq_q, seq_len, B, Hkv, APPEND};

  const int g4 = lane >> 4, n16 = lane & 15;
  // lane l: block-table entry of page l/8 of the step (entries past the sequence repeat its
  // last page; ids are range-checked where they are used)
  auto load_bt = [&](const StreamCursor& c) -> int {
    const int npg = (c.L + P - 1) / P;
    const int i = min(c.ls * STEP + (lane >> 3), npg - 1);
    return block_tables[int64_t(c.b) * bt_stride + i];
  };
  auto page_ok = [&](int p) -> int64_t {
    return (p < 0 || int64_t(p) >= num_pages) ? 0 : int64_t(p);
  };
  // B operand of S^T: lane l holds q row l % 16 (zero for rows >= G) at d = 32 kc + 8 (l / 16)
  // .. + 7 (dword loads: q is only 4-byte aligned)
  auto load_q = [&](const StreamCursor& c, uint4 (&r)[4]) {
#pragma unroll
    for (int kc = 0; kc < 4; ++kc) {
      r[kc] = make_uint4(0u, 0u, 0u, 0u);
      if (n16 < G) {
        const uint32_t* qw = reinterpret_cast<const uint32_t*>(
            q + int64_t(c.b) * q_seq_stride + int64_t(c.h * G + n16) * D + 32 * kc + 8 * g4);
        r[kc] = make_uint4(qw[0], qw[1], qw[2], qw[3]);
      }
    }
  };
  // Swizzled LDS offsets as per-lane bases XORed with compile-time terms: the store of K load
  // 4 p + r lands at (st_base ^ 16 p) + 2048 r; the transposing read (mb, kc, hi) at
  // (k_base[hi] ^ 16 mb) + 2048 kc.
  int st_base, k_base[2];
  {
    const int d = lane >> 1, f = tile::swz64_row_term(d);
    st_base = (d * KT + 8 * ((lane & 1) ^ (f & 1))) | (16 * (f >> 1));
#pragma unroll
    for (int hi = 0; hi < 2; ++hi) {
      const int fk = ((2 * g4 + hi) ^ ((n16 >> 2) << 1)) & 7;
      const int row = 8 * g4 + 4 * hi + (n16 >> 2);
      k_base[hi] = (row * KT + 4 * (n16 & 1) + 8 * (((n16 >> 1) & 1) ^ (fk & 1))) |
                   (16 * (fk >> 1));
    }
  }
  const int64_t page_stride = int64_t(Hkv) * TILE;
  const uint16_t* klane = kpool + 8 * lane;
  const uint16_t* vlane = vpool + n16 * P + 4 * g4;

  // K of tile t of a step into registers
  auto load_k = [&](uint4 (&kr)[16], int h, int bt, int t) {
#pragma unroll
    for (int pi = 0; pi < 4; ++pi) {
      const int64_t id = page_ok(__builtin_amdgcn_readlane(bt, 8 * (4 * t + pi)));
      const uint16_t* kp = klane + int64_t(h) * TILE + id * page_stride;
#pragma unroll
      for (int r = 0; r < 4; ++r) kr[4 * pi + r] = load16_nt(kp + 512 * r);
    }
  };
  auto stage_k = [&](const uint4 (&kr)[16]) {
#pragma unroll
    for (int pi = 0; pi < 4; ++pi)
#pragma unroll
      for (int r = 0; r < 4; ++r)
        *reinterpret_cast<uint4*>(&ks[(st_base ^ (16 * pi)) + 2048 * r]) = kr[4 * pi + r];
  };
  // V operands of tile t: vr[8 c + nb] holds row 16 nb + l % 16 at tokens 4 (l / 16) .. + 3 of
  // pages 2c (.x, .y) and 2c + 1 (.z, .w) of the tile
  auto load_v = [&](uint4 (&vr)[16], int h, int bt, int t) {
#pragma unroll
    for (int c = 0; c < 2; ++c)
#pragma unroll
      for (int s = 0; s < 2; ++s) {
        const int64_t id = page_ok(__builtin_amdgcn_readlane(bt, 8 * (4 * t + 2 * c + s)));
        const uint16_t* vp = vlane + int64_t(h) * TILE + id * page_stride;
#pragma unroll
        for (int nb = 0; nb < 8; ++nb) {
          const u32x2_t x =
              __builtin_nontemporal_load(reinterpret_cast<const u32x2_t*>(vp + 256 * nb));
          if (s == 0) {
            vr[8 * c + nb].x = x.x;
            vr[8 * c + nb].y = x.y;
          } else {
            vr[8 * c + nb].z = x.x;
            vr[8 * c + nb].w = x.y;
          }
        }
      }
  };

  float m = kNegBig;  // running reference point of row l % 16 (log2 units)
  f32x4_t acc[8], lsum = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int nb = 0; nb < 8; ++nb) acc[nb] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  const uint4 ones = tile::ones16<DT>();
  uint4 qreg[4];

  // d chunk outermost: consecutive products of one accumulator are four MFMAs apart
  auto qk_tile = [&](f32x4_t (&sc)[4]) {
#pragma unroll
    for (int kc = 0; kc < 4; ++kc)
#pragma unroll
      for (int mb = 0; mb < 4; ++mb) {
        const uint2 lo = tile::read_tr16(&ks[(k_base[0] ^ (16 * mb)) + 2048 * kc]);
        const uint2 hi = tile::read_tr16(&ks[(k_base[1] ^ (16 * mb)) + 2048 * kc]);
        sc[mb] = tile::mfma16<DT>(make_uint4(lo.x, lo.y, hi.x, hi.y), qreg[kc],
                                 kc == 0 ? f32x4_t{0.f, 0.f, 0.f, 0.f} : sc[mb]);
      }
  };
  // scores of tile t -> log2 units; on masked steps tokens at or past `valid` and tokens of
  // pages with an id outside the pool (bit 8 pg of `bad`) -> -inf. Returns the lane's max.
  auto prep = [&](f32x4_t (&sc)[4], int t, bool masked, int valid, uint64_t bad) -> float {
    float mx = -INFINITY;
    if (masked) {
#pragma unroll
      for (int mb = 0; mb < 4; ++mb) {
        const int pg = 4 * t + mb;
        const int lim = ((bad >> (8 * pg)) & 1ull) ? 0 : valid - (16 * pg + 4 * g4);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const float x = j < lim ? sc[mb][j] * scale_log2 : -INFINITY;
          sc[mb][j] = x;
          mx = fmaxf(mx, x);
        }
      }
    } else {
#pragma unroll
      for (int mb = 0; mb < 4; ++mb)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const float x = sc[mb][j] * scale_log2;
          sc[mb][j] = x;
          mx = fmaxf(mx, x);
        }
    }
    return mx;
  };
  // probabilities of tile t as the A operands of its two 32-token chunks
  auto probs = [&](const f32x4_t (&sc)[4], float mref, uint4 (&pk)[2]) {
#pragma unroll
    for (int c = 0; c < 2; ++c) {
      float p[2][4];
#pragma unroll
      for (int hh = 0; hh < 2; ++hh)
#pragma unroll
        for (int j = 0; j < 4; ++j) p[hh][j] = fast_exp2(sc[2 * c + hh][j] - mref);
      pk[c] = make_uint4(tile::pack16x2<DT>(p[0][0], p[0][1]), tile::pack16x2<DT>(p[0][2], p[0][3]),
                         tile::pack16x2<DT>(p[1][0], p[1][1]), tile::pack16x2<DT>(p[1][2], p[1][3]));
    }
  };
  // V words of tokens at or past `valid` or in pages outside the pool -> 0 (stale memory may
  // hold non-finite values, and 0 * inf is not 0)
  auto mask_v = [&](uint4 (&vr)[16], int t, int valid, uint64_t bad) {
#pragma unroll
    for (int c = 0; c < 2; ++c)
#pragma unroll
      for (int s = 0; s < 2; ++s) {
        const int pg = 4 * t + 2 * c + s;
        const int nvalid = ((bad >> (8 * pg)) & 1ull) ? 0 : valid - (16 * pg + 4 * g4);
#pragma unroll
        for (int nb = 0; nb < 8; ++nb) {
          uint4& x = vr[8 * c + nb];
          if (s == 0) {
            x.x = mask_pair(x.x, 0, nvalid);
            x.y = mask_pair(x.y, 2, nvalid);
          } else {
            x.z = mask_pair(x.z, 0, nvalid);
            x.w = mask_pair(x.w, 2, nvalid);
          }
        }
      }
  };
  // chunk outermost: consecutive products of one accumulator are eight MFMAs apart
  auto pv_tile = [&](const uint4 (&vr)[16], const uint4 (&pk)[2]) {
#pragma unroll
    for (int c = 0; c < 2; ++c)
#pragma unroll
      for (int nb = 0; nb < 8; ++nb) acc[nb] = tile::mfma16<DT>(pk[c], vr[8 * c + nb], acc[nb]);
  };

  int gs = start;
  StreamCursor cur = plan.seg_of(gs);
  // partials this wave writes (slot 0, slot 1): the first global step, step count and row of
  // their segments, for the arrivals after the range (arr_first -1: no partial in that slot)
  int arr_first[2] = {-1, -1}, arr_ns[2] = {0, 0}, arr_row[2] = {0, 0};
  load_q(cur, qreg);
  int bt_cur = load_bt(cur);
  uint4 bufA[16], bufB[16];
  load_k(bufA, cur.h, bt_cur, 0);
  load_k(bufB, cur.h, bt_cur, 1);

  for (;;) {
    {  // issue priority from progress: quartile 0 of the range -> 3, quartile 3 -> 0
      const int quarter = (4 * (gs - start)) / span;
      if (quarter <= 0) __builtin_amdgcn_s_setprio(3);
      else if (quarter == 1) __builtin_amdgcn_s_setprio(2);
      else if (quarter == 2) __builtin_amdgcn_s_setprio(1);
      else __builtin_amdgcn_s_setprio(0);
    }
    const bool has_next = gs + 1 < end;
    const StreamCursor nxt = has_next ? plan.next_of(cur) : cur;
    const bool nxt_opens = has_next && nxt.ls == 0;
    const int bt_nxt = load_bt(nxt);
    uint4 q_nxt[4];
#pragma unroll
    for (int kc = 0; kc < 4; ++kc) q_nxt[kc] = make_uint4(0u, 0u, 0u, 0u);
    if (nxt_opens) load_q(nxt, q_nxt);
    const int valid = min(SD_STEP_TOKENS, cur.L - cur.ls * SD_STEP_TOKENS);

    // append mode, the segment's last step: token tn of the step is the new one; lane l takes
    // k_new[l], k_new[l + 64] (its LDS column) and v_new[16 nb + l % 16] (its V operand rows)
    const bool app_step = APPEND && cur.app && cur.ls == cur.ns - 1;
    const int tn = valid - 1;
    const int64_t app_src = int64_t(cur.b) * new_seq_stride + int64_t(cur.h) * D;
    uint16_t kn0 = 0, kn1 = 0, vn[8];
#pragma unroll
    for (int nb = 0; nb < 8; ++nb) vn[nb] = 0;
    if (app_step) {
      kn0 = k_new[app_src + lane];
      kn1 = k_new[app_src + 64 + lane];
#pragma unroll
      for (int nb = 0; nb < 8; ++nb) vn[nb] = v_new[app_src + 16 * nb + n16];
    }
    auto put_knew = [&](int t) {
      if (app_step && (tn >> 6) == t) {
        ks[tile::swz64(lane, tn & (KT - 1))] = kn0;
        ks[tile::swz64(lane + 64, tn & (KT - 1))] = kn1;
      }
    };
    auto put_vnew = [&](uint4 (&vr)[16], int t) {
      if (!(app_step && (tn >> 6) == t)) return;
      const int cn = (tn >> 5) & 1, wsel = 2 * ((tn >> 4) & 1) + ((tn >> 1) & 1);
      const uint32_t sh = (tn & 1) ? 16u : 0u, keep = ~(0xffffu << sh);
      const bool mine = g4 == ((tn >> 2) & 3);
#pragma unroll
      for (int c = 0; c < 2; ++c) {
        const bool sel = mine && c == cn;  // per-element selects: the indices stay static
#pragma unroll
        for (int nb = 0; nb < 8; ++nb) {
          uint4& x = vr[8 * c + nb];
          const uint32_t nv = uint32_t(vn[nb]) << sh;
          x.x = (sel && wsel == 0) ? ((x.x & keep) | nv) : x.x;
          x.y = (sel && wsel == 1) ? ((x.y & keep) | nv) : x.y;
          x.z = (sel && wsel == 2) ? ((x.z & keep) | nv) : x.z;
          x.w = (sel && wsel == 3) ? ((x.w & keep) | nv) : x.w;
        }
      }
    };

    // pages of this step whose id is outside the pool: their tokens are not keys
    const bool pg_ok = bt_cur >= 0 && int64_t(bt_cur) < num_pages;
    const uint64_t bad = __ballot(!pg_ok);
    const bool masked = valid < SD_STEP_TOKENS || bad != 0;

    __builtin_amdgcn_sched_barrier(0);
    stage_k(bufA);
    put_knew(0);
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_sched_barrier(0);
    load_v(bufA, cur.h, bt_cur, 0);
    __builtin_amdgcn_sched_barrier(0);
    f32x4_t sA[4], sB[4];
    qk_tile(sA);
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_sched_barrier(0);
    stage_k(bufB);
    put_knew(1);
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_sched_barrier(0);
    load_v(bufB, cur.h, bt_cur, 1);
    __builtin_amdgcn_sched_barrier(0);
    qk_tile(sB);

    // softmax: row max over the step (lanes l, l ^ 16, l ^ 32, l ^ 48 hold one row)
    float mx = tile::max_col4(
        fmaxf(prep(sA, 0, masked, valid, bad), prep(sB, 1, masked, valid, bad)));
    const float mref = (mx - m > SD_RESCALE) ? mx : m;
    const float alpha = m == mref ? 1.f : fast_exp2(m - mref);
    const bool moved = m != mref;
    m = mref;
    uint4 pkA[2], pkB[2];
    probs(sA, mref, pkA);
    probs(sB, mref, pkB);
    // rescale O and the sums when some row's reference point moved: lane l's accumulator rows
    // are 4 (l / 16) + j; their alpha sits in lane 4 (l / 16) + j
    if (__ballot(moved)) {
      float aj[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) aj[j] = __shfl(alpha, 4 * g4 + j, 64);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        lsum[j] *= aj[j];
#pragma unroll
        for (int nb = 0; nb < 8; ++nb) acc[nb][j] *= aj[j];
      }
    }
#pragma unroll
    for (int c = 0; c < 2; ++c) {
      lsum = tile::mfma16<DT>(pkA[c], ones, lsum);
      lsum = tile::mfma16<DT>(pkB[c], ones, lsum);
    }
    __builtin_amdgcn_sched_barrier(0);
    put_vnew(bufA, 0);
    if (masked) mask_v(bufA, 0, valid, bad);
    pv_tile(bufA, pkA);
    __builtin_amdgcn_sched_barrier(0);
    // the next step's K (none after the range's last step: the wave's end waits for its
    // outstanding loads before it counts its partials in)
    if (has_next) load_k(bufA, nxt.h, bt_nxt, 0);
    __builtin_amdgcn_sched_barrier(0);
    put_vnew(bufB, 1);
    if (masked) mask_v(bufB, 1, valid, bad);
    pv_tile(bufB, pkB);
    __builtin_amdgcn_sched_barrier(0);
    if (has_next) load_k(bufB, nxt.h, bt_nxt, 1);

    if (app_step) {  // the new token goes into its slot after the range (page ids checked)
      const int idn = __builtin_amdgcn_readlane(bt_cur, 8 * (tn >> 4));
      if (idn >= 0 && int64_t(idn) < num_pages) {
        const int64_t slot = int64_t(idn) * page_stride + int64_t(cur.h) * TILE + (tn & 15);
        if (n_rec < SD_APP_REC) {
          if (lane == 0) {
            app_rec[n_rec][0] = slot;
            app_rec[n_rec][1] = app_src;
          }
          ++n_rec;
        } else {
          sd_store_new_token(k_new, v_new, kpool_w, vpool_w, slot, app_src, lane);
        }
      }
    }

    const bool seg_last = cur.ls == cur.ns - 1;
    if (seg_last || !has_next) {
      const int seg_first = gs - cur.ls;  // global index of the segment's first step
      const int64_t row0 = int64_t(cur.b) * Hq + int64_t(cur.h) * G;
      if (seg_last && seg_first >= start) {
        if (4 * g4 < G) {  // lane l holds rows 4 (l / 16) + j
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            if (4 * g4 + j >= G) continue;
            const float inv = lsum[j] > 0.f ? 1.f / lsum[j] : 0.f;
            uint16_t* o = out + (row0 + 4 * g4 + j) * D + n16;
#pragma unroll
            for (int nb = 0; nb < 8; ++nb) o[16 * nb] = to16<DT>(acc[nb][j] * inv);
          }
        }
      } else {
        const int slot = seg_first < start ? 0 : 1;
        arr_first[slot] = seg_first;
        arr_ns[slot] = cur.ns;
        arr_row[slot] = cur.b * Hkv + cur.h;
        // device-coherent partial stores (see paged_decode_stream)
        float* part = ws_part + (int64_t(w) * 2 + slot) * G * (D + 2);
        if (4 * g4 < G) {
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            if (4 * g4 + j >= G) continue;
#pragma unroll
            for (int nb = 0; nb < 8; ++nb)
              sd_store(part + (4 * g4 + j) * (D + 2) + 16 * nb + n16, acc[nb][j]);
            if (n16 == 0) sd_store(part + (4 * g4 + j) * (D + 2) + D + 1, lsum[j]);
          }
        }
        if (g4 == 0 && n16 < G) sd_store(part + n16 * (D + 2) + D, m);
      }
      m = kNegBig;
      lsum = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int nb = 0; nb < 8; ++nb) acc[nb] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    }
    if (!has_next) break;
    if (nxt_opens) {
#pragma unroll
      for (int kc = 0; kc < 4; ++kc) qreg[kc] = q_nxt[kc];
    }
    cur = nxt;
    bt_cur = bt_nxt;
    ++gs;
  }
  if constexpr (APPEND) sd_flush_appends(app_rec, n_rec, k_new, v_new, kpool_w, vpool_w, lane);
  sd_arrive_and_merge<G, DT>(arr_first, arr_ns, arr_row, Dp, Ce, ws_part, ws_meta, token, out, Hkv,
                         lane);
}

// ---------------------------------------------------------------------------------------------
// General kernel
// ---------------------------------------------------------------------------------------------
template <int DT, int DPL>
__global__ __launch_bounds__(64) void paged_attention_generic(
    void* __restrict__ out_, const void* __restrict__ q_, int64_t q_row_stride,
    const void* __restrict__ kp_, const void* __restrict__ vp_,
    const int32_t* __restrict__ bt, int64_t bt_stride, const int32_t* __restrict__ kv_lens,
    const int32_t* __restrict__ cu_q, const int32_t* __restrict__ offsets, int num_seqs, int Hq,
    int Hkv, int D, int P, int64_t num_pages, float scale_log2) {
  using E = Elem<DT>;
  using T = typename E::T;
  T* out = reinterpret_cast<T*>(out_);
  const T* q = reinterpret_cast<const T*>(q_);
  const T* kp = reinterpret_cast<const T*>(kp_);
  const T* vp = reinterpret_cast<const T*>(vp_);
  __shared__ float q_s[64 * DPL];
  __shared__ float p_s[64];
  __shared__ int64_t base_s[64];

  const int64_t row = blockIdx.x;
  const int hq = blockIdx.y, lane = threadIdx.x;
  int b = int(row), s = 0;
  if (cu_q) {
    int lo = 0, hi = num_seqs - 1;  // largest b with cu_q[b] <= row
    while (lo < hi) {
      const int mid = (lo + hi + 1) >> 1;
      if (int64_t(cu_q[mid]) <= row) lo = mid; else hi = mid - 1;
    }
    b = lo;
    s = int(row - cu_q[b]);
  }
  const int kv_len = clamp_len(kv_lens[b], bt_stride, P);
  int limit = kv_len;
  if (offsets) limit = min(limit, offsets[b] + s + 1);
  if (limit < 0) limit = 0;
  const int G = Hq / Hkv;
  const int hk = hq / G;
  const int64_t qoff = row * q_row_stride + int64_t(hq) * D;
  for (int d = lane; d < 64 * DPL; d += 64) q_s[d] = d < D ? E::load(q, qoff + d) : 0.f;
  __syncthreads();

  float m = kNegBig, l = 0.f, acc[DPL];
#pragma unroll
  for (int i = 0; i < DPL; ++i) acc[i] = 0.f;
  const int32_t* btb = bt + int64_t(b) * bt_stride;
  const int64_t DP = int64_t(D) * P;

  for (int j0 = 0; j0 < limit; j0 += 64) {
    const int j = j0 + lane;
    const bool valid = j < limit;
    int64_t base = -1;  // -1: not a key (past the limit, or its page id is out of the pool)
    float sc = 0.f;
    if (valid) {
      const int lp = j / P, off = j - lp * P;
      const int64_t phys = btb[lp];
      if (phys >= 0 && phys < num_pages) {
        base = (phys * Hkv + hk) * DP + off;
        for (int d = 0; d < D; ++d) sc = fmaf(q_s[d], E::load(kp, base + int64_t(d) * P), sc);
      }
    }
    const float x = base >= 0 ? sc * scale_log2 : -INFINITY;
    const float mnew = fmaxf(m, wave_max(x));
    const float alpha = fast_exp2(m - mnew);
    const float p = fast_exp2(x - mnew);
    l = l * alpha + wave_sum(p);
#pragma unroll
    for (int i = 0; i < DPL; ++i) acc[i] *= alpha;
    p_s[lane] = p;
    base_s[lane] = base;
    __syncthreads();
    const int cnt = min(64, limit - j0);
    for (int jj = 0; jj < cnt; ++jj) {
      const float pj = p_s[jj];
      const int64_t bj = base_s[jj];
      if (bj < 0) continue;  // wave-uniform: every lane reads the same LDS entry
#pragma unroll
      for (int i = 0; i < DPL; ++i) {
        const int d = lane + 64 * i;
        if (d < D) acc[i] = fmaf(pj, E::load(vp, bj + int64_t(d) * P), acc[i]);
      }
    }
    __syncthreads();
    m = mnew;
  }
  const int64_t ooff = (row * Hq + hq) * D;
#pragma unroll
  for (int i = 0; i < DPL; ++i) {
    const int d = lane + 64 * i;
    if (d < D) E::store(out, ooff + d, l > 0.f ? acc[i] / l : 0.f);
  }
}

// ---------------------------------------------------------------------------------------------
// Tiled general kernel (paged_attention_tiled<DT, C, VEC, R>): what the fast kernels do not take
// (any storage type, head_dim <= 512, any page size, any Hq / Hkv with G * head_dim <= 8192,
// several rows per sequence with causal offsets). One 256-thread workgroup per (query row, kv
// head) serves the kv head's G q heads, so each key and value is read once per row instead of
// once per q head. Keys go in chunks of C tokens (32; 16 above head_dim 128): the chunk's K and
// V rows are staged in LDS as fp32, [C][Dp] with Dp = D4 + 4 and D4 = head_dim rounded up to 4
// (the pad columns stay zero; the 4-word row skew keeps a quarter-wave's 16-byte reads on
// distinct banks), with one 16-byte load of VEC consecutive tokens of one d when the page size
// is a multiple of VEC (else one element per load). S lanes (S = 1, 2 or 4, as many as leave no
// thread idle) score key t for head g against q pre-scaled by scale * log2(e), each over every
// S-th 4-word group of d, in fp32; a head's C * S lanes are consecutive lanes of one wave, so
// its chunk max and sum are lane-xor reductions; online softmax in fp32, base 2 (a NaN score
// makes its row's output NaN). Thread (g, d pair) accumulates O[g][d], O[g][d + 1] in
// registers, up to R pairs per thread. Keys past a row's limit and on pages whose id is outside
// the pool are not keys; their K / V words are zeros in LDS. Latency is hidden by several
// workgroups per CU (small LDS and register footprint), not by prefetching the next chunk into
// registers, which measured slower for the registers it holds.
// ---------------------------------------------------------------------------------------------
constexpr int PT_THREADS = 256;
constexpr int PT_MAX_GD = 8192;            // G * head_dim limit: 16 pairs per thread
constexpr size_t PT_MAX_LDS = 128 * 1024;  // dynamic LDS limit (of 160 KiB per CU)

// Workgroup barrier after this wave's LDS accesses are done, with no memory fence: the kernel
// shares nothing through global memory. The empty asm statements keep the compiler from moving
// LDS accesses across it.
__device__ __forceinline__ void pt_lds_sync() {
  asm volatile("" ::: "memory");
  // s_waitcnt fields: vmcnt [3:0] and [15:14] (63: no wait), expcnt [6:4] (7: no wait),
  // lgkmcnt [11:8] (0)
  __builtin_amdgcn_s_waitcnt(0xF | (7 << 4) | (3 << 14));
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

__device__ __forceinline__ float pt_xor_max(float v, int from, int to) {
  for (int o = from; o >= to; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  return v;
}
__device__ __forceinline__ float pt_xor_sum(float v, int from, int to) {
  for (int o = from; o >= to; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

template <int DT, int C, int VEC, int R>
__global__ __launch_bounds__(PT_THREADS) void paged_attention_tiled(
    void* __restrict__ out_, const void* __restrict__ q_, int64_t q_row_stride,
    const void* __restrict__ kp_, const void* __restrict__ vp_,
    const int32_t* __restrict__ bt, int64_t bt_stride, const int32_t* __restrict__ kv_lens,
    const int32_t* __restrict__ cu_q, const int32_t* __restrict__ offsets, int num_seqs, int Hq,
    int Hkv, int D, int P, int64_t num_pages, float scale_log2, int S) {
  using E = Elem<DT>;
  using T = typename E::T;
  static_assert(64 % C == 0, "a head's lanes must lie in one wave");
  T* out = reinterpret_cast<T*>(out_);
  const T* q = reinterpret_cast<const T*>(q_);
  const T* kp = reinterpret_cast<const T*>(kp_);
  const T* vp = reinterpret_cast<const T*>(vp_);
  extern __shared__ float4 pt_lds4[];
  __shared__ int64_t tok_base[C];  // element offset of key t (its page tile + slot), -1: no key
  const int G = Hq / Hkv, D4 = (D + 3) & ~3, Dp = D4 + 4, D2 = D4 / 2;
  float* ks = reinterpret_cast<float*>(pt_lds4);  // [C][Dp]
  float* vs = ks + C * Dp;                         // [C][Dp]
  float* qs = vs + C * Dp;                         // [G][D4], pre-scaled, zero past D
  float* ps = qs + G * D4;                         // [G][C]: the chunk's probabilities
  float* hm = ps + G * C;                          // [G]: running max (log2 units)
  float* hl = hm + G;                              // [G]: running sum
  float* ha = hl + G;                              // [G]: the chunk's rescale factor
  const int tid = threadIdx.x;
  const int64_t row = blockIdx.x;
  const int h = blockIdx.y;
  int b = int(row), s = 0;
  if (cu_q) {
    int lo = 0, hi = num_seqs - 1;  // largest b with cu_q[b] <= row
    while (lo < hi) {
      const int mid = (lo + hi + 1) >> 1;
      if (int64_t(cu_q[mid]) <= row) lo = mid; else hi = mid - 1;
    }
    b = lo;
    s = int(row - cu_q[b]);
  }
  const int kv_len = clamp_len(kv_lens[b], bt_stride, P);
  int limit = kv_len;
  if (offsets) limit = min(limit, offsets[b] + s + 1);
  if (limit < 0) limit = 0;
  const int64_t qoff = row * q_row_stride + int64_t(h) * G * D;
  for (int i = tid; i < 2 * C * Dp; i += PT_THREADS) ks[i] = 0.f;  // pad columns stay zero
  for (int i = tid; i < G * D4; i += PT_THREADS) {
    const int g = i / D4, d = i - g * D4;
    qs[i] = d < D ? E::load(q, qoff + int64_t(g) * D + d) * scale_log2 : 0.f;
  }
  for (int g = tid; g < G; g += PT_THREADS) {
    hm[g] = -INFINITY;
    hl[g] = 0.f;
  }
  float2 acc[R];
#pragma unroll
  for (int r = 0; r < R; ++r) acc[r] = make_float2(0.f, 0.f);
  const int32_t* btb = bt + int64_t(b) * bt_stride;
  const int64_t DP = int64_t(D) * P;
  const int lanes = C * S;  // lanes of one head in the scoring phase
  const int sl = tid % S, t_me = (tid / S) % C;

  for (int c0 = 0; c0 < limit; c0 += C) {
    if (tid < C) {
      const int j = c0 + tid;
      int64_t base = -1;
      if (j < limit) {
        const int lp = j / P, off = j - lp * P;
        const int64_t phys = btb[lp];
        if (phys >= 0 && phys < num_pages) base = (phys * Hkv + h) * DP + off;
      }
      tok_base[tid] = base;
    }
    pt_lds_sync();  // also: the previous chunk's products are done with ks / vs / ps
    if constexpr (VEC > 1) {
      // VEC consecutive keys of one d per 16-byte load: the group lies in one page (the page
      // size is a multiple of VEC and so is c0); keys of it past the limit are zeroed
      for (int i = tid; i < (C / VEC) * D; i += PT_THREADS) {
        const int tg = i % (C / VEC), d = i / (C / VEC), t0 = tg * VEC;
        const int64_t b0 = tok_base[t0];
        uint4 kw = make_uint4(0u, 0u, 0u, 0u), vw = make_uint4(0u, 0u, 0u, 0u);
        if (b0 >= 0) {
          kw = *reinterpret_cast<const uint4*>(kp + b0 + int64_t(d) * P);
          vw = *reinterpret_cast<const uint4*>(vp + b0 + int64_t(d) * P);
        }
        const T* ke = reinterpret_cast<const T*>(&kw);
        const T* ve = reinterpret_cast<const T*>(&vw);
#pragma unroll
        for (int e = 0; e < VEC; ++e) {
          const bool ok = c0 + t0 + e < limit;
          ks[(t0 + e) * Dp + d] = ok ? E::load(ke, e) : 0.f;
          vs[(t0 + e) * Dp + d] = ok ? E::load(ve, e) : 0.f;
        }
      }
    } else {
      for (int i = tid; i < C * D; i += PT_THREADS) {
        const int t = i % C, d = i / C;
        const int64_t b0 = tok_base[t];
        ks[t * Dp + d] = b0 >= 0 ? E::load(kp, b0 + int64_t(d) * P) : 0.f;
        vs[t * Dp + d] = b0 >= 0 ? E::load(vp, b0 + int64_t(d) * P) : 0.f;
      }
    }
    pt_lds_sync();
    // scores of the chunk, its max and sum per head; the head's running max, sum and rescale
    for (int g0 = 0; g0 < G; g0 += PT_THREADS / lanes) {
      const int g = g0 + tid / lanes, t = t_me;
      float x = -INFINITY;
      if (g < G) {
        const float4* qg = reinterpret_cast<const float4*>(qs + g * D4);
        const float4* kt = reinterpret_cast<const float4*>(ks + t * Dp);
        float a0 = 0.f, a1 = 0.f, a2 = 0.f, a3 = 0.f;
#pragma unroll 4
        for (int i = sl; i < D4 / 4; i += S) {
          const float4 qv = qg[i], kv = kt[i];
          a0 = fmaf(qv.x, kv.x, a0);
          a1 = fmaf(qv.y, kv.y, a1);
          a2 = fmaf(qv.z, kv.z, a2);
          a3 = fmaf(qv.w, kv.w, a3);
        }
        x = pt_xor_sum((a0 + a1) + (a2 + a3), S / 2, 1);
        if (tok_base[t] < 0) x = -INFINITY;
      }
      const float mx = pt_xor_max(x, lanes / 2, S);
      const float mo = g < G ? hm[g] : -INFINITY;
      const float mn = fmaxf(mo, mx);
      const float pr = x == -INFINITY ? 0.f : fast_exp2(x - mn);
      const float sum = pt_xor_sum(sl == 0 ? pr : 0.f, lanes / 2, 1);
      if (g < G && sl == 0) {
        ps[g * C + t] = pr;
        if (t == 0) {  // every lane of the head has read hm[g] above
          const float al = mo == -INFINITY ? 0.f : fast_exp2(mo - mn);
          hm[g] = mn;
          hl[g] = hl[g] * al + sum;
          ha[g] = al;
        }
      }
    }
    pt_lds_sync();
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int idx = tid + r * PT_THREADS;
      if (idx < G * D2) {
        const int g = idx / D2, d = 2 * (idx - g * D2);
        const float al = ha[g];
        float2 a = make_float2(acc[r].x * al, acc[r].y * al);
        const float4* pg = reinterpret_cast<const float4*>(ps + g * C);
#pragma unroll 2
        for (int t4 = 0; t4 < C / 4; ++t4) {
          const float4 pw = pg[t4];
          const float* v0 = vs + (4 * t4) * Dp + d;
          const float2 w0 = *reinterpret_cast<const float2*>(v0);
          const float2 w1 = *reinterpret_cast<const float2*>(v0 + Dp);
          const float2 w2 = *reinterpret_cast<const float2*>(v0 + 2 * Dp);
          const float2 w3 = *reinterpret_cast<const float2*>(v0 + 3 * Dp);
          a.x = fmaf(pw.x, w0.x, a.x);
          a.y = fmaf(pw.x, w0.y, a.y);
          a.x = fmaf(pw.y, w1.x, a.x);
          a.y = fmaf(pw.y, w1.y, a.y);
          a.x = fmaf(pw.z, w2.x, a.x);
          a.y = fmaf(pw.z, w2.y, a.y);
          a.x = fmaf(pw.w, w3.x, a.x);
          a.y = fmaf(pw.w, w3.y, a.y);
        }
        acc[r] = a;
      }
    }
  }
  pt_lds_sync();  // hl final
  const int64_t ooff = (row * Hq + int64_t(h) * G) * D;
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int idx = tid + r * PT_THREADS;
    if (idx < G * D2) {
      const int g = idx / D2, d = 2 * (idx - g * D2);
      const float l = hl[g];
      const float inv = l > 0.f ? 1.f / l : 0.f;
      if (d < D) E::store(out, ooff + int64_t(g) * D + d, acc[r].x * inv);
      if (d + 1 < D) E::store(out, ooff + int64_t(g) * D + d + 1, acc[r].y * inv);
    }
  }
}

// Dynamic LDS of paged_attention_tiled: K and V chunks, q, probabilities, per-head running
// max / sum / rescale.
inline size_t tiled_lds_bytes(int C, int G, int D) {
  const int D4 = (D + 3) & ~3;
  return size_t(2 * C * (D4 + 4) + G * D4 + G * C + 3 * G) * sizeof(float);
}

template <int DT>
int launch_generic(void* out, const void* q, int64_t q_row_stride, const void* kp, const void* vp,
                   const int32_t* bt, int64_t bt_stride, const int32_t* kv_lens,
                   const int32_t* cu_q, const int32_t* offsets, int num_seqs, int64_t rows, int Hq,
                   int Hkv, int D, int P, int64_t num_pages, float scale_log2, hipStream_t s) {
  const int G = Hq / Hkv;
  const int C = D <= 128 ? 32 : 16;  // 16 above 128: four workgroups' chunks fit one CU's LDS
  const size_t lds = tiled_lds_bytes(C, G, D);
  const int64_t pairs = int64_t(G) * (((D + 3) & ~3) / 2);  // (g, d pair) items
  if (pairs <= PT_MAX_GD / 2 && D <= 512 && lds <= PT_MAX_LDS) {
    using T = typename Elem<DT>::T;
    constexpr int VEC = 16 / int(sizeof(T));
    const bool vec = P % VEC == 0 && aligned(kp, 16) && aligned(vp, 16);
    int S = 1;  // lanes per (head, key) score: as many as leave no thread idle, <= 64 / C
    while (S < 4 && int64_t(G) * C * S * 2 <= PT_THREADS && C * S * 2 <= 64) S *= 2;
    const bool small = pairs <= 4 * PT_THREADS;
    const dim3 tgrid = dim3(unsigned(rows), unsigned(Hkv));
#define PIA_TILED(CC, VV, RR)                                                                  \
  {                                                                                            \
    auto* kern = &paged_attention_tiled<DT, CC, VV, RR>;                                       \
    if (lds > 65536)                                                                           \
      if (int rc = check_hip(hipFuncSetAttribute(reinterpret_cast<const void*>(kern),          \
                                                 hipFuncAttributeMaxDynamicSharedMemorySize,   \
                                                 int(lds)),                                    \
                             "paged_attention_tiled: LDS size"))                               \
        return rc;                                                                             \
    hipLaunchKernelGGL(kern, tgrid, dim3(PT_THREADS), lds, s, out, q, q_row_stride, kp, vp,   \
                       bt, bt_stride, kv_lens, cu_q, offsets, num_seqs, Hq, Hkv, D, P,         \
                       num_pages, scale_log2, S);                                              \
  }
#define PIA_TILED_R(CC, VV) \
  if (small) PIA_TILED(CC, VV, 4) else PIA_TILED(CC, VV, 16)
    if (C == 32) {
      if (vec) PIA_TILED_R(32, VEC) else PIA_TILED_R(32, 1)
    } else {
      if (vec) PIA_TILED_R(16, VEC) else PIA_TILED_R(16, 1)
    }
#undef PIA_TILED_R
#undef PIA_TILED
    return check_launch("paged_attention_tiled");
  }
  dim3 grid = dim3(unsigned(rows), unsigned(Hq));
#define PIA_GEN(DPL)                                                                        \
  hipLaunchKernelGGL((paged_attention_generic<DT, DPL>), grid, dim3(64), 0, s, out, q,      \
                     q_row_stride, kp, vp, bt, bt_stride, kv_lens, cu_q, offsets, num_seqs, \
                     Hq, Hkv, D, P, num_pages, scale_log2)
  if (D <= 64) PIA_GEN(1);
  else if (D <= 128) PIA_GEN(2);
  else if (D <= 256) PIA_GEN(4);
  else PIA_GEN(8);
#undef PIA_GEN
  return check_launch("paged_attention_generic");
}

int launch_generic_any(int dtype, void* out, const void* q, int64_t q_row_stride, const void* kp,
                       const void* vp, const int32_t* bt, int64_t bt_stride,
                       const int32_t* kv_lens, const int32_t* cu_q, const int32_t* offsets,
                       int num_seqs, int64_t rows, int Hq, int Hkv, int D, int P,
                       int64_t num_pages, float scale_log2, hipStream_t s) {
  switch (dtype) {
    case PIA_DTYPE_F32:
      return launch_generic<PIA_DTYPE_F32>(out, q, q_row_stride, kp, vp, bt, bt_stride, kv_lens,
                                           cu_q, offsets, num_seqs, rows, Hq, Hkv, D, P,
                                           num_pages, scale_log2, s);
    case PIA_DTYPE_F16:
      return launch_generic<PIA_DTYPE_F16>(out, q, q_row_stride, kp, vp, bt, bt_stride, kv_lens,
                                           cu_q, offsets, num_seqs, rows, Hq, Hkv, D, P,
                                           num_pages, scale_log2, s);
    case PIA_DTYPE_BF16:
      return launch_generic<PIA_DTYPE_BF16>(out, q, q_row_stride, kp, vp, bt, bt_stride,
                                            kv_lens, cu_q, offsets, num_seqs, rows, Hq, Hkv, D,
                                            P, num_pages, scale_log2, s);
  }
  return fail(PIA_EINVAL, "paged attention: unknown dtype");
}

// The new tokens of a decode step into their slots (any dtype, head_dim, page size): row b's
// k_new / v_new [Hkv, D] go to position L_b - 1 of its block table, for 1 <= L_b <= the table's
// width in tokens and a page id inside the pool (other rows write nothing). One workgroup per
// row, thread i over the row's Hkv * D elements.
template <typename T>
__global__ __launch_bounds__(256) void kv_append_kernel(
    T* __restrict__ kpool, T* __restrict__ vpool, const T* __restrict__ k_new,
    const T* __restrict__ v_new, int64_t new_seq_stride, const int32_t* __restrict__ bt,
    int64_t bt_stride, const int32_t* __restrict__ context_lens, int Hkv, int D, int P,
    int64_t num_pages) {
  const int b = blockIdx.x;
  const int L = context_lens[b];
  if (L < 1 || int64_t(L) > bt_stride * P) return;
  const int64_t page = bt[int64_t(b) * bt_stride + (L - 1) / P];
  if (page < 0 || page >= num_pages) return;
  const int off = (L - 1) % P;
  const int n = Hkv * D;
  for (int i = threadIdx.x; i < n; i += 256) {
    const int h = i / D, d = i - h * D;
    const int64_t dst = ((page * Hkv + h) * D + d) * P + off;
    const int64_t src = int64_t(b) * new_seq_stride + i;
    kpool[dst] = k_new[src];
    vpool[dst] = v_new[src];
  }
}

int launch_kv_append(int dtype, void* kp, void* vp, const void* k_new, const void* v_new,
                     int64_t new_seq_stride, const int32_t* bt, int64_t bt_stride,
                     const int32_t* context_lens, int B, int Hkv, int D, int P,
                     int64_t num_pages, hipStream_t s) {
#define PIA_KA(T)                                                                            \
  hipLaunchKernelGGL(kv_append_kernel<T>, dim3(unsigned(B)), dim3(256), 0, s,                \
                     reinterpret_cast<T*>(kp), reinterpret_cast<T*>(vp),                     \
                     reinterpret_cast<const T*>(k_new), reinterpret_cast<const T*>(v_new),   \
                     new_seq_stride, bt, bt_stride, context_lens, Hkv, D, P, num_pages)
  if (dtype == PIA_DTYPE_F32) PIA_KA(float);
  else PIA_KA(uint16_t);
#undef PIA_KA
  return check_launch("kv_append_kernel");
}

int check_heads(int Hq, int Hkv, int D, int P, int64_t num_pages, int dtype) {
  if (Hq <= 0 || Hkv <= 0 || D <= 0 || P <= 0 || num_pages <= 0)
    return fail(PIA_EINVAL, "paged attention: heads, head_dim, page_size, num_pages must be > 0");
  if (Hq % Hkv) return fail(PIA_EINVAL, "paged attention: num_heads % num_kv_heads != 0");
  if (D > 512) return fail(PIA_EUNSUPPORTED, "paged attention: head_dim > 512");
  if (Hq > 65535) return fail(PIA_EINVAL, "paged attention: num_heads > 65535");
  if (dtype != PIA_DTYPE_F32 && dtype != PIA_DTYPE_F16 && dtype != PIA_DTYPE_BF16)
    return fail(PIA_EINVAL, "paged attention: unknown dtype");
  return 0;
}

bool fast_path(int dtype, int Hq, int Hkv, int D, int P) {
  const int G = Hq / Hkv;
  return (dtype == PIA_DTYPE_BF16 || dtype == PIA_DTYPE_F16) && D == FD_D && P == FD_P &&
         Hq % Hkv == 0 && stream_group_ok(G);
}

// Whether a decode launch with G q rows per kv head runs the matrix-core engine: every fast
// group size but 1, 2 and 4. At G = 4 (Qwen3-8B, batch 256) the vector-ALU engine at two waves
// per SIMD measured 0.718 ms per step against 0.740 ms for the matrix-core engine at one (its
// registers), so the powers of two up to 4 stay on paged_decode_stream.
bool stream_uses_mfma(int G) { return !(G == 1 || G == 2 || G == 4); }

// Waves of a stream launch (CU count cached per device), capped by the partial slots the
// workspace holds: two single-wave workgroups per SIMD for the vector-ALU engine, one for the
// matrix-core engine (its registers).
int stream_waves(int G) {
  const int n = std::min(device_cus() * (stream_uses_mfma(G) ? SD_WAVES_PER_CU / 2
                                                              : SD_WAVES_PER_CU),
                         SD_MAX_WAVES);
  return std::max(2, n & ~1);  // whole (even, odd) pairs
}

}  // namespace
}  // namespace pia

using namespace pia;

namespace pia {
namespace {

// Argument checks shared by both decode entry points (nothing enqueued on failure).
int check_decode_args(const void* out, const void* q, int64_t q_seq_stride, const void* k_pages,
                      const void* v_pages, const int32_t* block_tables, int64_t bt_stride,
                      const int32_t* context_lens, int num_seqs, int num_heads, int num_kv_heads,
                      int head_dim, int page_size, int64_t num_pages, int dtype) {
  if (int rc = check_heads(num_heads, num_kv_heads, head_dim, page_size, num_pages, dtype))
    return rc;
  if (num_seqs < 0 || bt_stride < 0) return fail(PIA_EINVAL, "paged_decode: negative size");
  if (num_seqs == 0) return 0;
  if (!out || !q || !k_pages || !v_pages || !block_tables || !context_lens)
    return fail(PIA_EINVAL, "paged_decode: null pointer");
  if (bt_stride == 0) return fail(PIA_EINVAL, "paged_decode: bt_stride == 0");
  if (num_seqs > 65535) return fail(PIA_EINVAL, "paged_decode: num_seqs > 65535");
  if (q_seq_stride < int64_t(num_heads) * head_dim)
    return fail(PIA_EINVAL, "paged_decode: q_seq_stride < num_heads*head_dim");
  if (fast_path(dtype, num_heads, num_kv_heads, head_dim, page_size)) {
    if (!aligned(q, 4) || !aligned(k_pages, 16) || !aligned(v_pages, 16) || (q_seq_stride & 1))
      return fail(PIA_EINVAL, "paged_decode: q must be 4-byte and pools 16-byte aligned");
    // The stream kernel's step arithmetic is int32: Hkv * (sequences of a launch) * (steps per
    // sequence) plus a wave count must stay below 2^31.
    const int NW = stream_waves(num_heads / num_kv_heads);
    if (int64_t(num_kv_heads) * std::min(num_seqs, SD_MAX_SEQS) * ceil_div(bt_stride, 8) +
            2 * int64_t(NW) >= (int64_t(1) << 31))
      return fail(PIA_EUNSUPPORTED, "paged_decode: batch too large for int32 step indices");
  }
  return 0;
}

// The fast path (checked arguments): the stream kernel, in launches of up to SD_MAX_SEQS
// sequences that reuse the same scratch (`scratch`, laid out by decode_scratch_layout for
// `scratch_waves` waves, at least the NW waves of a launch). Launches on one stream are ordered,
// so the reuse is safe; each launch takes a fresh token for its counters.
// k_new != nullptr: append mode (the new tokens of the step in k_new / v_new, written into the
// pools by the kernel; k_pages / v_pages are then written too).
// Launch tokens for the arrival counters: the upper 48 bits of a 64-bit word, a process-wide
// sequence from a random start (a workspace never used before matches one with probability
// 2^-48 per counter).
uint64_t next_stream_token() {
  static std::atomic<uint64_t> seq{(uint64_t(std::random_device{}()) << 32) ^
                                   uint64_t(std::random_device{}())};
  return (seq.fetch_add(1, std::memory_order_relaxed) & 0xffffffffffffull) << 16;
}

template <int DT>
int launch_stream_decode_dt(void* out, const void* q, int64_t q_seq_stride, const void* k_pages,
                            const void* v_pages, const int32_t* block_tables, int64_t bt_stride,
                            const int32_t* context_lens, int num_seqs, int num_heads,
                            int num_kv_heads, int64_t num_pages, float scale_log2,
                            unsigned char* scratch, int scratch_waves, hipStream_t s,
                            const void* k_new, const void* v_new, int64_t new_seq_stride) {
  const int G = num_heads / num_kv_heads;
  const int NW = stream_waves(G);
  if (NW > scratch_waves) {
    set_error("paged_decode: %d waves, the scratch holds %d", NW, scratch_waves);
    return PIA_EUNSUPPORTED;
  }
  int32_t* ws_meta = reinterpret_cast<int32_t*>(scratch);
  float* ws_part =
      reinterpret_cast<float*>(scratch + decode_scratch_layout(G, scratch_waves).part_offset);
  uint16_t* kw = const_cast<uint16_t*>(reinterpret_cast<const uint16_t*>(k_pages));
  uint16_t* vw = const_cast<uint16_t*>(reinterpret_cast<const uint16_t*>(v_pages));
  for (int b0 = 0; b0 < num_seqs; b0 += SD_MAX_SEQS) {
    const int Bs = std::min(SD_MAX_SEQS, num_seqs - b0);
    uint16_t* o = reinterpret_cast<uint16_t*>(out) + int64_t(b0) * num_heads * FD_D;
    const uint16_t* qq = reinterpret_cast<const uint16_t*>(q) + int64_t(b0) * q_seq_stride;
    const int32_t* bt = block_tables + int64_t(b0) * bt_stride;
    const int32_t* cl = context_lens + b0;
    const uint16_t* kn =
        k_new ? reinterpret_cast<const uint16_t*>(k_new) + int64_t(b0) * new_seq_stride : nullptr;
    const uint16_t* vn =
        k_new ? reinterpret_cast<const uint16_t*>(v_new) + int64_t(b0) * new_seq_stride : nullptr;
    const size_t lds = size_t(2 * Bs + 1) * sizeof(int32_t);
    const uint64_t token = next_stream_token();
#define PIA_SD(GG, AP)                                                                         \
  hipLaunchKernelGGL((paged_decode_stream<GG, AP, DT>), dim3(unsigned(NW)), dim3(64), lds, s, o, \
                     qq, q_seq_stride, (const uint16_t*)k_pages, (const uint16_t*)v_pages, bt, \
                     bt_stride, cl, Bs, num_kv_heads, num_pages, ws_part, ws_meta, scale_log2, \
                     kw, vw, kn, vn, new_seq_stride, token)
#define PIA_SDM(GG, AP)                                                                        \
  hipLaunchKernelGGL((paged_decode_mfma<GG, AP, DT>), dim3(unsigned(NW)), dim3(64), lds, s, o, qq, \
                     q_seq_stride, (const uint16_t*)k_pages, (const uint16_t*)v_pages, bt,     \
                     bt_stride, cl, Bs, num_kv_heads, num_pages, ws_part, ws_meta, scale_log2, \
                     kw, vw, kn, vn, new_seq_stride, token)
    if (kn) {
      switch (G) {
        case 1: PIA_SD(1, true); break;
        case 2: PIA_SD(2, true); break;
        case 4: PIA_SD(4, true); break;
        case 3: PIA_SDM(3, true); break;
        case 5: PIA_SDM(5, true); break;
        case 6: PIA_SDM(6, true); break;
        case 7: PIA_SDM(7, true); break;
        case 16: PIA_SDM(16, true); break;
        default: PIA_SDM(8, true); break;
      }
    } else {
      switch (G) {
        case 1: PIA_SD(1, false); break;
        case 2: PIA_SD(2, false); break;
        case 4: PIA_SD(4, false); break;
        case 3: PIA_SDM(3, false); break;
        case 5: PIA_SDM(5, false); break;
        case 6: PIA_SDM(6, false); break;
        case 7: PIA_SDM(7, false); break;
        case 16: PIA_SDM(16, false); break;
        default: PIA_SDM(8, false); break;
      }
    }
#undef PIA_SD
#undef PIA_SDM
    if (int rc = check_launch("paged_decode_stream")) return rc;
  }
  return 0;
}

// The fast decode launch for a 16-bit dtype (PIA_DTYPE_BF16 or PIA_DTYPE_F16, see fast_path).
int launch_stream_decode(int dtype, void* out, const void* q, int64_t q_seq_stride,
                         const void* k_pages, const void* v_pages, const int32_t* block_tables,
                         int64_t bt_stride, const int32_t* context_lens, int num_seqs,
                         int num_heads, int num_kv_heads, int64_t num_pages, float scale_log2,
                         unsigned char* scratch, int scratch_waves, hipStream_t s,
                         const void* k_new = nullptr, const void* v_new = nullptr,
                         int64_t new_seq_stride = 0) {
  auto* launch = dtype == PIA_DTYPE_F16 ? &launch_stream_decode_dt<PIA_DTYPE_F16>
                                        : &launch_stream_decode_dt<PIA_DTYPE_BF16>;
  return launch(out, q, q_seq_stride, k_pages, v_pages, block_tables, bt_stride, context_lens,
                num_seqs, num_heads, num_kv_heads, num_pages, scale_log2, scratch, scratch_waves,
                s, k_new, v_new, new_seq_stride);
}

// ---------------------------------------------------------------------------------------------
// Library-owned scratch for pia_paged_decode_attention_noalloc: the meta ints (arrival
// counters), then the wave partials, in one static device array per GPU (held until the process
// ends). It is never cleared: each launch writes the partials it reads, and the counters carry
// a launch token, so whatever an earlier call left in them reads as stale. Every call on one
// GPU shares that GPU's array: calls that overlap (two streams, or two host threads without
// ordering) race on it.
// ---------------------------------------------------------------------------------------------
constexpr int64_t kNoAllocScratchBytes = int64_t(32) << 20;                  // 32 MiB per GPU
static __device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];

constexpr int kMaxDevices = 64;
std::atomic<unsigned char*> g_scratch_of[kMaxDevices];
std::mutex g_scratch_mu;

// Device address of `scratch` on the current device, resolved once per device with
// hipGetSymbolAddress (in host code the array's name is not a device address).
int scratch_ptr(unsigned char** ptr) {
  int dev = 0;
  if (int rc = check_hip(hipGetDevice(&dev), "paged_decode_noalloc: hipGetDevice")) return rc;
  if (dev < 0 || dev >= kMaxDevices) return fail(PIA_EUNSUPPORTED, "paged_decode_noalloc: device id >= 64");
  unsigned char* p = g_scratch_of[dev].load(std::memory_order_acquire);
  if (!p) {
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    p = g_scratch_of[dev].load(std::memory_order_relaxed);
    if (!p) {
      void* addr = nullptr;
      if (int rc = check_hip(hipGetSymbolAddress(&addr, HIP_SYMBOL(scratch)),
                             "paged_decode_noalloc: hipGetSymbolAddress(scratch)"))
        return rc;
      p = static_cast<unsigned char*>(addr);
      g_scratch_of[dev].store(p, std::memory_order_release);
    }
  }
  *ptr = p;
  return 0;
}

}  // namespace
}  // namespace pia

extern "C" int64_t pia_paged_decode_workspace_bytes(int num_seqs, int num_heads, int num_kv_heads,
                                                    int head_dim, int page_size,
                                                    int64_t bt_stride) {
  if (head_dim != FD_D || page_size != FD_P || num_seqs <= 0 || num_heads <= 0 ||
      num_kv_heads <= 0 || num_heads % num_kv_heads || bt_stride <= 0)
    return 0;
  const int G = num_heads / num_kv_heads;
  if (!stream_group_ok(G)) return 0;
  return decode_scratch_layout(G, SD_MAX_WAVES).total_bytes;
}

extern "C" int pia_paged_decode_scratch_layout(int num_heads, int num_kv_heads, int waves,
                                               int64_t* partials_offset, int64_t* total_bytes) {
  if (!partials_offset || !total_bytes) return fail(PIA_EINVAL, "decode_scratch_layout: null pointer");
  if (num_heads <= 0 || num_kv_heads <= 0 || num_heads % num_kv_heads ||
      !stream_group_ok(num_heads / num_kv_heads))
    return fail(PIA_EUNSUPPORTED, "decode_scratch_layout: Hq / Hkv must be 1..8 or 16");
  if (waves < 2 || waves > SD_MAX_WAVES)
    return fail(PIA_EINVAL, "decode_scratch_layout: waves must be in [2, 4096]");
  const DecodeScratchLayout lay = decode_scratch_layout(num_heads / num_kv_heads, waves);
  *partials_offset = lay.part_offset;
  *total_bytes = lay.total_bytes;
  return 0;
}

extern "C" int pia_paged_decode_attention(void* out, const void* q, int64_t q_seq_stride,
                                          const void* k_pages, const void* v_pages,
                                          const int32_t* block_tables, int64_t bt_stride,
                                          const int32_t* context_lens, int num_seqs,
                                          int num_heads, int num_kv_heads, int head_dim,
                                          int page_size, int64_t num_pages, float scale,
                                          int dtype, void* workspace, int64_t workspace_bytes,
                                          void* stream) {
  if (int rc = check_decode_args(out, q, q_seq_stride, k_pages, v_pages, block_tables, bt_stride,
                                 context_lens, num_seqs, num_heads, num_kv_heads, head_dim,
                                 page_size, num_pages, dtype))
    return rc;
  if (num_seqs == 0) return 0;
  const float scale_log2 = scale * kLog2e;
  hipStream_t s = as_stream(stream);
  if (fast_path(dtype, num_heads, num_kv_heads, head_dim, page_size)) {
    const int64_t need = pia_paged_decode_workspace_bytes(num_seqs, num_heads, num_kv_heads,
                                                          head_dim, page_size, bt_stride);
    if (!workspace || workspace_bytes < need) {
      set_error("paged_decode: workspace of %lld bytes needed, %lld given", (long long)need,
                (long long)workspace_bytes);
      return PIA_EINVAL;
    }
    if (!aligned(workspace, 4)) return fail(PIA_EINVAL, "paged_decode: workspace not 4-byte aligned");
    return launch_stream_decode(dtype, out, q, q_seq_stride, k_pages, v_pages, block_tables,
                                bt_stride, context_lens, num_seqs, num_heads, num_kv_heads,
                                num_pages, scale_log2, static_cast<unsigned char*>(workspace),
                                SD_MAX_WAVES, s);
  }
  return launch_generic_any(dtype, out, q, q_seq_stride, k_pages, v_pages, block_tables,
                            bt_stride, context_lens, nullptr, nullptr, num_seqs, num_seqs,
                            num_heads, num_kv_heads, head_dim, page_size, num_pages, scale_log2,
                            s);
}

extern "C" int pia_paged_decode_append_attention(
    void* out, const void* q, int64_t q_seq_stride, void* k_pages, void* v_pages,
    const int32_t* block_tables, int64_t bt_stride, const int32_t* context_lens,
    const void* k_new, const void* v_new, int64_t new_seq_stride, int num_seqs, int num_heads,
    int num_kv_heads, int head_dim, int page_size, int64_t num_pages, float scale, int dtype,
    void* workspace, int64_t workspace_bytes, void* stream) {
  if (int rc = check_decode_args(out, q, q_seq_stride, k_pages, v_pages, block_tables, bt_stride,
                                 context_lens, num_seqs, num_heads, num_kv_heads, head_dim,
                                 page_size, num_pages, dtype))
    return rc;
  if (num_seqs == 0) return 0;
  if (!k_new || !v_new) return fail(PIA_EINVAL, "paged_decode_append: null k_new / v_new");
  if (new_seq_stride < int64_t(num_kv_heads) * head_dim)
    return fail(PIA_EINVAL, "paged_decode_append: new_seq_stride < num_kv_heads*head_dim");
  const float scale_log2 = scale * kLog2e;
  hipStream_t s = as_stream(stream);
  if (fast_path(dtype, num_heads, num_kv_heads, head_dim, page_size)) {
    if (!aligned(k_new, 2) || !aligned(v_new, 2))
      return fail(PIA_EINVAL, "paged_decode_append: k_new / v_new must be 2-byte aligned");
    const int64_t need = pia_paged_decode_workspace_bytes(num_seqs, num_heads, num_kv_heads,
                                                          head_dim, page_size, bt_stride);
    if (!workspace || workspace_bytes < need) {
      set_error("paged_decode_append: workspace of %lld bytes needed, %lld given",
                (long long)need, (long long)workspace_bytes);
      return PIA_EINVAL;
    }
    if (!aligned(workspace, 4))
      return fail(PIA_EINVAL, "paged_decode_append: workspace not 4-byte aligned");
    return launch_stream_decode(dtype, out, q, q_seq_stride, k_pages, v_pages, block_tables,
                                bt_stride, context_lens, num_seqs, num_heads, num_kv_heads,
                                num_pages, scale_log2, static_cast<unsigned char*>(workspace),
                                SD_MAX_WAVES, s, k_new, v_new, new_seq_stride);
  }
  // any other shape: the new tokens into their slots, then the decode over the pool
  if (int rc = launch_kv_append(dtype, k_pages, v_pages, k_new, v_new, new_seq_stride,
                                block_tables, bt_stride, context_lens, num_seqs, num_kv_heads,
                                head_dim, page_size, num_pages, s))
    return rc;
  return launch_generic_any(dtype, out, q, q_seq_stride, k_pages, v_pages, block_tables,
                            bt_stride, context_lens, nullptr, nullptr, num_seqs, num_seqs,
                            num_heads, num_kv_heads, head_dim, page_size, num_pages, scale_log2,
                            s);
}

extern "C" int64_t pia_paged_decode_noalloc_scratch_bytes(int num_heads, int num_kv_heads) {
  if (num_heads <= 0 || num_kv_heads <= 0 || num_heads % num_kv_heads) return 0;
  const int G = num_heads / num_kv_heads;
  if (!stream_group_ok(G)) return 0;
  return decode_scratch_layout(G, stream_waves(G)).total_bytes;
}

extern "C" int pia_paged_decode_attention_noalloc(void* out, const void* q, int64_t q_seq_stride,
                                                  const void* k_pages, const void* v_pages,
                                                  const int32_t* block_tables, int64_t bt_stride,
                                                  const int32_t* context_lens, int num_seqs,
                                                  int num_heads, int num_kv_heads, int head_dim,
                                                  int page_size, int64_t num_pages, float scale,
                                                  int dtype, void* stream) {
  if (int rc = check_decode_args(out, q, q_seq_stride, k_pages, v_pages, block_tables, bt_stride,
                                 context_lens, num_seqs, num_heads, num_kv_heads, head_dim,
                                 page_size, num_pages, dtype))
    return rc;
  if (num_seqs == 0) return 0;
  const float scale_log2 = scale * kLog2e;
  hipStream_t s = as_stream(stream);
  if (!fast_path(dtype, num_heads, num_kv_heads, head_dim, page_size))  // no scratch needed
    return launch_generic_any(dtype, out, q, q_seq_stride, k_pages, v_pages, block_tables,
                              bt_stride, context_lens, nullptr, nullptr, num_seqs, num_seqs,
                              num_heads, num_kv_heads, head_dim, page_size, num_pages,
                              scale_log2, s);
  const int64_t need = pia_paged_decode_noalloc_scratch_bytes(num_heads, num_kv_heads);
  if (need > kNoAllocScratchBytes) {
    set_error("paged_decode_noalloc: %lld bytes of scratch needed (%d waves), the library's "
              "static scratch holds %lld", (long long)need,
              stream_waves(num_heads / num_kv_heads), (long long)kNoAllocScratchBytes);
    return PIA_EUNSUPPORTED;
  }
  unsigned char* base = nullptr;
  if (int rc = scratch_ptr(&base)) return rc;
  return launch_stream_decode(dtype, out, q, q_seq_stride, k_pages, v_pages, block_tables,
                              bt_stride, context_lens, num_seqs, num_heads, num_kv_heads,
                              num_pages, scale_log2, base, stream_waves(num_heads / num_kv_heads),
                              s);
}

extern "C" int pia_paged_attention(void* out, const void* q, const void* k_pages,
                                   const void* v_pages, const int32_t* block_tables,
                                   int64_t bt_stride, const int32_t* kv_lens, const int32_t* cu_q,
                                   const int32_t* q_pos_offsets, int num_seqs,
                                   int64_t total_q_rows, int num_heads, int num_kv_heads,
                                   int head_dim, int page_size, int64_t num_pages, float scale,
                                   int dtype, void* stream) {
  if (int rc = check_heads(num_heads, num_kv_heads, head_dim, page_size, num_pages, dtype))
    return rc;
  if (num_seqs < 0 || total_q_rows < 0 || bt_stride < 0)
    return fail(PIA_EINVAL, "paged_attention: negative size");
  if (num_seqs == 0 || total_q_rows == 0) return 0;
  if (!out || !q || !k_pages || !v_pages || !block_tables || !kv_lens)
    return fail(PIA_EINVAL, "paged_attention: null pointer");
  if (bt_stride == 0) return fail(PIA_EINVAL, "paged_attention: bt_stride == 0");
  if (!cu_q && total_q_rows != num_seqs)
    return fail(PIA_EINVAL, "paged_attention: without cu_q, total_q_rows must equal num_seqs");
  if (total_q_rows > 0x7fffffff) return fail(PIA_EINVAL, "paged_attention: too many rows");
  if (prefill_mfma_path(dtype, num_heads, num_kv_heads, head_dim, page_size, num_seqs,
                        total_q_rows, cu_q, scale) &&
      aligned(q, 16) && aligned(out, 16) && aligned(k_pages, 16) && aligned(v_pages, 16))
    return launch_prefill_mfma(dtype, out, q, k_pages, v_pages, block_tables, bt_stride, kv_lens,
                               cu_q, q_pos_offsets, num_seqs, total_q_rows, num_heads,
                               num_kv_heads, num_pages, scale * kLog2e, as_stream(stream));
  return launch_generic_any(dtype, out, q, int64_t(num_heads) * head_dim, k_pages, v_pages,
                            block_tables, bt_stride, kv_lens, cu_q, q_pos_offsets, num_seqs,
                            total_q_rows, num_heads, num_kv_heads, head_dim, page_size,
                            num_pages, scale * kLog2e, as_stream(stream));
}
