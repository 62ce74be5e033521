// Matrix-core building blocks shared by the paged attention kernels (gfx950): the bf16 / fp16
// 16x16x32 MFMA, the transposing LDS read, the swizzled [d][64 tokens] K/V tile layout and the
// pair pack and masking.
//
// Operand layouts of v_mfma_f32_16x16x32_bf16 (lane l, g4 = l / 16, n16 = l % 16):
//   A (16 x 32): lane l holds A[n16][8 g4 .. 8 g4 + 7]
//   B (32 x 16): lane l holds B[8 g4 .. 8 g4 + 7][n16]
//   C (16 x 16): lane l holds C[4 g4 + j][n16], j < 4
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "plastic_infer_amd.h"

namespace pia {
namespace tile {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

__device__ __forceinline__ f32x4_t mfma_bf16(const uint4& a, const uint4& b, f32x4_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                 __builtin_bit_cast(bf16x8_t, b), c, 0, 0, 0);
}

// ds_read_b64_tr_b16 at an 8-byte aligned LDS address: within each 16-lane group the eight-byte
// reads of the lanes form a 16 x 4 matrix of b16 elements, and lane i receives elements
// (4 k + i / 4, i % 4), k < 4.
__device__ __forceinline__ uint2 read_tr16(const uint16_t* p) {
  typedef short v4i16 __attribute__((ext_vector_type(4)));
  typedef __attribute__((address_space(3))) v4i16 lds_v4i16;
  const v4i16 v = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4i16*)(const_cast<uint16_t*>(p)));
  return __builtin_bit_cast(uint2, v);
}

// Tiles of 64 tokens (four 16-token pages) in their pool layout [d][token]: a tile row (one d,
// 64 tokens, eight 16-byte chunks) is stored unpadded with chunk c at c ^ ((d / 4) ^ 2 (d % 4))
// % 8. With that swizzle the transposing K reads and the 16-byte row stores of the prefill
// kernel run without LDS bank conflicts (SQ_LDS_BANK_CONFLICT 0 over a whole launch).
constexpr int kTileTokens = 64;

// element offset of (row d, token t) in a swizzled [d][64 tokens] tile
__device__ __forceinline__ int swz64(int d, int t) {
  return d * kTileTokens + ((((t >> 3) ^ (d >> 2) ^ ((d & 3) << 1)) & 7) << 3) + (t & 7);
}

// Swizzle term of row d (the chunk index is XORed with it).
__device__ __forceinline__ int swz64_row_term(int d) { return ((d >> 2) ^ ((d & 3) << 1)) & 7; }

// Two f32 -> one bf16x2 word, round to nearest even (one v_cvt_pk_bf16_f32).
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
  const bf16x2_t p = {static_cast<__bf16>(lo), static_cast<__bf16>(hi)};
  return __builtin_bit_cast(uint32_t, p);
}

// Zero the bf16 tokens of a dword pair (t, t+1) that lie at or beyond nvalid.
__device__ __forceinline__ uint32_t mask_pair(uint32_t x, int t, int nvalid) {
  const uint32_t lo = (t < nvalid) ? 0x0000ffffu : 0u;
  const uint32_t hi = (t + 1 < nvalid) ? 0xffff0000u : 0u;
  return x & (lo | hi);
}

// Max over lanes l, l ^ 16, l ^ 32, l ^ 48 (the four lanes that hold one column of an MFMA
// output) by two lane swaps on the vector ALU, without the LDS crossbar of a shuffle. Called
// with both operands equal, v_permlane16_swap returns (x[l & ~16], x[l | 16]) and
// v_permlane32_swap (x[l & 31], x[l | 32]) (measured on gfx950).
__device__ __forceinline__ float max_col4(float v) {
  const unsigned u = __float_as_uint(v);
  const auto a = __builtin_amdgcn_permlane16_swap(u, u, false, false);
  const float m = fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));
  const unsigned w = __float_as_uint(m);
  const auto b = __builtin_amdgcn_permlane32_swap(w, w, false, false);
  return fmaxf(__uint_as_float(b[0]), __uint_as_float(b[1]));
}

// NaN-propagating max over lanes l, l ^ 16, l ^ 32, l ^ 48, as max_col4 (IEEE 754-2019 maximum:
// a NaN in any of the four gives NaN; on gfx950 v_maximum3_f32, which needs no quieting of its
// inputs).
__device__ __forceinline__ float maximum_col4(float v) {
  const unsigned u = __float_as_uint(v);
  const auto a = __builtin_amdgcn_permlane16_swap(u, u, false, false);
  const float m = __builtin_elementwise_maximum(__uint_as_float(a[0]), __uint_as_float(a[1]));
  const unsigned w = __float_as_uint(m);
  const auto b = __builtin_amdgcn_permlane32_swap(w, w, false, false);
  return __builtin_elementwise_maximum(__uint_as_float(b[0]), __uint_as_float(b[1]));
}

// bf16 1.0 in every element: the B operand of a row sum by the matrix cores.
__device__ __forceinline__ uint4 bf16_ones() {
  return make_uint4(0x3f803f80u, 0x3f803f80u, 0x3f803f80u, 0x3f803f80u);
}

// The same three for either 16-bit storage type, DT = PIA_DTYPE_BF16 or PIA_DTYPE_F16: the
// 16x16x32 MFMA (fp32 accumulate), two f32 -> one pair (round to nearest even) and 1.0 in every
// element.
typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
template <int DT>
__device__ __forceinline__ f32x4_t mfma16(const uint4& a, const uint4& b, f32x4_t c) {
  if constexpr (DT == PIA_DTYPE_F16)
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8_t, a),
                                                  __builtin_bit_cast(f16x8_t, b), c, 0, 0, 0);
  else
    return mfma_bf16(a, b, c);
}
template <int DT>
__device__ __forceinline__ uint32_t pack16x2(float lo, float hi) {
  if constexpr (DT == PIA_DTYPE_F16) {
    typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));
    const f16x2_t p = {static_cast<_Float16>(lo), static_cast<_Float16>(hi)};
    return __builtin_bit_cast(uint32_t, p);
  } else {
    return pack_bf16x2(lo, hi);
  }
}
template <int DT>
__device__ __forceinline__ uint4 ones16() {
  if constexpr (DT == PIA_DTYPE_F16)
    return make_uint4(0x3c003c00u, 0x3c003c00u, 0x3c003c00u, 0x3c003c00u);
  else
    return bf16_ones();
}

}  // namespace tile
}  // namespace pia
