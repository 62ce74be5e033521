// Internal helpers shared by the HIP translation units of libplastic_infer_amd.so (gfx950 only).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdarg.h>
#include <stdio.h>

#include "plastic_infer_amd.h"

namespace pia {

// Thread-local last-error text behind pia_last_error().
void set_error(const char* fmt, ...) __attribute__((format(printf, 1, 2)));

inline int fail(int code, const char* what) {
  set_error("%s", what);
  return code;
}

// Checks a HIP launch / runtime call; records the text and returns the hipError_t as int.
inline int check_hip(hipError_t e, const char* where) {
  if (e == hipSuccess) return 0;
  set_error("%s: %s", where, hipGetErrorString(e));
  return (int)e;
}

// Compute units of the current device (cached per device; 256 if the query fails).
int device_cus();

inline int check_launch(const char* where) { return check_hip(hipGetLastError(), where); }

inline hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

inline bool aligned(const void* p, uintptr_t a) { return (reinterpret_cast<uintptr_t>(p) % a) == 0; }

inline int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }

// Multi-row paged attention on the matrix cores (paged_prefill.hip): whether a call takes it,
// and its launch (arguments already checked by pia_paged_attention).
bool prefill_mfma_path(int dtype, int Hq, int Hkv, int D, int P, int num_seqs,
                       int64_t total_q_rows, const int32_t* cu_q, float scale);
int launch_prefill_mfma(int dtype, void* out, const void* q, const void* k_pages,
                        const void* v_pages,
                        const int32_t* bt, int64_t bt_stride, const int32_t* kv_lens,
                        const int32_t* cu_q, const int32_t* offsets, int num_seqs,
                        int64_t total_q_rows, int Hq, int Hkv, int64_t num_pages,
                        float scale_log2, hipStream_t s);

// ---------------------------------------------------------------------------------------------
// Device helpers
// ---------------------------------------------------------------------------------------------

// bf16 <-> f32 by bit manipulation (bf16 is the upper half of an IEEE binary32).
__device__ __forceinline__ float bf16_lo(uint32_t x) { return __uint_as_float(x << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t x) { return __uint_as_float(x & 0xffff0000u); }
__device__ __forceinline__ float bf16_to_f32(uint16_t x) { return __uint_as_float(uint32_t(x) << 16); }

// Round-to-nearest-even f32 -> bf16 (NaN kept quiet), same rounding as torch's .to(bfloat16).
__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return uint16_t((u >> 16) | 0x40u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return uint16_t(u >> 16);
}

__device__ __forceinline__ float half_to_f32(uint16_t x) {
  return float(__builtin_bit_cast(_Float16, x));
}
__device__ __forceinline__ uint16_t f32_to_half(float f) {
  return __builtin_bit_cast(uint16_t, _Float16(f));  // round to nearest even
}

// Element load/store as f32 for the three storage types (dtype codes of the public header).
template <int DT> struct Elem;
template <> struct Elem<PIA_DTYPE_F32> {
  using T = float;
  __device__ __forceinline__ static float load(const T* p, int64_t i) { return p[i]; }
  __device__ __forceinline__ static void store(T* p, int64_t i, float v) { p[i] = v; }
};
template <> struct Elem<PIA_DTYPE_BF16> {
  using T = uint16_t;
  __device__ __forceinline__ static float load(const T* p, int64_t i) { return bf16_to_f32(p[i]); }
  __device__ __forceinline__ static void store(T* p, int64_t i, float v) { p[i] = f32_to_bf16(v); }
};
template <> struct Elem<PIA_DTYPE_F16> {
  using T = uint16_t;
  __device__ __forceinline__ static float load(const T* p, int64_t i) { return half_to_f32(p[i]); }
  __device__ __forceinline__ static void store(T* p, int64_t i, float v) { p[i] = f32_to_half(v); }
};

// Wave64 reductions through ds_swizzle/bpermute-backed shuffles.
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  return v;
}

}  // namespace pia
