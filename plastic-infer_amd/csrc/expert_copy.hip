// Expert-weight row movement between pinned host banks and HBM slot caches.
//   index_copy_rows_kernel : device-planned row copy (indices on device, optional device count);
//                            reads/writes any device-accessible memory, including pinned host
//                            memory mapped into the GPU address space.
//   pia_copy_rows_async    : host-planned copies issued to the DMA engines with hipMemcpyAsync,
//                            merging runs of consecutive rows into one transfer.
#include "pia_internal.h"

#include <algorithm>

namespace pia {
namespace {

template <typename IdT, typename W>
__global__ __launch_bounds__(256) void index_copy_rows_kernel(
    W* __restrict__ dst, const IdT* __restrict__ di, int64_t dst_rows, const W* __restrict__ src,
    const IdT* __restrict__ si, int64_t src_rows, int64_t length,
    const int64_t* __restrict__ num_indices, int64_t row_words) {
  int64_t n = length;
  if (num_indices) n = min(n, num_indices[0]);
  const int64_t total = n * row_words;
  for (int64_t w = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; w < total;
       w += int64_t(gridDim.x) * blockDim.x) {
    const int64_t r = w / row_words, c = w - r * row_words;
    const int64_t s = int64_t(si[r]), d = int64_t(di[r]);
    if (s < 0 || d < 0 || s >= src_rows || d >= dst_rows) continue;
    dst[d * row_words + c] = src[s * row_words + c];
  }
}

// One grid row (blockIdx.y) per bank; per-bank pointers and row sizes are read from device
// arrays so the launch is independent of host-side pointer values.
template <typename IdT>
__global__ __launch_bounds__(256) void index_copy_rows_multi_kernel(
    const int64_t* __restrict__ dst_ptrs, const int64_t* __restrict__ src_ptrs,
    const int64_t* __restrict__ row_bytes, const IdT* __restrict__ di,
    const IdT* __restrict__ si, int64_t length, const int64_t* __restrict__ num_indices) {
  const int bank = blockIdx.y;
  uint4* dst = reinterpret_cast<uint4*>(dst_ptrs[bank]);
  const uint4* src = reinterpret_cast<const uint4*>(src_ptrs[bank]);
  const int64_t row_words = row_bytes[bank] / 16;
  int64_t n = length;
  if (num_indices) n = min(n, num_indices[0]);
  const int64_t total = n * row_words;
  for (int64_t w = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; w < total;
       w += int64_t(gridDim.x) * blockDim.x) {
    const int64_t r = w / row_words, c = w - r * row_words;
    const int64_t s = int64_t(si[r]), d = int64_t(di[r]);
    if (s < 0 || d < 0) continue;
    dst[d * row_words + c] = src[s * row_words + c];
  }
}

// Device-side address of p: device/managed memory as is, pinned host memory via its mapping.
int resolve_device_ptr(const void* p, void** out, const char* what) {
  hipPointerAttribute_t attr;
  const hipError_t e = hipPointerGetAttributes(&attr, p);
  if (e != hipSuccess) {
    (void)hipGetLastError();  // clear the sticky error of the failed query
    set_error("%s: memory is not known to HIP (pageable host memory cannot be read by a "
              "kernel; pin it first)", what);
    return PIA_EINVAL;
  }
  if (attr.type == hipMemoryTypeHost) {
    void* d = nullptr;
    const hipError_t e2 = hipHostGetDevicePointer(&d, const_cast<void*>(p), 0);
    if (e2 != hipSuccess || d == nullptr) {
      (void)hipGetLastError();
      set_error("%s: pinned host memory has no device mapping", what);
      return PIA_EINVAL;
    }
    *out = d;
    return 0;
  }
  if (attr.type == hipMemoryTypeDevice || attr.type == hipMemoryTypeManaged ||
      attr.type == hipMemoryTypeUnified) {
    *out = const_cast<void*>(p);
    return 0;
  }
  set_error("%s: unsupported memory type %d", what, int(attr.type));
  return PIA_EINVAL;
}

template <typename IdT>
int launch_rows(void* dst, const void* di, int64_t dst_rows, const void* src, const void* si,
                int64_t src_rows, int64_t length, const int64_t* num_indices, int64_t row_bytes,
                hipStream_t s) {
  const bool v16 = row_bytes % 16 == 0 && aligned(dst, 16) && aligned(src, 16);
  const int64_t words = v16 ? row_bytes / 16 : row_bytes;
  const int64_t blocks = std::max<int64_t>(1, std::min<int64_t>(ceil_div(length * words, 256), 2048));
  if (v16)
    hipLaunchKernelGGL((index_copy_rows_kernel<IdT, uint4>), dim3(unsigned(blocks)), dim3(256), 0,
                       s, (uint4*)dst, (const IdT*)di, dst_rows, (const uint4*)src,
                       (const IdT*)si, src_rows, length, num_indices, words);
  else
    hipLaunchKernelGGL((index_copy_rows_kernel<IdT, uint8_t>), dim3(unsigned(blocks)), dim3(256),
                       0, s, (uint8_t*)dst, (const IdT*)di, dst_rows, (const uint8_t*)src,
                       (const IdT*)si, src_rows, length, num_indices, words);
  return check_launch("index_copy_rows");
}

}  // namespace
}  // namespace pia

using namespace pia;

extern "C" int pia_index_copy_rows(void* dst, const void* dst_indices, int64_t dst_num_rows,
                                   const void* src, const void* src_indices, int64_t src_num_rows,
                                   int64_t length, const int64_t* num_indices, int64_t row_bytes,
                                   int index_is_int32, void* stream) {
  if (length < 0 || row_bytes <= 0 || dst_num_rows < 0 || src_num_rows < 0)
    return fail(PIA_EINVAL, "index_copy_rows: invalid size");
  if (length == 0 || dst_num_rows == 0 || src_num_rows == 0) return 0;
  if (!dst || !src || !dst_indices || !src_indices)
    return fail(PIA_EINVAL, "index_copy_rows: null pointer");
  hipStream_t s = as_stream(stream);
  void* dst_d = nullptr;
  void* src_d = nullptr;
  if (int rc = resolve_device_ptr(dst, &dst_d, "index_copy_rows dst")) return rc;
  if (int rc = resolve_device_ptr(src, &src_d, "index_copy_rows src")) return rc;
  dst = dst_d;
  src = src_d;
  return index_is_int32
             ? launch_rows<int32_t>(dst, dst_indices, dst_num_rows, src, src_indices,
                                    src_num_rows, length, num_indices, row_bytes, s)
             : launch_rows<int64_t>(dst, dst_indices, dst_num_rows, src, src_indices,
                                    src_num_rows, length, num_indices, row_bytes, s);
}

extern "C" int pia_device_pointer(const void* ptr, void** device_ptr) {
  if (!ptr || !device_ptr) return fail(PIA_EINVAL, "device_pointer: null pointer");
  return resolve_device_ptr(ptr, device_ptr, "device_pointer");
}

extern "C" int pia_index_copy_rows_multi(const int64_t* dst_ptrs, const int64_t* src_ptrs,
                                         const int64_t* row_bytes, int num_banks,
                                         const void* dst_indices, const void* src_indices,
                                         int64_t length, const int64_t* num_indices,
                                         int index_is_int32, void* stream) {
  if (length < 0 || num_banks < 0) return fail(PIA_EINVAL, "index_copy_rows_multi: invalid size");
  if (length == 0 || num_banks == 0) return 0;
  if (num_banks > 65535) return fail(PIA_EINVAL, "index_copy_rows_multi: too many banks");
  if (!dst_ptrs || !src_ptrs || !row_bytes || !dst_indices || !src_indices)
    return fail(PIA_EINVAL, "index_copy_rows_multi: null pointer");
  hipStream_t s = as_stream(stream);
  // Grid-stride per bank; 64 blocks per bank keep enough rows in flight for host-mapped reads.
  dim3 grid = dim3(64, unsigned(num_banks));
  if (index_is_int32)
    hipLaunchKernelGGL(index_copy_rows_multi_kernel<int32_t>, grid, dim3(256), 0, s, dst_ptrs,
                       src_ptrs, row_bytes, (const int32_t*)dst_indices,
                       (const int32_t*)src_indices, length, num_indices);
  else
    hipLaunchKernelGGL(index_copy_rows_multi_kernel<int64_t>, grid, dim3(256), 0, s, dst_ptrs,
                       src_ptrs, row_bytes, (const int64_t*)dst_indices,
                       (const int64_t*)src_indices, length, num_indices);
  return check_launch("index_copy_rows_multi");
}

extern "C" int pia_copy_rows_async(void* dst, const int64_t* dst_rows, const void* src,
                                   const int64_t* src_rows, int64_t n, int64_t row_bytes,
                                   int64_t* copies_issued, void* stream) {
  if (copies_issued) *copies_issued = 0;
  if (n < 0 || row_bytes <= 0) return fail(PIA_EINVAL, "copy_rows_async: invalid size");
  if (n == 0) return 0;
  if (!dst || !src || !dst_rows || !src_rows) return fail(PIA_EINVAL, "copy_rows_async: null pointer");
  hipStream_t s = as_stream(stream);
  char* d = static_cast<char*>(dst);
  const char* sp = static_cast<const char*>(src);
  int64_t issued = 0;
  int64_t i = 0;
  while (i < n) {
    if (dst_rows[i] < 0 || src_rows[i] < 0) {
      ++i;
      continue;
    }
    int64_t run = 1;
    while (i + run < n && dst_rows[i + run] == dst_rows[i] + run &&
           src_rows[i + run] == src_rows[i] + run)
      ++run;
    const hipError_t e =
        hipMemcpyAsync(d + dst_rows[i] * row_bytes, sp + src_rows[i] * row_bytes,
                       size_t(run * row_bytes), hipMemcpyDefault, s);
    if (int rc = check_hip(e, "copy_rows_async: hipMemcpyAsync")) return rc;
    ++issued;
    i += run;
  }
  if (copies_issued) *copies_issued = issued;
  return 0;
}
