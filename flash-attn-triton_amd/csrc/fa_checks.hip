// fa_check_ranges: the range checks on device integer arrays that a call
// validates its arguments with (cache lengths, page tables, cache rows, left
// pads), reduced in one launch.
//
// Workgroup i reduces array i (plus an optional elementwise addend, or as the
// differences of adjacent elements) to its minimum and maximum as int64 and
// writes them to minmax[2i], minmax[2i + 1].
// minmax may be pinned host memory, so the host reads the results after an
// event on the stream without a separate device-to-host copy.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "fa_api_internal.h"
#include "fa_gfx950.h"

namespace {

constexpr int kThreads = 256;

struct RangeJob {
  const void* a;   // int32 or int64 elements
  const void* b;   // nullable addend, int32 or int64
  int64_t n;       // values reduced: numel, or numel - 1 for differences
  int a_wide, b_wide, diff;
};

struct RangeJobs {
  RangeJob job[FA_MAX_RANGE_CHECKS];
  int64_t* minmax;
};

__device__ inline int64_t load_int(const void* p, int wide, int64_t i) {
  return wide ? static_cast<const int64_t*>(p)[i]
              : static_cast<int64_t>(static_cast<const int32_t*>(p)[i]);
}

__global__ __launch_bounds__(kThreads) void range_minmax_kernel(RangeJobs jobs) {
  const RangeJob j = jobs.job[blockIdx.x];
  int64_t lo = INT64_MAX, hi = INT64_MIN;
  for (int64_t i = threadIdx.x; i < j.n; i += kThreads) {
    int64_t x = load_int(j.a, j.a_wide, i + (j.diff ? 1 : 0));
    if (j.diff)
      x -= load_int(j.a, j.a_wide, i);
    else if (j.b)
      x += load_int(j.b, j.b_wide, i);
    lo = x < lo ? x : lo;
    hi = x > hi ? x : hi;
  }
  for (int off = 32; off > 0; off >>= 1) {
    const int64_t ol = __shfl_xor(lo, off);
    const int64_t oh = __shfl_xor(hi, off);
    lo = ol < lo ? ol : lo;
    hi = oh > hi ? oh : hi;
  }
  __shared__ int64_t s_lo[kThreads / 64], s_hi[kThreads / 64];
  if ((threadIdx.x & 63) == 0) {
    s_lo[threadIdx.x >> 6] = lo;
    s_hi[threadIdx.x >> 6] = hi;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int w = 1; w < kThreads / 64; ++w) {
      lo = s_lo[w] < lo ? s_lo[w] : lo;
      hi = s_hi[w] > hi ? s_hi[w] : hi;
    }
    jobs.minmax[2 * blockIdx.x] = lo;
    jobs.minmax[2 * blockIdx.x + 1] = hi;
  }
}

}  // namespace

extern "C" int fa_check_ranges(int n, const void* const* a, const int* a_bytes,
                               const void* const* b, const int* b_bytes, const int* diff,
                               const int64_t* numel, int64_t* minmax, fa_stream_t stream) {
  if (n < 1 || n > FA_MAX_RANGE_CHECKS)
    return fa_set_error(FA_ERR_INVALID, "fa_check_ranges: n must be in [1, FA_MAX_RANGE_CHECKS]");
  if (!a || !a_bytes || !numel || !minmax)
    return fa_set_error(FA_ERR_INVALID, "fa_check_ranges: null pointer argument");
  if (reinterpret_cast<uintptr_t>(minmax) % 8 != 0)
    return fa_set_error(FA_ERR_INVALID, "fa_check_ranges: minmax must be 8-byte aligned");
  RangeJobs jobs{};
  for (int i = 0; i < n; ++i) {
    const bool dif = diff && diff[i];
    const bool has_b = !dif && b && b[i];
    if (!a[i] || numel[i] < 0 || (a_bytes[i] != 4 && a_bytes[i] != 8) ||
        (has_b && (!b_bytes || (b_bytes[i] != 4 && b_bytes[i] != 8))))
      return fa_set_error(FA_ERR_INVALID,
                          "fa_check_ranges: each array needs a pointer, a size >= 0 and 4- or "
                          "8-byte elements");
    jobs.job[i] = RangeJob{a[i], has_b ? b[i] : nullptr,
                           dif ? (numel[i] > 0 ? numel[i] - 1 : 0) : numel[i], a_bytes[i] == 8,
                           has_b && b_bytes[i] == 8, dif ? 1 : 0};
  }
  // The results go to device memory or to pinned host memory, through the
  // address the device sees; pageable host memory would fault the kernel.
  hipPointerAttribute_t attr{};
  void* dst = minmax;
  hipError_t e = hipPointerGetAttributes(&attr, minmax);
  if (e == hipSuccess && attr.type == hipMemoryTypeHost)
    e = hipHostGetDevicePointer(&dst, minmax, 0);
  else if (e == hipSuccess && attr.type != hipMemoryTypeDevice)
    e = hipErrorInvalidValue;
  if (e != hipSuccess || dst == nullptr) {
    (void)hipGetLastError();
    return fa_set_error(FA_ERR_INVALID,
                        "fa_check_ranges: minmax must be device memory or pinned host memory");
  }
  jobs.minmax = static_cast<int64_t*>(dst);
  hipLaunchKernelGGL(range_minmax_kernel, dim3(n), dim3(kThreads), 0, (hipStream_t)stream, jobs);
  e = hipGetLastError();
  if (e != hipSuccess) return fa_set_error(FA_ERR_HIP, hipGetErrorString(e));
  fa_set_error(FA_OK, "");
  return FA_OK;
}
