// fa_fwd_kvcache_noalloc: fa_fwd_kvcache for callers that cannot allocate
// device memory (code under HIP graph capture, tight serving loops).
//
// fa_fwd_kvcache takes its split-KV workspace (fp32 partial rows and LSEs of
// every key split, written by the split kernel and read by the combine
// kernel) from the caller.  This variant keeps that workspace in a
// file-scope device array instead, so a call allocates nothing: no hipMalloc,
// no hipFree, no allocating library routine.  Every GPU the library runs on
// holds one copy of the array (kScratchBytes) until the process ends.
//
// The array's name is a host-side stand-in, not a device address: host code
// uses only the per-device address hipGetSymbolAddress returns, fetched once
// per device on the first call with that device current.
//
// The split kernel writes every partial the combine kernel reads (each split
// that holds keys of a sequence, and split 0 of every sequence), so nothing
// in the array needs clearing between calls.  All calls on one GPU share its
// array: calls that overlap on one GPU (concurrent streams, or host threads
// launching at once) race and must be serialized by the caller.
#include <hip/hip_runtime.h>
#include <stdio.h>

#include <mutex>

#include "fa_api_internal.h"
#include "fa_gfx950.h"

constexpr int64_t kScratchBytes = FA_NOALLOC_SCRATCH_BYTES;

static __device__ __align__(256) unsigned char scratch[kScratchBytes];

namespace {

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

// This device's copy of `scratch` (set up on the device's first call).
int scratch_on_current_device(void** out) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return fa_set_error(FA_ERR_HIP, hipGetErrorString(e));
  if (dev < 0 || dev >= kMaxDevices)
    return fa_set_error(FA_ERR_UNSUPPORTED, "fa_fwd_kvcache_noalloc: device index beyond 63");
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    void* ptr = nullptr;
    e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess || ptr == nullptr)
      return fa_set_error(FA_ERR_HIP, "fa_fwd_kvcache_noalloc: hipGetSymbolAddress failed");
    g_scratch_ptr[dev] = ptr;
  }
  *out = g_scratch_ptr[dev];
  return FA_OK;
}

}  // namespace

extern "C" int fa_fwd_kvcache_noalloc(
    const void* q, const void* k_cache, const void* v_cache, void* out, float* lse,
    const int32_t* cache_seqlens, const int32_t* block_table, int64_t block_table_stride,
    int64_t page_size, int64_t cache_blocks, const int32_t* cache_batch_idx,
    const int32_t* cache_leftpad, int64_t batch, int64_t seqlen_q, int64_t max_keys,
    int64_t heads_q, int64_t heads_k, int64_t head_dim, const int64_t* q_stride,
    const int64_t* k_cache_stride, const int64_t* v_cache_stride, const int64_t* o_stride,
    const int64_t* lse_stride, int dtype, float softmax_scale, int causal, int64_t window_left,
    int64_t window_right, const float* alibi_slopes, int64_t alibi_batch_stride,
    fa_stream_t stream) {
  int32_t splits = 0;
  int64_t need = 0;
  int st = fa_fwd_kvcache_plan(batch, seqlen_q, heads_q, heads_k, head_dim, max_keys,
                               block_table ? page_size : 0, &splits, &need);
  if (st != FA_OK) return st;
  // fp32 never splits the keys of a row (no workspace is read), and an empty
  // call launches nothing: neither needs the scratch array.
  if (dtype == FA_DTYPE_F32 || batch == 0 || seqlen_q == 0) need = 0;
  if (need > kScratchBytes) {
    char msg[200];
    snprintf(msg, sizeof(msg),
             "fa_fwd_kvcache_noalloc: the split workspace needs %lld bytes, beyond the %lld-byte "
             "scratch array; use fa_fwd_kvcache with a workspace",
             (long long)need, (long long)kScratchBytes);
    return fa_set_error(FA_ERR_UNSUPPORTED, msg);
  }
  void* ws = nullptr;
  if (need > 0) {
    st = scratch_on_current_device(&ws);
    if (st != FA_OK) return st;
  }
  return fa_kvcache_run("fa_fwd_kvcache_noalloc", q, k_cache, v_cache, out, lse, cache_seqlens,
                        block_table, block_table_stride, page_size, cache_blocks,
                        cache_batch_idx, cache_leftpad, batch, seqlen_q, max_keys, heads_q,
                        heads_k, head_dim, q_stride, k_cache_stride, v_cache_stride, o_stride,
                        lse_stride, dtype, softmax_scale, causal, window_left, window_right,
                        alibi_slopes, alibi_batch_stride, splits, ws, need, stream);
}
