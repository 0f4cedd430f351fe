// Parameter blocks of the KV-cache append and rotary kernels (fa_kvappend.hip),
// shared with the C ABI (fa_api.hip).  Strides are in elements.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace fa {

struct AppendParams {
  const void* k_new; const void* v_new; void* k_cache; void* v_cache;
  int64_t kn_sb, kn_ss, kn_sh, vn_sb, vn_ss, vn_sh;
  int64_t kc_sb, kc_ss, kc_sh, vc_sb, vc_ss, vc_sh;
  const int* seqlens; const int* block_table; int64_t bt_stride; int page_size; int num_pages;
  const int* cache_rows; int cache_rows_n; const int* leftpad; int64_t capacity;
  const float* cos; const float* sin; int rot; int interleaved; int64_t table_rows;
  int batch, n_new, heads_k, head_dim;
};

struct RotaryQParams {
  const void* q; void* out;
  int64_t q_sb, q_ss, q_sh, o_sb, o_ss, o_sh;
  const int* seqlens; const int* leftpad;
  const float* cos; const float* sin; int rot; int interleaved; int64_t table_rows;
  int batch, seqlen_q, heads, head_dim;
};

}  // namespace fa

hipError_t fa_launch_kv_append(int dtype, const fa::AppendParams& p, hipStream_t st);
hipError_t fa_launch_rotary_q(int dtype, const fa::RotaryQParams& p, hipStream_t st);
