// Parameter block of the KV-cache decode kernels (fa_decode.hip), shared with
// the C ABI (fa_api.hip).  Strides are in elements.
#pragma once

#include <stdint.h>

namespace fa {

struct DecodeParams {
  const void* q; const void* k; const void* v; void* o; float* lse;
  int64_t q_sb, q_ss, q_sh;
  int64_t k_sb, k_ss, k_sh;    // {page or cache row, slot, head}
  int64_t v_sb, v_ss, v_sh;
  int64_t o_sb, o_ss, o_sh;
  int64_t lse_sb, lse_ss, lse_sh;   // {batch, query, head}
  const int* seqlens; const int* block_table; int64_t bt_stride; int page_size;
  const int* cache_rows; const int* leftpad;
  int batch, seqlen_q, heads_q, heads_k, group, max_keys;
  float scale, scale_log2;
  const float* alibi; int64_t alibi_sb;
  int causal, window_left, window_right;
  int split_keys, num_splits;
  float* o_part; float* lse_part;
};

}  // namespace fa
