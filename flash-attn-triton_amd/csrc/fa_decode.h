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
  // Leading extent of the caches: pages of a paged cache, rows of a batched
  // one.  Out-of-range pages and rows read as zeros (decode_keys).
  int cache_blocks;
  int batch, seqlen_q, heads_q, heads_k, group, max_keys;
  float scale, scale_log2;
  const float* alibi; int64_t alibi_sb;
  int causal, window_left, window_right;
  int split_keys, num_splits;
  float* o_part; float* lse_part;
};

// Visible keys of sequence b, clamped so that no read leaves the caches or the
// block table whatever the device arrays hold: cache_seqlens[b] (max_keys
// without it) within [0, max_keys - leftpad], leftpad within [0, max_keys],
// and zero keys for a batched-cache row outside [0, cache_blocks).  For a
// paged cache max_keys is at most the block table's columns times page_size,
// so every table read stays in row b.  The split and combine kernels use the
// same count.
__device__ inline int decode_keys(const DecodeParams& p, int b, int* row, int* pad) {
  int L = p.seqlens != nullptr ? p.seqlens[b] : p.max_keys;
  int lp = 0, r = b;
  if (p.block_table == nullptr) {
    r = p.cache_rows != nullptr ? p.cache_rows[b] : b;
    lp = p.leftpad != nullptr ? p.leftpad[b] : 0;
    lp = lp < 0 ? 0 : (lp > p.max_keys ? p.max_keys : lp);
    if (r < 0 || r >= p.cache_blocks) L = 0;
  }
  const int cap = p.max_keys - lp;
  L = L < 0 ? 0 : (L > cap ? cap : L);
  if (row != nullptr) *row = r;
  if (pad != nullptr) *pad = lp;
  return L;
}

}  // namespace fa
