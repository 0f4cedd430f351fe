// Functions shared between the C ABI's source files (not exported).
#pragma once

#include <stdint.h>

#include "fa_gfx950.h"

// Argument checks plus the split and combine launches of fa_fwd_kvcache,
// with the split partials in `workspace` (checked against the plan); `name`
// prefixes every error message.  Defined in fa_api.hip.
int fa_kvcache_run(const char* name, const void* q, const void* k_cache, const void* v_cache,
                   void* out, float* lse, const int32_t* cache_seqlens,
                   const int32_t* block_table, int64_t block_table_stride, int64_t page_size,
                   int64_t cache_blocks, const int32_t* cache_batch_idx,
                   const int32_t* cache_leftpad, int64_t batch, int64_t seqlen_q,
                   int64_t max_keys, int64_t heads_q, int64_t heads_k, int64_t head_dim,
                   const int64_t* q_stride, const int64_t* k_cache_stride,
                   const int64_t* v_cache_stride, const int64_t* o_stride,
                   const int64_t* lse_stride, int dtype, float softmax_scale, int causal,
                   int64_t window_left, int64_t window_right, const float* alibi_slopes,
                   int64_t alibi_batch_stride, int32_t num_splits, void* workspace,
                   int64_t workspace_bytes, fa_stream_t stream);

// Records `msg` as the calling thread's last error and returns `code`.
int fa_set_error(int code, const char* msg);
