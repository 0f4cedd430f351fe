/* C ABI of libfa_gfx950.so: FlashAttention-2 forward kernels for AMD MI355X (gfx950).
 *
 * Every entry point takes raw device pointers, element strides, sizes and the
 * HIP stream to launch on, and returns an int status (FA_OK on success).  No
 * entry point allocates device memory: outputs and workspaces are provided by
 * the caller.  Launches are asynchronous on `stream`.  On failure
 * fa_last_error_string() describes the error for the calling thread.
 *
 * The reference (luyanaa/flash-attn-triton) is pure Python + Triton; it has no
 * FFI.  Each function below replaces one Triton launch site of the reference's
 * forward path (cited per function); the Python layer of this package
 * (flash_attn_triton/) calls these through ctypes at exactly those sites.
 *
 * Tensor layouts.  `dtype` is FA_DTYPE_F16, FA_DTYPE_BF16 or FA_DTYPE_F32 (the
 * reference accepts fp16 and fp32, flash_attn_interface.py:95-96; fp32 runs in
 * fp32 throughout, on the fp32 matrix core; fa_quant_k_int8 / fa_fwd_int8 take
 * fp16 only).  Strides are in elements and the innermost (head-dim) stride must
 * be 1; rows must be 16-byte aligned.
 */
#ifndef FA_GFX950_H_
#define FA_GFX950_H_

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct ihipStream_t* fa_stream_t; /* == hipStream_t */

#define FA_OK 0
#define FA_ERR_INVALID 1     /* argument rejected before any launch */
#define FA_ERR_UNSUPPORTED 2 /* shape/dtype combination not built */
#define FA_ERR_HIP 3         /* HIP runtime reported an error */

#define FA_DTYPE_F16 0
#define FA_DTYPE_BF16 1
#define FA_DTYPE_F32 2

/* Library version (major*10000 + minor*100 + patch). */
int fa_version(void);

/* Description of the last error raised on the calling thread ("" if none). */
const char* fa_last_error_string(void);

/* Dense (and cross) forward attention on [B, S, H, D] strided tensors.
 *
 * Replaces the `_attn_fwd[grid](...)` launch of
 * flash_attn_triton/triton_kernel/attention_kernel.py:1082 (through
 * `_launch_dense_forward`, :1057-1101, and `attention`, :1201-1259).
 *
 * q [B, Sq, Hq, D], k/v [B, Sk, Hk, D], out [B, Sq, Hq, D]; *_stride[3] =
 * {batch, seq, head} element strides.  Hq % Hk == 0; query head h reads KV
 * head h / (Hq / Hk).  Query row i sits at position i + q_pos_offset; keys are
 * at positions 0..Sk-1 (upper-left alignment when the offset is 0).
 * causal keeps kpos <= qpos; window_left/right >= 0 keep
 * qpos-left <= kpos <= qpos+right (negative = unbounded).  alibi_slopes
 * (nullable, fp32) holds slope[b * alibi_batch_stride + h]; softcap > 0 caps
 * scores with softcap*tanh(s/softcap).  attn_bias (nullable, fp32) is added
 * to the scaled scores after ALiBi and before softcap, as the reference's
 * materialized path does (flash_attn_interface.py:36-42):
 * attn_bias[b*bias_stride[0] + h*bias_stride[1] + i*bias_stride[2] +
 * j*bias_stride[3]] (stride 0 broadcasts).  lse (nullable, fp32) receives the
 * natural-log logsumexp at lse[b*lse_stride[0] + h*lse_stride[1] +
 * i*lse_stride[2]]; rows with no visible key get out = 0 and lse = -inf.
 *
 * dropout_p in [0, 1) drops probabilities before the product with V
 * (attention_kernel.py:344-358): element (b, h, i, j) is kept iff its 16-bit
 * Philox4x32-10 draw under dropout_seed is >= t16 = min(round(p * 65536),
 * 65535), and kept values are scaled by 65536 / (65536 - t16), the
 * reciprocal of the keep probability (1 / (1 - p) to within 2^-17 / (1 - p)
 * below p = 1 - 2^-17), so the mask is unbiased; p < 2^-17 keeps everything.  The LSE is that of the undropped
 * scores.
 * The draw of (b, h, i, j) is half j%4 + 4((j%16)/8) of the Philox call with
 * counter {2(j/16) + (j/4)%2, i, h, b} and key {seed, seed >> 32}; rows and
 * keys are local to the sequence (varlen: b is the sequence index).  The
 * backward and fa_attn_probs reproduce the same mask from the same seed.
 */
int fa_fwd_dense(const void* q, const void* k, const void* v, void* out, float* lse,
                 int64_t batch, int64_t seqlen_q, int64_t seqlen_k, int64_t heads_q,
                 int64_t heads_k, int64_t head_dim, const int64_t* q_stride,
                 const int64_t* k_stride, const int64_t* v_stride, const int64_t* o_stride,
                 const int64_t* lse_stride, int dtype, float softmax_scale, int causal,
                 int64_t q_pos_offset, int64_t window_left, int64_t window_right, float softcap,
                 const float* alibi_slopes, int64_t alibi_batch_stride, const float* attn_bias,
                 const int64_t* bias_stride, float dropout_p, uint64_t dropout_seed,
                 fa_stream_t stream);

/* Packed variable-length forward attention.
 *
 * Replaces the `_varlen_fwd[grid](...)` launch of attention_kernel.py:1298
 * (through `_attention_varlen.forward`, :1283-1320).  q [Tq, Hq, D],
 * k/v [Tk, Hk, D] with *_stride[2] = {token, head}; sequence b owns query
 * rows [cu_seqlens_q[b], cu_seqlens_q[b+1]) and key rows
 * [cu_seqlens_k[b], cu_seqlens_k[b+1]) (device int32 arrays of batch+1
 * entries); positions are local to each sequence.  max_seqlen_q must bound
 * every query length.  lse (nullable) is [Tq, Hq] at
 * lse[t*lse_stride[0] + h*lse_stride[1]].  Other arguments as fa_fwd_dense.
 *
 * seqused_q / seqused_k (nullable, int32 [batch]; flash_attn_interface.py:551-580)
 * limit sequence b to its first seqused_q[b] queries / seqused_k[b] keys
 * (0 <= used <= length, checked by the caller).  cu_seqlens_out (nullable,
 * int32 [batch+1]) places sequence b's output and LSE rows at
 * [cu_seqlens_out[b], ...) instead of cu_seqlens_q[b] (the reference packs the
 * outputs of the used queries).  block_table (nullable; int32
 * [batch, block_table_stride]) makes k/v paged caches [pages, page_size, Hk, D]
 * with *_stride[3] = {page, slot, head}: key j of sequence b is slot
 * j % page_size of page block_table[b][j / page_size], the length of sequence
 * b still being cu_seqlens_k[b+1] - cu_seqlens_k[b] (paged varlen prefill,
 * flash_attn_interface.py:533-550, without the reference's gather).  With a
 * block table, num_pages is the caches' page count and block_table_cols the
 * table's columns: a page index outside [0, num_pages) reads as zeros and a
 * sequence's keys are clamped to block_table_cols * page_size, so no read
 * leaves the caches or the table whatever the table holds (the Python layer
 * rejects such tables first, flash_attn_interface.py:543-546).  cu_seqlens_*
 * must describe rows inside q/k/v (they are not bounds-checked here).
 */
int fa_fwd_varlen(const void* q, const void* k, const void* v, void* out, float* lse,
                  const int32_t* cu_seqlens_q, const int32_t* cu_seqlens_k, int64_t batch,
                  int64_t max_seqlen_q, int64_t max_seqlen_k, int64_t heads_q, int64_t heads_k,
                  int64_t head_dim, const int64_t* q_stride, const int64_t* k_stride,
                  const int64_t* v_stride, const int64_t* o_stride, const int64_t* lse_stride,
                  int dtype, float softmax_scale, int causal, int64_t window_left,
                  int64_t window_right, float softcap, const float* alibi_slopes,
                  int64_t alibi_batch_stride, const int32_t* seqused_q,
                  const int32_t* seqused_k, const int32_t* cu_seqlens_out,
                  const int32_t* block_table, int64_t block_table_stride, int64_t page_size,
                  int64_t num_pages, int64_t block_table_cols, float dropout_p,
                  uint64_t dropout_seed, fa_stream_t stream);

/* Backward of fa_fwd_dense: dq, dk, dv from dout.
 *
 * Replaces `_dense_backward` (attention_kernel.py:1104-1155: the
 * `_attn_bwd_preprocess` and `_attn_bwd` launches, :536-566 and :809-1054).
 * q, k, v, out, dout, dq, dk, dv are [B, S, H, D] with *_stride[3] = {batch,
 * seq, head} (k, v, dk, dv with Hk heads); lse is the natural-log LSE the
 * forward returned ([B, Hq, Sq] at lse_stride {batch, head, seq}); delta is an
 * fp32 workspace of the same shape and strides (written, then read).  The
 * score options (scale, causal, q_pos_offset, window, softcap, ALiBi,
 * attn_bias) must be those of the forward call.  dq / dk / dv are written, not
 * accumulated; grouped KV heads are reduced inside the kernel (no atomics,
 * deterministic).  dtype fp16, bf16 or fp32, head_dim 32, 64, 128 or 256
 * (the reference's Triton backward is dtype-generic,
 * attention_kernel.py:1104-1198).
 *
 * attn_bias / bias_stride[4]: the forward's fp32 bias (may be null).  dbias /
 * dbias_stride[4] (may be null): an fp32 buffer, zero-filled by the caller,
 * that receives d loss / d bias, i.e. dS = P (dP - delta) (times the softcap
 * derivative) at dbias[b*s0 + h*s1 + i*s2 + j*s3]; give broadcast dimensions
 * stride 0 and their gradients are summed (atomically: with a broadcast bias
 * the summation order, and so the last bits, vary between calls).  The
 * reference differentiates its torch path through the bias
 * (flash_attn_interface.py:15-49).  Launches two kernels on `stream`.
 */
int fa_bwd_dense(const void* q, const void* k, const void* v, const void* out, const void* dout,
                 const float* lse, void* dq, void* dk, void* dv, float* delta, int64_t batch,
                 int64_t seqlen_q, int64_t seqlen_k, int64_t heads_q, int64_t heads_k,
                 int64_t head_dim, const int64_t* q_stride, const int64_t* k_stride,
                 const int64_t* v_stride, const int64_t* o_stride, const int64_t* do_stride,
                 const int64_t* dq_stride, const int64_t* dk_stride, const int64_t* dv_stride,
                 const int64_t* lse_stride, int dtype, float softmax_scale, int causal,
                 int64_t q_pos_offset, int64_t window_left, int64_t window_right, float softcap,
                 const float* alibi_slopes, int64_t alibi_batch_stride, const float* attn_bias,
                 const int64_t* bias_stride, float* dbias, const int64_t* dbias_stride,
                 float dropout_p, uint64_t dropout_seed, fa_stream_t stream);

/* Backward of fa_fwd_varlen (without seqused / block table).
 *
 * Replaces `_attention_varlen.backward` (attention_kernel.py:1322-1361: the
 * `_varlen_bwd` and `_varlen_bwd_dkdv` launches, :107-272).  Packed tensors
 * with *_stride[2] = {token, head}; lse / delta [Tq, Hq] at lse_stride
 * {token, head}.  Other arguments as fa_bwd_dense.
 */
int fa_bwd_varlen(const void* q, const void* k, const void* v, const void* out,
                  const void* dout, const float* lse, void* dq, void* dk, void* dv, float* delta,
                  const int32_t* cu_seqlens_q, const int32_t* cu_seqlens_k, int64_t batch,
                  int64_t max_seqlen_q, int64_t max_seqlen_k, int64_t heads_q, int64_t heads_k,
                  int64_t head_dim, const int64_t* q_stride, const int64_t* k_stride,
                  const int64_t* v_stride, const int64_t* o_stride, const int64_t* do_stride,
                  const int64_t* dq_stride, const int64_t* dk_stride, const int64_t* dv_stride,
                  const int64_t* lse_stride, int dtype, float softmax_scale, int causal,
                  int64_t window_left, int64_t window_right, float softcap,
                  const float* alibi_slopes, int64_t alibi_batch_stride, float dropout_p,
                  uint64_t dropout_seed, fa_stream_t stream);

/* Split-KV plan for fa_fwd_kvcache: the number of key splits the launch will
 * use and the workspace bytes it needs (0 when num_splits == 1).
 * max_keys bounds every sequence's visible key count (e.g. the cache
 * capacity); page_size is the paged cache's page size, 0 for a batched cache
 * (it decides whether the bandwidth-bound decode kernel can run: up to 32
 * query rows per KV head, head_dim 64 or 128, page_size % 32 == 0).
 * Host-only, no device work.  No counterpart in the reference, whose
 * KV-cache path loops over the batch in Python.
 */
int fa_fwd_kvcache_plan(int64_t batch, int64_t seqlen_q, int64_t heads_q, int64_t heads_k,
                        int64_t head_dim, int64_t max_keys, int64_t page_size,
                        int32_t* num_splits, int64_t* workspace_bytes);

/* Attention of q against a KV cache, paged or batched (decode and chunked
 * prefill against a cache).
 *
 * Replaces the per-sequence Python loop of
 * flash_attn_triton/flash_attn_interface.py:501-525 (gather + pad +
 * `flash_attn_func_cross` + `_attn_fwd` launch per batch item) with one
 * split-KV launch plus a combine launch.
 *
 * q [B, Sq, Hq, D] (q_stride {batch, seq, head}); out likewise.
 * Paged (block_table != NULL): k_cache/v_cache [cache_blocks, page_size, Hk, D]
 * with cache_stride {page, slot, head}; logical key t of sequence b lives in
 * page block_table[b*block_table_stride + t/page_size], slot t%page_size.
 * Batched (block_table == NULL): caches [cache_blocks, capacity, Hk, D] with
 * cache_stride {row, slot, head}; sequence b reads cache row
 * cache_batch_idx[b] (nullable: b) from slot cache_leftpad[b] (nullable: 0).
 * cache_seqlens[b] (device int32, nullable: max_keys for every b) visible
 * keys.  max_keys is the capacity: the slots of a batched row, and for a
 * paged cache at most the block table's columns times page_size.  Whatever
 * the device arrays hold, no read leaves the caches or the table: lengths
 * are clamped to [0, max_keys - leftpad], leftpad to [0, max_keys], and a
 * page or cache row outside [0, cache_blocks) reads as zeros (a row: no keys).
 * When causal, query i sits at position i + L_b - Sq (bottom-right);
 * otherwise at i.  window/alibi as fa_fwd_dense.  lse (nullable) is
 * [B, Hq, Sq] at lse[b*s0 + h*s1 + i*s2].  num_splits/workspace come from
 * fa_fwd_kvcache_plan (workspace may be NULL when its size is 0).
 */
int fa_fwd_kvcache(const void* q, const void* k_cache, const void* v_cache, void* out,
                   float* lse, const int32_t* cache_seqlens, const int32_t* block_table,
                   int64_t block_table_stride, int64_t page_size, int64_t cache_blocks,
                   const int32_t* cache_batch_idx, const int32_t* cache_leftpad, int64_t batch,
                   int64_t seqlen_q, int64_t max_keys, int64_t heads_q, int64_t heads_k,
                   int64_t head_dim,
                   const int64_t* q_stride, const int64_t* k_cache_stride,
                   const int64_t* v_cache_stride, const int64_t* o_stride,
                   const int64_t* lse_stride, int dtype, float softmax_scale, int causal,
                   int64_t window_left, int64_t window_right, const float* alibi_slopes,
                   int64_t alibi_batch_stride, int32_t num_splits, void* workspace,
                   int64_t workspace_bytes, fa_stream_t stream);

/* fa_fwd_kvcache for callers that cannot allocate device memory (code under
 * HIP graph capture, serving loops, harnesses that forbid hipMalloc).
 *
 * No counterpart in the reference (its KV-cache path is a Python loop).  The
 * arguments are those of fa_fwd_kvcache without num_splits / workspace: the
 * split-KV partials live in a device array inside the library, of
 * FA_NOALLOC_SCRATCH_BYTES per GPU, held from the library's load until the
 * process ends.  A call allocates nothing.  Shapes whose split workspace
 * (fa_fwd_kvcache_plan's workspace_bytes) exceeds that size are rejected with
 * FA_ERR_UNSUPPORTED before any launch.  All calls on one GPU share its
 * array, which keeps the last call's contents: calls that overlap on one GPU
 * (several streams or host threads) race and must be serialized by the
 * caller.  Call with the stream's device current.
 */
#define FA_NOALLOC_SCRATCH_BYTES (16 << 20)
int fa_fwd_kvcache_noalloc(const void* q, const void* k_cache, const void* v_cache, void* out,
                           float* lse, const int32_t* cache_seqlens, const int32_t* block_table,
                           int64_t block_table_stride, int64_t page_size, int64_t cache_blocks,
                           const int32_t* cache_batch_idx, const int32_t* cache_leftpad,
                           int64_t batch, int64_t seqlen_q, int64_t max_keys, int64_t heads_q,
                           int64_t heads_k, int64_t head_dim, const int64_t* q_stride,
                           const int64_t* k_cache_stride, const int64_t* v_cache_stride,
                           const int64_t* o_stride, const int64_t* lse_stride, int dtype,
                           float softmax_scale, int causal, int64_t window_left,
                           int64_t window_right, const float* alibi_slopes,
                           int64_t alibi_batch_stride, fa_stream_t stream);

/* Materialized attention probabilities (return_attn_probs=True).
 *
 * Replaces the dense torch math of `_attention_with_probs`
 * (flash_attn_interface.py:15-49, called at :139-148, :289-298 and, per
 * sequence, :642-659).  Given the natural-log LSE the forward kernels return,
 * writes probs[b][h][i][j] = exp(score - lse) as fp32
 * [batch, heads_q, max_seqlen_q, max_seqlen_k] contiguous, zero for masked
 * keys, padding and rows whose LSE is -inf.  Dense (cu_seqlens_* NULL): q
 * [B, Sq, Hq, D] and k [B, Sk, Hk, D] with {batch, seq, head} strides, lse at
 * {batch, query, head} strides, queries at position i + q_pos_offset.
 * Varlen: q [Tq, Hq, D], k [Tk, Hk, D] ({unused, token, head} strides), lse
 * [Tq, Hq] ({unused, token, head}), positions local to each sequence.
 * lse_out (nullable) receives the LSE as [batch, heads_q, max_seqlen_q] with
 * -inf padding (the varlen return layout, :644).  Score epilogue and masks as
 * fa_fwd_dense.
 */
int fa_attn_probs(const void* q, const void* k, const float* lse, float* probs, float* lse_out,
                  const int32_t* cu_seqlens_q, const int32_t* cu_seqlens_k, int64_t batch,
                  int64_t max_seqlen_q, int64_t max_seqlen_k, int64_t heads_q, int64_t heads_k,
                  int64_t head_dim, const int64_t* q_stride, const int64_t* k_stride,
                  const int64_t* lse_stride, int dtype, float softmax_scale, int causal,
                  int64_t q_pos_offset, int64_t window_left, int64_t window_right, float softcap,
                  const float* alibi_slopes, int64_t alibi_batch_stride, const float* attn_bias,
                  const int64_t* bias_stride, float dropout_p,
                  uint64_t dropout_seed, fa_stream_t stream);

/* KV-cache append, the cache write of flash_attn_with_kvcache(k=, v=, ...)
 * (replaces the reference's append at flash_attn_interface.py:468-493, which
 * writes into an advanced-indexing copy and is lost; here the cache is
 * written in place, as upstream FlashAttention-2 does).  Token t of batch b
 * (k_new/v_new [batch, n_new, heads_k, head_dim]) goes to logical position
 * pos = cache_seqlens[b] + cache_leftpad[b] + t (cache_seqlens / cache_leftpad
 * nullable = 0): slot pos % page_size of page block_table[b*block_table_stride
 * + pos/page_size] (paged, num_pages pages), else position pos of cache row
 * cache_batch_idx[b] (nullable = b; cache_rows rows of capacity positions).
 * With rotary_cos/rotary_sin (fp32 [rotary_rows, rotary_dim/2], row-major,
 * already rounded to the element type) k is rotated at position pos before the
 * write (flash_attn_interface.py:52-66: interleaved pairs (2j, 2j+1) or
 * half-split pairs (j, j + rotary_dim/2); dims past rotary_dim are copied).
 * Positions outside [0, capacity), pages outside [0, num_pages) and rows
 * outside the tables are skipped (the caller validates them first). */
int fa_kvcache_append(const void* k_new, const void* v_new, void* k_cache, void* v_cache,
                      const int32_t* cache_seqlens, const int32_t* block_table,
                      int64_t block_table_stride, int64_t page_size, int64_t num_pages,
                      const int32_t* cache_batch_idx, int64_t cache_rows,
                      const int32_t* cache_leftpad, int64_t capacity, const float* rotary_cos,
                      const float* rotary_sin, int64_t rotary_dim, int64_t rotary_rows,
                      int rotary_interleaved, int64_t batch, int64_t n_new, int64_t heads_k,
                      int64_t head_dim, const int64_t* k_new_stride, const int64_t* v_new_stride,
                      const int64_t* k_cache_stride, const int64_t* v_cache_stride, int dtype,
                      fa_stream_t stream);

/* Rotary embedding of the queries of flash_attn_with_kvcache(rotary_cos=...)
 * (replaces flash_attn_interface.py:515-518): out[b][i][h] = q[b][i][h] rotated
 * at position cache_seqlens[b] - seqlen_q + cache_leftpad[b] + i, where
 * cache_seqlens holds the lengths after any append; a negative position
 * counts from the end of the tables (torch indexing in the reference); tables
 * and pairing as in fa_kvcache_append.  q and out are
 * [batch, seqlen_q, heads, head_dim]. */
int fa_rotary_q(const void* q, void* out, const int32_t* cache_seqlens,
                const int32_t* cache_leftpad, const float* rotary_cos, const float* rotary_sin,
                int64_t rotary_dim, int64_t rotary_rows, int rotary_interleaved, int64_t batch,
                int64_t seqlen_q, int64_t heads, int64_t head_dim, const int64_t* q_stride,
                const int64_t* out_stride, int dtype, fa_stream_t stream);

/* Range checks of integer device arrays in one launch: the validation of the
 * KV-cache call's device arguments (replaces the `torch.any(...)` / `.item()`
 * chain of flash_attn_interface.py:428-453 that checks the block table,
 * cache_seqlens, cache_batch_idx and cache_leftpad, one host synchronization
 * each).  For i < n (1 <= n <= FA_MAX_RANGE_CHECKS): array a[i] holds numel[i]
 * integers of a_bytes[i] (4 or 8) bytes; b[i] (b or b[i] may be NULL) an
 * addend of the same length and b_bytes[i] bytes; minmax[2i] and minmax[2i+1]
 * receive min and max of a[i][j] + b[i][j] over j as int64 (INT64_MAX and
 * INT64_MIN for an empty array).  diff (nullable) selects, where diff[i] is
 * nonzero, the differences of adjacent elements a[i][j+1] - a[i][j],
 * j < numel[i] - 1, instead (b[i] ignored): the monotonicity check of
 * cu_seqlens (flash_attn_interface.py:583-598).  minmax is device memory or pinned host
 * memory (checked with hipPointerGetAttributes; anything else is rejected),
 * so a host that passes pinned memory reads the results after an event on the
 * stream, with no copy.  a/b are device arrays.  One workgroup per array. */
#define FA_MAX_RANGE_CHECKS 8
int fa_check_ranges(int n, const void* const* a, const int* a_bytes, const void* const* b,
                    const int* b_bytes, const int* diff, const int64_t* numel, int64_t* minmax,
                    fa_stream_t stream);

/* Per-token INT8 quantization of K (fp16), bit-exact with
 * `_quantize_k_rows` (attention_kernel_int8.py:58-79, launched at :232):
 *   s = fp32(max(amax_row, 1)) / 127;  k8 = round_half_away(fp32(k) * (1/s)).
 * k [B, H, S, D] fp16 with k_stride {batch, head, seq}; k8 [B*H, S, D] int8
 * contiguous; s_k [B*H, S] fp32.  D in {32, 64, 128, 256}.
 */
int fa_quant_k_int8(const void* k, int8_t* k8, float* s_k, int64_t batch, int64_t heads,
                    int64_t seqlen, int64_t head_dim, const int64_t* k_stride,
                    fa_stream_t stream);

/* INT8-QK^T attention forward (`_attn_fwd_int8`, attention_kernel_int8.py:167-217,
 * launched at :237).  q/v/out [B, H, S, D] fp16 with strides
 * {batch, head, seq}; k8/s_k from fa_quant_k_int8.  Q is quantized per row in
 * the kernel (division form); QK^T runs on int8 MFMA with i32 accumulation,
 * PV on fp16 MFMA.  Keys >= seq_len_k are masked; for causal, query i sits at
 * position i + seq_len_k - seq_len_q.  lse (nullable) receives the natural-log
 * logsumexp [B, H, S] contiguous.
 */
int fa_fwd_int8(const void* q, const int8_t* k8, const float* s_k, const void* v, void* out,
                float* lse, int64_t batch, int64_t heads, int64_t seqlen, int64_t head_dim,
                const int64_t* q_stride, const int64_t* v_stride, const int64_t* o_stride,
                float sm_scale, int causal, int64_t seq_len_k, int64_t seq_len_q,
                fa_stream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* FA_GFX950_H_ */
