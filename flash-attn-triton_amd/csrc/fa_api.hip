// C ABI of libfa_gfx950.so (declarations and contracts: include/fa_gfx950.h).
//
// Each entry point validates its arguments, fills a kernel parameter block
// and launches on the caller's stream.  Nothing here allocates device memory
// or synchronizes.
#include <math.h>
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include <string>

#include "fa_gfx950.h"
#include "fa_api_internal.h"
#include "fa_decode.h"
#include "fa_probs.h"
#include "fa_kvappend.h"
#include "fa_fwd_launch.h"
#include "fa_bwd.h"

namespace {

thread_local std::string g_last_error;

int fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
int fail(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_last_error = buf;
  return code;
}

int hip_status(hipError_t e, const char* what) {
  if (e == hipSuccess) {
    g_last_error.clear();
    return FA_OK;
  }
  return fail(FA_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
}

// Positions are 32-bit inside the kernels: lengths and the query position
// offset stay within 2^29 and windows are clamped to 2^30 - 1, which is
// unbounded at those lengths, so qpos +- window never overflows.
constexpr int64_t kMaxLen = int64_t(1) << 29;
int clamp_window(int64_t w) {
  const int64_t cap = (int64_t(1) << 30) - 1;
  return w < 0 ? -1 : (int)(w > cap ? cap : w);
}

bool supported_head_dim(int64_t d) { return d == 16 || d == 32 || d == 64 || d == 128 || d == 256; }

// 16-byte vector loads need 16-byte aligned rows: base pointer aligned and
// every stride a multiple of 16 bytes (8 two-byte or 4 four-byte elements).
bool aligned16(const void* ptr, const int64_t* strides, int n, int64_t elem = 2) {
  if (reinterpret_cast<uintptr_t>(ptr) % 16 != 0) return false;
  for (int i = 0; i < n; ++i)
    if ((strides[i] * elem) % 16 != 0) return false;
  return true;
}

hipError_t launch_fwd(int dtype, const fa::FwdParams& p, int mode, int head_dim, bool generic,
                      hipStream_t st) {
  if (dtype == FA_DTYPE_F32) return fa_launch_fwd_f32(p, mode, head_dim, generic, st);
  return dtype == FA_DTYPE_F16 ? fa_launch_fwd_f16(p, mode, head_dim, generic, st)
                               : fa_launch_fwd_bf16(p, mode, head_dim, generic, st);
}

bool supported_dtype(int dtype) {
  return dtype == FA_DTYPE_F16 || dtype == FA_DTYPE_BF16 || dtype == FA_DTYPE_F32;
}

int64_t elem_bytes(int dtype) { return dtype == FA_DTYPE_F32 ? 4 : 2; }

void fill_scale(fa::FwdParams& p, float scale, float softcap, const float* alibi) {
  p.scale = scale;
  p.scale_log2 = scale * fa::kLog2e;
  p.softcap = softcap;
  p.softcap_k = softcap > 0.f ? 2.f * fa::kLog2e / softcap : 0.f;
  p.alibi = alibi;
}

bool needs_generic(const fa::FwdParams& p) {
  return p.alibi != nullptr || p.softcap > 0.f || !(p.scale > 0.f) || p.drop.enabled;
}

// Dropout of probability p with a 64-bit seed (the mask is defined in
// fa_common.h); p = 0 disables it.  An element is kept with probability
// (65536 - t16) / 65536, so kept values are scaled by the reciprocal of that,
// which makes the mask unbiased for the 16-bit threshold (1 / (1 - p) up to
// 2^-17 / (1 - p)).  Every p in [0, 1) is accepted, as the reference does
// (flash_attn_interface.py:99): a p within 2^-17 of 1 would round to
// t16 = 65536 and keep nothing, so t16 stops at 65535 (one element in 65536
// kept, scaled by 65536).  p outside [0, 1) is rejected.
bool fill_dropout(fa::DropoutCfg& d, float p, uint64_t seed) {
  if (!(p >= 0.f && p < 1.f)) return false;
  d.t16 = (int)nearbyint((double)p * 65536.0);
  if (d.t16 > 65535) d.t16 = 65535;
  d.enabled = d.t16 > 0;
  d.seed_lo = (uint32_t)(seed & 0xffffffffu);
  d.seed_hi = (uint32_t)(seed >> 32);
  d.scale = (float)(65536.0 / (65536.0 - (double)d.t16));
  return true;
}

struct KvPlan {
  bool decode;                       // decode_kernel (fa_decode.hip) instead of fwd_kernel
  int num_splits, split_tiles, split_keys;
  int64_t o_part_bytes, lse_part_bytes;
};

KvPlan kvcache_plan(int64_t batch, int64_t seqlen_q, int64_t heads_q, int64_t heads_k,
                    int64_t head_dim, int64_t max_keys, int64_t page_size) {
  const int64_t group = heads_q / heads_k;
  const int64_t rows = seqlen_q * group;
  KvPlan plan{};
  int64_t splits;
  if (fa_decode_eligible(rows, head_dim, page_size)) {
    plan.decode = true;
    plan.split_keys = fa_decode_split_keys(batch, heads_k, max_keys);
    splits = max_keys > 0 ? (max_keys + plan.split_keys - 1) / plan.split_keys : 1;
    plan.split_tiles = 0;
  } else {
    const int tile = fa::kvcache_tile_keys((int)rows, (int)head_dim);
    const int64_t bm = (rows <= 32 && head_dim <= 128) ? 32 : 128;
    const int64_t max_tiles = max_keys > 0 ? (max_keys + tile - 1) / tile : 1;
    const int64_t base = batch * heads_k * ((rows + bm - 1) / bm);
    // Enough workgroups to cover 256 CUs several times over; at least four key
    // tiles per split so the merge stays a small fraction of the traffic.
    const int64_t target = bm == 32 ? 8192 : 1024;
    splits = base > 0 ? (target + base - 1) / base : 1;
    const int64_t cap = max_tiles / 4 > 1 ? max_tiles / 4 : 1;
    if (splits > cap) splits = cap;
    if (splits > 256) splits = 256;
    if (splits < 1) splits = 1;
    int64_t split_tiles = (max_tiles + splits - 1) / splits;
    splits = (max_tiles + split_tiles - 1) / split_tiles;
    plan.split_tiles = (int)split_tiles;
  }
  if (splits < 1) splits = 1;
  plan.num_splits = (int)splits;
  const int64_t prow = splits * batch * seqlen_q * heads_q;
  plan.o_part_bytes = splits > 1 ? ((prow * head_dim * 4 + 255) / 256) * 256 : 0;
  plan.lse_part_bytes = splits > 1 ? prow * 4 : 0;
  return plan;
}

}  // namespace

hipError_t fa_launch_combine(int dtype, const float* o_part, const float* lse_part, void* out,
                             float* lse, int num_splits, int batch, int seqlen_q, int heads,
                             int head_dim, const int64_t* o_stride, const int64_t* lse_stride,
                             hipStream_t st) {
  const int64_t threads = (int64_t)batch * seqlen_q * heads * (head_dim / 4);
  const int64_t blocks = (threads + 255) / 256;
  if (blocks <= 0) return hipSuccess;
  const int64_t l0 = lse_stride ? lse_stride[0] : 0, l1 = lse_stride ? lse_stride[2] : 0,
                l2 = lse_stride ? lse_stride[1] : 0;
  if (dtype == FA_DTYPE_F16)
    hipLaunchKernelGGL(fa::combine_kernel<fa::F16>, dim3((unsigned)blocks), dim3(256), 0, st,
                       o_part, lse_part, out, lse, num_splits, batch, seqlen_q, heads, head_dim,
                       o_stride[0], o_stride[1], o_stride[2], l0, l1, l2);
  else
    hipLaunchKernelGGL(fa::combine_kernel<fa::BF16>, dim3((unsigned)blocks), dim3(256), 0, st,
                       o_part, lse_part, out, lse, num_splits, batch, seqlen_q, heads, head_dim,
                       o_stride[0], o_stride[1], o_stride[2], l0, l1, l2);
  return hipGetLastError();
}

namespace {

// Shared part of fa_bwd_dense / fa_bwd_varlen: checks, scale fields, launch.
int bwd_launch(const char* name, fa::BwdParams& p, int dtype, int64_t head_dim,
               float softmax_scale, float softcap, const float* alibi_slopes,
               int64_t alibi_batch_stride, int causal, int64_t window_left, int64_t window_right,
               float dropout_p, uint64_t dropout_seed, hipStream_t st) {
  if (!fill_dropout(p.drop, dropout_p, dropout_seed))
    return fail(FA_ERR_INVALID, "%s: dropout_p must be in [0, 1 - 2^-17]", name);
  p.scale = softmax_scale;
  p.scale_log2 = softmax_scale * fa::kLog2e;
  p.softcap = softcap;
  p.softcap_k = softcap > 0.f ? 2.f * fa::kLog2e / softcap : 0.f;
  p.alibi = alibi_slopes;
  p.alibi_sb = alibi_batch_stride;
  p.causal = causal != 0;
  p.window_left = clamp_window(window_left);
  p.window_right = clamp_window(window_right);
  const bool generic = alibi_slopes != nullptr || softcap > 0.f || p.drop.enabled ||
                       p.bias != nullptr || p.dbias != nullptr;
  const hipError_t e = dtype == FA_DTYPE_F16   ? fa_launch_bwd_f16(p, (int)head_dim, generic, st)
                       : dtype == FA_DTYPE_BF16 ? fa_launch_bwd_bf16(p, (int)head_dim, generic, st)
                                                : fa_launch_bwd_f32(p, (int)head_dim, generic, st);
  return hip_status(e, name);
}

int bwd_check_common(const char* name, const void* q, const void* k, const void* v,
                     const void* out, const void* dout, const float* lse, const void* dq,
                     const void* dk, const void* dv, const float* delta, int dtype,
                     int64_t head_dim, int64_t heads_q, int64_t heads_k) {
  if (!q || !k || !v || !out || !dout || !lse || !dq || !dk || !dv || !delta)
    return fail(FA_ERR_INVALID, "%s: null pointer argument", name);
  if (dtype != FA_DTYPE_F16 && dtype != FA_DTYPE_BF16 && dtype != FA_DTYPE_F32)
    return fail(FA_ERR_UNSUPPORTED, "%s: dtype %d not supported (fp16 / bf16 / fp32)", name, dtype);
  if (head_dim != 32 && head_dim != 64 && head_dim != 128 && head_dim != 256)
    return fail(FA_ERR_UNSUPPORTED, "%s: head_dim %lld not in {32,64,128,256}", name,
                (long long)head_dim);
  if (heads_q <= 0 || heads_k <= 0 || heads_q % heads_k != 0)
    return fail(FA_ERR_INVALID, "%s: bad head counts Hq=%lld Hk=%lld", name, (long long)heads_q,
                (long long)heads_k);
  return FA_OK;
}

}  // namespace

int fa_set_error(int code, const char* msg) { return fail(code, "%s", msg); }

extern "C" {

int fa_version(void) { return 100; }

const char* fa_last_error_string(void) { return g_last_error.c_str(); }

int fa_fwd_dense(const void* q, const void* k, const void* v, void* out, float* lse,
                 int64_t batch, int64_t seqlen_q, int64_t seqlen_k, int64_t heads_q,
                 int64_t heads_k, int64_t head_dim, const int64_t* q_stride,
                 const int64_t* k_stride, const int64_t* v_stride, const int64_t* o_stride,
                 const int64_t* lse_stride, int dtype, float softmax_scale, int causal,
                 int64_t q_pos_offset, int64_t window_left, int64_t window_right, float softcap,
                 const float* alibi_slopes, int64_t alibi_batch_stride, const float* attn_bias,
                 const int64_t* bias_stride, float dropout_p, uint64_t dropout_seed,
                 fa_stream_t stream) {
  if (!q || !k || !v || !out || !q_stride || !k_stride || !v_stride || !o_stride)
    return fail(FA_ERR_INVALID, "fa_fwd_dense: null pointer argument");
  if (attn_bias && !bias_stride)
    return fail(FA_ERR_INVALID, "fa_fwd_dense: attn_bias without bias_stride");
  if (lse && !lse_stride) return fail(FA_ERR_INVALID, "fa_fwd_dense: lse without lse_stride");
  if (!supported_dtype(dtype))
    return fail(FA_ERR_UNSUPPORTED, "fa_fwd_dense: dtype %d not supported", dtype);
  if (!supported_head_dim(head_dim))
    return fail(FA_ERR_UNSUPPORTED, "fa_fwd_dense: head_dim %lld not in {16,32,64,128,256}",
                (long long)head_dim);
  if (batch < 0 || seqlen_q < 0 || seqlen_k < 0 || heads_q <= 0 || heads_k <= 0 ||
      heads_q % heads_k != 0)
    return fail(FA_ERR_INVALID, "fa_fwd_dense: bad sizes B=%lld Sq=%lld Sk=%lld Hq=%lld Hk=%lld",
                (long long)batch, (long long)seqlen_q, (long long)seqlen_k, (long long)heads_q,
                (long long)heads_k);
  if (seqlen_q > kMaxLen || seqlen_k > kMaxLen || q_pos_offset > kMaxLen ||
      q_pos_offset < -kMaxLen || batch * heads_q > INT32_MAX)
    return fail(FA_ERR_UNSUPPORTED, "fa_fwd_dense: sizes or position offset exceed 2^29");
  const int64_t eb = elem_bytes(dtype);
  if (!aligned16(q, q_stride, 3, eb) || !aligned16(k, k_stride, 3, eb) ||
      !aligned16(v, v_stride, 3, eb) || !aligned16(out, o_stride, 3, eb))
    return fail(FA_ERR_UNSUPPORTED, "fa_fwd_dense: tensors must be 16-byte aligned with strides "
                                    "that are multiples of 16 bytes");
  if (batch == 0 || seqlen_q == 0) return hip_status(hipSuccess, "");
  fa::FwdParams p{};
  p.q = q; p.k = k; p.v = v; p.o = out; p.lse = lse;
  p.q_sb = q_stride[0]; p.q_ss = q_stride[1]; p.q_sh = q_stride[2];
  p.k_sb = k_stride[0]; p.k_ss = k_stride[1]; p.k_sh = k_stride[2];
  p.v_sb = v_stride[0]; p.v_ss = v_stride[1]; p.v_sh = v_stride[2];
  p.o_sb = o_stride[0]; p.o_ss = o_stride[1]; p.o_sh = o_stride[2];
  if (lse) { p.lse_sb = lse_stride[0]; p.lse_sh = lse_stride[1]; p.lse_ss = lse_stride[2]; }
  p.batch = (int)batch; p.seqlen_q = (int)seqlen_q; p.seqlen_k = (int)seqlen_k;
  p.heads_q = (int)heads_q; p.heads_k = (int)heads_k; p.group = (int)(heads_q / heads_k);
  fill_scale(p, softmax_scale, softcap, alibi_slopes);
  p.alibi_sb = alibi_batch_stride;
  p.causal = causal != 0;
  p.window_left = clamp_window(window_left);
  p.window_right = clamp_window(window_right);
  p.q_offset = q_pos_offset;
  if (attn_bias) {
    p.bias = attn_bias;
    p.bias_sb = bias_stride[0]; p.bias_sh = bias_stride[1];
    p.bias_sq = bias_stride[2]; p.bias_sk = bias_stride[3];
  }
  if (!fill_dropout(p.drop, dropout_p, dropout_seed))
    return fail(FA_ERR_INVALID, "fa_fwd_dense: dropout_p must be in [0, 1 - 2^-17]");
  p.num_splits = 1;
  p.heavy_first = p.causal || p.window_right >= 0;
  return hip_status(launch_fwd(dtype, p, fa::kModePrefill, (int)head_dim,
                               needs_generic(p) || attn_bias != nullptr, (hipStream_t)stream),
                    "fa_fwd_dense launch");
}

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
                  uint64_t dropout_seed, fa_stream_t stream) {
  if (!q || !k || !v || !out || !cu_seqlens_q || !cu_seqlens_k || !q_stride || !k_stride ||
      !v_stride || !o_stride)
    return fail(FA_ERR_INVALID, "fa_fwd_varlen: null pointer argument");
  if (block_table && (page_size <= 0 || num_pages <= 0 || block_table_cols <= 0 ||
                      num_pages > INT32_MAX || block_table_cols > INT32_MAX))
    return fail(FA_ERR_INVALID, "fa_fwd_varlen: a block table needs positive page_size, "
                                "num_pages and block_table_cols");
  if (lse && !lse_stride) return fail(FA_ERR_INVALID, "fa_fwd_varlen: lse without lse_stride");
  if (!supported_dtype(dtype))
    return fail(FA_ERR_UNSUPPORTED, "fa_fwd_varlen: dtype %d not supported", dtype);
  if (!supported_head_dim(head_dim))
    return fail(FA_ERR_UNSUPPORTED, "fa_fwd_varlen: head_dim %lld not in {16,32,64,128,256}",
                (long long)head_dim);
  if (batch < 0 || max_seqlen_q < 0 || max_seqlen_k < 0 || heads_q <= 0 || heads_k <= 0 ||
      heads_q % heads_k != 0)
    return fail(FA_ERR_INVALID, "fa_fwd_varlen: bad sizes");
  if (max_seqlen_q > kMaxLen || max_seqlen_k > kMaxLen || batch * heads_q > INT32_MAX)
    return fail(FA_ERR_UNSUPPORTED, "fa_fwd_varlen: sizes exceed 2^29");
  const int64_t eb = elem_bytes(dtype);
  const int nkv = block_table ? 3 : 2;   // paged K/V: {page, slot, head} strides
  if (!aligned16(q, q_stride, 2, eb) || !aligned16(k, k_stride, nkv, eb) ||
      !aligned16(v, v_stride, nkv, eb) || !aligned16(out, o_stride, 2, eb))
    return fail(FA_ERR_UNSUPPORTED, "fa_fwd_varlen: tensors must be 16-byte aligned with strides "
                                    "that are multiples of 16 bytes");
  if (batch == 0 || max_seqlen_q == 0) return hip_status(hipSuccess, "");
  fa::FwdParams p{};
  p.q = q; p.k = k; p.v = v; p.o = out; p.lse = lse;
  p.q_ss = q_stride[0]; p.q_sh = q_stride[1];
  if (block_table) {
    p.k_sb = k_stride[0]; p.k_ss = k_stride[1]; p.k_sh = k_stride[2];
    p.v_sb = v_stride[0]; p.v_ss = v_stride[1]; p.v_sh = v_stride[2];
    p.block_table = block_table; p.bt_stride = block_table_stride; p.page_size = (int)page_size;
    p.cache_blocks = (int)num_pages; p.bt_cols = (int)block_table_cols;
  } else {
    p.k_ss = k_stride[0]; p.k_sh = k_stride[1];
    p.v_ss = v_stride[0]; p.v_sh = v_stride[1];
  }
  p.o_ss = o_stride[0]; p.o_sh = o_stride[1];
  if (lse) { p.lse_ss = lse_stride[0]; p.lse_sh = lse_stride[1]; }
  p.cu_q = cu_seqlens_q; p.cu_k = cu_seqlens_k;
  p.seqused_q = seqused_q; p.seqused_k = seqused_k; p.cu_o = cu_seqlens_out;
  if (!fill_dropout(p.drop, dropout_p, dropout_seed))
    return fail(FA_ERR_INVALID, "fa_fwd_varlen: dropout_p must be in [0, 1 - 2^-17]");
  p.batch = (int)batch; p.seqlen_q = (int)max_seqlen_q; p.seqlen_k = (int)max_seqlen_k;
  p.heads_q = (int)heads_q; p.heads_k = (int)heads_k; p.group = (int)(heads_q / heads_k);
  fill_scale(p, softmax_scale, softcap, alibi_slopes);
  p.alibi_sb = alibi_batch_stride;
  p.causal = causal != 0;
  p.window_left = clamp_window(window_left);
  p.window_right = clamp_window(window_right);
  p.num_splits = 1;
  p.heavy_first = p.causal || p.window_right >= 0;
  return hip_status(launch_fwd(dtype, p, fa::kModePrefill, (int)head_dim, needs_generic(p),
                               (hipStream_t)stream),
                    "fa_fwd_varlen launch");
}

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
                 float dropout_p, uint64_t dropout_seed, fa_stream_t stream) {
  const char* name = "fa_bwd_dense";
  int rc = bwd_check_common(name, q, k, v, out, dout, lse, dq, dk, dv, delta, dtype, head_dim,
                            heads_q, heads_k);
  if (rc != FA_OK) return rc;
  if (!q_stride || !k_stride || !v_stride || !o_stride || !do_stride || !dq_stride ||
      !dk_stride || !dv_stride || !lse_stride)
    return fail(FA_ERR_INVALID, "%s: null stride argument", name);
  if ((attn_bias && !bias_stride) || (dbias && !dbias_stride))
    return fail(FA_ERR_INVALID, "%s: attn_bias / dbias without its strides", name);
  if (batch < 0 || seqlen_q < 0 || seqlen_k < 0)
    return fail(FA_ERR_INVALID, "%s: bad sizes B=%lld Sq=%lld Sk=%lld", name, (long long)batch,
                (long long)seqlen_q, (long long)seqlen_k);
  if (seqlen_q > kMaxLen || seqlen_k > kMaxLen || q_pos_offset > kMaxLen ||
      q_pos_offset < -kMaxLen || batch * heads_q > INT32_MAX)
    return fail(FA_ERR_UNSUPPORTED, "%s: sizes or position offset exceed 2^29", name);
  if (!aligned16(q, q_stride, 3) || !aligned16(k, k_stride, 3) || !aligned16(v, v_stride, 3) ||
      !aligned16(out, o_stride, 3) || !aligned16(dout, do_stride, 3) ||
      !aligned16(dq, dq_stride, 3) || !aligned16(dk, dk_stride, 3) || !aligned16(dv, dv_stride, 3))
    return fail(FA_ERR_UNSUPPORTED, "%s: tensors must be 16-byte aligned with strides that are "
                                    "multiples of 16 bytes", name);
  if (batch == 0) return hip_status(hipSuccess, "");
  fa::BwdParams p{};
  p.q = q; p.k = k; p.v = v; p.o = out; p.dout = dout; p.dq = dq; p.dk = dk; p.dv = dv;
  p.lse = lse; p.delta = delta;
  p.q_sb = q_stride[0]; p.q_ss = q_stride[1]; p.q_sh = q_stride[2];
  p.k_sb = k_stride[0]; p.k_ss = k_stride[1]; p.k_sh = k_stride[2];
  p.v_sb = v_stride[0]; p.v_ss = v_stride[1]; p.v_sh = v_stride[2];
  p.o_sb = o_stride[0]; p.o_ss = o_stride[1]; p.o_sh = o_stride[2];
  p.do_sb = do_stride[0]; p.do_ss = do_stride[1]; p.do_sh = do_stride[2];
  p.dq_sb = dq_stride[0]; p.dq_ss = dq_stride[1]; p.dq_sh = dq_stride[2];
  p.dk_sb = dk_stride[0]; p.dk_ss = dk_stride[1]; p.dk_sh = dk_stride[2];
  p.dv_sb = dv_stride[0]; p.dv_ss = dv_stride[1]; p.dv_sh = dv_stride[2];
  p.lse_sb = lse_stride[0]; p.lse_sh = lse_stride[1]; p.lse_ss = lse_stride[2];
  p.batch = (int)batch; p.seqlen_q = (int)seqlen_q; p.seqlen_k = (int)seqlen_k;
  p.heads_q = (int)heads_q; p.heads_k = (int)heads_k; p.group = (int)(heads_q / heads_k);
  p.q_offset = q_pos_offset;
  p.bias = attn_bias;
  if (attn_bias) {
    p.bias_sb = bias_stride[0]; p.bias_sh = bias_stride[1];
    p.bias_sq = bias_stride[2]; p.bias_sk = bias_stride[3];
  }
  p.dbias = dbias;
  if (dbias) {
    p.dbias_sb = dbias_stride[0]; p.dbias_sh = dbias_stride[1];
    p.dbias_sq = dbias_stride[2]; p.dbias_sk = dbias_stride[3];
  }
  return bwd_launch(name, p, dtype, head_dim, softmax_scale, softcap, alibi_slopes,
                    alibi_batch_stride, causal, window_left, window_right, dropout_p,
                    dropout_seed, (hipStream_t)stream);
}

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
                  uint64_t dropout_seed, fa_stream_t stream) {
  const char* name = "fa_bwd_varlen";
  int rc = bwd_check_common(name, q, k, v, out, dout, lse, dq, dk, dv, delta, dtype, head_dim,
                            heads_q, heads_k);
  if (rc != FA_OK) return rc;
  if (!cu_seqlens_q || !cu_seqlens_k || !q_stride || !k_stride || !v_stride || !o_stride ||
      !do_stride || !dq_stride || !dk_stride || !dv_stride || !lse_stride)
    return fail(FA_ERR_INVALID, "%s: null pointer argument", name);
  if (batch < 0 || max_seqlen_q < 0 || max_seqlen_k < 0)
    return fail(FA_ERR_INVALID, "%s: bad sizes", name);
  if (max_seqlen_q > kMaxLen || max_seqlen_k > kMaxLen || batch * heads_q > INT32_MAX)
    return fail(FA_ERR_UNSUPPORTED, "%s: sizes exceed 2^29", name);
  if (!aligned16(q, q_stride, 2) || !aligned16(k, k_stride, 2) || !aligned16(v, v_stride, 2) ||
      !aligned16(out, o_stride, 2) || !aligned16(dout, do_stride, 2) ||
      !aligned16(dq, dq_stride, 2) || !aligned16(dk, dk_stride, 2) || !aligned16(dv, dv_stride, 2))
    return fail(FA_ERR_UNSUPPORTED, "%s: tensors must be 16-byte aligned with strides that are "
                                    "multiples of 16 bytes", name);
  if (batch == 0) return hip_status(hipSuccess, "");
  fa::BwdParams p{};
  p.q = q; p.k = k; p.v = v; p.o = out; p.dout = dout; p.dq = dq; p.dk = dk; p.dv = dv;
  p.lse = lse; p.delta = delta;
  p.q_ss = q_stride[0]; p.q_sh = q_stride[1];
  p.k_ss = k_stride[0]; p.k_sh = k_stride[1];
  p.v_ss = v_stride[0]; p.v_sh = v_stride[1];
  p.o_ss = o_stride[0]; p.o_sh = o_stride[1];
  p.do_ss = do_stride[0]; p.do_sh = do_stride[1];
  p.dq_ss = dq_stride[0]; p.dq_sh = dq_stride[1];
  p.dk_ss = dk_stride[0]; p.dk_sh = dk_stride[1];
  p.dv_ss = dv_stride[0]; p.dv_sh = dv_stride[1];
  p.lse_ss = lse_stride[0]; p.lse_sh = lse_stride[1];
  p.cu_q = cu_seqlens_q; p.cu_k = cu_seqlens_k;
  p.batch = (int)batch; p.seqlen_q = (int)max_seqlen_q; p.seqlen_k = (int)max_seqlen_k;
  p.heads_q = (int)heads_q; p.heads_k = (int)heads_k; p.group = (int)(heads_q / heads_k);
  return bwd_launch(name, p, dtype, head_dim, softmax_scale, softcap, alibi_slopes,
                    alibi_batch_stride, causal, window_left, window_right, dropout_p,
                    dropout_seed, (hipStream_t)stream);
}

int fa_fwd_kvcache_plan(int64_t batch, int64_t seqlen_q, int64_t heads_q, int64_t heads_k,
                        int64_t head_dim, int64_t max_keys, int64_t page_size,
                        int32_t* num_splits, int64_t* workspace_bytes) {
  if (!num_splits || !workspace_bytes)
    return fail(FA_ERR_INVALID, "fa_fwd_kvcache_plan: null output pointer");
  if (batch < 0 || seqlen_q < 0 || heads_q <= 0 || heads_k <= 0 || heads_q % heads_k != 0 ||
      max_keys < 0 || page_size < 0)
    return fail(FA_ERR_INVALID, "fa_fwd_kvcache_plan: bad sizes");
  if (!supported_head_dim(head_dim))
    return fail(FA_ERR_UNSUPPORTED, "fa_fwd_kvcache_plan: head_dim %lld not supported",
                (long long)head_dim);
  const KvPlan plan = kvcache_plan(batch, seqlen_q, heads_q, heads_k, head_dim, max_keys,
                                   page_size);
  *num_splits = plan.num_splits;
  *workspace_bytes = plan.o_part_bytes + plan.lse_part_bytes;
  g_last_error.clear();
  return FA_OK;
}

}  // extern "C"

// fa_fwd_kvcache and fa_fwd_kvcache_noalloc: argument checks, then the split
// and combine launches.  `workspace` holds the split partials (checked
// against the plan here); `name` prefixes every error message.
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
                   int64_t workspace_bytes, fa_stream_t stream) {
  if (!q || !k_cache || !v_cache || !out || !q_stride || !k_cache_stride || !v_cache_stride ||
      !o_stride)
    return fail(FA_ERR_INVALID, "%s: null pointer argument", name);
  if (lse && !lse_stride) return fail(FA_ERR_INVALID, "%s: lse without lse_stride", name);
  if (!supported_dtype(dtype))
    return fail(FA_ERR_UNSUPPORTED, "%s: dtype %d not supported", name, dtype);
  if (!supported_head_dim(head_dim))
    return fail(FA_ERR_UNSUPPORTED, "%s: head_dim %lld not supported", name,
                (long long)head_dim);
  if (batch < 0 || seqlen_q < 0 || max_keys < 0 || heads_q <= 0 || heads_k <= 0 ||
      heads_q % heads_k != 0 || cache_blocks < 0 || cache_blocks > INT32_MAX)
    return fail(FA_ERR_INVALID, "%s: bad sizes", name);
  if (block_table && page_size <= 0)
    return fail(FA_ERR_INVALID, "%s: page_size must be positive", name);
  if (seqlen_q * (heads_q / heads_k) > kMaxLen || max_keys > kMaxLen)
    return fail(FA_ERR_UNSUPPORTED, "%s: sizes exceed 2^29", name);
  const int64_t eb = elem_bytes(dtype);
  if (!aligned16(q, q_stride, 3, eb) || !aligned16(k_cache, k_cache_stride, 3, eb) ||
      !aligned16(v_cache, v_cache_stride, 3, eb) || !aligned16(out, o_stride, 3, eb))
    return fail(FA_ERR_UNSUPPORTED, "%s: tensors must be 16-byte aligned with "
                                    "strides that are multiples of 16 bytes", name);
  const KvPlan plan = kvcache_plan(batch, seqlen_q, heads_q, heads_k, head_dim, max_keys,
                                   block_table ? page_size : 0);
  if (num_splits != plan.num_splits)
    return fail(FA_ERR_INVALID, "%s: num_splits %d does not match the plan (%d)", name,
                (int)num_splits, plan.num_splits);
  // Nothing to compute: no launch, and no workspace is read.
  if (batch == 0 || seqlen_q == 0) return hip_status(hipSuccess, "");
  // fp32 runs every key of a row in one workgroup: the plan's split count is
  // checked above (the contract is dtype-independent) but no split is used,
  // so the workspace is neither needed nor read.
  const bool f32 = dtype == FA_DTYPE_F32;
  if (plan.num_splits > 1 && !f32 &&
      (!workspace || workspace_bytes < plan.o_part_bytes + plan.lse_part_bytes ||
       reinterpret_cast<uintptr_t>(workspace) % 16 != 0))
    return fail(FA_ERR_INVALID, "%s: workspace too small or misaligned (%lld < %lld)", name,
                (long long)workspace_bytes, (long long)(plan.o_part_bytes + plan.lse_part_bytes));
  if (plan.decode && !f32) {
    fa::DecodeParams d{};
    d.q = q; d.k = k_cache; d.v = v_cache; d.o = out; d.lse = lse;
    d.q_sb = q_stride[0]; d.q_ss = q_stride[1]; d.q_sh = q_stride[2];
    d.k_sb = k_cache_stride[0]; d.k_ss = k_cache_stride[1]; d.k_sh = k_cache_stride[2];
    d.v_sb = v_cache_stride[0]; d.v_ss = v_cache_stride[1]; d.v_sh = v_cache_stride[2];
    d.o_sb = o_stride[0]; d.o_ss = o_stride[1]; d.o_sh = o_stride[2];
    if (lse) { d.lse_sb = lse_stride[0]; d.lse_sh = lse_stride[1]; d.lse_ss = lse_stride[2]; }
    d.seqlens = cache_seqlens;
    d.block_table = block_table; d.bt_stride = block_table_stride; d.page_size = (int)page_size;
    d.cache_rows = cache_batch_idx; d.leftpad = cache_leftpad;
    d.cache_blocks = (int)cache_blocks;
    d.batch = (int)batch; d.seqlen_q = (int)seqlen_q; d.heads_q = (int)heads_q;
    d.heads_k = (int)heads_k; d.group = (int)(heads_q / heads_k); d.max_keys = (int)max_keys;
    d.scale = softmax_scale; d.scale_log2 = softmax_scale * fa::kLog2e;
    d.alibi = alibi_slopes; d.alibi_sb = alibi_batch_stride;
    d.causal = causal != 0;
    d.window_left = clamp_window(window_left);
    d.window_right = clamp_window(window_right);
    d.split_keys = plan.split_keys; d.num_splits = plan.num_splits;
    if (plan.num_splits > 1) {
      d.o_part = static_cast<float*>(workspace);
      d.lse_part = reinterpret_cast<float*>(static_cast<char*>(workspace) + plan.o_part_bytes);
    }
    const bool generic = alibi_slopes != nullptr || !(softmax_scale > 0.f);
    return hip_status(fa_launch_decode(dtype, d, (int)head_dim, generic, (hipStream_t)stream),
                      name);
  }
  fa::FwdParams p{};
  p.q = q; p.k = k_cache; p.v = v_cache; p.o = out; p.lse = lse;
  p.q_sb = q_stride[0]; p.q_ss = q_stride[1]; p.q_sh = q_stride[2];
  p.k_sb = k_cache_stride[0]; p.k_ss = k_cache_stride[1]; p.k_sh = k_cache_stride[2];
  p.v_sb = v_cache_stride[0]; p.v_ss = v_cache_stride[1]; p.v_sh = v_cache_stride[2];
  p.o_sb = o_stride[0]; p.o_ss = o_stride[1]; p.o_sh = o_stride[2];
  if (lse) { p.lse_sb = lse_stride[0]; p.lse_sh = lse_stride[1]; p.lse_ss = lse_stride[2]; }
  p.batch = (int)batch; p.seqlen_q = (int)seqlen_q; p.seqlen_k = (int)max_keys;
  p.heads_q = (int)heads_q; p.heads_k = (int)heads_k; p.group = (int)(heads_q / heads_k);
  fill_scale(p, softmax_scale, 0.f, alibi_slopes);
  p.alibi_sb = alibi_batch_stride;
  p.causal = causal != 0;
  p.kv_causal_offset = causal != 0;
  p.window_left = clamp_window(window_left);
  p.window_right = clamp_window(window_right);
  p.seqlens_k = cache_seqlens;
  p.block_table = block_table; p.bt_stride = block_table_stride; p.page_size = (int)page_size;
  p.cache_rows = cache_batch_idx; p.leftpad = cache_leftpad;
  p.cache_blocks = (int)cache_blocks;
  p.num_splits = f32 ? 1 : plan.num_splits; p.split_tiles = plan.split_tiles;
  if (p.num_splits > 1) {
    p.o_part = static_cast<float*>(workspace);
    p.lse_part = reinterpret_cast<float*>(static_cast<char*>(workspace) + plan.o_part_bytes);
  }
  p.heavy_first = 0;
  hipError_t e = launch_fwd(dtype, p, fa::kModeKvcache, (int)head_dim, needs_generic(p),
                            (hipStream_t)stream);
  if (e == hipSuccess && p.num_splits > 1)
    e = fa_launch_combine(dtype, p.o_part, p.lse_part, out, lse, plan.num_splits, (int)batch,
                          (int)seqlen_q, (int)heads_q, (int)head_dim, o_stride, lse_stride,
                          (hipStream_t)stream);
  return hip_status(e, name);
}

extern "C" {

int fa_fwd_kvcache(const void* q, const void* k_cache, const void* v_cache, void* out,
                   float* lse, const int32_t* cache_seqlens, const int32_t* block_table,
                   int64_t block_table_stride, int64_t page_size, int64_t cache_blocks,
                   const int32_t* cache_batch_idx, const int32_t* cache_leftpad, int64_t batch,
                   int64_t seqlen_q, int64_t max_keys, int64_t heads_q, int64_t heads_k,
                   int64_t head_dim, const int64_t* q_stride, const int64_t* k_cache_stride,
                   const int64_t* v_cache_stride, const int64_t* o_stride,
                   const int64_t* lse_stride, int dtype, float softmax_scale, int causal,
                   int64_t window_left, int64_t window_right, const float* alibi_slopes,
                   int64_t alibi_batch_stride, int32_t num_splits, void* workspace,
                   int64_t workspace_bytes, fa_stream_t stream) {
  return fa_kvcache_run("fa_fwd_kvcache", q, k_cache, v_cache, out, lse, cache_seqlens,
                        block_table, block_table_stride, page_size, cache_blocks,
                        cache_batch_idx, cache_leftpad, batch, seqlen_q, max_keys, heads_q,
                        heads_k, head_dim, q_stride, k_cache_stride, v_cache_stride, o_stride,
                        lse_stride, dtype, softmax_scale, causal, window_left, window_right,
                        alibi_slopes, alibi_batch_stride, num_splits, workspace,
                        workspace_bytes, stream);
}

int fa_attn_probs(const void* q, const void* k, const float* lse, float* probs, float* lse_out,
                  const int32_t* cu_seqlens_q, const int32_t* cu_seqlens_k, int64_t batch,
                  int64_t max_seqlen_q, int64_t max_seqlen_k, int64_t heads_q, int64_t heads_k,
                  int64_t head_dim, const int64_t* q_stride, const int64_t* k_stride,
                  const int64_t* lse_stride, int dtype, float softmax_scale, int causal,
                  int64_t q_pos_offset, int64_t window_left, int64_t window_right, float softcap,
                  const float* alibi_slopes, int64_t alibi_batch_stride, const float* attn_bias,
                  const int64_t* bias_stride, float dropout_p, uint64_t dropout_seed,
                  fa_stream_t stream) {
  if (!q || !k || !lse || !probs || !q_stride || !k_stride || !lse_stride)
    return fail(FA_ERR_INVALID, "fa_attn_probs: null pointer argument");
  if ((cu_seqlens_q == nullptr) != (cu_seqlens_k == nullptr))
    return fail(FA_ERR_INVALID, "fa_attn_probs: cu_seqlens_q and cu_seqlens_k go together");
  if (attn_bias && !bias_stride)
    return fail(FA_ERR_INVALID, "fa_attn_probs: attn_bias without bias_stride");
  if (!supported_dtype(dtype))
    return fail(FA_ERR_UNSUPPORTED, "fa_attn_probs: dtype %d not supported", dtype);
  if (!supported_head_dim(head_dim))
    return fail(FA_ERR_UNSUPPORTED, "fa_attn_probs: head_dim %lld not supported",
                (long long)head_dim);
  if (batch < 0 || max_seqlen_q < 0 || max_seqlen_k < 0 || heads_q <= 0 || heads_k <= 0 ||
      heads_q % heads_k != 0 || batch * heads_q > 65535)
    return fail(FA_ERR_INVALID, "fa_attn_probs: bad sizes");
  if (max_seqlen_q > kMaxLen || max_seqlen_k > kMaxLen || q_pos_offset > kMaxLen ||
      q_pos_offset < -kMaxLen)
    return fail(FA_ERR_UNSUPPORTED, "fa_attn_probs: lengths or offset exceed 2^29");
  if (max_seqlen_q > 4 * 65535)
    return fail(FA_ERR_UNSUPPORTED, "fa_attn_probs: max_seqlen_q above 262140 is not supported");
  if (!aligned16(q, q_stride, 3, elem_bytes(dtype)) || !aligned16(k, k_stride, 3, elem_bytes(dtype)))
    return fail(FA_ERR_UNSUPPORTED, "fa_attn_probs: q/k must be 16-byte aligned with strides "
                                    "that are multiples of 16 bytes");
  fa::ProbsParams p{};
  p.q = q; p.k = k; p.lse = lse; p.probs = probs; p.lse_out = lse_out;
  p.q_sb = q_stride[0]; p.q_ss = q_stride[1]; p.q_sh = q_stride[2];
  p.k_sb = k_stride[0]; p.k_ss = k_stride[1]; p.k_sh = k_stride[2];
  p.lse_sb = lse_stride[0]; p.lse_ss = lse_stride[1]; p.lse_sh = lse_stride[2];
  p.cu_q = cu_seqlens_q; p.cu_k = cu_seqlens_k;
  p.batch = (int)batch; p.max_q = (int)max_seqlen_q; p.max_k = (int)max_seqlen_k;
  p.heads_q = (int)heads_q; p.group = (int)(heads_q / heads_k); p.head_dim = (int)head_dim;
  p.scale = softmax_scale; p.softcap = softcap;
  p.alibi = alibi_slopes; p.alibi_sb = alibi_batch_stride;
  if (attn_bias) {
    p.bias = attn_bias;
    p.bias_sb = bias_stride[0]; p.bias_sh = bias_stride[1];
    p.bias_sq = bias_stride[2]; p.bias_sk = bias_stride[3];
  }
  p.causal = causal != 0; p.q_offset = (int)q_pos_offset;
  p.window_left = clamp_window(window_left);
  p.window_right = clamp_window(window_right);
  if (!fill_dropout(p.drop, dropout_p, dropout_seed))
    return fail(FA_ERR_INVALID, "fa_attn_probs: dropout_p must be in [0, 1 - 2^-17]");
  return hip_status(fa_launch_probs(dtype, p, (hipStream_t)stream), "fa_attn_probs launch");
}

int fa_kvcache_append(const void* k_new, const void* v_new, void* k_cache, void* v_cache,
                      const int32_t* cache_seqlens, const int32_t* block_table,
                      int64_t block_table_stride, int64_t page_size, int64_t num_pages,
                      const int32_t* cache_batch_idx, int64_t cache_rows,
                      const int32_t* cache_leftpad, int64_t capacity, const float* rotary_cos,
                      const float* rotary_sin, int64_t rotary_dim, int64_t rotary_rows,
                      int rotary_interleaved, int64_t batch, int64_t n_new, int64_t heads_k,
                      int64_t head_dim, const int64_t* k_new_stride, const int64_t* v_new_stride,
                      const int64_t* k_cache_stride, const int64_t* v_cache_stride, int dtype,
                      fa_stream_t stream) {
  if (!k_new || !v_new || !k_cache || !v_cache || !k_new_stride || !v_new_stride ||
      !k_cache_stride || !v_cache_stride)
    return fail(FA_ERR_INVALID, "fa_kvcache_append: null pointer argument");
  if (!supported_dtype(dtype))
    return fail(FA_ERR_UNSUPPORTED, "fa_kvcache_append: dtype %d not supported", dtype);
  if (batch < 0 || n_new < 0 || heads_k <= 0 || head_dim <= 0 || capacity < 0 ||
      (block_table && (page_size <= 0 || num_pages <= 0)) || (!block_table && cache_rows <= 0))
    return fail(FA_ERR_INVALID, "fa_kvcache_append: bad sizes");
  if ((rotary_cos == nullptr) != (rotary_sin == nullptr))
    return fail(FA_ERR_INVALID, "fa_kvcache_append: rotary_cos and rotary_sin go together");
  if (rotary_cos && (rotary_dim <= 0 || rotary_dim % 2 != 0 || rotary_dim > head_dim ||
                     rotary_rows <= 0))
    return fail(FA_ERR_INVALID, "fa_kvcache_append: rotary_dim %lld must be even, positive and "
                                "at most head_dim", (long long)rotary_dim);
  if (batch * n_new * heads_k * head_dim > INT64_C(1) << 40 || capacity > kMaxLen)
    return fail(FA_ERR_UNSUPPORTED, "fa_kvcache_append: sizes too large");
  fa::AppendParams p{};
  p.k_new = k_new; p.v_new = v_new; p.k_cache = k_cache; p.v_cache = v_cache;
  p.kn_sb = k_new_stride[0]; p.kn_ss = k_new_stride[1]; p.kn_sh = k_new_stride[2];
  p.vn_sb = v_new_stride[0]; p.vn_ss = v_new_stride[1]; p.vn_sh = v_new_stride[2];
  p.kc_sb = k_cache_stride[0]; p.kc_ss = k_cache_stride[1]; p.kc_sh = k_cache_stride[2];
  p.vc_sb = v_cache_stride[0]; p.vc_ss = v_cache_stride[1]; p.vc_sh = v_cache_stride[2];
  p.seqlens = cache_seqlens; p.block_table = block_table; p.bt_stride = block_table_stride;
  p.page_size = (int)page_size; p.num_pages = (int)num_pages;
  p.cache_rows = cache_batch_idx; p.cache_rows_n = (int)cache_rows; p.leftpad = cache_leftpad;
  p.capacity = capacity;
  p.cos = rotary_cos; p.sin = rotary_sin; p.rot = (int)rotary_dim;
  p.interleaved = rotary_interleaved != 0; p.table_rows = rotary_rows;
  p.batch = (int)batch; p.n_new = (int)n_new; p.heads_k = (int)heads_k; p.head_dim = (int)head_dim;
  return hip_status(fa_launch_kv_append(dtype, p, (hipStream_t)stream), "fa_kvcache_append launch");
}

int fa_rotary_q(const void* q, void* out, const int32_t* cache_seqlens,
                const int32_t* cache_leftpad, const float* rotary_cos, const float* rotary_sin,
                int64_t rotary_dim, int64_t rotary_rows, int rotary_interleaved, int64_t batch,
                int64_t seqlen_q, int64_t heads, int64_t head_dim, const int64_t* q_stride,
                const int64_t* out_stride, int dtype, fa_stream_t stream) {
  if (!q || !out || !cache_seqlens || !rotary_cos || !rotary_sin || !q_stride || !out_stride)
    return fail(FA_ERR_INVALID, "fa_rotary_q: null pointer argument");
  if (!supported_dtype(dtype))
    return fail(FA_ERR_UNSUPPORTED, "fa_rotary_q: dtype %d not supported", dtype);
  if (batch < 0 || seqlen_q < 0 || heads <= 0 || head_dim <= 0 || rotary_rows <= 0 ||
      rotary_dim <= 0 || rotary_dim % 2 != 0 || rotary_dim > head_dim)
    return fail(FA_ERR_INVALID, "fa_rotary_q: bad sizes");
  fa::RotaryQParams p{};
  p.q = q; p.out = out;
  p.q_sb = q_stride[0]; p.q_ss = q_stride[1]; p.q_sh = q_stride[2];
  p.o_sb = out_stride[0]; p.o_ss = out_stride[1]; p.o_sh = out_stride[2];
  p.seqlens = cache_seqlens; p.leftpad = cache_leftpad;
  p.cos = rotary_cos; p.sin = rotary_sin; p.rot = (int)rotary_dim;
  p.interleaved = rotary_interleaved != 0; p.table_rows = rotary_rows;
  p.batch = (int)batch; p.seqlen_q = (int)seqlen_q; p.heads = (int)heads; p.head_dim = (int)head_dim;
  return hip_status(fa_launch_rotary_q(dtype, p, (hipStream_t)stream), "fa_rotary_q launch");
}

int fa_quant_k_int8(const void* k, int8_t* k8, float* s_k, int64_t batch, int64_t heads,
                    int64_t seqlen, int64_t head_dim, const int64_t* k_stride,
                    fa_stream_t stream) {
  if (!k || !k8 || !s_k || !k_stride) return fail(FA_ERR_INVALID, "fa_quant_k_int8: null pointer");
  if (head_dim != 32 && head_dim != 64 && head_dim != 128 && head_dim != 256)
    return fail(FA_ERR_UNSUPPORTED, "fa_quant_k_int8: head_dim %lld not in {32,64,128,256}",
                (long long)head_dim);
  if (batch < 0 || heads <= 0 || seqlen < 0 || batch * heads * seqlen > INT32_MAX)
    return fail(FA_ERR_INVALID, "fa_quant_k_int8: bad sizes");
  if (!aligned16(k, k_stride, 3) || reinterpret_cast<uintptr_t>(k8) % 8 != 0 ||
      reinterpret_cast<uintptr_t>(s_k) % 4 != 0)
    return fail(FA_ERR_UNSUPPORTED, "fa_quant_k_int8: misaligned tensors");
  return hip_status(fa_launch_quant_k_int8(k, k8, s_k, (int)batch, (int)heads, (int)seqlen,
                                           (int)head_dim, k_stride, (hipStream_t)stream),
                    "fa_quant_k_int8 launch");
}

int fa_fwd_int8(const void* q, const int8_t* k8, const float* s_k, const void* v, void* out,
                float* lse, int64_t batch, int64_t heads, int64_t seqlen, int64_t head_dim,
                const int64_t* q_stride, const int64_t* v_stride, const int64_t* o_stride,
                float sm_scale, int causal, int64_t seq_len_k, int64_t seq_len_q,
                fa_stream_t stream) {
  if (!q || !k8 || !s_k || !v || !out || !q_stride || !v_stride || !o_stride)
    return fail(FA_ERR_INVALID, "fa_fwd_int8: null pointer argument");
  if (head_dim != 32 && head_dim != 64 && head_dim != 128 && head_dim != 256)
    return fail(FA_ERR_UNSUPPORTED, "fa_fwd_int8: head_dim %lld not in {32,64,128,256}",
                (long long)head_dim);
  if (batch < 0 || heads <= 0 || seqlen < 0 || batch * heads > INT32_MAX)
    return fail(FA_ERR_INVALID, "fa_fwd_int8: bad sizes");
  if (seqlen > kMaxLen || seq_len_k < 0 || seq_len_k > kMaxLen || seq_len_q < 0 ||
      seq_len_q > kMaxLen)
    return fail(FA_ERR_UNSUPPORTED, "fa_fwd_int8: lengths exceed 2^29");
  if (!aligned16(q, q_stride, 3) || !aligned16(v, v_stride, 3) || !aligned16(out, o_stride, 3) ||
      reinterpret_cast<uintptr_t>(k8) % 16 != 0)
    return fail(FA_ERR_UNSUPPORTED, "fa_fwd_int8: misaligned tensors");
  if (batch == 0 || seqlen == 0) return hip_status(hipSuccess, "");
  return hip_status(fa_launch_int8_fwd(q, k8, s_k, v, out, lse, (int)batch, (int)heads,
                                       (int)seqlen, (int)head_dim, q_stride, v_stride, o_stride,
                                       sm_scale, causal, (int)seq_len_k, (int)seq_len_q,
                                       (hipStream_t)stream),
                    "fa_fwd_int8 launch");
}

}  // extern "C"
