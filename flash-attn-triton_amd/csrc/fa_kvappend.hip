// KV-cache append and rotary embedding for flash_attn_with_kvcache(k, v,
// rotary_cos, rotary_sin, ...).
//
// Behaviour of /root/reference/flash_attn_triton/flash_attn_interface.py:468-493
// (append) and :52-66 (rotary), with the append performed in place (the
// reference indexes the cache with advanced indexing and writes into the
// temporary copy, so its append is lost; upstream FlashAttention-2 writes the
// cache):
//   * token t of batch b goes to logical cache position
//     pos = cache_seqlens[b] + cache_leftpad[b] + t: slot pos % page_size of
//     page block_table[b][pos / page_size] (paged), or position pos of cache
//     row cache_batch_idx[b] (batched);
//   * with rotary tables, k is rotated at position pos before it is written,
//     and q row i at cache_seqlens_after[b] - seqlen_q + cache_leftpad[b] + i;
//   * rotary_dim = 2 * (columns of cos): interleaved pairs (2j, 2j + 1) or the
//     half-split pairs (j, j + rotary_dim / 2) rotate by (cos[pos][j],
//     sin[pos][j]); dims past rotary_dim are copied.
// The tables arrive in fp32 already rounded to the input dtype (the reference
// casts them to x.dtype before multiplying); the rotation is computed in fp32
// and rounded once to the element type.
//
// One thread per output element.  Out-of-range slots, pages or table rows
// (which the Python layer rejects before calling) are skipped, never read or
// written.
#include <type_traits>

#include "fa_common.h"
#include "fa_kvappend.h"

namespace fa {

namespace {

template <class T>
__device__ inline float ld(const void* base, int64_t i) {
  if constexpr (std::is_same<T, float>::value) return static_cast<const float*>(base)[i];
  else return T::to_float(static_cast<const uint16_t*>(base)[i]);
}

template <class T>
__device__ inline void st(void* base, int64_t i, float x) {
  if constexpr (std::is_same<T, float>::value) static_cast<float*>(base)[i] = x;
  else static_cast<uint16_t*>(base)[i] = (uint16_t)(T::pack2(x, 0.f) & 0xffffu);
}

// Element d of the rotated row: `row(j)` reads element j of the source row.
template <class F>
__device__ inline float rotate(F row, int d, const float* cs, const float* sn, int rot, int inter) {
  if (d >= rot) return row(d);
  if (inter) {
    const int j = d >> 1;
    return (d & 1) ? row(d - 1) * sn[j] + row(d) * cs[j] : row(d) * cs[j] - row(d + 1) * sn[j];
  }
  const int h = rot >> 1;
  return d < h ? row(d) * cs[d] - row(d + h) * sn[d] : row(d - h) * sn[d - h] + row(d) * cs[d - h];
}

}  // namespace

template <class T>
__global__ __launch_bounds__(256) void kv_append_kernel(const AppendParams p) {
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int64_t total = (int64_t)p.batch * p.n_new * p.heads_k * p.head_dim;
  if (idx >= total) return;
  const int d = (int)(idx % p.head_dim);
  int64_t r = idx / p.head_dim;
  const int h = (int)(r % p.heads_k);
  r /= p.heads_k;
  const int t = (int)(r % p.n_new);
  const int b = (int)(r / p.n_new);
  const int64_t pos = (int64_t)(p.seqlens != nullptr ? p.seqlens[b] : 0) +
                      (p.leftpad != nullptr ? p.leftpad[b] : 0) + t;
  if (pos < 0 || pos >= p.capacity) return;
  int64_t kc, vc;
  if (p.block_table != nullptr) {
    const int page = p.block_table[(int64_t)b * p.bt_stride + pos / p.page_size];
    if (page < 0 || page >= p.num_pages) return;
    const int slot = (int)(pos % p.page_size);
    kc = (int64_t)page * p.kc_sb + (int64_t)slot * p.kc_ss + (int64_t)h * p.kc_sh + d;
    vc = (int64_t)page * p.vc_sb + (int64_t)slot * p.vc_ss + (int64_t)h * p.vc_sh + d;
  } else {
    const int row = p.cache_rows != nullptr ? p.cache_rows[b] : b;
    if (row < 0 || row >= p.cache_rows_n) return;
    kc = (int64_t)row * p.kc_sb + pos * p.kc_ss + (int64_t)h * p.kc_sh + d;
    vc = (int64_t)row * p.vc_sb + pos * p.vc_ss + (int64_t)h * p.vc_sh + d;
  }
  const int64_t kn = (int64_t)b * p.kn_sb + (int64_t)t * p.kn_ss + (int64_t)h * p.kn_sh;
  const int64_t vn = (int64_t)b * p.vn_sb + (int64_t)t * p.vn_ss + (int64_t)h * p.vn_sh + d;
  float kx;
  if (p.cos != nullptr) {
    if (pos >= p.table_rows) return;
    const int half = p.rot >> 1;
    kx = rotate([&](int j) { return ld<T>(p.k_new, kn + j); }, d, p.cos + pos * half,
                p.sin + pos * half, p.rot, p.interleaved);
  } else {
    kx = ld<T>(p.k_new, kn + d);
  }
  st<T>(p.k_cache, kc, kx);
  st<T>(p.v_cache, vc, ld<T>(p.v_new, vn));
}

template <class T>
__global__ __launch_bounds__(256) void rotary_q_kernel(const RotaryQParams p) {
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int64_t total = (int64_t)p.batch * p.seqlen_q * p.heads * p.head_dim;
  if (idx >= total) return;
  const int d = (int)(idx % p.head_dim);
  int64_t r = idx / p.head_dim;
  const int h = (int)(r % p.heads);
  r /= p.heads;
  const int i = (int)(r % p.seqlen_q);
  const int b = (int)(r / p.seqlen_q);
  int64_t pos = (int64_t)p.seqlens[b] - p.seqlen_q + (p.leftpad != nullptr ? p.leftpad[b] : 0) + i;
  // Negative positions count from the end of the tables (torch indexing in
  // the reference, flash_attn_interface.py:56).
  if (pos < 0) pos += p.table_rows;
  const int64_t qi = (int64_t)b * p.q_sb + (int64_t)i * p.q_ss + (int64_t)h * p.q_sh;
  const int64_t oi = (int64_t)b * p.o_sb + (int64_t)i * p.o_ss + (int64_t)h * p.o_sh + d;
  if (pos < 0 || pos >= p.table_rows) {
    // A query row before the first or past the last table row has no
    // rotation to apply (the Python layer rejects such calls).
    st<T>(p.out, oi, ld<T>(p.q, qi + d));
    return;
  }
  const int half = p.rot >> 1;
  st<T>(p.out, oi, rotate([&](int j) { return ld<T>(p.q, qi + j); }, d, p.cos + pos * half,
                          p.sin + pos * half, p.rot, p.interleaved));
}

}  // namespace fa

hipError_t fa_launch_kv_append(int dtype, const fa::AppendParams& p, hipStream_t st) {
  const int64_t total = (int64_t)p.batch * p.n_new * p.heads_k * p.head_dim;
  if (total <= 0) return hipSuccess;
  const dim3 grid((unsigned)((total + 255) / 256));
  if (dtype == 0) hipLaunchKernelGGL(fa::kv_append_kernel<fa::F16>, grid, dim3(256), 0, st, p);
  else if (dtype == 1) hipLaunchKernelGGL(fa::kv_append_kernel<fa::BF16>, grid, dim3(256), 0, st, p);
  else hipLaunchKernelGGL(fa::kv_append_kernel<float>, grid, dim3(256), 0, st, p);
  return hipGetLastError();
}

hipError_t fa_launch_rotary_q(int dtype, const fa::RotaryQParams& p, hipStream_t st) {
  const int64_t total = (int64_t)p.batch * p.seqlen_q * p.heads * p.head_dim;
  if (total <= 0) return hipSuccess;
  const dim3 grid((unsigned)((total + 255) / 256));
  if (dtype == 0) hipLaunchKernelGGL(fa::rotary_q_kernel<fa::F16>, grid, dim3(256), 0, st, p);
  else if (dtype == 1) hipLaunchKernelGGL(fa::rotary_q_kernel<fa::BF16>, grid, dim3(256), 0, st, p);
  else hipLaunchKernelGGL(fa::rotary_q_kernel<float>, grid, dim3(256), 0, st, p);
  return hipGetLastError();
}
