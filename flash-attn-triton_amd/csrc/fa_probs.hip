// Materialized attention probabilities for flash_attn_*(return_attn_probs=True).
//
// The reference computes this testing option with dense torch math
// (/root/reference/flash_attn_triton/flash_attn_interface.py:15-49 for dense and
// cross, :642-659 for varlen).  Here the output and the natural-log LSE come
// from the flash kernels (which also take the additive attn_bias), and
// probs_kernel recomputes every score with the same epilogue (scale, ALiBi,
// bias, softcap, mask) and writes p = exp(s - lse): the softmax of the row
// without ever holding the row.
//
// Layout: probs [batch, heads_q, max_q, max_k] fp32 contiguous, zero where
// i >= q_len(b), j >= k_len(b) or the key is masked; lse_out (optional)
// [batch, heads_q, max_q] fp32 contiguous, -inf past q_len(b) (the padding of
// the reference's varlen return, :644).  Rows whose LSE is -inf get all-zero
// probabilities (nan_to_num of an empty softmax, :44).
#include <type_traits>

#include "fa_probs.h"
#include "fa_common.h"

namespace fa {

// q . k over the head dim for 16-bit element types (T = F16 / BF16) or fp32
// (T = float), accumulated in fp32.
template <class T>
__device__ inline float row_dot(const void* qv, const void* kv, int head_dim) {
  float s = 0.f;
  if constexpr (std::is_same<T, float>::value) {
    const float* qp = static_cast<const float*>(qv);
    const float* kp = static_cast<const float*>(kv);
    for (int d = 0; d < head_dim; d += 4) {
      const f32x4 qa = *reinterpret_cast<const f32x4*>(qp + d);
      const f32x4 ka = *reinterpret_cast<const f32x4*>(kp + d);
#pragma unroll
      for (int e = 0; e < 4; ++e) s = fmaf(qa[e], ka[e], s);
    }
  } else {
    const uint16_t* qp = static_cast<const uint16_t*>(qv);
    const uint16_t* kp = static_cast<const uint16_t*>(kv);
    for (int d = 0; d < head_dim; d += 8) {
      const u32x4 qa = load16(qp + d), ka = load16(kp + d);
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int sh = (e & 1) * 16;
        s = fmaf(T::to_float((uint16_t)(qa[e >> 1] >> sh)), T::to_float((uint16_t)(ka[e >> 1] >> sh)), s);
      }
    }
  }
  return s;
}

template <class T>
__global__ __launch_bounds__(256) void probs_kernel(const ProbsParams p) {
  constexpr int64_t kElem = std::is_same<T, float>::value ? 4 : 2;
  const int j = blockIdx.x * 64 + (threadIdx.x & 63);
  const int i = blockIdx.y * 4 + (threadIdx.x >> 6);
  const int bz = blockIdx.z;
  const int h = bz % p.heads_q;
  const int b = bz / p.heads_q;
  if (i >= p.max_q || j >= p.max_k) return;
  const int kvh = h / p.group;

  int Sq, Sk;
  int64_t qrow, krow, lse_i;
  if (p.cu_q != nullptr) {
    const int qs = p.cu_q[b], ks = p.cu_k[b];
    Sq = p.cu_q[b + 1] - qs;
    Sk = p.cu_k[b + 1] - ks;
    qrow = (int64_t)(qs + i) * p.q_ss;
    krow = (int64_t)(ks + j) * p.k_ss;
    lse_i = (int64_t)(qs + i) * p.lse_ss;
  } else {
    Sq = p.max_q;
    Sk = p.max_k;
    qrow = (int64_t)b * p.q_sb + (int64_t)i * p.q_ss;
    krow = (int64_t)b * p.k_sb + (int64_t)j * p.k_ss;
    lse_i = (int64_t)b * p.lse_sb + (int64_t)i * p.lse_ss;
  }
  const bool valid = i < Sq && j < Sk;
  float prob = 0.f;
  float lse = -INFINITY;
  if (i < Sq) lse = p.lse[lse_i + (int64_t)h * p.lse_sh];
  if (valid && lse != -INFINITY) {
    const char* qp = static_cast<const char*>(p.q) + (qrow + (int64_t)h * p.q_sh) * kElem;
    const char* kp = static_cast<const char*>(p.k) + (krow + (int64_t)kvh * p.k_sh) * kElem;
    const float s = row_dot<T>(qp, kp, p.head_dim);
    const int qpos = i + (p.cu_q != nullptr ? 0 : p.q_offset);
    float x = s * p.scale;
    if (p.alibi != nullptr) x -= p.alibi[(int64_t)b * p.alibi_sb + h] * fabsf((float)(qpos - j));
    if (p.bias != nullptr)
      x += p.bias[(int64_t)b * p.bias_sb + (int64_t)h * p.bias_sh + (int64_t)i * p.bias_sq +
                  (int64_t)j * p.bias_sk];
    if (p.softcap > 0.f) x = p.softcap * tanhf(x / p.softcap);
    bool keep = true;
    if (p.causal) keep = keep && j <= qpos;
    if (p.window_left >= 0) keep = keep && j >= qpos - p.window_left;
    if (p.window_right >= 0) keep = keep && j <= qpos + p.window_right;
    if (keep) prob = expf(x - lse);
    if (p.drop.enabled) prob *= dropout_factor_at(p.drop, i, j, h, b);
  }
  p.probs[(((int64_t)b * p.heads_q + h) * p.max_q + i) * p.max_k + j] = prob;
  if (p.lse_out != nullptr && j == 0)
    p.lse_out[((int64_t)b * p.heads_q + h) * p.max_q + i] = lse;
}

}  // namespace fa

hipError_t fa_launch_probs(int dtype, const fa::ProbsParams& p, hipStream_t st) {
  const dim3 grid((unsigned)((p.max_k + 63) / 64), (unsigned)((p.max_q + 3) / 4),
                  (unsigned)(p.batch * p.heads_q));
  if (grid.x == 0 || grid.y == 0 || grid.z == 0) return hipSuccess;
  if (dtype == 0)
    hipLaunchKernelGGL(fa::probs_kernel<fa::F16>, grid, dim3(256), 0, st, p);
  else if (dtype == 1)
    hipLaunchKernelGGL(fa::probs_kernel<fa::BF16>, grid, dim3(256), 0, st, p);
  else
    hipLaunchKernelGGL(fa::probs_kernel<float>, grid, dim3(256), 0, st, p);
  return hipGetLastError();
}
