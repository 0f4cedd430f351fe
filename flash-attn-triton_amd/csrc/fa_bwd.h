// Parameters of the attention backward kernels (fa_bwd_kernel.h) and their
// host launch entry points (fa_bwd_f16.hip / fa_bwd_bf16.hip).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "fa_common.h"

namespace fa {

// All strides are in elements.  Layouts as in the forward:
//   dense : x[b*x_sb + i*x_ss + h*x_sh + d]
//   varlen: x[(cu[b] + i)*x_ss + h*x_sh + d]   (cu_q != nullptr)
// lse (natural log, fp32) and delta (fp32, rowsum(dO * O), written by the dQ
// kernel and read by the dK/dV kernel) share the lse strides.
struct BwdParams {
  const void* q; const void* k; const void* v; const void* o; const void* dout;
  void* dq; void* dk; void* dv;
  const float* lse; float* delta;
  int64_t q_sb, q_ss, q_sh;
  int64_t k_sb, k_ss, k_sh;
  int64_t v_sb, v_ss, v_sh;
  int64_t o_sb, o_ss, o_sh;
  int64_t do_sb, do_ss, do_sh;
  int64_t dq_sb, dq_ss, dq_sh;
  int64_t dk_sb, dk_ss, dk_sh;
  int64_t dv_sb, dv_ss, dv_sh;
  int64_t lse_sb, lse_ss, lse_sh;
  int batch, seqlen_q, seqlen_k, heads_q, heads_k, group;
  float scale, scale_log2, softcap, softcap_k;   // softcap_k = 2 log2(e) / softcap
  const float* alibi; int64_t alibi_sb;
  int causal, window_left, window_right;
  int64_t q_offset;                               // query row i sits at position i + q_offset
  const int* cu_q; const int* cu_k;
  DropoutCfg drop;                                // the forward's dropout (GENERIC only)
  // Optional fp32 additive bias of the dense forward (after ALiBi, before
  // softcap), bias[b*bias_sb + h*bias_sh + i*bias_sq + j*bias_sk], and the
  // fp32 buffer that receives its gradient dS, added at the same index form
  // (dense layout only, GENERIC only; broadcast dims have stride 0, so their
  // gradients sum).
  const float* bias; int64_t bias_sb, bias_sh, bias_sq, bias_sk;
  float* dbias; int64_t dbias_sb, dbias_sh, dbias_sq, dbias_sk;
  int n_blocks, total_blocks;                     // filled by the launcher
};

}  // namespace fa

// dQ (and delta) first, then dK / dV, both on `st`.  D in {32, 64, 128, 256}.
hipError_t fa_launch_bwd_f16(const fa::BwdParams& p, int head_dim, bool generic, hipStream_t st);
hipError_t fa_launch_bwd_bf16(const fa::BwdParams& p, int head_dim, bool generic, hipStream_t st);
// fp32 (fa_bwd_f32.hip): D in {32, 64, 128}.
hipError_t fa_launch_bwd_f32(const fa::BwdParams& p, int head_dim, bool generic, hipStream_t st);
