// Parameter block of probs_kernel (fa_probs.hip), shared with the C ABI.
// Strides are in elements.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "fa_common.h"

namespace fa {

struct ProbsParams {
  const void* q; const void* k; const float* lse; float* probs; float* lse_out;
  int64_t q_sb, q_ss, q_sh;      // dense {batch, seq, head}; varlen {-, token, head}
  int64_t k_sb, k_ss, k_sh;
  int64_t lse_sb, lse_ss, lse_sh;   // dense {batch, query, head}; varlen {-, token, head}
  const int* cu_q; const int* cu_k;
  int batch, max_q, max_k, heads_q, group, head_dim;
  float scale, softcap;
  const float* alibi; int64_t alibi_sb;
  const float* bias; int64_t bias_sb, bias_sh, bias_sq, bias_sk;
  int causal, q_offset, window_left, window_right;
  DropoutCfg drop;   // probabilities are returned after dropout, as the forward used them
};

}  // namespace fa

hipError_t fa_launch_probs(int dtype, const fa::ProbsParams& p, hipStream_t st);
