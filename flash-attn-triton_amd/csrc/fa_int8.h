// Parameters and quantization helpers of the INT8-QK^T attention kernels
// (fa_int8.hip, fa_int8_pp.h).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace fa {

// x >= 0 ? floor(x + 0.5) : ceil(x - 0.5) in fp32 (the reference's _round_i8,
// attention_kernel_int8.py:27-39), computed as trunc(x + copysign(0.5, x)):
// the sum is the same single fp32 addition in both branches (x + 0.5 for
// x >= 0, including +0 and -0, whose sum -0.5 truncates to 0 as floor(0.5)
// does; x - 0.5 for x < 0), and truncation equals floor for the positive sums
// and ceil for the negative ones.  No contraction: the rounding of the sum is
// part of the definition.
__device__ inline float round_half_away(float x) {
#pragma clang fp contract(off)
  return __builtin_truncf(x + __builtin_copysignf(0.5f, x));
}

__device__ inline uint32_t pack_i8x4(float a, float b, float c, float d) {
  return ((uint32_t)(uint8_t)(int8_t)(int)a) | ((uint32_t)(uint8_t)(int8_t)(int)b << 8) |
         ((uint32_t)(uint8_t)(int8_t)(int)c << 16) | ((uint32_t)(uint8_t)(int8_t)(int)d << 24);
}

// q, v, o: [B, H, S, D] with the given strides (elements); k8: [B*H, S, D]
// contiguous int8; s_k: [B*H, S]; lse: [B, H, S].
struct Int8Params {
  const void* q; const int8_t* k8; const float* s_k; const void* v; void* o; float* lse;
  int64_t q_sb, q_sh, q_ss;
  int64_t v_sb, v_sh, v_ss;
  int64_t o_sb, o_sh, o_ss;
  int batch, heads, seqlen;
  float scale_log2;
  int causal, seq_len_k, seq_len_q;
  int n_mblocks, total_blocks;
};

}  // namespace fa
