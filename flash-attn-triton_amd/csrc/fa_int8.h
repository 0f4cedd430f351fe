// Parameters and quantization helpers of the INT8-QK^T attention kernels
// (fa_int8.hip, fa_int8_pp.h).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "fa_fastdiv.h"

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

// round_half_away(x) as an integer: the truncating convert of x +- 0.5 (the
// same single fp32 addition, then the truncation the convert performs).
__device__ inline int round_half_away_i(float x) {
#pragma clang fp contract(off)
  return (int)(x + __builtin_copysignf(0.5f, x));
}

// Low bytes of four ints in [-128, 127] as one dword (a in byte 0): two byte
// permutes and a shift-or.
__device__ inline uint32_t pack_i8x4_i(int a, int b, int c, int d) {
  const uint32_t ab = __builtin_amdgcn_perm((uint32_t)b, (uint32_t)a, 0x0c0c0400u);
  const uint32_t cd = __builtin_amdgcn_perm((uint32_t)d, (uint32_t)c, 0x0c0c0400u);
  return ab | (cd << 16);
}

// x / s of the Q quantizer (s = fp32(max(amax, 1)) / 127, |x| <= amax, x and
// amax fp16 values) from inv = 1 / s (IEEE division, once per row): q0 = x inv
// is within an ulp of x / s, and one correction with the exact remainder
// x - q0 s gives the correctly rounded quotient (Markstein's theorem for a
// correctly rounded reciprocal).  Checked equal to the IEEE division for every
// such (x, amax) pair, 7.7e8 of them (tests/test_int8_division.py).
__device__ inline float quant_div(float x, float s, float inv) {
  const float q0 = x * inv;
  const float r = __builtin_fmaf(-q0, s, x);
  return __builtin_fmaf(r, inv, q0);
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
  int persist_rounds;   // int8_persist_kernel: row blocks per workgroup
  // int8_persist_kernel: divisions by the row blocks (causal: pairs) per
  // group and by the head count (set by its launcher).
  FastDiv fd_blk, fd_heads;
};

}  // namespace fa
