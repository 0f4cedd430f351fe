// Row staging through LDS for the forward kernels at head dim 128
// (fa_prefill_kernel.h, fa_prefill_pp.h, fa_prefill_persist.h).
#pragma once

#include "fa_common.h"

namespace fa {

// Row staging through LDS.  The MFMA layouts hold a 32-row x 128 block in
// 16-byte pieces of 32 different rows per instruction; read or written that
// way, every global instruction touches 32 partial cache lines (measured on
// MI355X: 16 output stores of one wave took 2.3 us to issue).  These helpers
// move one wave's 32 rows through LDS instead, so that each global
// instruction covers four whole 256-byte rows (16 bytes per lane).  Staged Q
// rows (8 KiB per wave) keep 16-byte chunk c of row r at chunk position
// c ^ (r & 15), as the K tiles do.

// DMA of 32 rows (row_b bytes apart, from the resource's base) into the
// staging area at LDS address `lds`; rows past the resource read as zeros.
__device__ inline void stage_rows_load(const u32x4& rs, uint32_t lds, uint32_t row_b, int lane) {
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int r = 4 * i + (lane >> 4);
    const uint32_t c = (uint32_t)((lane & 15) ^ (r & 15));
    buf_load16_lds(rs, lds + i * 1024, (uint32_t)r * row_b + c * 16);
  }
}

// Row c32 of the staged block in the MFMA B-operand layout of S^T = K Q^T:
// lane (c32, g) gets dims 16 kc + 8 g .. + 7 of its row for each kc.
template <int NKC>
__device__ inline void stage_rows_read_operand(const uint8_t* st, int c32, int g, u32x4* out) {
#pragma unroll
  for (int kc = 0; kc < NKC; ++kc)
    out[kc] = *reinterpret_cast<const u32x4*>(st + c32 * 256 + (((2 * kc + g) ^ (c32 & 15)) * 16));
}

// O^T accumulators (lane (c32, g): dims 32 db + 8 (v / 4) + 4 g + v % 4 of row
// c32) times inv_l, packed to 16 bits, written to a staging area of
// kStageOutBytes and read back as whole rows: out[i] is chunk lane % 16 of row
// 4 i + lane / 16.  Rows are kStageOutPitch bytes apart (one 16-byte pad per
// 256-byte row spreads the 32 rows of a write over the banks), so every LDS
// address is a per-lane base plus an immediate (a swizzle would need one
// register per chunk).
constexpr int kStageOutPitch = 272;
constexpr int kStageOutBytes = 32 * kStageOutPitch;
template <class T, int NDB>
__device__ inline void stage_rows_gather(const f32x16* acc, float inv_l, uint8_t* st, int c32,
                                         int g, int lane, u32x4* out) {
  uint8_t* const wr = st + c32 * kStageOutPitch + 8 * g;
#pragma unroll
  for (int db = 0; db < NDB; ++db) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      u32x2 val;
      val[0] = T::pack2(acc[db][4 * r] * inv_l, acc[db][4 * r + 1] * inv_l);
      val[1] = T::pack2(acc[db][4 * r + 2] * inv_l, acc[db][4 * r + 3] * inv_l);
      *reinterpret_cast<u32x2*>(wr + (db * 4 + r) * 16) = val;
    }
  }
  // The wave's LDS writes are visible to its own later reads (all lanes).
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  const uint8_t* const rd = st + (lane >> 4) * kStageOutPitch + (lane & 15) * 16;
#pragma unroll
  for (int i = 0; i < 8; ++i)
    out[i] = *reinterpret_cast<const u32x4*>(rd + i * 4 * kStageOutPitch);
}

// Stores of stage_rows_gather's rows [0, rows_ok) at `orow0` (row stride
// o_ss elements): four whole rows per instruction.
__device__ inline void stage_rows_put(const u32x4* rows, uint16_t* orow0, int64_t o_ss, int lane,
                                      int rows_ok = 32) {
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int r = 4 * i + (lane >> 4);
    if (r < rows_ok) store16(orow0 + (int64_t)r * o_ss + (lane & 15) * 8, rows[i]);
  }
}

template <class T, int NDB>
__device__ inline void stage_rows_store(const f32x16* acc, float inv_l, uint8_t* st, int c32,
                                        int g, int lane, uint16_t* orow0, int64_t o_ss,
                                        int rows_ok) {
  u32x4 rows[8];
  stage_rows_gather<T, NDB>(acc, inv_l, st, c32, g, lane, rows);
  stage_rows_put(rows, orow0, o_ss, lane, rows_ok);
}

}  // namespace fa
