// Shared device-side types and helpers for the gfx950 (CDNA4) attention kernels.
//
// Everything here targets one architecture: 64-wide wavefronts, the CDNA4
// matrix cores (v_mfma_f32_32x32x16_{f16,bf16}, v_mfma_i32_32x32x32_i8) and
// v_permlane32_swap for exchanging values between the two 32-lane halves of a
// wave.  There is no portability layer.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "fa_fastdiv.h"

#include <atomic>

namespace fa {

// Raises a kernel's dynamic-LDS limit to `bytes` on the current device, once
// per device: the attribute is device state, so a process that launches on
// several devices sets it on each.  `devices` is one bit per device
// (devices 0..63; others set it on every call), a static of the call site;
// concurrent first calls both set the attribute, which is harmless.
template <class Kern>
inline hipError_t set_lds_limit(std::atomic<uint64_t>& devices, Kern kern, int bytes) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  const uint64_t bit = dev >= 0 && dev < 64 ? (uint64_t)1 << dev : 0;
  if (bit != 0 && (devices.load(std::memory_order_acquire) & bit) != 0) return hipSuccess;
  e = hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                          hipFuncAttributeMaxDynamicSharedMemorySize, bytes);
  if (e == hipSuccess && bit != 0) devices.fetch_or(bit, std::memory_order_acq_rel);
  return e;
}

// Compute units of the current device (cached per device).
inline hipError_t device_cus(int* n) {
  static std::atomic<int> cus[64];
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  if (dev >= 0 && dev < 64) {
    const int c = cus[dev].load(std::memory_order_relaxed);
    if (c > 0) {
      *n = c;
      return hipSuccess;
    }
  }
  e = hipDeviceGetAttribute(n, hipDeviceAttributeMultiprocessorCount, dev);
  if (e == hipSuccess && dev >= 0 && dev < 64) cus[dev].store(*n, std::memory_order_relaxed);
  return e;
}

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef int i32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;

// Element-type tags.  Storage is handled as raw 16-bit words; the MFMA and
// conversion wrappers reinterpret them.
struct F16 {
  static constexpr int kBytes = 2;
  // Row sums may be taken over the rounded P: fp16 rounding (2^-12 relative)
  // keeps the log-sum-exp within 3e-4.
  static constexpr bool kSumRounded = true;
  __device__ static inline f32x16 mfma32(u32x4 a, u32x4 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a),
                                                   __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
  }
  // Round-to-nearest-even pack of two floats (v_cvt_pk_f16_f32).
  __device__ static inline uint32_t pack2(float lo, float hi) {
    f32x2 x = {lo, hi};
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(x, f16x2));
  }
  __device__ static inline float to_float(uint16_t h) {
    return (float)__builtin_bit_cast(_Float16, h);
  }
  // acc + lo + hi of a packed pair (v_dot2c_f32_f16 against (1, 1)).
  __device__ static inline float sum2(uint32_t pk, float acc) {
    const f16x2 one = {(_Float16)1.0f, (_Float16)1.0f};
    return __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2, pk), one, acc, false);
  }
};

struct BF16 {
  static constexpr int kBytes = 2;
  // bf16 rounding (2^-9 relative) would move the log-sum-exp of short rows by
  // up to 2e-3: row sums are taken over the fp32 P instead.
  static constexpr bool kSumRounded = false;
  __device__ static inline f32x16 mfma32(u32x4 a, u32x4 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a),
                                                    __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
  }
  // Round-to-nearest-even pack of two floats (v_cvt_pk_bf16_f32).
  __device__ static inline uint32_t pack2(float lo, float hi) {
    f32x2 x = {lo, hi};
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(x, bf16x2));
  }
  __device__ static inline float to_float(uint16_t h) {
    return __builtin_bit_cast(float, (uint32_t)h << 16);
  }
  // acc + lo + hi of a packed pair (v_dot2c_f32_bf16 against (1, 1)).
  __device__ static inline float sum2(uint32_t pk, float acc) {
    const bf16x2 one = {(__bf16)1.0f, (__bf16)1.0f};
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, pk), one, acc, false);
  }
};

// Exchange a value between lane l and lane l^32 and combine both copies:
// v_permlane32_swap moves the upper half of `a` and the lower half of `b`;
// with a == b == x the two results hold x[l % 32] and x[l % 32 + 32].
__device__ inline float halves_max(float x) {
  auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ inline float halves_sum(float x) {
  auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// blockIdx.x -> logical work id so that consecutive logical ids run on the
// same XCD.  Hardware dispatches workgroup L to XCD L % 8; grouping the work
// of one (batch, head) on one XCD keeps its K/V tiles in that XCD's L2.
__device__ inline int xcd_remap(int L, int total) {
  constexpr int kXcds = 8;
  const int per = total / kXcds;
  if (L >= per * kXcds) return L;
  return (L % kXcds) * per + L / kXcds;
}

// Work item (row block mb, group index grp) of launch item L, for a launch of
// n_mblocks row blocks per group (a group is one (batch, head)).  Each XCD
// (items L % 8 == x) owns a contiguous range of groups, so their K/V tiles
// stay in its L2.  heavy_first (causal: the last row blocks see the most
// keys): each XCD takes its groups `span` at a time (span 0: all of them at
// once) and dispatches the last row block of every group in the span first,
// then the next-to-last, ..., so light blocks fill the tail; a wider span
// evens out the tail, a narrower one keeps fewer groups' K/V in L2.
__device__ inline void work_item(int L, int total, int n_mblocks, bool heavy_first, int span,
                                 int& mb, int& grp) {
  constexpr int kXcds = 8;
  if (heavy_first && total % (kXcds * n_mblocks) == 0) {
    const int groups_per_xcd = total / kXcds / n_mblocks;
    const int w = span <= 0 || span > groups_per_xcd ? groups_per_xcd : span;
    if (groups_per_xcd % w == 0) {
      const int k = L / kXcds;
      const int r = k % (w * n_mblocks);
      mb = n_mblocks - 1 - r / w;
      grp = (L % kXcds) * groups_per_xcd + (k / (w * n_mblocks)) * w + r % w;
      return;
    }
  }
  const int id = xcd_remap(L, total);
  mb = id % n_mblocks;
  grp = id / n_mblocks;
  if (heavy_first) mb = n_mblocks - 1 - mb;
}

// Work item of a varlen launch, whose groups differ in work (their
// sequences' lengths): contiguous group ranges per XCD would load the XCDs
// unevenly (1.56x the mean on the busiest XCD at 32 random lengths).  Here
// XCD x owns the K/V heads c = grp / group with c % 8 == x, so the sequences
// spread over all XCDs while the query heads of one K/V head share its tiles
// in one L2, and runs them one K/V head at a time (row blocks of the head's
// query heads interleaved, the last first when heavy_first).  The last
// n_kv % 8 K/V heads, if any, follow with their items spread over all XCDs.
// Returns false (no item assigned) unless total = n_kv * group * n_mblocks.
__device__ inline bool work_item_kv_rr(int L, int total, int n_mblocks, int group,
                                       bool heavy_first, int& mb, int& grp) {
  constexpr int kXcds = 8;
  const int per_kv = group * n_mblocks;   // items per K/V head
  if (per_kv <= 0 || total % per_kv != 0) return false;
  const int main_items = total / per_kv / kXcds * kXcds * per_kv;
  int c, r;
  if (L < main_items) {
    const int k = L / kXcds;
    c = (k / per_kv) * kXcds + L % kXcds;
    r = k % per_kv;
  } else {
    c = L / per_kv;   // main_items is a multiple of per_kv
    r = L % per_kv;
  }
  mb = r / group;
  if (heavy_first) mb = n_mblocks - 1 - mb;
  grp = c * group + r % group;
  return true;
}

// work_item span of the causal launches of the ping-pong forward and INT8
// kernels (and of the fp32 backward): 4 groups measured best on MI355X at
// B=4 H=32 S=4096 (1: 5-7% slower, all groups of an XCD: 1-3% slower).
constexpr int kCausalSpan = 4;
// The 16-bit backward kernels' span: each group streams 2 MiB of K / V (dQ)
// or Q / dO (dK/dV) per XCD at that shape, so four groups at a time
// overflowed the 4 MiB L2 (causal dQ + dK/dV read 1882 MB for 672 MB of
// inputs); two read 1333 MB for 0.9% more time, one 1367 MB for 5.4%.
constexpr int kBwdCausalSpan = 2;

__device__ inline u32x4 load16(const void* p) { return *reinterpret_cast<const u32x4*>(p); }
__device__ inline void store16(void* p, u32x4 v) { *reinterpret_cast<u32x4*>(p) = v; }

// gfx950 LDS transpose read (ds_read_b64_tr_b16).  Every lane names 8 bytes
// (4 consecutive 16-bit elements) of LDS; within each group of 16 lanes the
// reads form a 4 x 16 block whose row r is supplied by lanes 4r..4r+3, and
// lane i of the group receives column i of that block (rows 0..3).
typedef short s16x4v __attribute__((__vector_size__(4 * sizeof(short))));
__device__ inline u32x2 lds_read_tr16(const uint16_t* p) {
  typedef __attribute__((address_space(3))) s16x4v lds_s16x4;
  return __builtin_bit_cast(u32x2, __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)p));
}

// Raw buffer addressing.  A buffer resource covers [base, base + num_bytes);
// a raw buffer load whose byte offset lies at or beyond num_bytes returns zero
// without touching memory, so tiles that run past the end of a sequence need
// no branch.  Word 3 is the gfx9-family raw-buffer configuration (32-bit
// dwords, no swizzle).  The base and size must be wave-uniform: they live in
// scalar registers.
__device__ inline __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t num_bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)num_bytes,
                                           0x00020000);
}
__device__ inline u32x4 buf_load16(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
  return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, 0));
}
// The same with the non-temporal hint (cache policy NT): for data read once.
// A plain streaming read measured 7.0 TB/s with it against 6.3 TB/s without
// on MI355X.
__device__ inline u32x4 buf_load16_nt(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
  return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, 2));
}

// Byte extent of rows [row0, rows) of a strided 2-byte tensor whose rows hold
// `row_elems` elements at `row_stride` elements apart, clamped to 32 bits;
// zero when no row is left.
__device__ inline uint32_t rows_extent(int row0, int rows, int64_t row_stride, int row_elems) {
  if (row0 >= rows) return 0;
  const int64_t bytes = ((int64_t)(rows - 1 - row0) * row_stride + row_elems) * 2;
  return bytes > 0xffffffffll ? 0xffffffffu : (uint32_t)bytes;
}

// Buffer resource as four scalar words (gfx9 raw buffer: base, stride 0,
// num_records = bytes, word 3 = 32-bit dword format, no swizzle).
__device__ inline u32x4 make_rsrc_words(const void* base, uint32_t num_bytes) {
  const uint64_t a = reinterpret_cast<uint64_t>(base);
  u32x4 r;
  r[0] = __builtin_amdgcn_readfirstlane((uint32_t)a);
  r[1] = __builtin_amdgcn_readfirstlane((uint32_t)(a >> 32) & 0xffffu);
  r[2] = __builtin_amdgcn_readfirstlane(num_bytes);
  r[3] = 0x00020000u;
  return r;
}

// LDS byte address of a pointer into dynamic shared memory.
__device__ inline uint32_t lds_address(const void* p) {
  return (uint32_t)reinterpret_cast<uintptr_t>((const __attribute__((address_space(3))) uint8_t*)p);
}

// Raw buffer load of 16 bytes per lane straight into LDS: lane l's bytes land
// at LDS address lds + 16 l (lds wave-uniform, through M0).  Written as
// inline assembly so that the compiler does not treat every later LDS read as
// dependent on it and wait for all outstanding loads; the kernel waits for
// these loads itself (s_waitcnt vmcnt) before the barrier that publishes them.
// (The readfirstlane states the uniformity the "s" constraint needs: the
// compiler does not always prove it for a computed address.)
__device__ inline void buf_load16_lds(const u32x4& r, uint32_t lds, uint32_t voff) {
  asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dwordx4 %1, %2, 0 offen lds"
               :
               : "s"(__builtin_amdgcn_readfirstlane(lds)), "v"(voff), "s"(r)
               : "memory", "m0");
}

// The 4-byte form: lane l's dword lands at LDS address lds + 4 l.
__device__ inline void buf_load4_lds(const u32x4& r, uint32_t lds, uint32_t voff) {
  asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dword %1, %2, 0 offen lds"
               :
               : "s"(__builtin_amdgcn_readfirstlane(lds)), "v"(voff), "s"(r)
               : "memory", "m0");
}

// s_waitcnt immediate that waits until at most n vector-memory instructions
// of this wave are outstanding (lgkm and exp counts left unconstrained).
constexpr int vmcnt_imm(int n) { return 0x0f70 | (n & 15) | ((n >> 4) << 14); }

// ------------------------------------------------------------------ dropout
// Counter-based random bits: Philox4x32-10 (Salmon, Moraes, Dror and Shaw,
// "Parallel random numbers: as easy as 1, 2, 3", SC 2011; the Random123
// reference parameters).  One call maps a 128-bit counter and a 64-bit key to
// 128 random bits.
__device__ inline u32x4 philox4x32_10(u32x4 c, uint32_t k0, uint32_t k1) {
  constexpr uint32_t kM0 = 0xD2511F53u, kM1 = 0xCD9E8D57u;
  constexpr uint32_t kW0 = 0x9E3779B9u, kW1 = 0xBB67AE85u;
#pragma unroll
  for (int r = 0; r < 10; ++r) {
    if (r) {
      k0 += kW0;
      k1 += kW1;
    }
    const uint64_t p0 = (uint64_t)kM0 * c[0];
    const uint64_t p1 = (uint64_t)kM1 * c[2];
    c = u32x4{(uint32_t)(p1 >> 32) ^ c[1] ^ k0, (uint32_t)p1, (uint32_t)(p0 >> 32) ^ c[3] ^ k1,
              (uint32_t)p0};
  }
  return c;
}

// Dropout mask.  Element (batch b, query head h, query row i, key j; rows and
// keys local to the sequence) keeps its probability iff its 16-bit draw is at
// least t16 = round(p * 65536), and a kept probability is scaled by
// 65536 / (65536 - t16), the reciprocal of the keep probability (an unbiased
// mask).  The draws come 8 to a Philox call: call
// (2 (j / 16) + (j / 4) % 2, i, h, b) under key (seed_lo, seed_hi) covers the
// keys 16 (j / 16) + 4 s + {0, 1, 2, 3, 8, 9, 10, 11} (s = (j / 4) % 2) in the
// order of its eight 16-bit halves, word e / 2 bits 16 (e % 2).  That is the
// key order of one lane's half of a 16-key product step, so a kernel whose
// lanes hold one query row draws once per 16 keys.
struct DropoutCfg {
  int enabled;
  uint32_t seed_lo, seed_hi;
  int t16;          // keep iff draw >= t16 (0 .. 65536)
  float scale;      // 65536 / (65536 - t16)
};

// Draws for keys 16 G + 4 s + {0..3, 8..11} of one row (one call).
__device__ inline u32x4 dropout_draws(const DropoutCfg& d, int G, int s, int row, int head,
                                      int batch) {
  return philox4x32_10(u32x4{(uint32_t)(2 * G + s), (uint32_t)row, (uint32_t)head, (uint32_t)batch},
                       d.seed_lo, d.seed_hi);
}

// Half e (0..7) of a call's draws, as the multiplier of the probability.
__device__ inline float dropout_factor(const DropoutCfg& d, u32x4 r, int e) {
  const uint32_t w = r[e >> 1];
  const int v = (int)((e & 1) ? (w >> 16) : (w & 0xffffu));
  return v >= d.t16 ? d.scale : 0.f;
}

// The multiplier of one element (one call per element).
__device__ inline float dropout_factor_at(const DropoutCfg& d, int row, int key, int head,
                                          int batch) {
  const int w = key & 15;
  const u32x4 r = dropout_draws(d, key >> 4, (w >> 2) & 1, row, head, batch);
  return dropout_factor(d, r, (w & 3) | ((w >> 3) << 2));
}

}  // namespace fa
