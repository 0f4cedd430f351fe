// FlashAttention-2 backward for gfx950, fp16 / bf16 inputs, fp32 accumulation.
//
// Gradients of the forward in fa_prefill_kernel.h, following the reference's
// backward (/root/reference/flash_attn_triton/triton_kernel/attention_kernel.py:
// 536-566 `_attn_bwd_preprocess`, :569-668 `_attn_bwd_dkdv`, :671-776
// `_attn_bwd_dq`, :809-1054 `_attn_bwd`; varlen :107-272):
//   P  = exp(s - lse)        s = scale * q.k  -> ALiBi -> softcap -> mask
//   dV = P^T dO              dP = dO V^T       delta = rowsum(dO * O)
//   dS = P * (dP - delta) * softcap'          (softcap' = 1 - tanh^2, else 1)
//   dQ = scale * dS K        dK = scale * dS^T Q
// with the forward's natural-log LSE, so P is exactly the forward's
// probabilities (rows with no visible key have LSE = -inf and P = 0).  With
// dropout (multipliers F of fa_common.h's mask): dV = (F P)^T dO and
// dS = P (F dP - delta) -- the derivative of O = (F P) V, where the
// reference's kernels use F P (dP - delta) (attention_kernel.py:661, :763).
//
// Two kernels, no atomics, deterministic:
// * bwd_dq_kernel: a workgroup owns BM = 32*NW query rows of one (batch,
//   head); wave w owns 32 rows and keeps Q and dO of its rows in VGPRs.  Per
//   tile of BN keys: S^T = K Q^T and dP^T = V dO^T (A = K / V rows from LDS,
//   B = Q^T / dO^T from VGPRs), dS^T in registers, dQ^T += K^T dS^T (A = K^T
//   by the LDS transpose read).  The accumulator layouts put one query row in
//   each lane, so LSE and delta are per-lane scalars and dS^T is already the
//   B operand of the dQ^T product (the same key permutation as the forward's
//   P^T).  It also writes delta, computed from its dO and O rows.
// * dK / dV: a workgroup owns 128 keys of one (batch, KV head), 32 per key
//   group.  Per tile of query rows (of every query head of the GQA group, so
//   each dK / dV element has one writer): S = Q K^T, dP = dO V^T (A = Q / dO
//   rows from LDS), P and dS in registers with one key per lane, dV^T +=
//   dO^T P and dK^T += Q^T dS (A = dO^T / Q^T by the transpose read).  Up to
//   D = 128 each key group has two waves (bwd_dkdv_split_kernel,
//   fa_bwd_split.h); at D = 256 one wave per group runs two passes
//   (bwd_dkdv_kernel below).
// Every LDS tile is read both row-wise (16-byte reads of one row per lane)
// and transposed (ds_read_b64_tr_b16), so tiles are stored unpadded with an
// XOR swizzle of their 16-byte chunks (swz_off) that keeps both patterns free
// of bank conflicts.
#pragma once

#include <type_traits>

#include "fa_bwd.h"
#include "fa_common.h"

namespace fa {

// Element offset of 16-byte chunk c of row r in a swizzled tile whose rows
// hold D 16-bit elements.  Chunks are grouped into 256-byte lines (the width
// of the 64 LDS banks); within a line the chunk position is XORed with a
// function of the line.  Row reads (16 lanes, 16 consecutive rows, one chunk
// each) and transpose reads (4 consecutive rows x 4 consecutive chunks per 16
// lanes) both land on 16 distinct chunk positions.
template <int D>
__device__ inline int swz_off(int r, int c) {
  constexpr int CPR = D / 8;
  if constexpr (CPR >= 16) {
    const int line = r * (CPR / 16) + (c >> 4);
    const int s = ((r & 3) << 2) | ((r >> 2) & 3);
    return (line << 7) + (((c & 15) ^ s) << 3);
  } else if constexpr (CPR == 8) {
    const int line = r >> 1;
    const int s = ((line & 1) << 2) | ((line >> 1) & 3);
    return (line << 7) + (((((r & 1) << 3) | c) ^ s) << 3);
  } else {
    static_assert(CPR == 4, "head dim must be 32, 64, 128 or 256");
    const int line = r >> 2;
    return (line << 7) + (((((r & 3) << 2) | c) ^ (line & 3)) << 3);
  }
}

// A operand of a 32x32x16 product read transposed from a swizzled tile: the
// lane gets column (col0 + lane % 32) of rows 16cc + {4g .. 4g+3, 8+4g .. 8+4g+3}
// (g = lane / 32), the key order of the score accumulators.
template <int D>
__device__ inline u32x4 tr_operand(const uint16_t* tile, int lane, int cc, int col0) {
  const int g = lane >> 5, j = lane & 15;
  const int r = 16 * cc + 4 * g + (j >> 2);
  const int d = col0 + 16 * ((lane & 31) >> 4) + 4 * (j & 3);
  const u32x2 lo = lds_read_tr16(tile + swz_off<D>(r, d >> 3) + (d & 7));
  const u32x2 hi = lds_read_tr16(tile + swz_off<D>(r + 8, d >> 3) + (d & 7));
  return u32x4{lo[0], lo[1], hi[0], hi[1]};
}

// Per-score transform shared by both kernels: the recomputed probability and
// the softcap derivative.  `lse2` is the row's LSE in log2 units (the dQ
// kernel passes +inf for a row that sees no key, giving P = 0; the dK/dV
// kernel passes the row's -inf and masks every pair of such a row); `bias_v`
// is the pair's attn_bias value (read only by the BIAS instantiations).
template <bool GENERIC, bool BIAS = false>
__device__ inline float bwd_prob(const BwdParams& p, float s, float lse2, float slope, int qpos,
                                 int key, float bias_v, float& cap_grad) {
  cap_grad = 1.f;
  if (!GENERIC) return __builtin_amdgcn_exp2f(fmaf(s, p.scale_log2, -lse2));
  float x = s * p.scale;
  if (p.alibi != nullptr) x = fmaf(-slope, fabsf((float)(qpos - key)), x);
  if (BIAS) x += bias_v;
  if (p.softcap > 0.f) {
    // tanh(x / softcap) = 1 - 2 / (1 + e^(2x/softcap))
    const float e2 = __builtin_amdgcn_exp2f(x * p.softcap_k);
    const float th = 1.f - 2.f * __builtin_amdgcn_rcpf(1.f + e2);
    x = p.softcap * th;
    cap_grad = 1.f - th * th;
  }
  return __builtin_amdgcn_exp2f(fmaf(x, kLog2e, -lse2));
}

// Row base offsets of one (batch, head) for the dense or varlen layout.
__device__ inline int64_t row_base(const BwdParams& p, int64_t sb, int64_t ss, int64_t sh, int b,
                                   int head, int start) {
  return (p.cu_q != nullptr ? (int64_t)start * ss : (int64_t)b * sb) + (int64_t)head * sh;
}

// Inverse of swz_off: the logical (row, chunk) stored at chunk position pos of
// 256-byte line `line` (what an LDS-DMA lane writing that position must load).
template <int D>
__device__ inline void swz_inverse(int line, int pos, int& r, int& c) {
  constexpr int CPR = D / 8;
  if constexpr (CPR >= 16) {
    r = line / (CPR / 16);
    const int s = ((r & 3) << 2) | ((r >> 2) & 3);
    c = (pos ^ s) | ((line % (CPR / 16)) << 4);
  } else if constexpr (CPR == 8) {
    const int x = pos ^ (((line & 1) << 2) | ((line >> 1) & 3));
    r = 2 * line + (x >> 3);
    c = x & 7;
  } else {
    const int x = pos ^ (line & 3);
    r = 4 * line + (x >> 2);
    c = x & 3;
  }
}

// K and V tiles of BN keys stream through NS LDS stages filled by LDS-DMA
// buffer loads issued NS - 1 tiles ahead.
template <class T, int D, int NW, int BN, int NS>
struct BwdDqTile {
  static constexpr int BM = 32 * NW;
  static constexpr int NT = 64 * NW;
  static constexpr int TILEB = BN * D * 2;       // bytes of one K or V stage
  static constexpr int IPS = TILEB / 1024;       // 1-KiB DMA instructions per K (or V) stage
  static constexpr int IPW = 2 * IPS / NW;       // per wave: waves [0, NW/2) load K, the rest V
  // The prologue stages each wave's 32 Q and dO rows (then its O rows) in
  // LDS before the K / V stages take it over.
  static constexpr int ROWS_B = 64 * D;          // bytes of 32 rows
  static constexpr int LDS_BYTES = NS * 2 * TILEB > 2 * NW * ROWS_B ? NS * 2 * TILEB : 2 * NW * ROWS_B;
  static_assert(IPW * NW == 2 * IPS && IPW > 0, "K and V tiles must split evenly over the waves");
};

// VARLEN: cu_seqlens launch (an instantiation of its own, so that the dense
// kernel carries none of the varlen work-item code).  BIAS: the dense
// attn_bias and its gradient (instantiations of their own, so that the other
// generic kernels keep their registers).
template <class T, int D, int NW, int BN, int NS, bool GENERIC, int WPE, bool VARLEN,
          bool BIAS = false>
__global__ __launch_bounds__(NW * 64) __attribute__((amdgpu_waves_per_eu(WPE, WPE)))
void bwd_dq_kernel(const BwdParams p) {
  static_assert(!BIAS || (GENERIC && !VARLEN), "attn_bias: generic dense kernels only");
  using Tile = BwdDqTile<T, D, NW, BN, NS>;
  constexpr int BM = Tile::BM, TILEB = Tile::TILEB, IPW = Tile::IPW;
  constexpr int NKC = D / 16, NDB = D / 32, NKB = BN / 32, NCC = BN / 16;

  extern __shared__ __attribute__((aligned(16))) uint16_t smem[];
  uint8_t* const smem_b = reinterpret_cast<uint8_t*>(smem);

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int c32 = lane & 31;
  const int g = lane >> 5;

  // ------------------------------------------------------------ work item
  // Causal: late (longer) rows first.  Varlen: K/V heads round-robin over
  // the XCDs, as in the forward (ragged sequences load contiguous ranges
  // unevenly).
  int mb, id;
  if (!VARLEN ||
      !work_item_kv_rr(blockIdx.x, p.total_blocks, p.n_blocks, p.group, p.causal != 0, mb, id))
    work_item(blockIdx.x, p.total_blocks, p.n_blocks, p.causal != 0, kBwdCausalSpan, mb, id);
  const int hh = id % p.heads_q;
  const int b = id / p.heads_q;
  const int kvh = hh / p.group;

  int Sq = p.seqlen_q, Sk = p.seqlen_k, qs = 0, ks = 0;
  if (p.cu_q != nullptr) {
    qs = p.cu_q[b];
    ks = p.cu_k[b];
    Sq = p.cu_q[b + 1] - qs;
    Sk = p.cu_k[b + 1] - ks;
  }
  const int row0 = mb * BM;
  if (row0 >= Sq) return;
  const int row_last = min(row0 + BM, Sq) - 1;
  const int qi = row0 + w * 32 + c32;
  const bool row_valid = qi < Sq;
  const int qoff = (int)p.q_offset;
  const int qpos = qi + qoff;

  const int64_t lse_base = row_base(p, p.lse_sb, p.lse_ss, p.lse_sh, b, hh, qs);
  float slope = 0.f;
  if (GENERIC && p.alibi != nullptr) slope = p.alibi[(int64_t)b * p.alibi_sb + hh];

  const int wrow0 = row0 + w * 32;
  const int qpos_w_min = wrow0 + qoff;
  const int qpos_w_max = min(wrow0 + 31, row_last) + qoff;
  const int wl = p.window_left, wr = p.window_right;
  const bool causal = p.causal != 0;
  int key_hi = Sk - 1;
  if (causal) key_hi = min(key_hi, qpos);
  if (wr >= 0) key_hi = min(key_hi, qpos + wr);
  const int key_lo = wl >= 0 ? qpos - wl : -(1 << 30);

  int k_hi = Sk;
  if (causal) k_hi = min(k_hi, row_last + qoff + 1);
  if (wr >= 0) k_hi = min(k_hi, row_last + qoff + wr + 1);
  int k_lo = 0;
  if (wl >= 0) k_lo = max(0, row0 + qoff - wl);
  const int t_begin = k_lo / BN;
  const int t_end = k_hi > k_lo ? (k_hi + BN - 1) / BN : t_begin;
  const int J = t_end - t_begin;

  // ------------------------------------------------------------ Q, dO rows; delta
  // The wave's 32 rows of Q and dO, then of O, go global -> LDS as whole
  // rows (LDS-DMA, 1 KiB of consecutive rows per instruction, the K / V
  // tile layout) and come back in the MFMA operand layout.  Read straight
  // in that layout (16 bytes of 32 rows per instruction, each 128-byte line
  // touched by four instructions) the rows were fetched from HBM about twice
  // (measured on MI355X: 792 MB for 402 MB of Q, dO and O at B=4 H=32
  // S=4096 D=128).  Rows past the sequence read as zeros.
  u32x4 qreg[NKC], doreg[NKC];
  float dsum = 0.f;
  {
    constexpr int NI = D / 16;   // 1-KiB DMA instructions per 32 rows
    uint8_t* const st_a = smem_b + w * Tile::ROWS_B;
    uint8_t* const st_b = smem_b + (NW + w) * Tile::ROWS_B;
    int sr[NI], sc[NI];
#pragma unroll
    for (int i = 0; i < NI; ++i) swz_inverse<D>(4 * i + (lane >> 4), lane & 15, sr[i], sc[i]);
    auto stage = [&](const void* t, int64_t sb, int64_t ss, int64_t sh, uint8_t* st) {
      const uint16_t* rows = static_cast<const uint16_t*>(t) + row_base(p, sb, ss, sh, b, hh, qs) +
                             (int64_t)wrow0 * ss;
      const u32x4 rs = make_rsrc_words(rows, rows_extent(wrow0, Sq, ss, D));
      const uint32_t dst = lds_address(st);
#pragma unroll
      for (int i = 0; i < NI; ++i)
        buf_load16_lds(rs, dst + i * 1024, (uint32_t)sr[i] * (uint32_t)(ss * 2) + (uint32_t)sc[i] * 16);
    };
    auto read = [&](const uint8_t* st, u32x4* out) {
#pragma unroll
      for (int kc = 0; kc < NKC; ++kc)
        out[kc] = *reinterpret_cast<const u32x4*>(reinterpret_cast<const uint16_t*>(st) +
                                                  swz_off<D>(c32, 2 * kc + g));
    };
    stage(p.q, p.q_sb, p.q_ss, p.q_sh, st_a);
    stage(p.dout, p.do_sb, p.do_ss, p.do_sh, st_b);
    __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));
    read(st_a, qreg);
    read(st_b, doreg);
    // The Q reads have returned before the O rows overwrite their area.
    __builtin_amdgcn_s_waitcnt(0x0070);   // vmcnt(0) lgkmcnt(0)
    stage(p.o, p.o_sb, p.o_ss, p.o_sh, st_a);
    __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));
    u32x4 oreg[NKC];
    read(st_a, oreg);
#pragma unroll
    for (int kc = 0; kc < NKC; ++kc) {
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        dsum = fmaf(T::to_float((uint16_t)(oreg[kc][e] & 0xffffu)),
                    T::to_float((uint16_t)(doreg[kc][e] & 0xffffu)), dsum);
        dsum = fmaf(T::to_float((uint16_t)(oreg[kc][e] >> 16)),
                    T::to_float((uint16_t)(doreg[kc][e] >> 16)), dsum);
      }
    }
  }
  const float delta = halves_sum(dsum);
  // attn_bias of this lane's row, and its gradient row (dense layout only).
  const float* bias_row = nullptr;
  float* dbias_row = nullptr;
  if (BIAS && row_valid) {
    if (p.bias != nullptr)
      bias_row = p.bias + (int64_t)b * p.bias_sb + (int64_t)hh * p.bias_sh + (int64_t)qi * p.bias_sq;
    if (p.dbias != nullptr)
      dbias_row = p.dbias + (int64_t)b * p.dbias_sb + (int64_t)hh * p.dbias_sh +
                  (int64_t)qi * p.dbias_sq;
  }
  float lse2 = INFINITY;
  if (row_valid) {
    const float l = p.lse[lse_base + (int64_t)qi * p.lse_ss];
    if (l != -INFINITY) lse2 = l * kLog2e;
    if (g == 0) p.delta[lse_base + (int64_t)qi * p.lse_ss] = delta;
  }
  // Retire these loads before the DMA stream starts (the compiler does not
  // count the DMA instructions), and every wave's staging reads before the
  // K / V stages overwrite the staging areas.
  __builtin_amdgcn_s_waitcnt(0x0070);   // vmcnt(0) lgkmcnt(0)
  __builtin_amdgcn_s_barrier();

  // ------------------------------------------------------------ DMA stream
  // Waves [0, NW/2) copy K tiles, the others V tiles; lane l writes chunk
  // position l % 16 of line 4 i' + l / 16 (see swz_inverse).
  const bool load_k = w < NW / 2;
  const int j0 = (w % (NW / 2)) * IPW;
  const int64_t x_ss = load_k ? p.k_ss : p.v_ss;
  const uint16_t* xg = load_k ? static_cast<const uint16_t*>(p.k) + row_base(p, p.k_sb, p.k_ss, p.k_sh, b, kvh, ks)
                              : static_cast<const uint16_t*>(p.v) + row_base(p, p.v_sb, p.v_ss, p.v_sh, b, kvh, ks);
  uint32_t voff[IPW];
#pragma unroll
  for (int i = 0; i < IPW; ++i) {
    int r, c;
    swz_inverse<D>(4 * (j0 + i) + (lane >> 4), lane & 15, r, c);
    voff[i] = (uint32_t)r * (uint32_t)(x_ss * 2) + (uint32_t)c * 16;
  }
  const uint32_t x_lds = lds_address(smem_b) + (load_k ? 0 : NS * TILEB) + j0 * 1024;
  auto issue = [&](int it, int stage) {   // tile t_begin + it into stage it % NS; past J an empty load
    const bool live = it < J;
    const int n0 = (t_begin + (live ? it : 0)) * BN;
    const u32x4 rs = make_rsrc_words(xg + (int64_t)n0 * x_ss, live ? rows_extent(n0, Sk, x_ss, D) : 0u);
    const uint32_t dst = x_lds + stage * TILEB;
#pragma unroll
    for (int i = 0; i < IPW; ++i) buf_load16_lds(rs, dst + i * 1024, voff[i]);
  };

  auto wave_masks = [&](int t) {
    const int n0 = t * BN, n1 = n0 + BN;
    bool need = n1 > Sk;
    if (causal) need = need || n1 - 1 > qpos_w_min;
    if (wr >= 0) need = need || n1 - 1 > qpos_w_min + wr;
    if (wl >= 0) need = need || n0 < qpos_w_max - wl;
    return need;
  };

  f32x16 acc[NDB];
#pragma unroll
  for (int db = 0; db < NDB; ++db) acc[db] = f32x16{};

  constexpr bool STAGE = D <= 128;

  // One tile: operands staged ahead of their products (all A operands of a
  // 32-key block of S^T / dP^T first; the transposed K reads of dQ^T before
  // the elementwise work, which hides their latency).
  auto tile_math = [&](int t, int stage, bool masked) {
    const uint16_t* Ks = reinterpret_cast<const uint16_t*>(smem_b + stage * TILEB);
    const uint16_t* Vs = reinterpret_cast<const uint16_t*>(smem_b + (NS + stage) * TILEB);
    f32x16 s[NKB], dp[NKB];
#pragma unroll
    for (int kb = 0; kb < NKB; ++kb) {
      s[kb] = f32x16{};
      dp[kb] = f32x16{};
      if constexpr (STAGE) {
        u32x4 ka[NKC], va[NKC];
#pragma unroll
        for (int kc = 0; kc < NKC; ++kc) {
          const int off = swz_off<D>(kb * 32 + c32, 2 * kc + g);
          ka[kc] = load16(Ks + off);
          va[kc] = load16(Vs + off);
        }
#pragma unroll
        for (int kc = 0; kc < NKC; ++kc) {
          s[kb] = T::mfma32(ka[kc], qreg[kc], s[kb]);
          dp[kb] = T::mfma32(va[kc], doreg[kc], dp[kb]);
        }
        // Half the reads up front, then one read behind every product.
        __builtin_amdgcn_sched_group_barrier(0x100, NKC, 0);   // LDS reads
#pragma unroll
        for (int i = 0; i < NKC; ++i) {
          __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);   // MFMA
          __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);   // LDS read
        }
        __builtin_amdgcn_sched_group_barrier(0x008, NKC, 0);
        __builtin_amdgcn_sched_barrier(0);
      } else {
#pragma unroll
        for (int kc = 0; kc < NKC; ++kc) {
          const int off = swz_off<D>(kb * 32 + c32, 2 * kc + g);
          s[kb] = T::mfma32(load16(Ks + off), qreg[kc], s[kb]);
          dp[kb] = T::mfma32(load16(Vs + off), doreg[kc], dp[kb]);
        }
      }
    }
    constexpr int NTA = STAGE ? NCC * NDB : 1;
    u32x4 ta[NTA];
    if constexpr (STAGE) {
#pragma unroll
      for (int cc = 0; cc < NCC; ++cc)
#pragma unroll
        for (int db = 0; db < NDB; ++db) ta[cc * NDB + db] = tr_operand<D>(Ks, lane, cc, db * 32);
      __builtin_amdgcn_sched_barrier(0);
    }
    const int n0 = t * BN;
    const bool drop = GENERIC && p.drop.enabled;
    u32x4 dsb[NCC];
    auto elementwise = [&](auto masked_c) {
      constexpr bool MASKED = decltype(masked_c)::value;
#pragma unroll
      for (int cc = 0; cc < NCC; ++cc) {
        const int kb = cc >> 1, o8 = (cc & 1) * 8;
        u32x4 rnd = {0, 0, 0, 0};
        if (drop) rnd = dropout_draws(p.drop, (n0 >> 4) + cc, g, qi, hh, b);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          float ds[2];
#pragma unroll
          for (int u = 0; u < 2; ++u) {
            const int v = o8 + 2 * j + u;
            const int key = n0 + kb * 32 + 8 * (v >> 2) + 4 * g + (v & 3);
            float cg;
            const float bv =
                BIAS && bias_row != nullptr && key < Sk ? bias_row[(int64_t)key * p.bias_sk] : 0.f;
            float pr = bwd_prob<GENERIC, BIAS>(p, s[kb][v], lse2, slope, qpos, key, bv, cg);
            if (MASKED) pr = (key < key_lo || key > key_hi) ? 0.f : pr;
            const float dpv = drop ? dp[kb][v] * dropout_factor(p.drop, rnd, 2 * j + u) : dp[kb][v];
            ds[u] = pr * (dpv - delta) * cg;
            // dS is the gradient of the biased score; broadcast dims of the
            // bias share an element, so the sum is accumulated atomically.
            if (BIAS && dbias_row != nullptr && key < Sk && ds[u] != 0.f)
              atomicAdd(dbias_row + (int64_t)key * p.dbias_sk, ds[u]);
          }
          dsb[cc][j] = T::pack2(ds[0], ds[1]);
        }
      }
    };
    if (masked)
      elementwise(std::true_type{});
    else
      elementwise(std::false_type{});
#pragma unroll
    for (int cc = 0; cc < NCC; ++cc) {
#pragma unroll
      for (int db = 0; db < NDB; ++db) {
        if constexpr (STAGE)
          acc[db] = T::mfma32(ta[cc * NDB + db], dsb[cc], acc[db]);
        else
          acc[db] = T::mfma32(tr_operand<D>(Ks, lane, cc, db * 32), dsb[cc], acc[db]);
      }
    }
  };

  // ------------------------------------------------------------ main loop
  // Tiles it .. it + NS - 2 are in flight at the top of iteration it; the
  // barrier after the wait publishes tile it and retires the reads of tile
  // it - 1, whose stage the next DMA refills.  The body is straight-line (a
  // wave whose rows see no key of a tile computes it masked).  With staged
  // operands it is unrolled by the stage count, so the stage bases are
  // immediate offsets of the reads.
#pragma unroll
  for (int s = 0; s < NS - 1; ++s) issue(s, s);
  auto iteration = [&](int it, int stage) {
    __builtin_amdgcn_s_waitcnt(vmcnt_imm((NS - 2) * IPW));
    __builtin_amdgcn_sched_barrier(0);
    asm volatile("s_barrier" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);
    issue(it + NS - 1, (stage + NS - 1) % NS);
    tile_math(t_begin + it, stage, wave_masks(t_begin + it));
  };
  if constexpr (STAGE) {
    static_assert(NS == 3, "the main loop is unrolled for three stages");
    int it = 0;
    for (; it + NS <= J; it += NS) {
      iteration(it, 0);
      iteration(it + 1, 1);
      iteration(it + 2, 2);
    }
    if (it < J) iteration(it, 0);
    if (it + 1 < J) iteration(it + 1, 1);
  } else {
    for (int it = 0; it < J; ++it) iteration(it, it % NS);
  }
  __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));

  // ------------------------------------------------------------ dQ = scale * acc
  if (!row_valid) return;
  uint16_t* dqrow = static_cast<uint16_t*>(p.dq) + row_base(p, p.dq_sb, p.dq_ss, p.dq_sh, b, hh, qs) +
                    (int64_t)qi * p.dq_ss;
#pragma unroll
  for (int db = 0; db < NDB; ++db) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int d = db * 32 + r * 8 + g * 4;
      u32x2 val;
      val[0] = T::pack2(acc[db][4 * r] * p.scale, acc[db][4 * r + 1] * p.scale);
      val[1] = T::pack2(acc[db][4 * r + 2] * p.scale, acc[db][4 * r + 3] * p.scale);
      *reinterpret_cast<u32x2*>(dqrow + d) = val;
    }
  }
}

// Whole-row stores of 32 rows held in the accumulator layout (lane (c32, g):
// dims 32 db + 8 (v / 4) + 4 g + v % 4 of row c32), times `scale`, packed to
// 16 bits: the values go through `st` (32 rows of 2 D + 16 bytes, the pad
// spreading a write's rows over the banks) and come back as 16-byte chunks of
// whole rows, so each store instruction writes D / 8 lanes' worth of every
// row it touches instead of 16 bytes of 32 rows.  (Stored directly, the dK /
// dV rows of a non-causal launch, all finishing at once, reached HBM as
// partial lines: 3.5x the bytes.)  Rows [0, rows_ok) are stored.
template <class T, int D>
__device__ inline void store_rows_staged(const f32x16* acc, float scale, uint8_t* st, int c32,
                                         int g, int lane, uint16_t* row0, int64_t ss,
                                         int rows_ok) {
  constexpr int NDB = D / 32, PITCH = 2 * D + 16, CPR = D / 8, RPI = 64 / CPR;
  uint8_t* const wr = st + c32 * PITCH + 8 * g;
#pragma unroll
  for (int db = 0; db < NDB; ++db) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      u32x2 val;
      val[0] = T::pack2(acc[db][4 * r] * scale, acc[db][4 * r + 1] * scale);
      val[1] = T::pack2(acc[db][4 * r + 2] * scale, acc[db][4 * r + 3] * scale);
      *reinterpret_cast<u32x2*>(wr + (db * 4 + r) * 16) = val;
    }
  }
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  const int rl = lane / CPR, cl = lane % CPR;
  const uint8_t* const rd = st + rl * PITCH + cl * 16;
#pragma unroll
  for (int i = 0; i < 32 / RPI; ++i) {
    const int r = RPI * i + rl;
    const u32x4 x = *reinterpret_cast<const u32x4*>(rd + i * RPI * PITCH);
    if (r < rows_ok) store16(row0 + (int64_t)r * ss + cl * 8, x);
  }
}

// Q and dO tiles of BM rows stream through NS LDS stages, filled by LDS-DMA
// buffer loads (no VGPR staging) issued NS - 1 tiles ahead; the LSE and delta
// of the tile's rows ride along (one 4-byte-per-lane DMA each).
template <class T, int D, int NW, int BM, int NS>
struct BwdDkvTile {
  static constexpr int BN = 32 * NW;
  static constexpr int NT = 64 * NW;
  static constexpr int TILEB = BM * D * 2;       // bytes of one Q or dO stage
  static constexpr int IPS = TILEB / 1024;       // 1-KiB DMA instructions per Q (or dO) stage
  static constexpr int IPW = 2 * IPS / NW;       // per wave: waves [0, NW/2) load Q, the rest dO
  static constexpr int LPS = IPW + 1;            // DMA instructions per wave per stage (+ LSE or delta)
  static constexpr int FB = 256;                 // bytes of one LSE / delta stage (64 lanes x 4 B)
  static constexpr int LDS_BYTES = NS * (2 * TILEB + 2 * FB);   // + 4 B per head of the group (ALiBi)
  static_assert(IPW * NW == 2 * IPS && IPW > 0, "Q and dO tiles must split evenly over the waves");
  static_assert(BM <= 64 && BM % 32 == 0, "one DMA lane per row for LSE / delta");
};

// dK / dV at D = 256, one wave per key group.  PASS 0 would accumulate dK and
// dV together; at D = 256 the two accumulators do not fit beside K and V, so
// the launcher runs PASS 1 (dV only) and PASS 2 (dK only), recomputing S in
// each.
template <class T, int D, int NW, int BM, int NS, bool GENERIC, int WPE, int PASS, bool VARLEN,
          bool BIAS = false>
__global__ __launch_bounds__(NW * 64) __attribute__((amdgpu_waves_per_eu(WPE, WPE)))
void bwd_dkdv_kernel(const BwdParams p) {
  static_assert(!BIAS || (GENERIC && !VARLEN), "attn_bias: generic dense kernels only");
  constexpr bool DO_DV = PASS != 2, DO_DK = PASS != 1;
  using Tile = BwdDkvTile<T, D, NW, BM, NS>;
  constexpr int BN = Tile::BN, TILEB = Tile::TILEB, IPW = Tile::IPW, LPS = Tile::LPS;
  constexpr int FB = Tile::FB;
  constexpr int NKC = D / 16, NDB = D / 32, NRB = BM / 32, NCC = BM / 16;

  extern __shared__ __attribute__((aligned(16))) uint16_t smem[];
  uint8_t* const smem_b = reinterpret_cast<uint8_t*>(smem);
  float* const slopes_lds = reinterpret_cast<float*>(smem_b + Tile::LDS_BYTES);

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int c32 = lane & 31;
  const int g = lane >> 5;

  // ------------------------------------------------------------ work item
  // Causal: early key blocks (seen by the most rows) first.  Varlen: K/V
  // heads round-robin over the XCDs.
  int nb, id;
  if (!VARLEN ||
      !work_item_kv_rr(blockIdx.x, p.total_blocks, p.n_blocks, 1, p.causal != 0, nb, id))
    work_item(blockIdx.x, p.total_blocks, p.n_blocks, p.causal != 0, kBwdCausalSpan, nb, id);
  if (p.causal) nb = p.n_blocks - 1 - nb;
  const int kvh = id % p.heads_k;
  const int b = id / p.heads_k;

  int Sq = p.seqlen_q, Sk = p.seqlen_k, qs = 0, ks = 0;
  if (p.cu_q != nullptr) {
    qs = p.cu_q[b];
    ks = p.cu_k[b];
    Sq = p.cu_q[b + 1] - qs;
    Sk = p.cu_k[b + 1] - ks;
  }
  const int key0 = nb * BN;
  if (key0 >= Sk) return;
  const int key_last = min(key0 + BN, Sk) - 1;
  const int kj = key0 + w * 32 + c32;
  const bool key_valid = kj < Sk;
  const int qoff = (int)p.q_offset;
  const int wl = p.window_left, wr = p.window_right;
  const bool causal = p.causal != 0;

  // K and V rows of this lane's key: B operands of S = Q K^T and dP = dO V^T.
  u32x4 kreg[NKC], vreg[NKC];
  {
    const uint16_t* krow = static_cast<const uint16_t*>(p.k) +
                           row_base(p, p.k_sb, p.k_ss, p.k_sh, b, kvh, ks) + (int64_t)kj * p.k_ss;
    const uint16_t* vrow = static_cast<const uint16_t*>(p.v) +
                           row_base(p, p.v_sb, p.v_ss, p.v_sh, b, kvh, ks) + (int64_t)kj * p.v_ss;
#pragma unroll
    for (int kc = 0; kc < NKC; ++kc) {
      const u32x4 z = {0, 0, 0, 0};
      kreg[kc] = key_valid ? load16(krow + kc * 16 + g * 8) : z;
      vreg[kc] = key_valid && DO_DK ? load16(vrow + kc * 16 + g * 8) : z;
    }
    // ALiBi slopes of the group's query heads go to LDS now, so that the main
    // loop issues no vector-memory load besides the DMA stream it counts.
    if (GENERIC && p.alibi != nullptr) {
      for (int gi = tid; gi < p.group; gi += NW * 64)
        slopes_lds[gi] = p.alibi[(int64_t)b * p.alibi_sb + kvh * p.group + gi];
    }
    // Retire these loads before the DMA stream starts: the compiler does not
    // count the DMA instructions and would otherwise wait for all of them at
    // the first use of kreg.
    __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));
  }

  // attn_bias column of this lane's key (dense layout only); the row and
  // query head are added per score.
  const float* bias_col = nullptr;
  if (BIAS && key_valid && p.bias != nullptr)
    bias_col = p.bias + (int64_t)b * p.bias_sb + (int64_t)kj * p.bias_sk;

  // Query rows i that see a key of this block: [q_lo, q_hi).
  int q_lo = 0, q_hi = Sq;
  if (causal) q_lo = max(q_lo, key0 - qoff);
  if (wr >= 0) q_lo = max(q_lo, key0 - qoff - wr);
  if (wl >= 0) q_hi = min(q_hi, key_last - qoff + wl + 1);
  const int m_begin = q_lo / BM;
  const int m_end = q_hi > q_lo ? (q_hi + BM - 1) / BM : m_begin;
  const int NM = m_end - m_begin;
  const int J = NM * p.group;

  // This wave's keys [wk0, wk1] and the tiles it must mask.
  const int wk0 = key0 + w * 32;
  const int wk1 = min(wk0 + 31, Sk - 1);
  auto wave_masks = [&](int m0) {
    const int p0 = m0 + qoff, p1 = m0 + BM - 1 + qoff;
    bool need = false;
    if (causal) need = need || p0 < wk1;
    if (wr >= 0) need = need || p0 + wr < wk1;
    if (wl >= 0) need = need || p1 - wl > wk0;
    return need;
  };
  // Work item it is (query head kvh * group + it / NM, m-block m_begin + it % NM).
  // The DMA stream and the products each visit the items in order, so each
  // side keeps a running (m-block, head) pair instead of dividing per tile.
  int ld_m = m_begin;               // m-block of the next tile to load
  int mm_m = m_begin, mm_h = 0;     // m-block and head-in-group of the next tile to compute

  // ------------------------------------------------------------ DMA stream
  // Waves [0, NW/2) copy Q tiles, the others dO tiles; each wave writes
  // IPW consecutive KiB (four 256-byte lines per instruction) of a stage.
  // Lane l writes chunk position l % 16 of line 4 i' + l / 16 and so loads
  // the logical (row, chunk) the swizzle puts there.
  const bool load_q = w < NW / 2;
  const int j0 = (w % (NW / 2)) * IPW;
  const int64_t x_ss = load_q ? p.q_ss : p.do_ss;
  uint32_t voff[IPW];
#pragma unroll
  for (int i = 0; i < IPW; ++i) {
    int r, c;
    swz_inverse<D>(4 * (j0 + i) + (lane >> 4), lane & 15, r, c);
    voff[i] = (uint32_t)r * (uint32_t)(x_ss * 2) + (uint32_t)c * 16;
  }
  const uint32_t f_voff = (uint32_t)lane * (uint32_t)(p.lse_ss * 4);
  const uint32_t x_lds = lds_address(smem_b) + (load_q ? 0 : NS * TILEB) + j0 * 1024;
  const uint32_t f_lds = lds_address(smem_b) + 2 * NS * TILEB + (w & 1) * NS * FB;
  // Running DMA sources: the next tile's first Q / dO row and LSE / delta
  // entry, and the byte extents from there to the end of the head's rows.
  // A step moves one m-block down; after the last m-block of a head the
  // pointers move to the first m-block of the next head.  Every live tile has
  // m0 < q_hi <= Sq, so its extents are positive.
  const int64_t x_sh = load_q ? p.q_sh : p.do_sh;
  const uint16_t* x_run =
      (load_q ? static_cast<const uint16_t*>(p.q) + row_base(p, p.q_sb, p.q_ss, p.q_sh, b, kvh * p.group, qs)
              : static_cast<const uint16_t*>(p.dout) +
                    row_base(p, p.do_sb, p.do_ss, p.do_sh, b, kvh * p.group, qs)) +
      (int64_t)m_begin * BM * x_ss;
  const float* f_run = ((w & 1) ? p.delta : p.lse) +
                       row_base(p, p.lse_sb, p.lse_ss, p.lse_sh, b, kvh * p.group, qs) +
                       (int64_t)m_begin * BM * p.lse_ss;
  const int64_t x_mstep = (int64_t)BM * x_ss, f_mstep = (int64_t)BM * p.lse_ss;
  const int64_t x_hstep = x_sh - (int64_t)(NM - 1) * x_mstep;
  const int64_t f_hstep = p.lse_sh - (int64_t)(NM - 1) * f_mstep;
  const int64_t x_ext0 = ((int64_t)(Sq - 1 - m_begin * BM) * x_ss + D) * 2;
  const int64_t f_ext0 = ((int64_t)(Sq - 1 - m_begin * BM) * p.lse_ss + 1) * 4;
  int64_t x_ext = x_ext0, f_ext = f_ext0;
  int ld_left = J;                  // live tiles not yet loaded
  auto clamp32 = [](int64_t v) { return v > 0xffffffffll ? 0xffffffffu : (uint32_t)v; };
  auto issue = [&](int stage) {     // the next tile into `stage`; past J an empty load
    const bool live = ld_left > 0;
    const u32x4 rs = make_rsrc_words(x_run, live ? clamp32(x_ext) : 0u);
    const uint32_t dst = x_lds + stage * TILEB;
#pragma unroll
    for (int i = 0; i < IPW; ++i) buf_load16_lds(rs, dst + i * 1024, voff[i]);
    buf_load4_lds(make_rsrc_words(f_run, live ? clamp32(f_ext) : 0u), f_lds + stage * FB, f_voff);
    --ld_left;
    if (++ld_m == m_end) {
      ld_m = m_begin;
      x_run += x_hstep;
      f_run += f_hstep;
      x_ext = x_ext0;
      f_ext = f_ext0;
    } else {
      x_run += x_mstep;
      f_run += f_mstep;
      x_ext -= 2 * x_mstep;
      f_ext -= 4 * f_mstep;
    }
  };

  f32x16 dk[NDB], dv[NDB];
#pragma unroll
  for (int db = 0; db < NDB; ++db) {
    dk[db] = f32x16{};
    dv[db] = f32x16{};
  }

  // One tile of BM query rows.  At D = 256 staged operand arrays would not
  // fit beside the accumulators, so the products read their A operands
  // straight from LDS.
  auto tile_math = [&](int stage, bool masked) {
    const uint16_t* Qs = reinterpret_cast<const uint16_t*>(smem_b + stage * TILEB);
    const uint16_t* Ds = reinterpret_cast<const uint16_t*>(smem_b + (NS + stage) * TILEB);
    const float* Ls = reinterpret_cast<const float*>(smem_b + 2 * NS * TILEB + stage * FB);
    const float* Es = reinterpret_cast<const float*>(smem_b + 2 * NS * TILEB + (NS + stage) * FB);
    const int hq = kvh * p.group + mm_h, m0 = mm_m * BM;
    float slope = 0.f;
    if (GENERIC && p.alibi != nullptr) slope = slopes_lds[mm_h];
    f32x16 s[NRB], dp[NRB];
#pragma unroll
    for (int rb = 0; rb < NRB; ++rb) {
      s[rb] = f32x16{};
      dp[rb] = f32x16{};
#pragma unroll
      for (int kc = 0; kc < NKC; ++kc) {
        const int off = swz_off<D>(rb * 32 + c32, 2 * kc + g);
        s[rb] = T::mfma32(load16(Qs + off), kreg[kc], s[rb]);
        if (DO_DK) dp[rb] = T::mfma32(load16(Ds + off), vreg[kc], dp[rb]);
      }
    }
    u32x4 pb[NCC], dsb[NCC];
    auto elementwise = [&](auto masked_c) {
      constexpr bool MASKED = decltype(masked_c)::value;
#pragma unroll
      for (int cc = 0; cc < NCC; ++cc) {
        const int rb = cc >> 1, o8 = (cc & 1) * 8;
        // Slots o8 .. o8+7 hold rows 16cc + 4g + {0..3} and 16cc + 8 + 4g + {0..3}.
        const int r0 = 16 * cc + 4 * g;
        const f32x4 l0 = *reinterpret_cast<const f32x4*>(Ls + r0);
        const f32x4 l1 = *reinterpret_cast<const f32x4*>(Ls + r0 + 8);
        const f32x4 e0 = *reinterpret_cast<const f32x4*>(Es + r0);
        const f32x4 e1 = *reinterpret_cast<const f32x4*>(Es + r0 + 8);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          float pv[2], ds[2];
#pragma unroll
          for (int u = 0; u < 2; ++u) {
            const int v = o8 + 2 * j + u;          // accumulator slot
            const int rr = 2 * j + u;              // rows r0 + rr%4 (+8 for rr >= 4)
            const float lse = rr < 4 ? l0[rr] : l1[rr - 4];
            const float dl = rr < 4 ? e0[rr] : e1[rr - 4];
            // Rows with no visible key (LSE -inf, so exp2 gives +inf here)
            // only occur in tiles that take the mask, which selects P = 0 for
            // every pair of such a row: an unmasked tile's rows all see every
            // key of this wave.  Rows past the sequence read LSE = delta = 0
            // next to zero Q / dO rows and contribute nothing.
            const float lse2 = lse * kLog2e;
            const int row = m0 + r0 + (rr & 3) + (rr >= 4 ? 8 : 0);
            const int qpos = row + qoff;
            float cg;
            const float bv = BIAS && bias_col != nullptr && row < Sq
                                 ? bias_col[(int64_t)hq * p.bias_sh + (int64_t)row * p.bias_sq]
                                 : 0.f;
            float pr = bwd_prob<GENERIC, BIAS>(p, s[rb][v], lse2, slope, qpos, kj, bv, cg);
            if (MASKED) {
              bool vis = true;
              if (causal) vis = vis && kj <= qpos;
              if (wr >= 0) vis = vis && kj <= qpos + wr;
              if (wl >= 0) vis = vis && kj >= qpos - wl;
              pr = vis ? pr : 0.f;
            }
            float dpv = dp[rb][v];
            pv[u] = pr;
            if (GENERIC && p.drop.enabled) {
              const float f = dropout_factor_at(p.drop, row, kj, hq, b);
              pv[u] = pr * f;
              dpv *= f;
            }
            ds[u] = pr * (dpv - dl) * cg;
          }
          pb[cc][j] = T::pack2(pv[0], pv[1]);
          dsb[cc][j] = T::pack2(ds[0], ds[1]);
        }
      }
    };
    if (masked)
      elementwise(std::true_type{});
    else
      elementwise(std::false_type{});
#pragma unroll
    for (int cc = 0; cc < NCC; ++cc) {
#pragma unroll
      for (int db = 0; db < NDB; ++db) {
        if (DO_DV) dv[db] = T::mfma32(tr_operand<D>(Ds, lane, cc, db * 32), pb[cc], dv[db]);
        if (DO_DK) dk[db] = T::mfma32(tr_operand<D>(Qs, lane, cc, db * 32), dsb[cc], dk[db]);
      }
    }
  };

  // ------------------------------------------------------------ main loop
  // At the top of iteration it this wave has tiles it .. it + NS - 2 in
  // flight; once at most NS - 2 tiles remain, tile it has landed, and the
  // barrier publishes every wave's share of it.  The barrier also retires
  // the reads of tile it - 1, whose stage the next DMA refills.
#pragma unroll
  for (int s = 0; s < NS - 1; ++s) issue(s);
  // Straight-line body: a tile that holds no visible (row, key) pair for
  // this wave is computed anyway with the mask (its P is all zero).  A
  // branch around it would make the dK / dV accumulators a join value that
  // the compiler copies between register files on every iteration.
  auto iteration = [&](int stage) {   // the next tile, held in `stage`
    __builtin_amdgcn_s_waitcnt(vmcnt_imm((NS - 2) * LPS));
    __builtin_amdgcn_sched_barrier(0);
    asm volatile("s_barrier" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);
    issue((stage + NS - 1) % NS);
    tile_math(stage, wave_masks(mm_m * BM));
    if (++mm_m == m_end) {
      mm_m = m_begin;
      ++mm_h;
    }
  };
  for (int it = 0; it < J; ++it) iteration(it % NS);
  // No DMA may still be writing LDS when the workgroup retires.
  __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));

  // ------------------------------------------------------------ dK = scale * dK^T, dV
  // Every wave's reads of the last tile are done once all waves pass the
  // barrier: the stages then hold each wave's 32 rows of staging.
  static_assert(4 * 32 * (2 * D + 16) <= Tile::LDS_BYTES, "output staging must fit the stages");
  __syncthreads();
  uint8_t* const st = smem_b + w * 32 * (2 * D + 16);
  const int rows_ok = Sk - wk0;
  if (DO_DK)
    store_rows_staged<T, D>(dk, p.scale, st, c32, g, lane,
                            static_cast<uint16_t*>(p.dk) +
                                row_base(p, p.dk_sb, p.dk_ss, p.dk_sh, b, kvh, ks) +
                                (int64_t)wk0 * p.dk_ss,
                            p.dk_ss, rows_ok);
  if (DO_DV)
    store_rows_staged<T, D>(dv, 1.f, st, c32, g, lane,
                            static_cast<uint16_t*>(p.dv) +
                                row_base(p, p.dv_sb, p.dv_ss, p.dv_sh, b, kvh, ks) +
                                (int64_t)wk0 * p.dv_ss,
                            p.dv_ss, rows_ok);
}

}  // namespace fa
