// FlashAttention-2 prefill forward for gfx950 (dense, cross and varlen), fp16 / bf16.
//
// Same semantics as fwd_kernel (fa_fwd_kernel.h), which it replaces for
// prefill at head dims that are multiples of 32; the behaviour follows the
// reference's dense and varlen forward kernels
// (/root/reference/flash_attn_triton/triton_kernel/attention_kernel.py:424-533,
// :275-372, :27-104).  What differs is the schedule:
//
// * K and V tiles are read with raw buffer loads whose resource ends at the
//   last valid key row of the (batch, head) slab: rows past the sequence come
//   back as zeros, so the loads carry no branch and no 64-bit address math.
//   Every thread's byte offsets are computed once; per tile only the scalar
//   base of the resource moves.
// * fp16 row sums are taken from the packed P operand with v_dot2 against
//   (1, 1): numerator (P V) and denominator (sum P) see the same rounded P,
//   at half the adds.  bf16 sums the fp32 P (its rounding is 8x coarser).
// * The running max is raised lazily: a row's max is only moved when a tile
//   exceeds it by more than kRescaleSlack (log2 units).  Until then
//   exp2(s - m) stays below 2^kRescaleSlack, which fp16/bf16 P and the fp32
//   accumulators hold exactly as well, and the whole-wave O^T rescale
//   (D/2 multiplies per lane) is skipped for the tile.  The final result is
//   normalized by the same sum, so it does not depend on when m moved.
//
// Layout per workgroup (NW waves, BM = 32*NW query rows, BN keys per tile):
//   S^T = K Q^T on v_mfma_f32_32x32x16 (A = K rows from LDS, B = Q^T in VGPRs),
//   O^T += V^T P^T (A = V^T gathered from the row-major V tile with the gfx950
//   LDS transpose read ds_read_b64_tr_b16, B = P^T from the score
//   accumulators), K/V double-buffered in LDS, one barrier per tile.
#pragma once

#include "fa_fwd_kernel.h"

namespace fa {

constexpr float kRescaleSlack = 8.0f;

template <int D, int NW, int BN>
struct PrefillTile {
  static constexpr int BM = NW * 32;
  static constexpr int NT = NW * 64;
  // Row pitches in LDS (elements).  K rows carry 16 B of padding: the 16 rows
  // a ds_read_b128 quarter-wave touches start on distinct 16-byte bank groups.
  // V rows carry 64 B: the four rows one transpose read covers per 16-lane
  // group (and the two column halves of a 32-lane group) land on distinct
  // banks.
  static constexpr int KSTR = D + 8;
  static constexpr int VSTR = D + 32;
  static constexpr int KTILE = BN * KSTR;
  static constexpr int VTILE = BN * VSTR;
  static constexpr int LDS_BYTES = 2 * (KTILE + VTILE) * 2;
  static constexpr int CPR = D / 8;                 // 16-byte chunks per row
  static constexpr int CHUNKS = BN * CPR;          // 16-byte chunks per tile (K and V each)
  static constexpr int KPT = (CHUNKS + NT - 1) / NT; // chunks per thread per tile
  static_assert(D % 32 == 0, "head dim must be a multiple of 32");
  static_assert(BN % 32 == 0, "tile must hold whole 32-key MFMA blocks");
  static_assert(CHUNKS % NT == 0 || CHUNKS < NT, "tiles must split evenly over threads");
};

// BIAS: the additive fp32 attn_bias is read in the score epilogue (GENERIC
// only).  It is a separate instantiation because its per-score loads raise
// register pressure past the budget of the 3-waves-per-SIMD tiles.
template <class T, int D, int NW, int BN, bool GENERIC, int WPE, bool BIAS = false>
__global__ __launch_bounds__(NW * 64) __attribute__((amdgpu_waves_per_eu(WPE, WPE)))
void prefill_kernel(const FwdParams p) {
  static_assert(GENERIC || !BIAS, "the bias is applied by the generic epilogue");
  using Tile = PrefillTile<D, NW, BN>;
  constexpr int BM = Tile::BM;
  constexpr int NT = Tile::NT;
  constexpr int KSTR = Tile::KSTR;
  constexpr int VSTR = Tile::VSTR;
  constexpr int KTILE = Tile::KTILE;
  constexpr int VTILE = Tile::VTILE;
  constexpr int CPR = Tile::CPR;
  constexpr int KPT = Tile::KPT;
  constexpr int CHUNKS = Tile::CHUNKS;
  constexpr int NKC = D / 16;      // 16-dim MFMA k-steps for S^T
  constexpr int NDB = D / 32;      // 32-dim output blocks of O^T
  constexpr int NKB = BN / 32;     // 32-key blocks per tile
  constexpr int NCC = BN / 16;     // 16-key k-steps for O^T

  extern __shared__ __attribute__((aligned(16))) uint16_t smem[];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);   // wave-uniform
  const int c32 = lane & 31;
  const int g = lane >> 5;

  // ------------------------------------------------------------ work item
  // Varlen: K/V heads dealt round-robin over the XCDs (ragged sequences would
  // load contiguous ranges unevenly), each K/V head's row blocks back to
  // back.  Otherwise span 1 (a group's row blocks back to back, heaviest
  // first): the wider span of the ping-pong kernels doubled the HBM reads at
  // the varlen configuration.
  int mb, id;
  if (p.cu_q == nullptr ||
      !work_item_kv_rr(blockIdx.x, p.total_blocks, p.n_mblocks, p.group, p.heavy_first != 0, mb, id))
    work_item(blockIdx.x, p.total_blocks, p.n_mblocks, p.heavy_first != 0, 1, mb, id);
  const int hh = id % p.heads_q;
  const int b = id / p.heads_q;
  const int kvh = hh / p.group;

  int Sq, Sk;
  int64_t q_base, o_base, lse_base, k_base, v_base;
  if (p.cu_q != nullptr) {
    const int qs = p.cu_q[b], ks = p.cu_k[b];
    Sq = p.cu_q[b + 1] - qs;
    Sk = p.cu_k[b + 1] - ks;
    if (p.seqused_q != nullptr) Sq = max(0, min(Sq, p.seqused_q[b]));
    if (p.seqused_k != nullptr) Sk = max(0, min(Sk, p.seqused_k[b]));
    const int os = p.cu_o != nullptr ? p.cu_o[b] : qs;
    q_base = (int64_t)qs * p.q_ss;
    o_base = (int64_t)os * p.o_ss;
    lse_base = (int64_t)os * p.lse_ss;
    k_base = (int64_t)ks * p.k_ss;
    v_base = (int64_t)ks * p.v_ss;
  } else {
    Sq = p.seqlen_q;
    Sk = p.seqlen_k;
    q_base = (int64_t)b * p.q_sb;
    o_base = (int64_t)b * p.o_sb;
    lse_base = (int64_t)b * p.lse_sb;
    k_base = (int64_t)b * p.k_sb;
    v_base = (int64_t)b * p.v_sb;
  }
  q_base += (int64_t)hh * p.q_sh;
  o_base += (int64_t)hh * p.o_sh;
  lse_base += (int64_t)hh * p.lse_sh;
  k_base += (int64_t)kvh * p.k_sh;
  v_base += (int64_t)kvh * p.v_sh;
  const int64_t qoff = p.q_offset;

  const int row0 = mb * BM;
  if (row0 >= Sq) return;   // varlen blocks past this sequence's queries
  const int row_last = min(row0 + BM, Sq) - 1;

  const int qi = row0 + w * 32 + c32;
  const bool row_valid = qi < Sq;
  const int qpos = qi + (int)qoff;
  float slope = 0.f;
  if (GENERIC && p.alibi != nullptr && row_valid) slope = p.alibi[(int64_t)b * p.alibi_sb + hh];
  const float* bias_row = nullptr;
  if (BIAS)
    bias_row = p.bias + (int64_t)b * p.bias_sb + (int64_t)hh * p.bias_sh + (int64_t)qi * p.bias_sq;

  const int wrow0 = row0 + w * 32;
  const bool wave_active = wrow0 <= row_last;
  // Positions fit in 32 bits (the host keeps lengths and offsets below 2^29).
  const int qoff32 = (int)qoff;
  const int qpos_w_min = wrow0 + qoff32;
  const int qpos_w_max = min(wrow0 + 31, row_last) + qoff32;

  const int wl = p.window_left, wr = p.window_right;
  const bool causal = p.causal != 0;
  // Keys this row may see on a masked tile: [key_lo, key_hi].
  const int qp32 = qpos;
  int key_hi = Sk - 1;
  if (causal) key_hi = min(key_hi, qp32);
  if (wr >= 0) key_hi = min(key_hi, qp32 + wr);
  const int key_lo = wl >= 0 ? qp32 - wl : INT32_MIN;

  // Key range [k_lo, k_hi) any row of the workgroup can see.
  int k_hi = Sk;
  if (causal) k_hi = min(k_hi, row_last + qoff32 + 1);
  if (wr >= 0) k_hi = min(k_hi, row_last + qoff32 + wr + 1);
  int k_lo = 0;
  if (wl >= 0) k_lo = max(0, row0 + qoff32 - wl);
  const int t_begin = k_lo / BN;
  const int t_end = k_hi > k_lo ? (k_hi + BN - 1) / BN : t_begin;

  // ------------------------------------------------------------ Q^T in VGPRs
  const uint16_t* qg = static_cast<const uint16_t*>(p.q);
  u32x4 qreg[NKC];
  {
    const uint16_t* qrow = qg + q_base + (int64_t)qi * p.q_ss;
#pragma unroll
    for (int kc = 0; kc < NKC; ++kc)
      qreg[kc] = row_valid ? load16(qrow + kc * 16 + g * 8) : u32x4{0, 0, 0, 0};
    // Retire the Q loads here: otherwise the loop's first use of qreg has to
    // assume they may still be in flight behind the tile prefetches and waits
    // for every outstanding load.
    __builtin_amdgcn_s_waitcnt(0x0f70);   // vmcnt(0)
  }

  // ------------------------------------------------------------ tile loads
  // K and V tiles are copied row-major: chunk c = tid + i*NT of a tile is key
  // row c / CPR, 16-byte column c % CPR.  Every byte offset goes into the VGPR
  // offset operand: the range check of a raw buffer load covers that operand
  // but not the scalar one.
  const uint16_t* kg = static_cast<const uint16_t*>(p.k) + k_base;
  const uint16_t* vg = static_cast<const uint16_t*>(p.v) + v_base;
  const uint32_t k_row_b = (uint32_t)(p.k_ss * 2);
  const uint32_t v_row_b = (uint32_t)(p.v_ss * 2);
  uint32_t k_off[KPT], v_off[KPT];
#pragma unroll
  for (int i = 0; i < KPT; ++i) {
    // Threads past the tile's chunk count load nothing: an offset at the top
    // of the 32-bit range is beyond any resource and reads zero.
    const int c = tid + i * NT;
    k_off[i] = c < CHUNKS ? (uint32_t)(c / CPR) * k_row_b + (uint32_t)(c % CPR) * 16 : 0xfffffff0u;
    v_off[i] = c < CHUNKS ? (uint32_t)(c / CPR) * v_row_b + (uint32_t)(c % CPR) * 16 : 0xfffffff0u;
  }

  u32x4 kreg[KPT], vreg[KPT];
  auto load_k = [&](int t) {
    const int n0 = t * BN;
    const auto rs = make_rsrc(kg + (int64_t)n0 * p.k_ss, rows_extent(n0, Sk, p.k_ss, D));
#pragma unroll
    for (int i = 0; i < KPT; ++i) kreg[i] = buf_load16(rs, k_off[i], 0);
  };
  auto load_v = [&](int t) {
    const int n0 = t * BN;
    const auto rs = make_rsrc(vg + (int64_t)n0 * p.v_ss, rows_extent(n0, Sk, p.v_ss, D));
#pragma unroll
    for (int i = 0; i < KPT; ++i) vreg[i] = buf_load16(rs, v_off[i], 0);
  };
  // LDS: [K slot 0][K slot 1][V slot 0][V slot 1].
  auto k_slot = [&](int i) { return smem + (i & 1) * KTILE; };
  auto v_slot = [&](int i) { return smem + 2 * KTILE + (i & 1) * VTILE; };
  auto store_k = [&](int slot) {
    uint16_t* Ks = k_slot(slot);
#pragma unroll
    for (int i = 0; i < KPT; ++i) {
      const int c = tid + i * NT;
      if (CHUNKS % NT == 0 || c < CHUNKS) store16(Ks + (c / CPR) * KSTR + (c % CPR) * 8, kreg[i]);
    }
  };
  auto store_v = [&](int slot) {
    uint16_t* Vs = v_slot(slot);
#pragma unroll
    for (int i = 0; i < KPT; ++i) {
      const int c = tid + i * NT;
      if (CHUNKS % NT == 0 || c < CHUNKS) store16(Vs + (c / CPR) * VSTR + (c % CPR) * 8, vreg[i]);
    }
  };

  // V^T operand of O^T += V^T P^T through ds_read_b64_tr_b16.  Within each
  // 16-lane group the instruction returns to lane i the i-th column of the 4x16
  // block whose row r is read by lanes 4r..4r+3 (4 elements each).  Lane
  // (c32, g) needs, for 16-key chunk cc and 32-dim block db, the keys
  // 16cc + 4g + r and 16cc + 8 + 4g + r (r < 4) at dim db*32 + c32, so lane j
  // of its group reads key row 16cc + 4g + j/4 (+8), dims 16(c32/16) + 4(j%4).
  const int vt_lane = (4 * g + (lane & 15) / 4) * VSTR + 16 * (c32 >> 4) + 4 * (lane & 3);

  // Per-wave tile classification: skipped (no key of the tile visible to any
  // row of this wave) or masked (some key hidden from some row).
  auto wave_skips = [&](int t) {
    const int n0 = t * BN, n1 = n0 + BN;
    bool skip = !wave_active || n0 >= Sk;
    if (causal) skip = skip || n0 > qpos_w_max;
    if (wr >= 0) skip = skip || n0 > qpos_w_max + wr;
    if (wl >= 0) skip = skip || n1 - 1 < qpos_w_min - wl;
    return skip;
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
  float m_run = -INFINITY;   // running (possibly stale) max, log2 units
  float l_run = 0.f;         // this lane's partial row sum

  // S^T of one tile from a K slot (v_mfma_f32_32x32x16: A = K rows, B = Q^T).
  auto qk = [&](const uint16_t* Ks, f32x16* sd) {
#pragma unroll
    for (int kb = 0; kb < NKB; ++kb) {
      sd[kb] = f32x16{};
#pragma unroll
      for (int kc = 0; kc < NKC; ++kc) {
        const u32x4 a = load16(Ks + (kb * 32 + c32) * KSTR + kc * 16 + g * 8);
        sd[kb] = T::mfma32(a, qreg[kc], sd[kb]);
      }
    }
  };
  // O^T += V^T P^T for one tile from a V slot.
  auto pv = [&](const uint16_t* Vs, const u32x4* pb) {
#pragma unroll
    for (int cc = 0; cc < NCC; ++cc) {
#pragma unroll
      for (int db = 0; db < NDB; ++db) {
        const uint16_t* vp = Vs + vt_lane + cc * 16 * VSTR + db * 32;
        const u32x2 lo = lds_read_tr16(vp);
        const u32x2 hi = lds_read_tr16(vp + 8 * VSTR);
        const u32x4 a = {lo[0], lo[1], hi[0], hi[1]};
        acc[db] = T::mfma32(a, pb[cc], acc[db]);
      }
    }
  };
  // Softmax of one tile of scores starting at key n0: GENERIC transform,
  // boundary mask, lazy max / rescale, P = exp2(s - m) packed to the element
  // type as the B operand of pv (pb[cc] holds keys 16cc .. 16cc + 15 in the
  // MFMA's k order), row sums.
  auto softmax_tile = [&](f32x16* sc, int n0, bool masked, u32x4* pb) {
    // GENERIC: scale, ALiBi and softcap, scores -> log2 units.  Otherwise the
    // scores stay raw (scale > 0) and the scale is folded into the exp2
    // argument and the max.
    // D = 256 keeps the direct form: its registers are already at the limit.
    if (GENERIC && (BIAS || D >= 256)) {
#pragma unroll
      for (int kb = 0; kb < NKB; ++kb) {
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          const int key = n0 + kb * 32 + 8 * (v >> 2) + 4 * g + (v & 3);
          float x = sc[kb][v] * p.scale;
          if (p.alibi != nullptr) x = fmaf(-slope, fabsf((float)(qp32 - key)), x);
          if (BIAS && row_valid && key < Sk) x += bias_row[(int64_t)key * p.bias_sk];
          if (p.softcap > 0.f) {
            // softcap * tanh(x / softcap) = softcap - 2 softcap / (1 + e^(2x/softcap))
            const float e2 = __builtin_amdgcn_exp2f(x * p.softcap_k);
            x = p.softcap - 2.f * p.softcap * __builtin_amdgcn_rcpf(1.f + e2);
          }
          sc[kb][v] = x * kLog2e;
        }
      }
    } else if (GENERIC) {
      // The same transform with its constants folded per tile (this epilogue
      // is VALU-bound): qpos - key = dq0 - koff with dq0 = qpos - n0 - 4g and
      // koff = 32 kb + 8 (v / 4) + v % 4 fixed per slot, and with softcap only
      // x k = x (2 log2 e / softcap) is needed:
      //   softcap log2(e) tanh(x / softcap) = c2 - 2 c2 / (1 + 2^(x k)),
      //   x k = s (scale k) - (slope k) |qpos - key|,  c2 = softcap log2(e).
      const int dq0 = qp32 - n0 - 4 * g;
      const bool alibi = p.alibi != nullptr;
      // |qpos - key| as a float: an integer subtract of the slot's offset (an
      // inline constant below 64) and one convert.
      auto dist = [&](int kb, int v) { return fabsf((float)(dq0 - (kb * 32 + 8 * (v >> 2) + (v & 3)))); };
      if (p.softcap > 0.f) {
        const float sk = p.scale * p.softcap_k, ak = -slope * p.softcap_k;
        const float c2 = p.softcap * kLog2e, m2c2 = -2.f * c2;
        auto cap = [&](float xk) {
          return fmaf(m2c2, __builtin_amdgcn_rcpf(1.f + __builtin_amdgcn_exp2f(xk)), c2);
        };
        // (One 32-key block at a time: interleaving the exp / rcp chains of
        // several blocks buys nothing and costs registers.)
        if (alibi) {
#pragma unroll
          for (int kb = 0; kb < NKB; ++kb) {
#pragma unroll
            for (int v = 0; v < 16; ++v)
              sc[kb][v] = cap(fmaf(ak, dist(kb, v), sc[kb][v] * sk));
            __builtin_amdgcn_sched_barrier(0);
          }
        } else {
#pragma unroll
          for (int kb = 0; kb < NKB; ++kb) {
#pragma unroll
            for (int v = 0; v < 16; ++v) sc[kb][v] = cap(sc[kb][v] * sk);
            __builtin_amdgcn_sched_barrier(0);
          }
        }
      } else {
        const float sl2 = p.scale * kLog2e, al2 = -slope * kLog2e;
        if (alibi) {
#pragma unroll
          for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
            for (int v = 0; v < 16; ++v)
              sc[kb][v] = fmaf(al2, dist(kb, v), sc[kb][v] * sl2);
        } else {
#pragma unroll
          for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
            for (int v = 0; v < 16; ++v) sc[kb][v] *= sl2;
        }
      }
    }
    // Boundary tiles only (a wave-uniform branch): keys outside
    // [key_lo, key_hi] -> -inf.
    if (masked) {
#pragma unroll
      for (int kb = 0; kb < NKB; ++kb) {
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          const int key = n0 + kb * 32 + 8 * (v >> 2) + 4 * g + (v & 3);
          if (key < key_lo || key > key_hi) sc[kb][v] = -INFINITY;
        }
      }
    }
    // Row max over this lane's scores: four independent max3 chains.
    float mq[4] = {-INFINITY, -INFINITY, -INFINITY, -INFINITY};
#pragma unroll
    for (int kb = 0; kb < NKB; ++kb) {
#pragma unroll
      for (int v = 0; v < 16; v += 8) {
#pragma unroll
        for (int q = 0; q < 4; ++q)
          mq[q] = fmaxf(fmaxf(mq[q], sc[kb][v + 2 * q]), sc[kb][v + 2 * q + 1]);
      }
    }
    const float sl = GENERIC ? 1.f : p.scale_log2;
    const float mx = halves_max(fmaxf(fmaxf(mq[0], mq[1]), fmaxf(mq[2], mq[3]))) * sl;
    const bool raise = mx > m_run + kRescaleSlack;
    if (__builtin_amdgcn_ballot_w64(raise)) {
      const float m_new = raise ? mx : m_run;
      const float alpha = m_new == m_run ? 1.f : __builtin_amdgcn_exp2f(m_run - m_new);
      l_run *= alpha;
#pragma unroll
      for (int db = 0; db < NDB; ++db) acc[db] *= alpha;
      m_run = m_new;
    }
    const float m_use = m_run == -INFINITY ? 0.f : m_run;
    float lq[4] = {0.f, 0.f, 0.f, 0.f};   // independent partial row sums
    if (GENERIC && p.drop.enabled) {
      // Dropout: the row sums take the undropped P, the product the dropped
      // one (one Philox call per 16 keys of this lane's row).
#pragma unroll
      for (int cc = 0; cc < NCC; ++cc) {
        const f32x16& sv = sc[cc >> 1];
        const int o8 = (cc & 1) * 8;
        const u32x4 r = dropout_draws(p.drop, (n0 >> 4) + cc, g, qi, hh, b);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const float e0 = __builtin_amdgcn_exp2f(fmaf(sv[o8 + 2 * j], sl, -m_use));
          const float e1 = __builtin_amdgcn_exp2f(fmaf(sv[o8 + 2 * j + 1], sl, -m_use));
          lq[j] += e0 + e1;
          pb[cc][j] = T::pack2(e0 * dropout_factor(p.drop, r, 2 * j),
                               e1 * dropout_factor(p.drop, r, 2 * j + 1));
        }
      }
      l_run += (lq[0] + lq[1]) + (lq[2] + lq[3]);
      return;
    }
#pragma unroll
    for (int cc = 0; cc < NCC; ++cc) {
      const f32x16& sv = sc[cc >> 1];
      const int o8 = (cc & 1) * 8;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const float e0 = __builtin_amdgcn_exp2f(fmaf(sv[o8 + 2 * j], sl, -m_use));
        const float e1 = __builtin_amdgcn_exp2f(fmaf(sv[o8 + 2 * j + 1], sl, -m_use));
        pb[cc][j] = T::pack2(e0, e1);
        if (T::kSumRounded)
          lq[j] = T::sum2(pb[cc][j], lq[j]);
        else
          lq[j] += e0 + e1;
      }
    }
    l_run += (lq[0] + lq[1]) + (lq[2] + lq[3]);
  };

  // ------------------------------------------------------------ main loop
  const int J = t_end - t_begin;
  // One wave group: per tile S = K Q^T, softmax, O^T += V^T P^T, with the
  // next tile's loads in flight; LDS slot i & 1 holds K_i and V_i.
  u32x4 pbuf[NCC];
  f32x16 s[NKB];
  if (J > 0) {
    load_k(t_begin);
    load_v(t_begin);
    store_k(0);
    store_v(0);
  }
  for (int it = 0; it < J; ++it) {
    const int t = t_begin + it;
    __syncthreads();
    const bool has_next = it + 1 < J;
    if (has_next) {
      load_k(t + 1);
      load_v(t + 1);
    }
    if (!wave_skips(t)) {
      qk(k_slot(it), s);
      softmax_tile(s, t * BN, wave_masks(t), pbuf);
      pv(v_slot(it), pbuf);
    }
    if (has_next) {
      store_k(it + 1);
      store_v(it + 1);
    }
  }

  // ------------------------------------------------------------ epilogue
  const float l_tot = halves_sum(l_run);
  const float inv_l = l_tot > 0.f ? 1.f / l_tot : 0.f;
  const float lse_val = l_tot > 0.f ? (m_run + __log2f(l_tot)) * kLn2 : -INFINITY;
  if (!row_valid) return;

  uint16_t* orow = static_cast<uint16_t*>(p.o) + o_base + (int64_t)qi * p.o_ss;
#pragma unroll
  for (int db = 0; db < NDB; ++db) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int d = db * 32 + r * 8 + g * 4;
      u32x2 val;
      val[0] = T::pack2(acc[db][4 * r] * inv_l, acc[db][4 * r + 1] * inv_l);
      val[1] = T::pack2(acc[db][4 * r + 2] * inv_l, acc[db][4 * r + 3] * inv_l);
      *reinterpret_cast<u32x2*>(orow + d) = val;
    }
  }
  if (p.lse != nullptr && g == 0) p.lse[lse_base + (int64_t)qi * p.lse_ss] = lse_val;
}

}  // namespace fa
