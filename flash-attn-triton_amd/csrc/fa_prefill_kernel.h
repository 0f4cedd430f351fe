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
//
// KS > 0 (D = 128, 32-key tiles, no attn_bias): the tiles go global -> LDS
// through the buffer loads' LDS mode instead of VGPR staging, unpadded with
// the XOR swizzle of the ping-pong kernel (16-byte chunk c of row r at
// c ^ (r & 15) for K, c ^ 4 (r & 3) for V), in a ring of KS K stages and
// KS - 1 V stages: the loads of K_{t+KS-1} and V_{t+KS-2} go out at the top
// of tile t, so K has KS - 1 tiles of compute to land in and V KS - 2 plus
// the S^T product and softmax of its own tile.  This form walks the key
// tiles downwards, from the last visible one: with ALiBi (and with the
// recency typical of real attention) scores grow towards the diagonal, and
// walking upwards the running max moved past the rescale slack on about
// 40 % of the tiles at BASELINE config 5 (64 multiplies of O^T each);
// downwards the first tiles set it (measured 1 % faster there).  The tile
// loads step running 64-bit bases and ring slots instead of forming each
// tile's address from its index: the 64-bit products and slot divisions were
// about 40 scalar instructions per tile, and dropping them made BASELINE
// config 5 3 % faster (848 -> 822 us per launch on one MI355X).
#pragma once

#include "fa_fwd_kernel.h"
#include "fa_stage_rows.h"

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

// Dynamic LDS of prefill_kernel: the padded double buffers, or with KS > 0
// the K ring (KS tiles) and the V ring (KS - 1 tiles) of unpadded rows.
template <int D, int NW, int BN, int KS>
constexpr int prefill_lds_bytes() {
  return KS > 0 ? (2 * KS - 1) * BN * D * 2 : PrefillTile<D, NW, BN>::LDS_BYTES;
}

// BIAS: the additive fp32 attn_bias is read in the score epilogue (GENERIC
// only).  It is a separate instantiation because its per-score loads raise
// register pressure past the budget of the 3-waves-per-SIMD tiles.
template <class T, int D, int NW, int BN, bool GENERIC, int WPE, bool BIAS = false, int KS = 0>
__global__ __launch_bounds__(NW * 64) __attribute__((amdgpu_waves_per_eu(WPE, WPE)))
void prefill_kernel(const FwdParams p) {
  static_assert(GENERIC || !BIAS, "the bias is applied by the generic epilogue");
  constexpr bool kDma = KS > 0;
  static_assert(!kDma || (D == 128 && BN == 32 && !BIAS && KS >= 3),
                "the LDS-DMA ring is laid out for head dim 128 and 32-key tiles");
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
  // One slope per (batch, head): wave-uniform, also on rows past the
  // sequence (their scores are discarded).
  float slope = 0.f;
  if (GENERIC && p.alibi != nullptr) slope = p.alibi[(int64_t)b * p.alibi_sb + hh];
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
  // (-2^30 for no lower bound: positions stay below 2^29, so key_lo - n0
  // cannot overflow.)
  constexpr int kNoKey = 1 << 30;
  const int key_lo = wl >= 0 ? qp32 - wl : -kNoKey;

  // Key range [k_lo, k_hi) any row of the workgroup can see.
  int k_hi = Sk;
  if (causal) k_hi = min(k_hi, row_last + qoff32 + 1);
  if (wr >= 0) k_hi = min(k_hi, row_last + qoff32 + wr + 1);
  int k_lo = 0;
  if (wl >= 0) k_lo = max(0, row0 + qoff32 - wl);
  const int t_begin = k_lo / BN;
  const int t_end = k_hi > k_lo ? (k_hi + BN - 1) / BN : t_begin;
  const int J_all = t_end - t_begin;

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

  // Register staging of the tile loads: one set (the next tile) or, for the
  // generic 4-wave tiles, two (the next two tiles: a load has two tiles of
  // compute to land in; these kernels wait on load latency otherwise).
  constexpr bool kDeep = GENERIC && NW == 4 && D <= 128;
  u32x4 kreg[KPT], vreg[KPT], kreg2[kDeep ? KPT : 1], vreg2[kDeep ? KPT : 1];
  auto load_k = [&](int t, u32x4* kr) {
    const int n0 = t * BN;
    const auto rs = make_rsrc(kg + (int64_t)n0 * p.k_ss, rows_extent(n0, Sk, p.k_ss, D));
#pragma unroll
    for (int i = 0; i < KPT; ++i) kr[i] = buf_load16(rs, k_off[i], 0);
  };
  auto load_v = [&](int t, u32x4* vr) {
    const int n0 = t * BN;
    const auto rs = make_rsrc(vg + (int64_t)n0 * p.v_ss, rows_extent(n0, Sk, p.v_ss, D));
#pragma unroll
    for (int i = 0; i < KPT; ++i) vr[i] = buf_load16(rs, v_off[i], 0);
  };
  // LDS: [K slot 0][K slot 1][V slot 0][V slot 1].
  auto k_slot = [&](int i) { return smem + (i & 1) * KTILE; };
  auto v_slot = [&](int i) { return smem + 2 * KTILE + (i & 1) * VTILE; };
  auto store_k = [&](int slot, const u32x4* kr) {
    uint16_t* Ks = k_slot(slot);
#pragma unroll
    for (int i = 0; i < KPT; ++i) {
      const int c = tid + i * NT;
      if (CHUNKS % NT == 0 || c < CHUNKS) store16(Ks + (c / CPR) * KSTR + (c % CPR) * 8, kr[i]);
    }
  };
  auto store_v = [&](int slot, const u32x4* vr) {
    uint16_t* Vs = v_slot(slot);
#pragma unroll
    for (int i = 0; i < KPT; ++i) {
      const int c = tid + i * NT;
      if (CHUNKS % NT == 0 || c < CHUNKS) store16(Vs + (c / CPR) * VSTR + (c % CPR) * 8, vr[i]);
    }
  };

  // LDS-DMA ring (kDma).  Wave w copies rows [4 (IPW w + i), +4) of every K
  // and V tile, i < IPW; lane l writes physical chunk l % 16 of row
  // 4 (IPW w + i) + l / 16, so it loads the logical chunk the swizzle puts
  // there.  Tiles at or past J get an empty resource: the instruction still
  // retires (keeping the wait counts uniform) and writes zeros.
  constexpr int DTILEB = BN * D * 2;                  // bytes of one K or V tile
  constexpr int IPW = kDma ? DTILEB / 1024 / NW : 1;  // DMA instructions per wave and tile
  static_assert(!kDma || IPW * NW * 1024 == DTILEB, "tile must split evenly over the waves");
  uint8_t* const k_ring = reinterpret_cast<uint8_t*>(smem);
  uint8_t* const v_ring = k_ring + (kDma ? KS : 0) * DTILEB;
  uint32_t kd_off[IPW], vd_off[IPW];
#pragma unroll
  for (int i = 0; i < IPW; ++i) {
    const int r = 4 * (IPW * w + i) + (lane >> 4);
    const int pc = lane & 15;
    kd_off[i] = (uint32_t)r * k_row_b + (uint32_t)((pc ^ (r & 15)) * 16);
    vd_off[i] = (uint32_t)r * v_row_b + (uint32_t)((pc ^ (4 * (r & 3))) * 16);
  }
  const uint32_t k_ring_a = lds_address(k_ring) + IPW * w * 1024;
  const uint32_t v_ring_a = lds_address(v_ring) + IPW * w * 1024;
  // issue_k and issue_v are each called for rel = 0, 1, 2, ... in order, so
  // they step a running tile base down one tile and a running ring slot on
  // per call (no per-tile 64-bit products or divisions).  Only the first
  // (highest) tile can run past the sequence's last key: it takes the
  // extent to that key, every lower tile exactly its BN rows, and tiles past
  // J_all an empty resource.
  const int n0_top = (t_end - 1) * BN;
  const uint32_t k_top = J_all > 0 ? rows_extent(n0_top, Sk, p.k_ss, D) : 0u;
  const uint32_t v_top = J_all > 0 ? rows_extent(n0_top, Sk, p.v_ss, D) : 0u;
  const uint32_t k_full = rows_extent(0, BN, p.k_ss, D);
  const uint32_t v_full = rows_extent(0, BN, p.v_ss, D);
  const uint16_t* k_next = kg + (int64_t)n0_top * p.k_ss;
  const uint16_t* v_next = vg + (int64_t)n0_top * p.v_ss;
  const int64_t k_step = (int64_t)BN * p.k_ss, v_step = (int64_t)BN * p.v_ss;
  int k_wslot = 0, v_wslot = 0;
  auto issue_k = [&](int rel) __attribute__((always_inline)) {
    const uint32_t ext = rel < J_all ? (rel == 0 ? k_top : k_full) : 0u;
    const u32x4 rs = make_rsrc_words(k_next, ext);
    k_next -= k_step;
    const uint32_t dst = k_ring_a + (uint32_t)k_wslot * DTILEB;
    k_wslot = k_wslot == (kDma ? KS : 1) - 1 ? 0 : k_wslot + 1;
#pragma unroll
    for (int i = 0; i < IPW; ++i) buf_load16_lds(rs, dst + i * 1024, kd_off[i]);
  };
  auto issue_v = [&](int rel) __attribute__((always_inline)) {
    const uint32_t ext = rel < J_all ? (rel == 0 ? v_top : v_full) : 0u;
    const u32x4 rs = make_rsrc_words(v_next, ext);
    v_next -= v_step;
    const uint32_t dst = v_ring_a + (uint32_t)v_wslot * DTILEB;
    v_wslot = v_wslot == (kDma ? KS - 1 : 1) - 1 ? 0 : v_wslot + 1;
#pragma unroll
    for (int i = 0; i < IPW; ++i) buf_load16_lds(rs, dst + i * 1024, vd_off[i]);
  };
  // Swizzled operand reads of the ring: K (16 B per lane) row kb*32 + c32,
  // logical chunk 2 kc + g; V^T (ds_read_b64_tr_b16) as vt_lane below.
  uint32_t kd_rd[NKC], vd_rd[NDB];
  {
    const int j16 = lane & 15;
    const uint32_t v_rd = (uint32_t)(4 * g + (j16 >> 2)) * (D * 2) + (uint32_t)((j16 & 1) * 8);
    const int v_cx = 2 * (c32 >> 4) + ((j16 & 3) >> 1);
    const int v_sw = j16 >> 2;
#pragma unroll
    for (int kc = 0; kc < NKC; ++kc)
      kd_rd[kc] = (uint32_t)c32 * (D * 2) + ((uint32_t)(2 * kc + g) ^ (uint32_t)(c32 & 15)) * 16;
#pragma unroll
    for (int db = 0; db < NDB; ++db)
      vd_rd[db] = v_rd + ((((uint32_t)db ^ (uint32_t)v_sw) << 2) + (uint32_t)v_cx) * 16;
  }

  // V^T operand of O^T += V^T P^T through ds_read_b64_tr_b16.  Within each
  // 16-lane group the instruction returns to lane i the i-th column of the 4x16
  // block whose row r is read by lanes 4r..4r+3 (4 elements each).  Lane
  // (c32, g) needs, for 16-key chunk cc and 32-dim block db, the keys
  // 16cc + 4g + r and 16cc + 8 + 4g + r (r < 4) at dim db*32 + c32, so lane j
  // of its group reads key row 16cc + 4g + j/4 (+8), dims 16(c32/16) + 4(j%4).
  const int vt_lane = (4 * g + (lane & 15) / 4) * VSTR + 16 * (c32 >> 4) + 4 * (lane & 3);

  // Per-wave tile classification from key bounds computed once (integers,
  // so the per-tile tests stay on the scalar unit): a tile is skipped when no
  // key of it lies in [kw_lo, kw_hi], the union of this wave's rows' visible
  // ranges, and needs the lower / upper mask when it reaches below kf_lo /
  // above kf_hi, their intersection.
  int kw_lo = 0, kw_hi = Sk - 1, kf_lo = 0, kf_hi = Sk - 1;
  if (causal) {
    kw_hi = min(kw_hi, qpos_w_max);
    kf_hi = min(kf_hi, qpos_w_min);
  }
  if (wr >= 0) {
    kw_hi = min(kw_hi, qpos_w_max + wr);
    kf_hi = min(kf_hi, qpos_w_min + wr);
  }
  if (wl >= 0) {
    kw_lo = max(kw_lo, qpos_w_min - wl);
    kf_lo = qpos_w_max - wl;
  }
  if (!wave_active) {
    kw_lo = kNoKey;
    kw_hi = -kNoKey;
  }

  f32x16 acc[NDB];
#pragma unroll
  for (int db = 0; db < NDB; ++db) acc[db] = f32x16{};
  float m_run = -INFINITY;   // running (possibly stale) max, log2 units
  float l_run = 0.f;         // this lane's partial row sum

  // S^T of one tile from a K slot (v_mfma_f32_32x32x16: A = K rows, B = Q^T).
  // C operand the S^T products start from: zero, or with causal ALiBi on the
  // fast transform below, the per-slot ALiBi term divided by the score
  // scale (set there).
  f32x16 cinit = f32x16{};
  auto qk = [&](const uint16_t* Ks, f32x16* sd) {
#pragma unroll
    for (int kb = 0; kb < NKB; ++kb) {
      sd[kb] = cinit;
#pragma unroll
      for (int kc = 0; kc < NKC; ++kc) {
        const u32x4 a =
            kDma ? *reinterpret_cast<const u32x4*>(reinterpret_cast<const uint8_t*>(Ks) +
                                                  kd_rd[kc] + kb * 32 * D * 2)
                 : load16(Ks + (kb * 32 + c32) * KSTR + kc * 16 + g * 8);
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
        const uint16_t* vp =
            kDma ? reinterpret_cast<const uint16_t*>(reinterpret_cast<const uint8_t*>(Vs) +
                                                     vd_rd[db] + cc * 16 * D * 2)
                 : Vs + vt_lane + cc * 16 * VSTR + db * 32;
        const u32x2 lo = lds_read_tr16(vp);
        const u32x2 hi = lds_read_tr16(vp + 8 * (kDma ? D : VSTR));
        const u32x4 a = {lo[0], lo[1], hi[0], hi[1]};
        acc[db] = T::mfma32(a, pb[cc], acc[db]);
      }
    }
  };
  // Score transform of the generic epilogue without attn_bias (D < 256):
  // every score first becomes t = x k, x = s scale - slope |qpos - key| the
  // scaled score with ALiBi and k = 2 log2(e) / softcap with softcap (log2(e)
  // without).  The row max is taken on t (the cap is increasing) and softcap
  // enters with the exponent,
  //   softcap log2(e) tanh(x / softcap) = c2 - 2 c2 / (1 + 2^t),  c2 = softcap log2(e),
  // so the exp2 argument is one FMA: (c2 - m) - 2 c2 / (1 + 2^t).
  // ALiBi: on tiles whose keys are at or before every row's position (all
  // of them under causal masking: the keys past it are masked),
  // -k slope |qpos - key| = A - akk with A = ak (qpos - n0 - 4g - 32 kb) per
  // lane and 32-key block, ak = -k slope, and akk = ak koff per score slot
  // (koff < 32 the slot's key offset in the block, the same in every lane).
  // Causal launches start the S^T products from C = -akk / k (cinit), so the
  // MFMAs add the per-slot term and the transform is one FMA per score;
  // otherwise one FMA and one more per score.  (The 8-wave D = 128 tiles
  // take the |qpos - key| form.)
  constexpr bool kFastT = GENERIC && !BIAS && D < 256;
  constexpr bool kAkk = kFastT && (NKB == 1 || D <= 64);
  const bool alibi_on = GENERIC && p.alibi != nullptr;
  const bool cap_on = kFastT && p.softcap > 0.f;
  const float tk = GENERIC ? p.scale * (p.softcap > 0.f ? p.softcap_k : kLog2e) : 1.f;
  const float ak = GENERIC ? -slope * (p.softcap > 0.f ? p.softcap_k : kLog2e) : 0.f;
  const float c2 = p.softcap * kLog2e, m2c2 = -2.f * c2;
  auto koff = [](int kb, int v) __attribute__((always_inline)) { return kb * 32 + 8 * (v >> 2) + (v & 3); };
  if (kAkk && alibi_on && causal) {
    const float akt = -ak / tk;
#pragma unroll
    for (int v = 0; v < 16; ++v) cinit[v] = akt * (float)koff(0, v);
  }

  // Softmax of one tile of scores starting at key n0: GENERIC transform,
  // boundary masks (keys below key_lo when mlo, above key_hi when mhi), lazy
  // max / rescale, P = exp2(s - m) packed to the element type as the B
  // operand of pv (pb[cc] holds keys 16cc .. 16cc + 15 in the MFMA's k
  // order), row sums.
  auto softmax_tile = [&](f32x16* sc, int n0, bool mlo, bool mhi, u32x4* pb) {
    // GENERIC: scale, ALiBi and softcap, scores -> log2 units.  Otherwise the
    // scores stay raw (scale > 0) and the scale is folded into the exp2
    // argument and the max.
    // With attn_bias or D = 256 the transform is applied in full here (those
    // kernels are at their register limit).
    if (GENERIC && !kFastT) {
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
    } else if (kFastT) {
      if (alibi_on) {
        const int dq0 = qp32 - n0 - 4 * g;   // qpos - key = dq0 - koff
        if (kAkk && causal) {
#pragma unroll
          for (int kb = 0; kb < NKB; ++kb) {
            const float A = ak * (float)(dq0 - 32 * kb);
#pragma unroll
            for (int v = 0; v < 16; ++v) sc[kb][v] = fmaf(sc[kb][v], tk, A);
          }
        } else if (kAkk && n0 + BN - 1 <= qpos_w_min) {
#pragma unroll
          for (int kb = 0; kb < NKB; ++kb) {
            const float A = ak * (float)(dq0 - 32 * kb);
#pragma unroll
            for (int v = 0; v < 16; ++v)
              sc[kb][v] = fmaf(-ak, (float)koff(0, v), fmaf(sc[kb][v], tk, A));
          }
        } else {
#pragma unroll
          for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
            for (int v = 0; v < 16; ++v)
              sc[kb][v] = fmaf(ak, fabsf((float)(dq0 - koff(kb, v))), sc[kb][v] * tk);
        }
      } else {
#pragma unroll
        for (int kb = 0; kb < NKB; ++kb) sc[kb] *= tk;
      }
    }
    // Boundary tiles only (wave-uniform branches): keys outside
    // [key_lo, key_hi] -> -inf, one compare per bound against the slot's key
    // offset (an inline constant).
    auto mask_tile = [&](auto lo_c, auto hi_c) __attribute__((always_inline)) {
      const int mbase = n0 + 4 * g;
      const int lo_rel = key_lo - mbase, hi_rel = key_hi - mbase;
#pragma unroll
      for (int kb = 0; kb < NKB; ++kb) {
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          const int ko = koff(kb, v);
          const bool hide = (decltype(lo_c)::value && ko < lo_rel) || (decltype(hi_c)::value && ko > hi_rel);
          if (hide) sc[kb][v] = -INFINITY;
        }
      }
    };
    if (D >= 256 ? (mlo || mhi) : (mlo && mhi))
      mask_tile(std::true_type{}, std::true_type{});
    else if (mlo)
      mask_tile(std::true_type{}, std::false_type{});
    else if (mhi)
      mask_tile(std::false_type{}, std::true_type{});
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
    float mx = halves_max(fmaxf(fmaxf(mq[0], mq[1]), fmaxf(mq[2], mq[3]))) * sl;
    if (cap_on && mx != -INFINITY)
      mx = fmaf(m2c2, __builtin_amdgcn_rcpf(1.f + __builtin_amdgcn_exp2f(mx)), c2);
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
    // P and the row sums.  With softcap (a uniform branch) the exp2
    // arguments are formed in place first: the cap, then - m; a masked score
    // stays -inf.
    auto finish = [&](auto cap_c) __attribute__((always_inline)) {
      constexpr bool CAP = decltype(cap_c)::value;
      if constexpr (CAP) {
        const float c2m = c2 - m_use;
        auto cap_arg = [&](auto masked_c) __attribute__((always_inline)) {
#pragma unroll
          for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
            for (int v = 0; v < 16; ++v) {
              const float x = sc[kb][v];
              const float y = fmaf(m2c2, __builtin_amdgcn_rcpf(1.f + __builtin_amdgcn_exp2f(x)), c2m);
              sc[kb][v] = decltype(masked_c)::value && x == -INFINITY ? -INFINITY : y;
            }
        };
        if (mlo || mhi)
          cap_arg(std::true_type{});
        else
          cap_arg(std::false_type{});
      }
      auto expo = [&](float x) __attribute__((always_inline)) { return CAP ? x : fmaf(x, sl, -m_use); };
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
            const float e0 = __builtin_amdgcn_exp2f(expo(sv[o8 + 2 * j]));
            const float e1 = __builtin_amdgcn_exp2f(expo(sv[o8 + 2 * j + 1]));
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
          const float e0 = __builtin_amdgcn_exp2f(expo(sv[o8 + 2 * j]));
          const float e1 = __builtin_amdgcn_exp2f(expo(sv[o8 + 2 * j + 1]));
          pb[cc][j] = T::pack2(e0, e1);
          if (T::kSumRounded)
            lq[j] = T::sum2(pb[cc][j], lq[j]);
          else
            lq[j] += e0 + e1;
        }
      }
      l_run += (lq[0] + lq[1]) + (lq[2] + lq[3]);
    };
    if (kFastT && cap_on)
      finish(std::integral_constant<bool, kFastT>{});
    else
      finish(std::false_type{});
  };

  // ------------------------------------------------------------ main loop
  const int J = t_end - t_begin;
  // One wave group: per tile S = K Q^T, softmax, O^T += V^T P^T, with the
  // next tile's loads in flight; LDS slot i & 1 holds K_i and V_i.
  u32x4 pbuf[NCC];
  f32x16 s[NKB];
  auto compute = [&](int it) __attribute__((always_inline)) {
    const int n0 = (kDma ? t_end - 1 - it : t_begin + it) * BN;
    if (n0 <= kw_hi && n0 + BN - 1 >= kw_lo) {
      const uint16_t* Ks = kDma ? reinterpret_cast<const uint16_t*>(k_ring + (it % (kDma ? KS : 1)) * DTILEB)
                                : k_slot(it);
      const uint16_t* Vs = kDma ? reinterpret_cast<const uint16_t*>(v_ring + (it % (kDma ? KS - 1 : 1)) * DTILEB)
                                : v_slot(it);
      qk(Ks, s);
      softmax_tile(s, n0, n0 < kf_lo, n0 + BN - 1 > kf_hi, pbuf);
      pv(Vs, pbuf);
    }
  };
  if constexpr (kDma) {
    // Prologue: K_0, V_0, ..., K_{KS-3}, V_{KS-3}, K_{KS-2}; tile it then
    // issues V_{it+KS-2} and K_{it+KS-1}.  At the top of tile it the loads
    // issued after K_it and V_it are those of 2 KS - 5 tiles (K_{it+1},
    // V_{it+1}, ..., K_{it+KS-2}): waiting until at most that many remain
    // makes this wave's part of tile it visible, and the barrier everyone's.
    // The slots refilled in tile it held K_{it-1} and V_{it-1}, whose reads
    // every wave finished before that barrier.
#pragma unroll
    for (int i = 0; i < KS - 2; ++i) {
      issue_k(i);
      issue_v(i);
    }
    issue_k(KS - 2);
    for (int it = 0; it < J; ++it) {
      __builtin_amdgcn_s_waitcnt(vmcnt_imm((2 * KS - 5) * IPW));
      __builtin_amdgcn_s_barrier();
      issue_v(it + KS - 2);
      issue_k(it + KS - 1);
      compute(it);
    }
    // Every load (including the empty ones past the last tile) has landed
    // before the ring is reused for the output staging below.
    __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));
  } else if (J > 0) {
    load_k(t_begin, kreg);
    load_v(t_begin, vreg);
    store_k(0, kreg);
    store_v(0, vreg);
  }
  if constexpr (kDma) {
    // (the ring loop above)
  } else if constexpr (kDeep) {
    // Tile it + 1 waits in one register set while tile it + 2 loads into the
    // other; the sets alternate, so the loop runs tiles in pairs.
    if (J > 1) {
      load_k(t_begin + 1, kreg2);
      load_v(t_begin + 1, vreg2);
    }
    auto step = [&](int it, u32x4* st_k, u32x4* st_v, u32x4* ld_k, u32x4* ld_v)
        __attribute__((always_inline)) {
      __syncthreads();
      if (it + 2 < J) {
        load_k(t_begin + it + 2, ld_k);
        load_v(t_begin + it + 2, ld_v);
      }
      compute(it);
      if (it + 1 < J) {
        store_k(it + 1, st_k);
        store_v(it + 1, st_v);
      }
    };
    for (int it = 0; it < J; it += 2) {
      step(it, kreg2, vreg2, kreg, vreg);
      if (it + 1 < J) step(it + 1, kreg, vreg, kreg2, vreg2);
    }
  } else {
    for (int it = 0; it < J; ++it) {
      const int t = t_begin + it;
      __syncthreads();
      const bool has_next = it + 1 < J;
      if (has_next) {
        load_k(t + 1, kreg);
        load_v(t + 1, vreg);
      }
      compute(it);
      if (has_next) {
        store_k(it + 1, kreg);
        store_v(it + 1, vreg);
      }
    }
  }

  // ------------------------------------------------------------ epilogue
  const float l_tot = halves_sum(l_run);
  const float inv_l = l_tot > 0.f ? 1.f / l_tot : 0.f;
  const float lse_val = l_tot > 0.f ? (m_run + __log2f(l_tot)) * kLn2 : -INFINITY;
  if constexpr (D == 128) {
    // The output goes through LDS (the tile area, once every wave's last
    // tile reads are done) and out as whole rows: stored straight from the
    // accumulators, each instruction wrote 8 bytes of 32 rows, and the
    // partial lines reached HBM piecemeal (measured at BASELINE config 5:
    // 290.6 MB written for a 134.2 MB output).
    static_assert(NW * kStageOutBytes <= prefill_lds_bytes<D, NW, BN, KS>(),
                  "output staging must fit the tile area");
    __syncthreads();
    if (wave_active)
      stage_rows_store<T, NDB>(acc, inv_l, reinterpret_cast<uint8_t*>(smem) + w * kStageOutBytes,
                               c32, g, lane,
                               static_cast<uint16_t*>(p.o) + o_base + (int64_t)wrow0 * p.o_ss,
                               p.o_ss, Sq - wrow0);
    if (p.lse != nullptr && g == 0 && row_valid) p.lse[lse_base + (int64_t)qi * p.lse_ss] = lse_val;
    return;
  }
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
