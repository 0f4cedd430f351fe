// dK / dV of the FlashAttention-2 backward for head dims up to 128, with two
// waves per key group so that every SIMD runs two waves.
//
// With one wave per group of 32 keys (as bwd_dkdv_kernel does at D = 256)
// the kernel is bound by how fast that wave streams its operands out of LDS:
// each product reads a 1-KiB A operand from LDS, and one wave per SIMD
// reaches about half of the LDS read rate that two waves reach (measured on
// MI355X: ~90 against ~155 bytes per clock per CU for 16-byte row reads).  Its
// registers (K and V of the wave's keys, both dK^T and dV^T accumulators)
// leave no room for a second wave.
// Here the work of a key group is split between two waves on the same SIMD:
// * the P-wave keeps K of the group's 32 keys and the dV^T accumulator:
//   S = Q K^T, P = exp(S - lse) (ALiBi, attn_bias, softcap, mask), dV^T +=
//   dO^T (F P) (F the dropout multipliers); it hands P times the softcap
//   derivative to its partner through LDS, in fp32;
// * the dS-wave keeps V and the dK^T accumulator: dP = dO V^T, dS =
//   (P softcap') (F dP - delta), dK^T += Q^T dS, one tile behind the P-wave.
// Each wave then holds half the registers, and while one wave works through
// its elementwise step the other can use the matrix core.  Per tile the
// P-wave reads Q rows and transposed dO, the dS-wave dO rows and transposed
// Q, each 1 KiB per product as before, plus 4 KiB of P per 32 rows.  dS is
// (P softcap') (F dP - delta) in fp32, the one-wave form's P (F dP - delta)
// softcap' with the softcap factor applied first.
#pragma once

#include <climits>
#include <type_traits>

#include "fa_bwd_kernel.h"

namespace fa {

// Q and dO tiles of BM rows in NS LDS stages (DMA issued two tiles ahead, so
// the stage of tile t - 1, which the dS-waves read while the P-waves work on
// tile t, is not refilled before both are done with it), followed by two P
// exchange buffers (tile parity) of 32 keys x BM rows in fp32 per key group.
template <class T, int D, int BM, int NS>
struct BwdDkvSplitTile {
  static constexpr int KG = 4;                   // key groups of 32 keys
  static constexpr int NW = 2 * KG;              // a P-wave and a dS-wave per group
  static constexpr int BN = 32 * KG;
  static constexpr int NT = 64 * NW;
  static constexpr int TILEB = BM * D * 2;       // bytes of one Q or dO stage
  static constexpr int IPS = TILEB / 1024;       // 1-KiB DMA instructions per Q (or dO) stage
  static constexpr int IPW = 2 * IPS / NW;       // per wave: waves [0, NW/2) load Q, the rest dO
  static constexpr int LPS = IPW + 1;            // DMA instructions per wave per stage (+ LSE or delta)
  static constexpr int FB = 256;                 // bytes of one LSE / delta stage
  static constexpr int PB = 32 * BM * 4;         // fp32 P of one key group and tile
  static constexpr int STAGES_B = NS * (2 * TILEB + 2 * FB);
  static constexpr int LDS_BYTES = STAGES_B + 2 * KG * PB;   // + 4 B per head of the group (ALiBi)
  static_assert(IPW * NW == 2 * IPS && IPW > 0, "Q and dO tiles must split evenly over the waves");
  static_assert(BM <= 64 && BM % 32 == 0, "one DMA lane per row for LSE / delta");
  static_assert(NW * 32 * (2 * D + 16) <= LDS_BYTES, "output staging must fit");
};

template <class T, int D, int BM, int NS, bool GENERIC, bool VARLEN, bool BIAS = false>
__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(2, 2)))
void bwd_dkdv_split_kernel(const BwdParams p) {
  static_assert(!BIAS || (GENERIC && !VARLEN), "attn_bias: generic dense kernels only");
  static_assert(NS == 4, "the loops are unrolled for four stages");
  using Tile = BwdDkvSplitTile<T, D, BM, NS>;
  constexpr int KG = Tile::KG, BN = Tile::BN, NW = Tile::NW, TILEB = Tile::TILEB;
  constexpr int IPW = Tile::IPW, LPS = Tile::LPS, FB = Tile::FB, PB = Tile::PB;
  constexpr int NKC = D / 16, NDB = D / 32, NRB = BM / 32, NCC = BM / 16;
  constexpr int PD = 2;                          // DMA distance in tiles

  extern __shared__ __attribute__((aligned(16))) uint16_t smem[];
  uint8_t* const smem_b = reinterpret_cast<uint8_t*>(smem);
  uint8_t* const pbuf = smem_b + Tile::STAGES_B;
  float* const slopes_lds = reinterpret_cast<float*>(smem_b + Tile::LDS_BYTES);

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int grp = w % KG;                        // key group
  const bool dsw = w >= KG;                      // the dS-wave of the group
  const int c32 = lane & 31;
  const int g = lane >> 5;

  // ------------------------------------------------------------ work item
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
  const int kj = key0 + grp * 32 + c32;
  const bool key_valid = kj < Sk;
  const int qoff = (int)p.q_offset;
  const int wl = p.window_left, wr = p.window_right;
  const bool causal = p.causal != 0;

  // K (P-wave) or V (dS-wave) row of this lane's key: the B operand of
  // S = Q K^T or dP = dO V^T.
  u32x4 kv[NKC];
  {
    const uint16_t* row =
        dsw ? static_cast<const uint16_t*>(p.v) + row_base(p, p.v_sb, p.v_ss, p.v_sh, b, kvh, ks) +
                  (int64_t)kj * p.v_ss
            : static_cast<const uint16_t*>(p.k) + row_base(p, p.k_sb, p.k_ss, p.k_sh, b, kvh, ks) +
                  (int64_t)kj * p.k_ss;
#pragma unroll
    for (int kc = 0; kc < NKC; ++kc) {
      const u32x4 z = {0, 0, 0, 0};
      kv[kc] = key_valid ? load16(row + kc * 16 + g * 8) : z;
    }
    if (GENERIC && p.alibi != nullptr) {
      for (int gi = tid; gi < p.group; gi += NW * 64)
        slopes_lds[gi] = p.alibi[(int64_t)b * p.alibi_sb + kvh * p.group + gi];
    }
    __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));
  }

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
  const int J = NM * p.group;   // work items: (query head kvh * group + it / NM, m-block m_begin + it % NM)

  const int wk0 = key0 + grp * 32;
  const int wk1 = min(wk0 + 31, Sk - 1);
  // Query positions that see this lane's key: [vis_lo, vis_hi] (causal: from
  // the key on; window (wl, wr): kj - wr .. kj + wl), never empty, so that a
  // position is visible iff (unsigned)(qpos - vis_lo) <= vis_span.
  int vis_lo = INT_MIN, vis_hi = INT_MAX;
  if (causal) vis_lo = kj;
  if (wr >= 0) vis_lo = max(vis_lo, kj - wr);
  if (wl >= 0) vis_hi = (int)min((int64_t)kj + wl, (int64_t)INT_MAX);
  const uint32_t vis_span = (uint32_t)vis_hi - (uint32_t)vis_lo;
  auto wave_masks = [&](int m0) {
    const int p0 = m0 + qoff, p1 = m0 + BM - 1 + qoff;
    bool need = false;
    if (causal) need = need || p0 < wk1;
    if (wr >= 0) need = need || p0 + wr < wk1;
    if (wl >= 0) need = need || p1 - wl > wk0;
    return need;
  };

  // ------------------------------------------------------------ DMA stream
  // As in bwd_dkdv_kernel: waves [0, NW/2) copy Q tiles, the others dO tiles,
  // with running sources; odd waves copy the delta rows, even waves the LSE.
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
  int ld_m = m_begin, ld_left = J;
  auto clamp32 = [](int64_t v) { return v > 0xffffffffll ? 0xffffffffu : (uint32_t)v; };
  auto issue = [&](int stage) {   // the next tile into `stage`; past J an empty load
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

  // Per-lane byte offsets within a stage: the row reads of S / dP (row
  // rb*32 + c32, chunk 2 kc + g) and the halves of the transposed reads.
  uint32_t rd_ofs[NRB * NKC];
  uint32_t tr_ofs[NCC * NDB * 2];
#pragma unroll
  for (int rb = 0; rb < NRB; ++rb)
#pragma unroll
    for (int kc = 0; kc < NKC; ++kc)
      rd_ofs[rb * NKC + kc] = 2u * (uint32_t)swz_off<D>(rb * 32 + c32, 2 * kc + g);
  {
    const int j = lane & 15;
#pragma unroll
    for (int cc = 0; cc < NCC; ++cc)
#pragma unroll
      for (int db = 0; db < NDB; ++db) {
        const int r = 16 * cc + 4 * g + (j >> 2);
        const int d = db * 32 + 16 * (c32 >> 4) + 4 * (j & 3);
        tr_ofs[(cc * NDB + db) * 2] = 2u * (uint32_t)(swz_off<D>(r, d >> 3) + (d & 7));
        tr_ofs[(cc * NDB + db) * 2 + 1] = 2u * (uint32_t)(swz_off<D>(r + 8, d >> 3) + (d & 7));
      }
  }
  auto tr_read = [&](const uint8_t* base, int cc, int db) {
    const u32x2 lo = lds_read_tr16(reinterpret_cast<const uint16_t*>(base + tr_ofs[(cc * NDB + db) * 2]));
    const u32x2 hi =
        lds_read_tr16(reinterpret_cast<const uint16_t*>(base + tr_ofs[(cc * NDB + db) * 2 + 1]));
    return u32x4{lo[0], lo[1], hi[0], hi[1]};
  };

  f32x16 acc[NDB];   // dV^T (P-wave) or dK^T (dS-wave)
#pragma unroll
  for (int db = 0; db < NDB; ++db) acc[db] = f32x16{};
  int mm_m = m_begin, mm_h = 0;   // m-block and head-in-group of this wave's next tile

  // Products with the row operand (Q rows for the P-wave, dO rows for the
  // dS-wave) of a stage: S or dP of one tile.
  auto row_products = [&](const uint8_t* Rb, f32x16 (&sp)[NRB]) __attribute__((always_inline)) {
#pragma unroll
    for (int rb = 0; rb < NRB; ++rb) {
      sp[rb] = f32x16{};
      u32x4 ra[NKC];
#pragma unroll
      for (int kc = 0; kc < NKC; ++kc) ra[kc] = *reinterpret_cast<const u32x4*>(Rb + rd_ofs[rb * NKC + kc]);
#pragma unroll
      for (int kc = 0; kc < NKC; ++kc) sp[rb] = T::mfma32(ra[kc], kv[kc], sp[rb]);
      __builtin_amdgcn_sched_group_barrier(0x100, NKC, 0);   // LDS reads
      __builtin_amdgcn_sched_group_barrier(0x008, NKC, 0);   // MFMAs
      __builtin_amdgcn_sched_barrier(0);
    }
  };
  constexpr int NTA = NCC * NDB;
  // Transposed operand (dO^T for the P-wave, Q^T for the dS-wave) and the
  // products that accumulate dV^T / dK^T.
  auto tr_operands = [&](const uint8_t* Tb, u32x4 (&ta)[NTA]) __attribute__((always_inline)) {
#pragma unroll
    for (int cc = 0; cc < NCC; ++cc)
#pragma unroll
      for (int db = 0; db < NDB; ++db) ta[cc * NDB + db] = tr_read(Tb, cc, db);
  };
  auto tr_products = [&](const u32x4 (&ta)[NTA], const u32x4 (&bop)[NCC]) __attribute__((always_inline)) {
#pragma unroll
    for (int cc = 0; cc < NCC; ++cc)
#pragma unroll
      for (int db = 0; db < NDB; ++db) acc[db] = T::mfma32(ta[cc * NDB + db], bop[cc], acc[db]);
  };
  auto advance = [&]() {
    if (++mm_m == m_end) {
      mm_m = m_begin;
      ++mm_h;
    }
  };
  auto p_of = [&](int pslot) {   // this lane's slice of a P exchange buffer
    return reinterpret_cast<float*>(pbuf + (pslot * KG + grp) * PB) + lane * 4;
  };

  // P-wave, one tile in stage `stage`: S, P (written to the exchange buffer
  // `pslot`, times the softcap derivative), dV^T += dO^T (F P).
  auto p_tile = [&](int stage, int pslot) __attribute__((always_inline)) {
    const uint8_t* Qb = smem_b + stage * TILEB;
    const uint8_t* Db = smem_b + (NS + stage) * TILEB;
    const float* Ls = reinterpret_cast<const float*>(smem_b + 2 * NS * TILEB + stage * FB);
    float* const Pw = p_of(pslot);
    const int hq = kvh * p.group + mm_h, m0 = mm_m * BM;
    f32x16 sp[NRB];
    row_products(Qb, sp);
    // The transposed reads go ahead of the elementwise step, which hides
    // their latency; the generic kernels read them after it, for registers.
    u32x4 ta[NTA];
    if constexpr (!GENERIC) tr_operands(Db, ta);
    __builtin_amdgcn_sched_barrier(0);
    u32x4 bop[NCC];
    float slope = 0.f;
    if (GENERIC && p.alibi != nullptr) slope = slopes_lds[mm_h];
    f32x4 pc[NRB * 4];   // P times the softcap derivative, in accumulator order
    auto elem = [&](auto masked_c) __attribute__((always_inline)) {
      constexpr bool MASKED = decltype(masked_c)::value;
#pragma unroll
      for (int cc = 0; cc < NCC; ++cc) {
        const int rb = cc >> 1, o8 = (cc & 1) * 8;
        const int r0 = 16 * cc + 4 * g;
        const f32x4 l0 = *reinterpret_cast<const f32x4*>(Ls + r0);
        const f32x4 l1 = *reinterpret_cast<const f32x4*>(Ls + r0 + 8);
        const uint32_t vis_x = (uint32_t)(m0 + r0 + qoff) - (uint32_t)vis_lo;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          float pv[2];
#pragma unroll
          for (int u = 0; u < 2; ++u) {
            const int v = o8 + 2 * j + u;
            const int rr = 2 * j + u;
            const float lse = rr < 4 ? l0[rr] : l1[rr - 4];
            const float lse2 = lse * kLog2e;
            const int row = m0 + r0 + (rr & 3) + (rr >= 4 ? 8 : 0);
            const int qpos = row + qoff;
            float cg;
            const float bv = BIAS && bias_col != nullptr && row < Sq
                                 ? bias_col[(int64_t)hq * p.bias_sh + (int64_t)row * p.bias_sq]
                                 : 0.f;
            float pr = bwd_prob<GENERIC, BIAS>(p, sp[rb][v], lse2, slope, qpos, kj, bv, cg);
            if (MASKED) {
              const uint32_t x = vis_x + (uint32_t)((rr & 3) + (rr >= 4 ? 8 : 0));   // qpos - vis_lo
              pr = x <= vis_span ? pr : 0.f;
            }
            pv[u] = pr;
            if (GENERIC && p.drop.enabled) pv[u] = pr * dropout_factor_at(p.drop, row, kj, hq, b);
            pc[(rb * 16 + v) >> 2][v & 3] = pr * cg;
          }
          bop[cc][j] = T::pack2(pv[0], pv[1]);
        }
      }
    };
    if (wave_masks(m0))
      elem(std::true_type{});
    else
      elem(std::false_type{});
#pragma unroll
    for (int q = 0; q < NRB * 4; ++q) *reinterpret_cast<f32x4*>(Pw + q * 256) = pc[q];
    if constexpr (GENERIC) tr_operands(Db, ta);
    tr_products(ta, bop);
    advance();
  };

  // dS-wave, the back half of a tile in stage `stage` whose dP is `dp`:
  // dS from the P in exchange buffer `pslot`, dK^T += Q^T dS.
  auto ds_tile = [&](const f32x16 (&dp)[NRB], int stage, int pslot) __attribute__((always_inline)) {
    const uint8_t* Qb = smem_b + stage * TILEB;
    const float* Es = reinterpret_cast<const float*>(smem_b + 2 * NS * TILEB + (NS + stage) * FB);
    const float* Pw = p_of(pslot);
    const int hq = kvh * p.group + mm_h, m0 = mm_m * BM;
    u32x4 ta[NTA];
    if constexpr (!GENERIC) tr_operands(Qb, ta);
    u32x4 bop[NCC];
#pragma unroll
    for (int cc = 0; cc < NCC; ++cc) {
      const int rb = cc >> 1, o8 = (cc & 1) * 8;
      const int r0 = 16 * cc + 4 * g;
      const f32x4 e0 = *reinterpret_cast<const f32x4*>(Es + r0);
      const f32x4 e1 = *reinterpret_cast<const f32x4*>(Es + r0 + 8);
      const f32x4 pa = *reinterpret_cast<const f32x4*>(Pw + ((rb * 16 + o8) >> 2) * 256);
      const f32x4 pbv = *reinterpret_cast<const f32x4*>(Pw + (((rb * 16 + o8) >> 2) + 1) * 256);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        float ds[2];
#pragma unroll
        for (int u = 0; u < 2; ++u) {
          const int rr = 2 * j + u;
          const float dl = rr < 4 ? e0[rr] : e1[rr - 4];
          const float pcv = rr < 4 ? pa[rr] : pbv[rr - 4];
          const int v = o8 + 2 * j + u;
          float dpv = dp[rb][v];
          if (GENERIC && p.drop.enabled) {
            const int row = m0 + r0 + (rr & 3) + (rr >= 4 ? 8 : 0);
            dpv *= dropout_factor_at(p.drop, row, kj, hq, b);
          }
          ds[u] = pcv * (dpv - dl);
        }
        bop[cc][j] = T::pack2(ds[0], ds[1]);
      }
    }
    if constexpr (GENERIC) tr_operands(Qb, ta);
    tr_products(ta, bop);
    advance();
  };

  // ------------------------------------------------------------ main loop
  // J + 1 rounds, each opened by one workgroup barrier.  In round t the
  // P-waves do tile t (t < J); the dS-waves finish tile t - 1 (t >= 1) with
  // the P that the P-waves wrote in round t - 1, then compute dP of tile t
  // (t < J), which tile t's stage already holds.  Their phases so differ:
  // while a P-wave computes S a dS-wave works through its elementwise step,
  // and while the P-wave computes P the dS-wave runs its dK products.  The
  // wait before each barrier covers the DMA of the round's tile (at most one
  // newer tile in flight) and the P-waves' LDS writes.
#pragma unroll
  for (int s = 0; s < PD; ++s) issue(s);
  auto top = [&](int ts) __attribute__((always_inline)) {
    __builtin_amdgcn_s_waitcnt(vmcnt_imm((PD - 1) * LPS) & ~0x3f00);   // and lgkmcnt(0)
    __builtin_amdgcn_sched_barrier(0);
    asm volatile("s_barrier" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);
    issue((ts + PD) % NS);
  };
  auto unrolled = [&](auto&& round) __attribute__((always_inline)) {
    int t = 0;
    for (; t + NS <= J + 1; t += NS) {
      round(t, 0);
      round(t + 1, 1);
      round(t + 2, 2);
      round(t + 3, 3);
    }
    if (t < J + 1) round(t, 0);
    if (t + 1 < J + 1) round(t + 1, 1);
    if (t + 2 < J + 1) round(t + 2, 2);
  };
  if (!dsw) {
    unrolled([&](int t, int ts) __attribute__((always_inline)) {
      top(ts);
      if (t < J) p_tile(ts, ts & 1);
    });
  } else {
    f32x16 dp[NRB];
#pragma unroll
    for (int rb = 0; rb < NRB; ++rb) dp[rb] = f32x16{};
    unrolled([&](int t, int ts) __attribute__((always_inline)) {
      top(ts);
      if (t >= 1) ds_tile(dp, (ts + NS - 1) % NS, (ts + 1) & 1);
      if (t < J) row_products(smem_b + (NS + ts) * TILEB, dp);
    });
  }
  __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));

  // ------------------------------------------------------------ dK = scale * dK^T, dV
  __syncthreads();
  uint8_t* const st = smem_b + w * 32 * (2 * D + 16);
  const int rows_ok = Sk - wk0;
  if (dsw)
    store_rows_staged<T, D>(acc, p.scale, st, c32, g, lane,
                            static_cast<uint16_t*>(p.dk) +
                                row_base(p, p.dk_sb, p.dk_ss, p.dk_sh, b, kvh, ks) +
                                (int64_t)wk0 * p.dk_ss,
                            p.dk_ss, rows_ok);
  else
    store_rows_staged<T, D>(acc, 1.f, st, c32, g, lane,
                            static_cast<uint16_t*>(p.dv) +
                                row_base(p, p.dv_sb, p.dv_ss, p.dv_sh, b, kvh, ks) +
                                (int64_t)wk0 * p.dv_ss,
                            p.dv_ss, rows_ok);
}

}  // namespace fa
