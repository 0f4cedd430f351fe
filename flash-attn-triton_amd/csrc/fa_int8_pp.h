// Ping-pong INT8-QK^T attention forward for gfx950 at head dim 128.
//
// Semantics are those of int8_fwd_kernel (fa_int8.hip), i.e. the reference's
// _attn_fwd_int8 / _attn_fwd_int8_inner
// (/root/reference/flash_attn_triton/triton_kernel/attention_kernel_int8.py:82-141,
// :167-217): Q quantized per row in the prologue (division form, bit-exact
// with :100), S^T = K8 Q8^T in int32, scores i32 * s_k[key] * s_q *
// sm_scale * log2(e), online softmax, O^T += V^T P^T in fp16 with P rounded
// to fp16.
//
// The schedule is that of prefill_pp_kernel (fa_prefill_pp.h): a 512-thread
// workgroup owns 256 query rows (32 per wave); waves 0-3 and 4-7 alternate
// between a GEMM phase (S^T_j on v_mfma_i32_32x32x32_i8 and
// O^T += V_{j-1}^T P_{j-1} on v_mfma_f32_32x32x16_f16: 8 + 16 MFMAs per wave
// and 64-key tile, against 16 + 16 with fp16 scores) and a softmax phase,
// separated by workgroup barriers, so each SIMD's matrix core is fed by one
// of its two waves while the other exponentiates.
//
// LDS, four stages per operand, filled by the buffer loads' LDS mode:
//   K8 tile : 64 rows x 128 B; 16-byte chunk c of row r at c ^ ((r >> 1) & 7),
//             so the 16 rows that one ds_read_b128 quarter-wave reads (one
//             chunk column) fall into 16 distinct 16-byte bank groups;
//   V tile  : 64 rows x 256 B, chunk c of row r at c ^ 4 (r & 3), as in the
//             fp16 kernel (ds_read_b64_tr_b16 transpose reads);
//   s_k     : the tile's 64 key scales.
#pragma once

#include "fa_int8.h"
#include "fa_prefill_pp.h"

namespace fa {

template <int D>
struct Int8PingPongTile {
  static constexpr int NW = 8;
  static constexpr int NT = 512;
  static constexpr int BM = 256;             // query rows per workgroup
  static constexpr int BN = 64;              // keys per tile
  static constexpr int NS = 4;               // LDS stages per operand
  static constexpr int KROWB = D;            // bytes per K8 row
  static constexpr int VROWB = 2 * D;        // bytes per V row
  static constexpr int KTILEB = BN * KROWB;
  static constexpr int VTILEB = BN * VROWB;
  static constexpr int SKB = BN * 4;
  static constexpr int V_OFF = NS * KTILEB;
  static constexpr int SK_OFF = V_OFF + NS * VTILEB;
  static constexpr int LDS_BYTES = SK_OFF + NS * SKB;
  static constexpr int KRPI = 1024 / KROWB;  // K8 rows per 1-KiB load instruction
  static constexpr int VRPI = 1024 / VROWB;  // V rows per 1-KiB load instruction
  static constexpr int KIPW = KTILEB / 1024 / NW;
  static constexpr int VIPW = VTILEB / 1024 / NW;
  static constexpr int LPS = KIPW + VIPW + 1;  // load instructions per wave per softmax step
  static_assert(D == 128, "the INT8 ping-pong tiles are laid out for head dim 128");
  static_assert(KIPW * NW * 1024 == KTILEB && VIPW * NW * 1024 == VTILEB,
                "tiles must split evenly over the waves");
};

template <int D>
__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(2, 2)))
void int8_pp_kernel(const Int8Params p) {
  using Tile = Int8PingPongTile<D>;
  constexpr int BM = Tile::BM;
  constexpr int BN = Tile::BN;
  constexpr int NS = Tile::NS;
  constexpr int KROWB = Tile::KROWB;
  constexpr int VROWB = Tile::VROWB;
  constexpr int KTILEB = Tile::KTILEB;
  constexpr int VTILEB = Tile::VTILEB;
  constexpr int SKB = Tile::SKB;
  constexpr int KIPW = Tile::KIPW;
  constexpr int VIPW = Tile::VIPW;
  constexpr int NKC = D / 32;      // 32-dim k-steps of the int8 S^T
  constexpr int NDB = D / 32;      // 32-dim blocks of O^T
  constexpr int NKB = BN / 32;     // 32-key blocks per tile
  constexpr int NCC = BN / 16;     // 16-key k-steps of O^T

  extern __shared__ __attribute__((aligned(1024))) uint8_t smem_i8pp[];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int grp = w >> 2;             // 0: GEMM first, 1: softmax first
  const int rb = 2 * (w & 3) + grp;   // this wave's 32-row block
  const int c32 = lane & 31;
  const int g = lane >> 5;

  // ------------------------------------------------------------ work item
  int mb, bh;
  work_item(blockIdx.x, p.total_blocks, p.n_mblocks, p.causal != 0, kCausalSpan, mb, bh);
  const int h = bh % p.heads;
  const int b = bh / p.heads;
  const int S = p.seqlen;
  const int qoff = p.seq_len_k - p.seq_len_q;
  const int Sk = p.seq_len_k < S ? p.seq_len_k : S;

  const int row0 = mb * BM;
  const int row_last = min(row0 + BM, S) - 1;
  const int wrow0 = row0 + 32 * rb;
  const int qi = wrow0 + c32;
  const bool row_valid = qi < S;
  const int qpos = qi + qoff;
  const int qpos_w_min = wrow0 + qoff;
  const bool causal = p.causal != 0;
  int key_hi = Sk - 1;
  if (causal) key_hi = min(key_hi, qpos);
  int k_hi = Sk;
  if (causal) k_hi = min(k_hi, row_last + qoff + 1);
  const int J = k_hi > 0 ? (k_hi + BN - 1) / BN : 0;

  // ------------------------------------------------------------ Q8^T in VGPRs
  // Lane (c32, g) holds dims [32 kc + 16 g, +16) of row qi: the B operand of
  // v_mfma_i32_32x32x32_i8.  The quotient x / s_q is the IEEE division's
  // (quant_div), bit-exact with the reference's division form.
  i32x4 q8[NKC];
  float row_scale;
  {
#pragma clang fp contract(off)
    const uint16_t* qrow = static_cast<const uint16_t*>(p.q) + (int64_t)b * p.q_sb +
                           (int64_t)h * p.q_sh + (int64_t)qi * p.q_ss;
    float qf[NKC][16];
    float amax = 0.f;
#pragma unroll
    for (int kc = 0; kc < NKC; ++kc) {
#pragma unroll
      for (int half = 0; half < 2; ++half) {
        const u32x4 raw =
            row_valid ? load16(qrow + kc * 32 + g * 16 + half * 8) : u32x4{0, 0, 0, 0};
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const float f = F16::to_float((uint16_t)(raw[e >> 1] >> ((e & 1) * 16)));
          qf[kc][half * 8 + e] = f;
          amax = fmaxf(amax, fabsf(f));
        }
      }
    }
    amax = halves_max(amax);
    const float s_q = fmaxf(amax, 1.0f) / 127.0f;
    const float inv_q = 1.0f / s_q;
#pragma unroll
    for (int kc = 0; kc < NKC; ++kc) {
#pragma unroll
      for (int wd = 0; wd < 4; ++wd) {
        q8[kc][wd] = (int)pack_i8x4_i(round_half_away_i(quant_div(qf[kc][4 * wd + 0], s_q, inv_q)),
                                      round_half_away_i(quant_div(qf[kc][4 * wd + 1], s_q, inv_q)),
                                      round_half_away_i(quant_div(qf[kc][4 * wd + 2], s_q, inv_q)),
                                      round_half_away_i(quant_div(qf[kc][4 * wd + 3], s_q, inv_q)));
      }
    }
    row_scale = s_q * p.scale_log2;
  }

  // ------------------------------------------------------------ tile loads
  const int8_t* k8g = p.k8 + (int64_t)bh * S * D;
  const float* skg = p.s_k + (int64_t)bh * S;
  const uint16_t* vg = static_cast<const uint16_t*>(p.v) + (int64_t)b * p.v_sb + (int64_t)h * p.v_sh;
  const uint32_t v_row_b = (uint32_t)(p.v_ss * 2);
  // Lane l of this wave's i-th instruction writes physical chunk l % (row
  // chunks) of a row, so it loads the logical chunk the swizzle puts there.
  uint32_t k_off[KIPW], v_off[VIPW];
#pragma unroll
  for (int i = 0; i < KIPW; ++i) {
    const int r = Tile::KRPI * (KIPW * w + i) + (lane >> 3);
    k_off[i] = (uint32_t)r * KROWB + (uint32_t)(((lane & 7) ^ ((r >> 1) & 7)) * 16);
  }
#pragma unroll
  for (int i = 0; i < VIPW; ++i) {
    const int r = Tile::VRPI * (VIPW * w + i) + (lane >> 4);
    v_off[i] = (uint32_t)r * v_row_b + (uint32_t)(((lane & 15) ^ (4 * (r & 3))) * 16);
  }
  uint8_t* const k_lds = smem_i8pp;
  uint8_t* const v_lds = smem_i8pp + Tile::V_OFF;
  const uint8_t* const sk_lds = smem_i8pp + Tile::SK_OFF;
  const uint32_t k_lds_a = lds_address(k_lds) + KIPW * w * 1024;
  const uint32_t v_lds_a = lds_address(v_lds) + VIPW * w * 1024;
  const uint32_t sk_lds_a = lds_address(sk_lds);
  const uint32_t sk_voff = (uint32_t)lane * 4;
  // K8 tile rel and its key scales (every wave copies the 64 scales; the
  // copies are identical).  Tiles past J get an empty resource: the
  // instructions still retire (keeping the wait counts uniform) and write
  // zeros.
  auto load_k = [&](int rel) {
    const int n0 = rel * BN;
    const bool live = rel < J;
    const uint32_t left = live && n0 < Sk ? (uint32_t)(Sk - n0) : 0u;
    const u32x4 rk = make_rsrc_words(k8g + (int64_t)(live ? n0 : 0) * D, left * D);
    const uint32_t dst = k_lds_a + (rel % NS) * KTILEB;
#pragma unroll
    for (int i = 0; i < KIPW; ++i) buf_load16_lds(rk, dst + i * 1024, k_off[i]);
    const u32x4 rs = make_rsrc_words(skg + (live ? n0 : 0), left * 4);
    buf_load4_lds(rs, sk_lds_a + (rel % NS) * SKB, sk_voff);
  };
  // The same for a tile the caller knows is whole and inside the key range
  // (no selects, fixed extents).
  const uint32_t v_tile_ext = rows_extent(0, BN, p.v_ss, D);
  auto load_k_full = [&](int rel) {
    const int n0 = rel * BN;
    const u32x4 rk = make_rsrc_words(k8g + (int64_t)n0 * D, (uint32_t)(BN * D));
    const uint32_t dst = k_lds_a + (rel % NS) * KTILEB;
#pragma unroll
    for (int i = 0; i < KIPW; ++i) buf_load16_lds(rk, dst + i * 1024, k_off[i]);
    const u32x4 rs = make_rsrc_words(skg + n0, (uint32_t)(BN * 4));
    buf_load4_lds(rs, sk_lds_a + (rel % NS) * SKB, sk_voff);
  };
  auto load_v_full = [&](int rel) {
    const u32x4 rs = make_rsrc_words(vg + (int64_t)(rel * BN) * p.v_ss, v_tile_ext);
    const uint32_t dst = v_lds_a + (rel % NS) * VTILEB;
#pragma unroll
    for (int i = 0; i < VIPW; ++i) buf_load16_lds(rs, dst + i * 1024, v_off[i]);
  };
  auto load_v = [&](int rel) {
    const int n0 = rel * BN;
    const uint32_t ext = rel < J ? rows_extent(n0, Sk, p.v_ss, D) : 0u;
    const u32x4 rs = make_rsrc_words(vg + (int64_t)(rel < J ? n0 : 0) * p.v_ss, ext);
    const uint32_t dst = v_lds_a + (rel % NS) * VTILEB;
#pragma unroll
    for (int i = 0; i < VIPW; ++i) buf_load16_lds(rs, dst + i * 1024, v_off[i]);
  };

  // LDS read offsets.  K8 (A operand, 16 B per lane): key row kb*32 + c32,
  // logical chunk 2 kc + g.  V^T: as prefill_pp_kernel.
  uint32_t k_ofs[NKC], v_ofs[NDB];
#pragma unroll
  for (int kc = 0; kc < NKC; ++kc)
    k_ofs[kc] = (uint32_t)c32 * KROWB +
                (((uint32_t)(2 * kc + g)) ^ (uint32_t)((c32 >> 1) & 7)) * 16;
  {
    const int j16 = lane & 15;
    const uint32_t v_rd = (uint32_t)(4 * g + (j16 >> 2)) * VROWB + (uint32_t)((j16 & 1) * 8);
    const int v_cx = 2 * (c32 >> 4) + ((j16 & 3) >> 1);
    const int v_sw = j16 >> 2;
#pragma unroll
    for (int db = 0; db < NDB; ++db)
      v_ofs[db] = v_rd + ((((uint32_t)db ^ (uint32_t)v_sw) << 2) + (uint32_t)v_cx) * 16;
  }
  auto v_read = [&](const uint8_t* Vs, int db, int cc) {
    const uint16_t* vp = reinterpret_cast<const uint16_t*>(Vs + v_ofs[db] + cc * 16 * VROWB);
    const u32x2 lo = lds_read_tr16(vp);
    const u32x2 hi = lds_read_tr16(vp + 8 * D);
    return u32x4{lo[0], lo[1], hi[0], hi[1]};
  };

  auto wave_masks = [&](int rel) {
    const int n1 = (rel + 1) * BN;
    bool need = n1 > Sk;
    if (causal) need = need || n1 - 1 > qpos_w_min;
    return need;
  };

  f32x16 acc[NDB];
#pragma unroll
  for (int db = 0; db < NDB; ++db) acc[db] = f32x16{};
  float m_run = -INFINITY;   // running (possibly stale) max, log2 units
  float m_c = 0.f;           // finite max P is taken against
  float l_run = 0.f;
  // Exponents of the current tile, i32 * s_k[key] * s_q * scale * log2(e) - m_c.
  f32x16 s[NKB];
  u32x4 pbuf[NCC];
  // B operand of the coefficient product below: this lane's row scale in
  // k-slot 0 (lanes 0-31), zero in k-slot 1 (lanes 32-63).
  const float coef_b = g == 0 ? row_scale : 0.f;

  constexpr int NQK = NKC * NKB;
  constexpr int NPV = NDB * NCC;
  // One GEMM phase: S^T = K8 Q8^T from K stage kst (DO_QK) and
  // O^T += V^T P^T from V stage vst (DO_PV), operand reads running ahead of
  // the products as in prefill_pp_kernel.  The wave then turns its own
  // int32 scores into exponents, fma(i32, coef, -m_c) with the per-(key, row)
  // coefficients from two fp32 outer products: that VALU work sits under
  // the PV products, where a wave hides a few VALU instructions behind each
  // of its own MFMAs, instead of in the softmax phase, where every VALU
  // instruction slows the other wave's products, and the softmax phase is
  // left with the max, exp2, packing and row sums of the fp16 kernel.
  auto gemm = [&](int kst, int vst, auto do_qk_c, auto do_pv_c) {
    constexpr bool DO_QK = decltype(do_qk_c)::value;
    constexpr bool DO_PV = decltype(do_pv_c)::value;
    // V^T operands read in the first scheduling region (with the S^T chain).
    constexpr int NVA0 = DO_QK ? 4 : NPV;
    __builtin_amdgcn_s_setprio(1);
    const uint8_t* Ks = k_lds + kst * KTILEB;
    const uint8_t* Vs = v_lds + vst * VTILEB;
    const float* skl = reinterpret_cast<const float*>(sk_lds + kst * SKB);
    u32x4 ka[DO_QK ? NQK : 1];
    float ska[DO_QK ? NKB : 1];
    u32x4 va[DO_PV ? NPV : 1];
    i32x16 si[DO_QK ? NKB : 1];
    f32x16 coef[DO_QK ? NKB : 1];
    // Region 1: the S^T chain (or, without it, the whole O^T update).
    if constexpr (DO_QK) {
#pragma unroll
      for (int i = 0; i < NQK; ++i)
        ka[i] = *reinterpret_cast<const u32x4*>(Ks + k_ofs[i / NKB] + (i % NKB) * 32 * KROWB);
      // A operand of the coefficient product: key kb*32 + c32's scale (the
      // same in both k-slots; the B operand's slot 1 is zero).
#pragma unroll
      for (int kb = 0; kb < NKB; ++kb) ska[kb] = skl[kb * 32 + c32];
    }
    if constexpr (DO_PV) {
#pragma unroll
      for (int i = 0; i < NVA0; ++i) va[i] = v_read(Vs, i / NCC, i % NCC);
    }
    if constexpr (DO_QK) {
#pragma unroll
      for (int kb = 0; kb < NKB; ++kb) si[kb] = i32x16{};
#pragma unroll
      for (int kc = 0; kc < NKC; ++kc)
#pragma unroll
        for (int kb = 0; kb < NKB; ++kb)
          si[kb] = __builtin_amdgcn_mfma_i32_32x32x32_i8(__builtin_bit_cast(i32x4, ka[kc * NKB + kb]),
                                                         q8[kc], si[kb], 0, 0, 0);
      // coef[kb] = s_k[key] * (s_q * scale * log2 e) for every (key, row) of
      // the S^T accumulator, as the outer product of the key scales and the
      // row scales on the fp32 matrix core (exact products, one rounding).
#pragma unroll
      for (int kb = 0; kb < NKB; ++kb)
        coef[kb] = __builtin_amdgcn_mfma_f32_32x32x2f32(ska[kb], coef_b, f32x16{}, 0, 0, 0);
      // Scheduling groups (0x100 = LDS read, 0x008 = MFMA, 0x002 = VALU).
      constexpr int NRD1 = NQK + NKB + (DO_PV ? 2 * NVA0 : 0);
      __builtin_amdgcn_sched_group_barrier(0x100, 8, 0);
#pragma unroll
      for (int i = 0; i < NQK; ++i) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        __builtin_amdgcn_sched_group_barrier(0x100, (NRD1 - 8 + NQK - 1) / NQK, 0);
      }
      __builtin_amdgcn_sched_group_barrier(0x008, NKB, 0);
      __builtin_amdgcn_sched_barrier(0);
    }
    // Region 2: the O^T update with the remaining V^T reads, and the
    // conversion of the S^T scores under it.
    if constexpr (DO_PV) {
#pragma unroll
      for (int i = NVA0; i < NPV; ++i) va[i] = v_read(Vs, i / NCC, i % NCC);
#pragma unroll
      for (int db = 0; db < NDB; ++db)
#pragma unroll
        for (int cc = 0; cc < NCC; ++cc)
          acc[db] = F16::mfma32(va[db * NCC + cc], pbuf[cc], acc[db]);
    }
    if constexpr (DO_QK) {
      // (The empty asm keeps each product in this region: left alone, the
      // compiler sinks the conversion to its first use after the barrier.)
#pragma unroll
      for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          float t = fmaf((float)si[kb][v], coef[kb][v], -m_c);
          asm volatile("" : "+v"(t));
          s[kb][v] = t;
        }
    }
    if constexpr (DO_PV) {
      constexpr int NRD2 = 2 * (NPV - NVA0);
      constexpr int NVALU = DO_QK ? 2 * 16 * NKB : 0;
      if constexpr (!DO_QK) __builtin_amdgcn_sched_group_barrier(0x100, 8, 0);
      constexpr int RPER = DO_QK ? 2 : 2;
      constexpr int NRDG = DO_QK ? NRD2 : NRD2 - 8;
#pragma unroll
      for (int i = 0; i < NPV; ++i) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        if (i * RPER < NRDG) __builtin_amdgcn_sched_group_barrier(0x100, RPER, 0);
        if (NVALU > 0 && i >= 1)
          __builtin_amdgcn_sched_group_barrier(0x002, (NVALU + NPV - 2) / (NPV - 1), 0);
      }
    }
    __builtin_amdgcn_sched_barrier(0);
    __builtin_amdgcn_s_setprio(0);
  };

  // Softmax of tile rel: boundary mask, lazy max / O rescale (the exponents
  // move with m_c), P = exp2(s) packed as the B operand of pv, row sums
  // over the rounded P.
  auto softmax_tile = [&](int rel, bool masked) {
    if (masked) {
      const int hi0 = key_hi - rel * BN - 4 * g;
#pragma unroll
      for (int kb = 0; kb < NKB; ++kb) {
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          const int ko = kb * 32 + 8 * (v >> 2) + (v & 3);
          const uint32_t m = (uint32_t)((hi0 - ko) >> 31);
          const float sv = s[kb][v];
          s[kb][v] = __uint_as_float((__float_as_uint(sv) & ~m) | (m & 0xff800000u));
        }
      }
    }
    float mq[4] = {-INFINITY, -INFINITY, -INFINITY, -INFINITY};
#pragma unroll
    for (int kb = 0; kb < NKB; ++kb) {
#pragma unroll
      for (int v = 0; v < 16; v += 8) {
#pragma unroll
        for (int q = 0; q < 4; ++q)
          mq[q] = fmaxf(fmaxf(mq[q], s[kb][v + 2 * q]), s[kb][v + 2 * q + 1]);
      }
    }
    const float mx = halves_max(fmaxf(fmaxf(mq[0], mq[1]), fmaxf(mq[2], mq[3]))) + m_c;
    const bool raise = mx > m_run + kRescaleSlack;
    if (__builtin_amdgcn_ballot_w64(raise)) {
      const float m_new = raise ? mx : m_run;
      const float alpha = m_new == m_run ? 1.f : __builtin_amdgcn_exp2f(m_run - m_new);
      l_run *= alpha;
#pragma unroll
      for (int db = 0; db < NDB; ++db) acc[db] *= alpha;
      m_run = m_new;
      const float m_use = m_run == -INFINITY ? 0.f : m_run;
      const float shift = m_use - m_c;
#pragma unroll
      for (int kb = 0; kb < NKB; ++kb) s[kb] -= shift;
      m_c = m_use;
    }
    float lq[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int cc = 0; cc < NCC; ++cc) {
      const f32x16& sv = s[cc >> 1];
      const int o8 = (cc & 1) * 8;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const float e0 = __builtin_amdgcn_exp2f(sv[o8 + 2 * j]);
        const float e1 = __builtin_amdgcn_exp2f(sv[o8 + 2 * j + 1]);
        pbuf[cc][j] = F16::pack2(e0, e1);
        lq[j] = F16::sum2(pbuf[cc][j], lq[j]);
      }
    }
    l_run += (lq[0] + lq[1]) + (lq[2] + lq[3]);
  };

  // ------------------------------------------------------------ prologue
  // The Q loads retired in the quantization above; stages 0..NS-2 of K8 / s_k
  // and 0..NS-3 of V.
#pragma unroll
  for (int r = 0; r < NS - 1; ++r) load_k(r);
#pragma unroll
  for (int r = 0; r < NS - 2; ++r) load_v(r);
  __builtin_amdgcn_s_waitcnt(0x0f70);   // vmcnt(0)
  pp_barrier();

  // ------------------------------------------------------------ phases
  // As prefill_pp_kernel: GEMM(0), softmax(0), ..., softmax(J-1), GEMM(J)
  // with a barrier after each step, group 1 one barrier behind group 0.
  using yes = std::true_type;
  using no = std::false_type;
  // The wait that ends a softmax step.  Tile t's rows (K8, s_k of tile t,
  // V of tile t - 1) are loaded by both groups in their softmax step t - 3,
  // and the first GEMM to read them, group 0's GEMM(t), follows group 0's
  // softmax step t - 1 and group 1's softmax step t - 2 (group 1 runs one
  // phase behind): group 0 waits for its loads of two steps back, group 1
  // for those of one step back.
  auto step_wait = [&]() {
    if (grp == 0)
      __builtin_amdgcn_s_waitcnt(vmcnt_imm(2 * Tile::LPS));
    else
      __builtin_amdgcn_s_waitcnt(vmcnt_imm(Tile::LPS));
  };
  auto softmax_step = [&](int j) {
    load_k(j + NS - 1);
    load_v(j + NS - 2);
    softmax_tile(j, wave_masks(j));
    step_wait();
  };
  // Steps j < j_full: tile j is unmasked for every wave of the workgroup
  // and the tiles loaded (K8 j + 3, V j + 2) are live, whole and inside the
  // key range.
  auto softmax_step_full = [&](int j) {
    load_k_full(j + NS - 1);
    load_v_full(j + NS - 2);
    softmax_tile(j, false);
    step_wait();
  };
  int j_full = min(J - (NS - 1), Sk / BN - (NS - 1));
  if (causal) j_full = min(j_full, (row0 + qoff + 1) / BN);
  if (grp == 1) pp_barrier();
  if (J > 0) {
    gemm(0, 0, yes{}, no{});
    pp_barrier();
    if (j_full > 0)
      softmax_step_full(0);
    else
      softmax_step(0);
    pp_barrier();
    for (int j = 1; j < j_full; ++j) {
      gemm(j % NS, (j - 1) % NS, yes{}, yes{});
      pp_barrier();
      softmax_step_full(j);
      pp_barrier();
    }
    for (int j = j_full > 1 ? j_full : 1; j < J; ++j) {
      gemm(j % NS, (j - 1) % NS, yes{}, yes{});
      pp_barrier();
      softmax_step(j);
      pp_barrier();
    }
    gemm(0, (J - 1) % NS, no{}, yes{});
  }
  pp_barrier();
  if (grp == 0) pp_barrier();
  // No LDS write may still be in flight when the workgroup retires.
  __builtin_amdgcn_s_waitcnt(0x0f70);

  // ------------------------------------------------------------ epilogue
  const float l_tot = halves_sum(l_run);
  const float inv_l = l_tot > 0.f ? 1.f / l_tot : 0.f;
  if (!row_valid) return;
  uint16_t* orow = static_cast<uint16_t*>(p.o) + (int64_t)b * p.o_sb + (int64_t)h * p.o_sh +
                   (int64_t)qi * p.o_ss;
#pragma unroll
  for (int db = 0; db < NDB; ++db) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int d = db * 32 + r * 8 + g * 4;
      u32x2 val;
      val[0] = F16::pack2(acc[db][4 * r] * inv_l, acc[db][4 * r + 1] * inv_l);
      val[1] = F16::pack2(acc[db][4 * r + 2] * inv_l, acc[db][4 * r + 3] * inv_l);
      *reinterpret_cast<u32x2*>(orow + d) = val;
    }
  }
  if (p.lse != nullptr && g == 0)
    p.lse[((int64_t)b * p.heads + h) * S + qi] =
        l_tot > 0.f ? (m_run + __log2f(l_tot)) * kLn2 : -INFINITY;
}

}  // namespace fa
