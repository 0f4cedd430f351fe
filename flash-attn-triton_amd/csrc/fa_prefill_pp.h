// Ping-pong FlashAttention-2 prefill forward for gfx950 at head dim 128,
// fp16 / bf16 (dense, cross and varlen).
//
// Semantics are those of prefill_kernel (fa_prefill_kernel.h), i.e. the
// reference's dense and varlen forward kernels
// (/root/reference/flash_attn_triton/triton_kernel/attention_kernel.py:424-533,
// :275-372, :27-104).  The schedule is built around two measured properties
// of the CDNA4 SIMD:
//
// * An MFMA issued by one wave and VALU work (exp2, max, pack) issued by
//   another wave on the same SIMD run concurrently; inside one wave only a
//   few VALU instructions hide under each MFMA.
// * The two waves w and w + 4 of a 512-thread workgroup share a SIMD.
//
// So the workgroup's 8 waves form two groups, G0 = waves 0-3 and G1 = waves
// 4-7, which alternate between a GEMM phase and a softmax phase, separated by
// workgroup barriers.  While G0 runs the GEMM phase of key tile j
// (S_j = K_j Q^T and O^T += V_{j-1}^T P_{j-1}: 32 MFMAs per wave), G1 runs the
// softmax of tile j - 1 (VALU only), and the other way round in the next
// phase: each SIMD's matrix core is fed by one of its two waves in every
// phase.
//
// Tiles: a wave owns 32 query rows (row block 2 (w % 4) + w / 4, so both
// groups reach the causal diagonal at the same tile); keys come in tiles of
// 64.  K and V tiles are copied global -> LDS by the buffer loads' LDS mode
// (no VGPR staging): one instruction moves 64 x 16 bytes to 1 KiB of
// consecutive LDS.  Four stages per operand; the loads of K_{j+3} and V_{j+2}
// are issued in the softmax phase of tile j and waited for one softmax phase
// later, two phases before their first use.  Rows past the end of the
// sequence come back as zeros (raw buffer range check), so no load branches.
//
// LDS layout: rows of D = 128 halfs (256 B) without padding; the 16-byte
// chunk c of row r is stored at chunk position c ^ (r & 15) for K and
// c ^ 4 (r & 3) for V, so the K reads of the S^T product (16 rows, one chunk
// column per 16 lanes) and the V^T transpose reads (ds_read_b64_tr_b16, 4 rows
// x 4 chunks per 32 lanes) touch distinct bank groups.
#pragma once

#include <type_traits>

#include "fa_prefill_kernel.h"

namespace fa {

template <int D>
struct PingPongTile {
  static constexpr int NW = 8;
  static constexpr int NT = 512;
  static constexpr int BM = 256;          // query rows per workgroup (32 per wave)
  static constexpr int BN = 64;           // keys per tile
  static constexpr int NS = 4;            // LDS stages per operand
  static constexpr int ROWB = D * 2;      // bytes per K / V row
  static constexpr int TILEB = BN * ROWB; // bytes per K or V tile
  // Past the K and V rings: 8 KiB per wave of one group for staging Q and
  // output rows (stage_rows_* below).
  static constexpr int STAGE_OFF = 2 * NS * TILEB;
  static constexpr int LDS_BYTES = STAGE_OFF + 4 * 8192;
  static constexpr int RPI = 1024 / ROWB;              // rows per 1-KiB load instruction
  static constexpr int IPW = TILEB / 1024 / NW;        // load instructions per wave per tile
  static_assert(D == 128, "ping-pong tiles are laid out for head dim 128");
  static_assert(IPW * NW * 1024 == TILEB, "tile must split evenly over the waves");
};

// Workgroup barrier that the scheduler may not move instructions across (the
// phase structure depends on every MFMA of a GEMM phase being issued before
// it).  LDS visibility is handled by the kernel's explicit waits.
__device__ inline void pp_barrier() {
  __builtin_amdgcn_sched_barrier(0);
  asm volatile("s_barrier" ::: "memory");
  __builtin_amdgcn_sched_barrier(0);
}

// VARLEN: cu_seqlens addressing (an instantiation of its own, so that the
// dense kernel carries none of its work-item code).
template <class T, int D, bool VARLEN>
__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(2, 2)))
void prefill_pp_kernel(const FwdParams p) {
  using Tile = PingPongTile<D>;
  constexpr int BM = Tile::BM;
  constexpr int BN = Tile::BN;
  constexpr int NS = Tile::NS;
  constexpr int ROWB = Tile::ROWB;
  constexpr int TILEB = Tile::TILEB;
  constexpr int IPW = Tile::IPW;
  constexpr int RPI = Tile::RPI;
  constexpr int NKC = D / 16;      // 16-dim k-steps of S^T
  constexpr int NDB = D / 32;      // 32-dim blocks of O^T
  constexpr int NKB = BN / 32;     // 32-key blocks per tile
  constexpr int NCC = BN / 16;     // 16-key k-steps of O^T

  extern __shared__ __attribute__((aligned(1024))) uint8_t smem_pp[];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int grp = w >> 2;             // 0: GEMM first, 1: softmax first
  const int sid = w & 3;
  const int rb = 2 * sid + grp;       // this wave's 32-row block
  const int c32 = lane & 31;
  const int g = lane >> 5;

  // ------------------------------------------------------------ work item
  // Varlen: K/V heads round-robin over the XCDs (ragged sequences load
  // contiguous group ranges unevenly).
  int mb, id;
  if (!VARLEN ||
      !work_item_kv_rr(blockIdx.x, p.total_blocks, p.n_mblocks, p.group, p.heavy_first != 0, mb, id))
    work_item(blockIdx.x, p.total_blocks, p.n_mblocks, p.heavy_first != 0, kCausalSpan, mb, id);
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

  const int row0 = mb * BM;
  if (row0 >= Sq) return;   // whole workgroup: varlen blocks past this sequence
  const int row_last = min(row0 + BM, Sq) - 1;

  const int wrow0 = row0 + 32 * rb;
  const int qi = wrow0 + c32;
  const bool row_valid = qi < Sq;
  // Positions fit in 32 bits (the host keeps lengths and offsets below 2^29).
  const int qoff32 = (int)p.q_offset;
  const int qpos = qi + qoff32;
  const int qpos_w_min = wrow0 + qoff32;
  const int qpos_w_max = min(wrow0 + 31, row_last) + qoff32;

  const int wl = p.window_left, wr = p.window_right;
  const bool causal = p.causal != 0;
  int key_hi = Sk - 1;
  if (causal) key_hi = min(key_hi, qpos);
  if (wr >= 0) key_hi = min(key_hi, qpos + wr);
  // key_lo stays above -2^30 so that key - key_lo cannot overflow.
  const int key_lo = wl >= 0 ? max(qpos - wl, -(1 << 30)) : -(1 << 30);

  // Key tiles [t_begin, t_end) any row of the workgroup can see.
  int k_hi = Sk;
  if (causal) k_hi = min(k_hi, row_last + qoff32 + 1);
  if (wr >= 0) k_hi = min(k_hi, row_last + qoff32 + wr + 1);
  int k_lo = 0;
  if (wl >= 0) k_lo = max(0, row0 + qoff32 - wl);
  const int t_begin = k_lo / BN;
  const int t_end = k_hi > k_lo ? (k_hi + BN - 1) / BN : t_begin;
  const int J = t_end - t_begin;

  // ------------------------------------------------------------ Q^T in VGPRs
  // fp16: Q is pre-scaled by scale * log2(e) and rounded back to fp16, as the
  // reference's forward kernel does (attention_kernel.py:492-495), so the
  // scores come out of the MFMAs in log2 units.  bf16 keeps Q as given (its
  // 8-bit mantissa would move the log-sum-exp by ~1.5e-3) and scales every
  // score in the softmax.
  constexpr bool kPre = std::is_same<T, F16>::value;
  const uint16_t* qg = static_cast<const uint16_t*>(p.q);
  u32x4 qreg[NKC];
  // This wave's 32 Q rows are staged through LDS with whole-row DMA (rows past
  // the sequence read as zeros): G0 in V stages 2-3, which the V loads first
  // fill in the softmax phases after G0 has read its rows, G1 in the staging
  // area past the rings.
  static_assert(D == 128, "Q staging holds 256-byte rows");
  uint8_t* const q_st = smem_pp + (grp == 0 ? NS * TILEB + 2 * TILEB : Tile::STAGE_OFF) + sid * 8192;
  stage_rows_load(make_rsrc_words(qg + q_base + (int64_t)wrow0 * p.q_ss,
                                  rows_extent(wrow0, Sq, p.q_ss, D)),
                  lds_address(q_st), (uint32_t)(p.q_ss * 2), lane);
  auto prescale_q = [&]() {
    if constexpr (kPre) {
      const float qs = p.scale_log2;
#pragma unroll
      for (int kc = 0; kc < NKC; ++kc)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const uint32_t w2 = qreg[kc][i];
          qreg[kc][i] = T::pack2(T::to_float((uint16_t)(w2 & 0xffffu)) * qs,
                                 T::to_float((uint16_t)(w2 >> 16)) * qs);
        }
    }
  };

  // ------------------------------------------------------------ tile loads
  // This wave copies rows [RPI * (IPW * w + i), +RPI) of every K and V tile,
  // i < IPW.  Lane l writes physical chunk l % 16 of row RPI*(...) + l / 16,
  // so it loads the logical chunk that the swizzle puts there.
  const uint16_t* kg = static_cast<const uint16_t*>(p.k) + k_base;
  const uint16_t* vg = static_cast<const uint16_t*>(p.v) + v_base;
  const uint32_t k_row_b = (uint32_t)(p.k_ss * 2);
  const uint32_t v_row_b = (uint32_t)(p.v_ss * 2);
  uint32_t k_off[IPW], v_off[IPW];
#pragma unroll
  for (int i = 0; i < IPW; ++i) {
    const int r = RPI * (IPW * w + i) + (lane >> 4);
    const int pc = lane & 15;
    k_off[i] = (uint32_t)r * k_row_b + (uint32_t)((pc ^ (r & 15)) * 16);
    v_off[i] = (uint32_t)r * v_row_b + (uint32_t)((pc ^ (4 * (r & 3))) * 16);
  }
  uint8_t* const k_lds = smem_pp;
  uint8_t* const v_lds = smem_pp + NS * TILEB;
  // Tile rel (relative to t_begin) of K / V into its stage.  Tiles past the
  // workgroup's range get an empty resource: the instruction still retires
  // (keeping the wait counts uniform) and writes zeros.
  const uint32_t k_lds_a = lds_address(k_lds) + IPW * w * 1024;
  const uint32_t v_lds_a = lds_address(v_lds) + IPW * w * 1024;
  auto load_k = [&](int rel) {
    const int n0 = (t_begin + rel) * BN;
    const uint32_t ext = rel < J ? rows_extent(n0, Sk, p.k_ss, D) : 0u;
    const u32x4 rs = make_rsrc_words(kg + (int64_t)(rel < J ? n0 : 0) * p.k_ss, ext);
    const uint32_t dst = k_lds_a + (rel % NS) * TILEB;
#pragma unroll
    for (int i = 0; i < IPW; ++i) buf_load16_lds(rs, dst + i * 1024, k_off[i]);
  };
  auto load_v = [&](int rel) {
    const int n0 = (t_begin + rel) * BN;
    const uint32_t ext = rel < J ? rows_extent(n0, Sk, p.v_ss, D) : 0u;
    const u32x4 rs = make_rsrc_words(vg + (int64_t)(rel < J ? n0 : 0) * p.v_ss, ext);
    const uint32_t dst = v_lds_a + (rel % NS) * TILEB;
#pragma unroll
    for (int i = 0; i < IPW; ++i) buf_load16_lds(rs, dst + i * 1024, v_off[i]);
  };

  // Per-lane LDS read offsets.  K (A operand of S^T, 16 B per lane): key row
  // kb*32 + c32, logical chunk 2 kc + g.  V^T (ds_read_b64_tr_b16, 8 B per
  // lane): lane j of its 16-lane group reads key row 16 cc + 4 g + j / 4 (+8),
  // dims db*32 + 16 (c32 / 16) + 4 (j % 4).
  const int kx = c32 & 15;
  const uint32_t k_rd = (uint32_t)c32 * ROWB;
  const int j16 = lane & 15;
  const uint32_t v_rd = (uint32_t)(4 * g + (j16 >> 2)) * ROWB + (uint32_t)((j16 & 1) * 8);
  const int v_cx = 2 * (c32 >> 4) + ((j16 & 3) >> 1);   // chunk within a 32-dim block
  const int v_sw = j16 >> 2;                             // row & 3 of every V^T read

  auto wave_masks = [&](int rel) {
    const int n0 = (t_begin + rel) * BN, n1 = n0 + BN;
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
  // m_c: the finite max that P is taken against (m_run, or 0 while the row
  // has seen no key).  fp16: the S^T products start from -m_c instead of
  // zero (every lane of cneg holds -m_c of its query row), so they produce
  // the exponent s - m_c of P directly.
  float m_c = 0.f;
  f32x16 cneg = f32x16{};
  const float sl = kPre ? 1.f : p.scale_log2;
  f32x16 s[NKB];
  u32x4 pbuf[NCC];

  // LDS operand reads.  The per-lane swizzled offsets are computed once
  // (8 for K, one per 16-dim step; 4 for V^T, one per 32-dim block), so that
  // a GEMM phase issues no VALU work of its own: it would queue behind the
  // other group's softmax on the shared VALU port and starve the MFMAs.
  uint32_t k_ofs[NKC], v_ofs[NDB];
#pragma unroll
  for (int kc = 0; kc < NKC; ++kc) k_ofs[kc] = k_rd + (((uint32_t)(2 * kc + g)) ^ (uint32_t)kx) * 16;
#pragma unroll
  for (int db = 0; db < NDB; ++db)
    v_ofs[db] = v_rd + ((((uint32_t)db ^ (uint32_t)v_sw) << 2) + (uint32_t)v_cx) * 16;
  auto k_read = [&](const uint8_t* Ks, int kc, int kb) {
    return *reinterpret_cast<const u32x4*>(Ks + k_ofs[kc] + kb * 32 * ROWB);
  };
  auto v_read = [&](const uint8_t* Vs, int db, int cc) {
    const uint16_t* vp = reinterpret_cast<const uint16_t*>(Vs + v_ofs[db] + cc * 16 * ROWB);
    const u32x2 lo = lds_read_tr16(vp);
    const u32x2 hi = lds_read_tr16(vp + 8 * D);
    return u32x4{lo[0], lo[1], hi[0], hi[1]};
  };
  constexpr int NQK = NKC * NKB;   // MFMAs of S^T per tile
  constexpr int NPV = NDB * NCC;   // MFMAs of O^T per tile
  // One GEMM phase: S^T = K Q^T from K stage kst (DO_QK) and O^T += V^T P^T
  // from V stage vst (DO_PV).  The operand reads run ahead of the MFMAs that
  // consume them (8 K reads before the first product, then one read per
  // product; the V^T reads under the second half of S^T), pinned with
  // scheduling groups: left to itself the scheduler keeps two reads in flight
  // and every pair of MFMAs waits out the LDS latency.
  auto gemm = [&](int kst, int vst, auto do_qk_c, auto do_pv_c) {
    constexpr bool DO_QK = decltype(do_qk_c)::value;
    constexpr bool DO_PV = decltype(do_pv_c)::value;
    // The matrix-core phase of the SIMD: its instructions go first.
    __builtin_amdgcn_s_setprio(1);
    const uint8_t* Ks = k_lds + kst * TILEB;
    const uint8_t* Vs = v_lds + vst * TILEB;
    u32x4 ka[DO_QK ? NQK : 1];
    u32x4 va[DO_PV ? NPV : 1];
    if constexpr (DO_QK) {
#pragma unroll
      for (int i = 0; i < NQK; ++i) ka[i] = k_read(Ks, i / NKB, i % NKB);
    }
    if constexpr (DO_PV) {
#pragma unroll
      for (int db = 0; db < NDB; ++db)
#pragma unroll
        for (int cc = 0; cc < NCC; ++cc) va[db * NCC + cc] = v_read(Vs, db, cc);
    }
    if constexpr (DO_QK) {
#pragma unroll
      for (int kb = 0; kb < NKB; ++kb) s[kb] = kPre ? cneg : f32x16{};
#pragma unroll
      for (int kc = 0; kc < NKC; ++kc)
#pragma unroll
        for (int kb = 0; kb < NKB; ++kb) s[kb] = T::mfma32(ka[kc * NKB + kb], qreg[kc], s[kb]);
    }
    if constexpr (DO_PV) {
#pragma unroll
      for (int db = 0; db < NDB; ++db)
#pragma unroll
        for (int cc = 0; cc < NCC; ++cc)
          acc[db] = T::mfma32(va[db * NCC + cc], pbuf[cc], acc[db]);
    }
    // Scheduling groups (mask 0x100 = LDS read, 0x008 = MFMA): 8 reads up
    // front, then two reads behind every product until all are issued, so
    // the reads run as far ahead as the 15-entry LDS counter allows (a
    // measured 1.46x over one read per product for this phase in isolation).
    constexpr int NRD = (DO_QK ? NQK : 0) + (DO_PV ? 2 * NPV : 0);   // LDS reads
    constexpr int NMF = (DO_QK ? NQK : 0) + (DO_PV ? NPV : 0);       // MFMAs
    constexpr int NPAIR = (NRD - 8 + 1) / 2;
    __builtin_amdgcn_sched_group_barrier(0x100, 8, 0);
#pragma unroll
    for (int i = 0; i < NPAIR; ++i) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
    }
    __builtin_amdgcn_sched_group_barrier(0x008, NMF - NPAIR, 0);
    __builtin_amdgcn_sched_barrier(0);
    __builtin_amdgcn_s_setprio(0);
  };
  using yes = std::true_type;
  using no = std::false_type;
  // Softmax of the tile starting at key n0 (s: the exponents s - m_c for
  // fp16, the raw scores for bf16): boundary mask, lazy max / O rescale,
  // P = exp2(s - m_c) packed as the B operand of pv, row sums.
  auto softmax_tile = [&](int n0, bool masked) {
    if (masked) {
      // Keys outside [key_lo, key_hi] -> -inf, branch-free: the sign of
      // (key_hi - key) | (key - key_lo) selects the -inf bit pattern.
      const int hi0 = key_hi - n0 - 4 * g;
      const int lo0 = n0 + 4 * g - key_lo;
#pragma unroll
      for (int kb = 0; kb < NKB; ++kb) {
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          const int ko = kb * 32 + 8 * (v >> 2) + (v & 3);
          const uint32_t m = (uint32_t)(((hi0 - ko) | (lo0 + ko)) >> 31);
          // (A scalar copy first: bit_cast of a vector element reference
          // reads element 0 with this compiler.)
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
    const float mq4 = halves_max(fmaxf(fmaxf(mq[0], mq[1]), fmaxf(mq[2], mq[3])));
    const float mx = kPre ? mq4 + m_c : mq4 * sl;
    const bool raise = mx > m_run + kRescaleSlack;
    if (__builtin_amdgcn_ballot_w64(raise)) {
      const float m_new = raise ? mx : m_run;
      const float alpha = m_new == m_run ? 1.f : __builtin_amdgcn_exp2f(m_run - m_new);
      l_run *= alpha;
#pragma unroll
      for (int db = 0; db < NDB; ++db) acc[db] *= alpha;
      m_run = m_new;
      const float m_use = m_run == -INFINITY ? 0.f : m_run;
      if constexpr (kPre) {
        const float shift = m_use - m_c;   // 0 on the lanes that did not raise
#pragma unroll
        for (int kb = 0; kb < NKB; ++kb) s[kb] -= shift;
#pragma unroll
        for (int v = 0; v < 16; ++v) cneg[v] = -m_use;
      }
      m_c = m_use;
    }
    // exp2 argument of score x.
    auto expo = [&](float x) { return kPre ? x : fmaf(x, sl, -m_c); };
    float lq[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int cc = 0; cc < NCC; ++cc) {
      const f32x16& sv = s[cc >> 1];
      const int o8 = (cc & 1) * 8;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const float e0 = __builtin_amdgcn_exp2f(expo(sv[o8 + 2 * j]));
        const float e1 = __builtin_amdgcn_exp2f(expo(sv[o8 + 2 * j + 1]));
        pbuf[cc][j] = T::pack2(e0, e1);
        if (T::kSumRounded)
          lq[j] = T::sum2(pbuf[cc][j], lq[j]);
        else
          lq[j] += e0 + e1;
      }
    }
    l_run += (lq[0] + lq[1]) + (lq[2] + lq[3]);
  };

  // ------------------------------------------------------------ prologue
  // Stages 0..NS-2 of K and 0..NS-3 of V; the Q rows retire with them.
#pragma unroll
  for (int r = 0; r < NS - 1; ++r) load_k(r);
#pragma unroll
  for (int r = 0; r < NS - 2; ++r) load_v(r);
  __builtin_amdgcn_s_waitcnt(0x0f70);   // vmcnt(0)
  pp_barrier();
  stage_rows_read_operand<NKC>(q_st, c32, g, qreg);
  prescale_q();

  // ------------------------------------------------------------ phases
  // Every wave runs the same straight-line sequence GEMM(0), softmax(0),
  // GEMM(1), ..., softmax(J-1), GEMM(J) with a barrier after each step; G1
  // enters one barrier later than G0 (and G0 leaves one later), so in every
  // phase one group multiplies while the other exponentiates.
  // GEMM(j) = S_j (j < J) and O^T += V_{j-1}^T P_{j-1} (j >= 1).  Tiles that
  // hold no visible key for some of this wave's rows are computed anyway with
  // the mask applied: in lockstep, skipping them would not shorten a phase.
  auto softmax_step = [&](int j) {
    load_k(j + NS - 1);
    load_v(j + NS - 2);
    softmax_tile((t_begin + j) * BN, wave_masks(j));
    // This wave's loads from the previous softmax step have landed.
    __builtin_amdgcn_s_waitcnt(0x0f70 | (2 * IPW));
  };
  if (grp == 1) pp_barrier();
  if (J > 0) {
    gemm(0, 0, yes{}, no{});
    pp_barrier();
    softmax_step(0);
    pp_barrier();
    for (int j = 1; j < J; ++j) {
      gemm(j % NS, (j - 1) % NS, yes{}, yes{});
      pp_barrier();
      softmax_step(j);
      pp_barrier();
    }
    gemm(0, (J - 1) % NS, no{}, yes{});
  }
  pp_barrier();
  if (grp == 0) pp_barrier();
  // Every wave's tile loads (including the empty ones past the last tile)
  // have landed before the rings are reused as the output staging area.
  __builtin_amdgcn_s_waitcnt(0x0f70);
  pp_barrier();

  // ------------------------------------------------------------ epilogue
  const float l_tot = halves_sum(l_run);
  const float inv_l = l_tot > 0.f ? 1.f / l_tot : 0.f;
  const float lse_val = l_tot > 0.f ? (m_run + __log2f(l_tot)) * kLn2 : -INFINITY;
  stage_rows_store<T, NDB>(acc, inv_l, smem_pp + w * kStageOutBytes, c32, g, lane,
                           static_cast<uint16_t*>(p.o) + o_base + (int64_t)wrow0 * p.o_ss,
                           p.o_ss, Sq - wrow0);
  if (p.lse != nullptr && g == 0 && row_valid) p.lse[lse_base + (int64_t)qi * p.lse_ss] = lse_val;
}

}  // namespace fa
