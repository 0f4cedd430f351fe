// Persistent ping-pong prefill forward for gfx950 at head dim 128, fp16 /
// bf16, for large dense launches (every row block full, key tiles a multiple
// of the four LDS stages).
//
// Semantics are those of prefill_pp_kernel (fa_prefill_pp.h), i.e. the
// reference's dense forward kernel
// (/root/reference/flash_attn_triton/triton_kernel/attention_kernel.py:424-533,
// :275-372), whose phase schedule this kernel keeps: 8 waves in two groups
// alternate between a GEMM phase (S_t = K_t Q^T and O^T += V_{t-1}^T P_{t-1})
// and a softmax phase, barrier to barrier.
//
// What differs is the life of a workgroup.  Measured with s_memrealtime on
// MI355X at B=4 H=32 S=4096 D=128, a fresh workgroup of prefill_pp_kernel
// spends about 13 us outside its key loop (Q load 3.5 us, first K/V tiles
// 1.8 us, first barrier 0.7 us, output stores 3 us) and the next workgroup
// starts 3.9 us after the previous one ends on its CU.  With 8 row blocks per
// CU that was 15 % of the causal launch.  Here one workgroup per CU runs a
// fixed list of row blocks:
//
// * The K/V loads of a block's last softmax phases already fetch the next
//   block's first tiles into the ring stages they would use anyway (tile
//   j + 3 of a block with J tiles is the next block's tile j + 3 - J), so a
//   new block starts with its tiles in LDS.
// * Four softmax phases before a block ends, the next block's Q rows are
//   fetched into L2.
// * Between blocks both groups finish the ping-pong (one phase each with the
//   other group idle), then load the next block's Q rows straight into the
//   Q registers and, while those loads are in flight, stage the finished
//   block's output through LDS (whole-row stores); no barrier separates the
//   blocks.  A block change still costs about 10k shader-clock cycles per
//   workgroup (measured with s_memtime; staging Q through LDS behind
//   barriers cost about the same): every workgroup changes blocks at about
//   the same time, and its output stores and Q loads go out together.
// * The softmax phases of a block's middle (all but its last four) use a
//   form of the tile loads with no selects between this block's and the
//   next block's bases and a fixed wait: 4-5 % fewer cycles per phase pair.
//
// The phase loop itself is prefill_pp_kernel's.
//
#pragma once

#include "fa_prefill_pp.h"

namespace fa {

template <class T, int D, bool CAUSAL>
__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(2, 2)))
void prefill_persist_kernel(const FwdParams p) {
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
  constexpr int TPB = BM / BN;     // key tiles per row block
  static_assert(NS == 4, "the stream loop is unrolled by the four LDS stages");

  extern __shared__ __attribute__((aligned(1024))) uint8_t smem_ps[];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int grp = w >> 2;             // 0: GEMM first, 1: softmax first
  const int sid = w & 3;
  const int rb = 2 * sid + grp;       // this wave's 32-row block
  const int c32 = lane & 31;
  const int g = lane >> 5;

  // ------------------------------------------------------------ work list
  const int xcd = blockIdx.x & 7;
  const int slot = blockIdx.x >> 3;
  const int slots = gridDim.x >> 3;
  const int n_mb = p.n_mblocks;
  const int gx = p.batch * p.heads_q / 8;   // groups per XCD
  const int rounds = p.persist_rounds;      // row blocks per workgroup
  // Block descriptors live in separate scalars (no struct copies or selects
  // between two structs, which would keep them, and the kernel arguments
  // they are computed from, in scratch memory).
  auto make_blk = [&](int r, int64_t& q_base, int64_t& o_base, int64_t& lse_base,
                      int64_t& k_base, int64_t& v_base, int& row0, int& J)
      __attribute__((always_inline)) {
    // The divisions go through fd_blk / fd_heads / fd_group (multiply-high and
    // shift): as runtime divisions they were a few hundred scalar instructions
    // per descriptor, and a block change computes five descriptors.
    int gi, mb;
    if (CAUSAL) {
      const int u = (r >> 1) * slots + slot;
      const int uq = (int)fdiv((uint32_t)u, p.fd_blk);
      const int j = u - uq * (n_mb >> 1);
      gi = xcd * gx + uq;
      mb = (r & 1) ? j : n_mb - 1 - j;
    } else {
      const int u = r * slots + slot;
      const int uq = (int)fdiv((uint32_t)u, p.fd_blk);
      gi = xcd * gx + uq;
      mb = u - uq * n_mb;
    }
    const int b = (int)fdiv((uint32_t)gi, p.fd_heads);
    const int hh = gi - b * p.heads_q;
    const int kvh = (int)fdiv((uint32_t)hh, p.fd_group);
    q_base = (int64_t)b * p.q_sb + (int64_t)hh * p.q_sh;
    o_base = (int64_t)b * p.o_sb + (int64_t)hh * p.o_sh;
    lse_base = (int64_t)b * p.lse_sb + (int64_t)hh * p.lse_sh;
    k_base = (int64_t)b * p.k_sb + (int64_t)kvh * p.k_sh;
    v_base = (int64_t)b * p.v_sb + (int64_t)kvh * p.v_sh;
    row0 = mb * BM;
    J = CAUSAL ? (mb + 1) * TPB : p.seqlen_k / BN;
  };
  // The current block's K/V bases, first row and tile count stay in scalars
  // through its phase loop; everything else (and the next block's
  // descriptor, needed only in the last phases and between blocks) is
  // recomputed where it is used, which keeps the loop within the register
  // budget.
  int r_cur = 0;
  int64_t c_k = 0, c_v = 0, t64 = 0;
  int c_row0 = 0, c_J = 0;
  make_blk(0, t64, t64, t64, c_k, c_v, c_row0, c_J);

  // This lane's query row of the current block (every row exists: the host
  // launches this kernel only for full row blocks) and its visible keys.
  int qi, key_hi, qpos_w_min;
  auto set_rows = [&]() __attribute__((always_inline)) {
    const int wrow0 = c_row0 + 32 * rb;
    qi = wrow0 + c32;
    qpos_w_min = wrow0;
    key_hi = CAUSAL ? qi : p.seqlen_k - 1;
  };
  set_rows();

  // ------------------------------------------------------------ Q^T in VGPRs
  // fp16: Q is pre-scaled by scale * log2(e) and rounded back to fp16 (as in
  // prefill_pp_kernel and the reference, attention_kernel.py:492-495), so the
  // scores come out of the MFMAs in log2 units; bf16 scales every score.
  constexpr bool kPre = std::is_same<T, F16>::value;
  const uint16_t* qg = static_cast<const uint16_t*>(p.q);
  u32x4 qreg[NKC];
  auto prescale_q = [&]() __attribute__((always_inline)) {
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
  // This wave copies rows [RPI * (IPW * w + i), +RPI) of every K and V tile
  // (lane l writes physical chunk l % 16 of row RPI*(...) + l / 16, so it
  // loads the logical chunk the swizzle puts there).  Stream tile t belongs to
  // the current block when j < J (block-local index), else tile j - J of the
  // next one (blocks hold at least four tiles, so the look-ahead of three never
  // skips a block); tiles past the last block get an empty resource and write
  // zeros.
  const uint16_t* kg = static_cast<const uint16_t*>(p.k);
  const uint16_t* vg = static_cast<const uint16_t*>(p.v);
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
  uint8_t* const k_lds = smem_ps;
  uint8_t* const v_lds = smem_ps + NS * TILEB;
  const uint32_t k_lds_a = lds_address(k_lds) + IPW * w * 1024;
  const uint32_t v_lds_a = lds_address(v_lds) + IPW * w * 1024;
  // Every tile of this kernel's blocks is full (the host launches it only
  // for whole row blocks and key lengths a multiple of the block), so a
  // tile's resource covers its own rows; the next block's K / V bases (n_k,
  // n_v) are set once per block, which keeps the per-tile address work to a
  // few scalar instructions.
  const uint32_t k_tile_ext = rows_extent(0, BN, p.k_ss, D);
  const uint32_t v_tile_ext = rows_extent(0, BN, p.v_ss, D);
  int64_t n_k = 0, n_v = 0;
  auto set_next = [&]() __attribute__((always_inline)) {
    if (r_cur + 1 < rounds) {
      int64_t a0, a1, a2;
      int r0, j0;
      make_blk(r_cur + 1, a0, a1, a2, n_k, n_v, r0, j0);
    }
  };
  // in_block_c (std::true_type): the caller knows tile jj is the current
  // block's, which saves the selects between this block's and the next
  // block's bases.
  auto load_tile = [&](int jj, int stage, bool is_k, auto in_block_c) __attribute__((always_inline)) {
    const bool in_cur = decltype(in_block_c)::value || jj < c_J;
    const bool live = in_cur || r_cur + 1 < rounds;
    const int j = in_cur ? jj : jj - c_J;
    const int64_t base = is_k ? (in_cur ? c_k : n_k) : (in_cur ? c_v : n_v);
    const int64_t ss = is_k ? p.k_ss : p.v_ss;
    const uint32_t ext = live ? (is_k ? k_tile_ext : v_tile_ext) : 0u;
    const u32x4 rs = make_rsrc_words((is_k ? kg : vg) + base + (int64_t)(j * BN) * ss, ext);
    const uint32_t dst = (is_k ? k_lds_a : v_lds_a) + stage * TILEB;
#pragma unroll
    for (int i = 0; i < IPW; ++i) buf_load16_lds(rs, dst + i * 1024, is_k ? k_off[i] : v_off[i]);
  };

  // Per-lane LDS read offsets (see prefill_pp_kernel): K rows for the S^T
  // A operand, V^T through the transposing read.
  const int kx = c32 & 15;
  const uint32_t k_rd = (uint32_t)c32 * ROWB;
  const int j16 = lane & 15;
  const uint32_t v_rd = (uint32_t)(4 * g + (j16 >> 2)) * ROWB + (uint32_t)((j16 & 1) * 8);
  const int v_cx = 2 * (c32 >> 4) + ((j16 & 3) >> 1);
  const int v_sw = j16 >> 2;
  uint32_t k_ofs[NKC], v_ofs[NDB];
#pragma unroll
  for (int kc = 0; kc < NKC; ++kc) k_ofs[kc] = k_rd + (((uint32_t)(2 * kc + g)) ^ (uint32_t)kx) * 16;
#pragma unroll
  for (int db = 0; db < NDB; ++db)
    v_ofs[db] = v_rd + ((((uint32_t)db ^ (uint32_t)v_sw) << 2) + (uint32_t)v_cx) * 16;
  auto k_read = [&](const uint8_t* Ks, int kc, int kb) __attribute__((always_inline)) {
    return *reinterpret_cast<const u32x4*>(Ks + k_ofs[kc] + kb * 32 * ROWB);
  };
  auto v_read = [&](const uint8_t* Vs, int db, int cc) __attribute__((always_inline)) {
    const uint16_t* vp = reinterpret_cast<const uint16_t*>(Vs + v_ofs[db] + cc * 16 * ROWB);
    const u32x2 lo = lds_read_tr16(vp);
    const u32x2 hi = lds_read_tr16(vp + 8 * D);
    return u32x4{lo[0], lo[1], hi[0], hi[1]};
  };

  f32x16 acc[NDB];
#pragma unroll
  for (int db = 0; db < NDB; ++db) acc[db] = f32x16{};
  float m_run = -INFINITY;   // running (possibly stale) max, log2 units
  float l_run = 0.f;         // this lane's partial row sum
  // m_c: the finite max P is taken against; fp16 starts the S^T products from
  // cneg = -m_c so they produce the exponent s - m_c directly.
  float m_c = 0.f;
  f32x16 cneg = f32x16{};
  const float sl = kPre ? 1.f : p.scale_log2;
  f32x16 s[NKB];
  u32x4 pbuf[NCC];

  constexpr int NQK = NKC * NKB;
  constexpr int NPV = NDB * NCC;
  // One GEMM phase (the schedule of prefill_pp_kernel's): operand reads run
  // ahead of the MFMAs that consume them, pinned with scheduling groups.
  auto gemm = [&](int kst, int vst, auto do_qk_c, auto do_pv_c) __attribute__((always_inline)) {
    constexpr bool DO_QK = decltype(do_qk_c)::value;
    constexpr bool DO_PV = decltype(do_pv_c)::value;
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
    constexpr int NRD = (DO_QK ? NQK : 0) + (DO_PV ? 2 * NPV : 0);
    constexpr int NMF = (DO_QK ? NQK : 0) + (DO_PV ? NPV : 0);
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

  // Softmax of the current block's tile j: causal mask on the diagonal tiles
  // (keys past this lane's row -> -inf), lazy max / O rescale,
  // P = exp2(s - m_c) packed as the B operand of the next O^T product, row
  // sums.
  auto softmax_tile = [&](int j) __attribute__((always_inline)) {
    const int n0 = j * BN;
    if (CAUSAL && n0 + BN - 1 > qpos_w_min) {
      const int hi0 = key_hi - n0 - 4 * g;
#pragma unroll
      for (int kb = 0; kb < NKB; ++kb) {
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          const int ko = kb * 32 + 8 * (v >> 2) + (v & 3);
          const float sv = s[kb][v];
          s[kb][v] = ko > hi0 ? -INFINITY : sv;
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
        const float shift = m_use - m_c;
#pragma unroll
        for (int kb = 0; kb < NKB; ++kb) s[kb] -= shift;
#pragma unroll
        for (int v = 0; v < 16; ++v) cneg[v] = -m_use;
      }
      m_c = m_use;
    }
    auto expo = [&](float x) __attribute__((always_inline)) { return kPre ? x : fmaf(x, sl, -m_c); };
    float lq[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int cc = 0; cc < NCC; ++cc) {
      const f32x16& sv = s[cc >> 1];
      const int o8 = (cc & 1) * 8;
#pragma unroll
      for (int j2 = 0; j2 < 4; ++j2) {
        const float e0 = __builtin_amdgcn_exp2f(expo(sv[o8 + 2 * j2]));
        const float e1 = __builtin_amdgcn_exp2f(expo(sv[o8 + 2 * j2 + 1]));
        pbuf[cc][j2] = T::pack2(e0, e1);
        if (T::kSumRounded)
          lq[j2] = T::sum2(pbuf[cc][j2], lq[j2]);
        else
          lq[j2] += e0 + e1;
      }
    }
    l_run += (lq[0] + lq[1]) + (lq[2] + lq[3]);
  };

  // The next block's Q rows into L2 (one 4-byte load per 128-byte line, 64
  // lines per wave, written as a throwaway into the last 2 KiB past the
  // rings, which no output staging uses).  It is issued after the phase's
  // tile loads, and the step waits leave it in flight until the tile loads
  // issued after it are waited for.
  auto prefetch_q = [&]() __attribute__((always_inline)) {
    int64_t n_q, n_o, n_l, n_k, n_v;
    int n_row0, n_J;
    make_blk(r_cur + 1, n_q, n_o, n_l, n_k, n_v, n_row0, n_J);
    const uint16_t* q0 = qg + n_q + (int64_t)(n_row0 + 32 * rb) * p.q_ss;
    const u32x4 rs = make_rsrc_words(q0, rows_extent(0, 32, p.q_ss, D));
    const uint32_t voff = (uint32_t)(lane >> 1) * (uint32_t)(p.q_ss * 2) + (uint32_t)(lane & 1) * 128;
    buf_load4_lds(rs, lds_address(smem_ps + Tile::STAGE_OFF + 4 * 8192 - 8 * 256 + w * 256), voff);
  };

  // The wait that ends a softmax step.  Tile t's rows are loaded by both
  // groups in their softmax step t - 3, and the first GEMM to read them,
  // group 0's GEMM(t), follows group 0's softmax step t - 1 and group 1's
  // softmax step t - 2 (group 1 runs one phase behind): group 0 waits for
  // its loads of two steps back, group 1 for those of one step back.  E
  // loads issued after those (a Q prefetch, the next block's Q rows) stay
  // in flight too.
  auto step_wait = [&](auto e_c) __attribute__((always_inline)) {
    constexpr int E = decltype(e_c)::value;
    if (grp == 0)
      __builtin_amdgcn_s_waitcnt(vmcnt_imm(4 * IPW + E));
    else
      __builtin_amdgcn_s_waitcnt(vmcnt_imm(2 * IPW + E));
  };
  using e0c = std::integral_constant<int, 0>;
  using e1c = std::integral_constant<int, 1>;

  // Softmax phase of the current block's tile j: the tile loads of K_{j+3}
  // and V_{j+2} (the next block's first tiles past the end), the softmax,
  // then the step wait (the Q prefetch of this step or the one before stays
  // in flight).
  auto softmax_step = [&](int j) __attribute__((always_inline)) {
    load_tile(j + NS - 1, (j + NS - 1) % NS, true, std::false_type{});
    load_tile(j + NS - 2, (j + NS - 2) % NS, false, std::false_type{});
    const bool more = r_cur + 1 < rounds;
    const bool pre = j == c_J - 4 && more;
    if (pre) prefetch_q();
    softmax_tile(j);
    if ((pre || (j > 0 && j == c_J - 3)) && more)
      step_wait(e1c{});
    else
      step_wait(e0c{});
  };

  // The same for a phase j < J - 4: both tiles are this block's, no Q
  // prefetch in this phase or the one before.
  // Running tile bases of the plain phases (non-causal): the plain phase of
  // tile j loads K_{j+3} and V_{j+2} of the current block, so each base steps
  // one tile per phase (set at the block's start) instead of being formed
  // from j: ten scalar instructions fewer per softmax phase, 0.8 % at BASELINE
  // config 2 non-causal.  The causal kernel keeps the indexed form: the two
  // running bases there raised its scalar-register spills from 16 to 27 and
  // it ran no faster.
  const uint16_t* k_run = kg;
  const uint16_t* v_run = vg;
  const int64_t k_step = (int64_t)BN * p.k_ss, v_step = (int64_t)BN * p.v_ss;
  auto load_run = [&](const uint16_t*& run, int stage, bool is_k) __attribute__((always_inline)) {
    const u32x4 rs = make_rsrc_words(run, is_k ? k_tile_ext : v_tile_ext);
    run += is_k ? k_step : v_step;
    const uint32_t dst = (is_k ? k_lds_a : v_lds_a) + stage * TILEB;
#pragma unroll
    for (int i = 0; i < IPW; ++i) buf_load16_lds(rs, dst + i * 1024, is_k ? k_off[i] : v_off[i]);
  };
  auto softmax_step_plain = [&](int j) __attribute__((always_inline)) {
    if constexpr (CAUSAL) {
      load_tile(j + NS - 1, (j + NS - 1) % NS, true, std::true_type{});
      load_tile(j + NS - 2, (j + NS - 2) % NS, false, std::true_type{});
    } else {
      load_run(k_run, (j + NS - 1) % NS, true);
      load_run(v_run, (j + NS - 2) % NS, false);
    }
    softmax_tile(j);
    step_wait(e0c{});
  };

  // A block's Q rows straight into the Q registers: lane (c32, g) loads dims
  // 16 kc + 8 g .. + 7 of its row (32 bytes of each row per instruction; the
  // rows were fetched into L2 four softmax phases before).  The compiler
  // waits for these loads where prescale_q first reads them.
  auto load_q_regs = [&](int64_t q_base, int row0) __attribute__((always_inline)) {
    const uint16_t* qrow = qg + q_base + (int64_t)(row0 + 32 * rb + c32) * p.q_ss + 8 * g;
#pragma unroll
    for (int kc = 0; kc < NKC; ++kc) qreg[kc] = *reinterpret_cast<const u32x4*>(qrow + 16 * kc);
  };

  // The block's last softmax phase.  The Q registers are free from here on
  // (the block's last S^T product is done), so the next block's Q rows go
  // into them first, ahead of the phase's tile loads, and the phase's own
  // wait leaves them in flight with those tile loads.
  auto softmax_step_last = [&](int j, bool more) __attribute__((always_inline)) {
    if (more) {
      int64_t n_q, n_o, n_l, n_k2, n_v2;
      int n_row0, n_J;
      make_blk(r_cur + 1, n_q, n_o, n_l, n_k2, n_v2, n_row0, n_J);
      load_q_regs(n_q, n_row0);
    }
    load_tile(j + NS - 1, (j + NS - 1) % NS, true, std::false_type{});
    load_tile(j + NS - 2, (j + NS - 2) % NS, false, std::false_type{});
    softmax_tile(j);
    if (more)
      step_wait(std::integral_constant<int, NKC>{});
    else
      step_wait(e0c{});
  };

  // ------------------------------------------------------------ prologue
  // The first block's Q rows, K tiles 0..2 and V tiles 0..1 of the stream.
  // Lane indices the compiler must not treat as loop invariants: the staging
  // addresses derived from them are recomputed per block instead of being
  // hoisted out of the block loop and held (or spilled) through it.
  auto opaque = [](int x) __attribute__((always_inline)) {
    asm volatile("" : "+v"(x));
    return x;
  };
  {
    int64_t q0, o0, l0;
    make_blk(0, q0, o0, l0, c_k, c_v, c_row0, c_J);
    load_q_regs(q0, c_row0);
  }
  set_next();
#pragma unroll
  for (int r = 0; r < NS - 1; ++r) load_tile(r, r, true, std::false_type{});
#pragma unroll
  for (int r = 0; r < NS - 2; ++r) load_tile(r, r, false, std::false_type{});
  prescale_q();
  __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));
  pp_barrier();

  uint16_t* const og = static_cast<uint16_t*>(p.o);
  // Output of block r, whose state is still in acc / l_run / m_run: staged
  // through the LDS area st_o (kStageOutBytes) and stored as whole rows,
  // with the block's LSE.
  auto finish_block = [&](int r, uint8_t* st_o) __attribute__((always_inline)) {
    const float l_tot = halves_sum(l_run);
    const float inv_l = l_tot > 0.f ? 1.f / l_tot : 0.f;
    const float lse_val = l_tot > 0.f ? (m_run + __log2f(l_tot)) * kLn2 : -INFINITY;
    int64_t f_q, f_o, f_l, f_k, f_v;
    int f_row0, f_J;
    make_blk(r, f_q, f_o, f_l, f_k, f_v, f_row0, f_J);
    const int lane_s = opaque(lane);
    u32x4 orows[8];
    stage_rows_gather<T, NDB>(acc, inv_l, st_o, lane_s & 31, lane_s >> 5, lane_s, orows);
    const int row_w = f_row0 + 32 * rb;
    stage_rows_put(orows, og + f_o + (int64_t)row_w * p.o_ss, p.o_ss, lane_s);
    if (p.lse != nullptr && g == 0) p.lse[f_l + (int64_t)(row_w + c32) * p.lse_ss] = lse_val;
  };
  auto reset_state = [&]() __attribute__((always_inline)) {
#pragma unroll
    for (int db = 0; db < NDB; ++db) acc[db] = f32x16{};
    m_run = -INFINITY;
    l_run = 0.f;
    m_c = 0.f;
    cneg = f32x16{};
  };
  // Output staging areas.  Group 0 stages in the phase of its last O^T
  // product (group 1 is in its last softmax phase, whose tile loads fill K
  // stage 2 and V stage 1): K stage 3 and V stage 2 hold tiles that both
  // groups have finished reading, and the area past the rings is free.
  // Group 1 stages one phase after its last O^T product, while group 0's
  // first softmax phase of the next block loads K stage 3 and V stage 2:
  // it uses V stage 3 (its own last O^T operand, next loaded two phases
  // later) and the area past the rings.  The Q-row prefetch writes its
  // throwaway bytes at the end of that area, clear of both.
  static_assert(kStageOutBytes <= TILEB && 3 * kStageOutBytes <= 4 * 8192 - 8 * 256,
                "output staging must fit the stages and the area past the rings");
  uint8_t* const past = smem_ps + Tile::STAGE_OFF;
  uint8_t* const st_own = grp == 0
      ? (sid == 0 ? k_lds + 3 * TILEB : sid == 1 ? v_lds + 2 * TILEB : past + (sid - 2) * kStageOutBytes)
      : (sid == 0 ? v_lds + 3 * TILEB : past + (sid - 1) * kStageOutBytes);

  // The block loop.  Group 1 runs one phase behind group 0 for the whole
  // life of the workgroup; nothing drains between blocks.  Per block each
  // group runs GEMM(0) (S^T only), softmax(0), ..., softmax(J-1) and
  // GEMM(J) (O^T only), one barrier after each, 2J + 1 phases.  The next
  // block's Q rows go into the Q registers at the start of softmax(J-1).  Group 0 stages its
  // output right after its GEMM(J); group 1 does so after the barrier that
  // ends its GEMM(J), i.e. in its next phase, before its GEMM(0) of the
  // next block.  So group 1's GEMM(J) shares a phase with group 0's next
  // GEMM(0) (16 + 16 MFMAs per SIMD, a full GEMM phase), and each group's
  // output stores and Q loads run beside the other group's work.
  if (grp == 1) pp_barrier();
  for (;;) {
    // ---------------------------------------------------------- one block
    const int J = c_J;
    const int j_tail = J - 4;   // the phases from J - 4 on prefetch Q rows or wait for them
    const bool more = r_cur + 1 < rounds;
    if constexpr (!CAUSAL) {
      k_run = kg + c_k + (int64_t)(NS - 1) * k_step;
      v_run = vg + c_v + (int64_t)(NS - 2) * v_step;
    }
    gemm(0, 0, yes{}, no{});
    pp_barrier();
    if (j_tail > 0)
      softmax_step_plain(0);
    else
      softmax_step(0);
    pp_barrier();
    for (int j = 1; j < j_tail; ++j) {
      gemm(j % NS, (j - 1) % NS, yes{}, yes{});
      pp_barrier();
      softmax_step_plain(j);
      pp_barrier();
    }
    for (int j = j_tail > 1 ? j_tail : 1; j < J - 1; ++j) {
      gemm(j % NS, (j - 1) % NS, yes{}, yes{});
      pp_barrier();
      softmax_step(j);
      pp_barrier();
    }
    gemm((J - 1) % NS, (J - 2) % NS, yes{}, yes{});
    pp_barrier();
    softmax_step_last(J - 1, more);
    pp_barrier();
    gemm(0, (J - 1) % NS, no{}, yes{});
    // Group 1 passes the barrier that ends this phase before its output,
    // group 0 after it: one barrier each.  Both scale the next block's Q
    // rows in their next phase, where the wait for them also covers the
    // tile loads of two phases back (the loads complete in order).
    if (grp == 1) pp_barrier();
    finish_block(r_cur, st_own);
    reset_state();
    if (grp == 0) pp_barrier();
    if (!more) break;
    prescale_q();
    ++r_cur;
    make_blk(r_cur, t64, t64, t64, c_k, c_v, c_row0, c_J);
    set_next();
    set_rows();
  }
  // Group 0 matches group 1's last barrier.
  if (grp == 0) pp_barrier();
}

}  // namespace fa
