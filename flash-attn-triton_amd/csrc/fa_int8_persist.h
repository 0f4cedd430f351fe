// Persistent INT8-QK^T ping-pong forward for gfx950 at head dim 128, for
// large dense launches (every row block full, no query offset).
//
// Semantics are those of int8_pp_kernel (fa_int8_pp.h), i.e. the reference's
// _attn_fwd_int8 / _attn_fwd_int8_inner
// (/root/reference/flash_attn_triton/triton_kernel/attention_kernel_int8.py:82-141,
// :167-217): Q quantized per row (division form), S^T = K8 Q8^T in int32,
// scores i32 * s_k[key] * s_q * sm_scale * log2(e), online softmax,
// O^T += V^T P^T in fp16.  Its phase schedule (GEMM and softmax phases of
// two wave groups, barrier to barrier) and tiles are int8_pp_kernel's; the
// workgroup life is prefill_persist_kernel's (fa_prefill_persist.h): one
// workgroup per CU runs a fixed list of row blocks (causal: row block mb
// paired with n - 1 - mb), the K8 / key-scale / V loads of a block's last
// softmax phases fetch the next block's first tiles, its Q rows are fetched
// into L2 four phases before the end, and the ping-pong runs on across
// blocks (group 1 one phase behind, each group staging its output in a phase
// where the other group computes).  A block's Q rows load into registers
// at the start of its predecessor's last softmax phase and are quantized
// where the next block's first GEMM phase needs them.
//
// LDS: K8 tiles 4 x 8 KiB (chunk c of row r at c ^ ((r >> 1) & 7)), V tiles
// 4 x 16 KiB (chunk c of row r at c ^ 4 (r & 3)), key scales 4 x 256 B, then
// 63 KiB for output staging (group 0's four waves, then three of group 1's;
// its first wave stages in V stage 3) and the Q prefetch's throwaway bytes.
#pragma once

#include "fa_int8_pp.h"
#include "fa_stage_rows.h"

namespace fa {

template <int D>
struct Int8PersistTile {
  static constexpr int NW = 8;
  static constexpr int NT = 512;
  static constexpr int BM = 256;             // query rows per row block
  static constexpr int BN = 64;              // keys per tile
  static constexpr int NS = 4;               // LDS stages per operand
  static constexpr int KROWB = D;            // bytes per K8 row
  static constexpr int VROWB = 2 * D;        // bytes per V row
  static constexpr int KTILEB = BN * KROWB;
  static constexpr int VTILEB = BN * VROWB;
  static constexpr int SKB = BN * 4;
  static constexpr int V_OFF = NS * KTILEB;
  static constexpr int SK_OFF = V_OFF + NS * VTILEB;
  static constexpr int PAST_OFF = SK_OFF + NS * SKB;
  static constexpr int LDS_BYTES = 160 * 1024;
  static constexpr int PF_OFF = LDS_BYTES - NW * 256;   // Q prefetch throwaway, 256 B per wave
  static constexpr int KRPI = 1024 / KROWB;  // K8 rows per 1-KiB load instruction
  static constexpr int VRPI = 1024 / VROWB;  // V rows per 1-KiB load instruction
  static constexpr int KIPW = KTILEB / 1024 / NW;
  static constexpr int VIPW = VTILEB / 1024 / NW;
  static constexpr int LPS = KIPW + VIPW + 1;  // load instructions per wave per softmax step
  static_assert(D == 128, "the INT8 persistent tiles are laid out for head dim 128");
  static_assert(KIPW * NW * 1024 == KTILEB && VIPW * NW * 1024 == VTILEB,
                "tiles must split evenly over the waves");
  static_assert(PAST_OFF + 7 * kStageOutBytes <= PF_OFF,
                "output staging of seven waves must fit past the rings");
  static_assert(kStageOutBytes <= VTILEB, "one wave's output staging must fit a V stage");
};

template <int D, bool CAUSAL>
__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(2, 2)))
void int8_persist_kernel(const Int8Params p) {
  using Tile = Int8PersistTile<D>;
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
  constexpr int LPS = Tile::LPS;
  constexpr int NKC = D / 32;      // 32-dim k-steps of the int8 S^T
  constexpr int NDB = D / 32;      // 32-dim blocks of O^T
  constexpr int NKB = BN / 32;     // 32-key blocks per tile
  constexpr int NCC = BN / 16;     // 16-key k-steps of O^T
  constexpr int TPB = BM / BN;     // key tiles per row block
  constexpr int NQL = 2 * NKC;     // 16-byte Q loads per lane
  static_assert(NS == 4, "the stream loop is unrolled by the four LDS stages");

  extern __shared__ __attribute__((aligned(1024))) uint8_t smem_ip[];

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
  const int gx = p.batch * p.heads / 8;     // groups per XCD
  const int rounds = p.persist_rounds;      // row blocks per workgroup
  const int S = p.seqlen;
  // Block r of this workgroup: (batch, head) group gi and first row row0.
  // Divisions by multiply-high and shift (fd_blk, fd_heads): as runtime
  // divisions they were a few hundred scalar instructions per descriptor.
  auto make_blk = [&](int r, int& gi, int& row0, int& J) __attribute__((always_inline)) {
    int mb;
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
    row0 = mb * BM;
    J = CAUSAL ? (mb + 1) * TPB : S / BN;
  };
  // Element offsets of group gi's Q / V / O rows (the [B, H, S, D] strides)
  // and its K8 (bytes) and key-scale (floats) rows.
  auto q_base_of = [&](int gi) __attribute__((always_inline)) {
    const int b = (int)fdiv((uint32_t)gi, p.fd_heads);
    return (int64_t)b * p.q_sb + (int64_t)(gi - b * p.heads) * p.q_sh;
  };
  auto o_base_of = [&](int gi) __attribute__((always_inline)) {
    const int b = (int)fdiv((uint32_t)gi, p.fd_heads);
    return (int64_t)b * p.o_sb + (int64_t)(gi - b * p.heads) * p.o_sh;
  };
  auto v_base_of = [&](int gi) __attribute__((always_inline)) {
    const int b = (int)fdiv((uint32_t)gi, p.fd_heads);
    return (int64_t)b * p.v_sb + (int64_t)(gi - b * p.heads) * p.v_sh;
  };
  int r_cur = 0;
  int c_gi = 0, c_row0 = 0, c_J = 0;
  make_blk(0, c_gi, c_row0, c_J);
  int64_t c_k = 0, c_s = 0, c_v = 0;   // current block's K8 (bytes), s_k, V bases
  int64_t n_k = 0, n_s = 0, n_v = 0;   // the next block's
  auto set_bases = [&]() __attribute__((always_inline)) {
    c_k = (int64_t)c_gi * S * D;
    c_s = (int64_t)c_gi * S;
    c_v = v_base_of(c_gi);
    if (r_cur + 1 < rounds) {
      int gi, r0, j0;
      make_blk(r_cur + 1, gi, r0, j0);
      n_k = (int64_t)gi * S * D;
      n_s = (int64_t)gi * S;
      n_v = v_base_of(gi);
    }
  };
  set_bases();

  int qi, key_hi, qpos_w_min;
  auto set_rows = [&]() __attribute__((always_inline)) {
    const int wrow0 = c_row0 + 32 * rb;
    qi = wrow0 + c32;
    qpos_w_min = wrow0;
    key_hi = CAUSAL ? qi : S - 1;
  };
  set_rows();

  // ------------------------------------------------------------ Q rows
  // Lane (c32, g) loads dims [32 kc + 16 g, +16) of its row (two 16-byte
  // loads per kc) and quantizes them into the B operand of
  // v_mfma_i32_32x32x32_i8; the quotient x / s_q is the IEEE division's
  // (quant_div), bit-exact with the reference's division form.
  const uint16_t* qg = static_cast<const uint16_t*>(p.q);
  u32x4 qraw[NQL];
  i32x4 q8[NKC];
  float row_scale = 0.f, coef_b = 0.f;
  auto load_q_raw = [&](int gi, int row0) __attribute__((always_inline)) {
    const uint16_t* qrow = qg + q_base_of(gi) + (int64_t)(row0 + 32 * rb + c32) * p.q_ss + 16 * g;
#pragma unroll
    for (int i = 0; i < NQL; ++i) qraw[i] = load16(qrow + 32 * (i >> 1) + 8 * (i & 1));
  };
  auto quantize_q = [&]() __attribute__((always_inline)) {
#pragma clang fp contract(off)
    float amax = 0.f;
#pragma unroll
    for (int i = 0; i < NQL; ++i)
#pragma unroll
      for (int e = 0; e < 8; ++e)
        amax = fmaxf(amax, fabsf(F16::to_float((uint16_t)(qraw[i][e >> 1] >> ((e & 1) * 16)))));
    amax = halves_max(amax);
    const float s_q = fmaxf(amax, 1.0f) / 127.0f;
    const float inv_q = 1.0f / s_q;
    auto qv = [&](int i, int e) __attribute__((always_inline)) {
      return round_half_away_i(
          quant_div(F16::to_float((uint16_t)(qraw[i][e >> 1] >> ((e & 1) * 16))), s_q, inv_q));
    };
#pragma unroll
    for (int kc = 0; kc < NKC; ++kc)
#pragma unroll
      for (int wd = 0; wd < 4; ++wd) {
        const int i = 2 * kc + (wd >> 1), e0 = 4 * (wd & 1);
        q8[kc][wd] = (int)pack_i8x4_i(qv(i, e0), qv(i, e0 + 1), qv(i, e0 + 2), qv(i, e0 + 3));
      }
    row_scale = s_q * p.scale_log2;
    coef_b = g == 0 ? row_scale : 0.f;
  };

  // ------------------------------------------------------------ tile loads
  // Stream tile jj belongs to the current block when jj < J, else it is tile
  // jj - J of the next one; past the last block an empty resource (zeros).
  const int8_t* k8g = p.k8;
  const float* skg = p.s_k;
  const uint16_t* vg = static_cast<const uint16_t*>(p.v);
  const uint32_t v_row_b = (uint32_t)(p.v_ss * 2);
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
  uint8_t* const k_lds = smem_ip;
  uint8_t* const v_lds = smem_ip + Tile::V_OFF;
  const uint8_t* const sk_lds = smem_ip + Tile::SK_OFF;
  const uint32_t k_lds_a = lds_address(k_lds) + KIPW * w * 1024;
  const uint32_t v_lds_a = lds_address(v_lds) + VIPW * w * 1024;
  const uint32_t sk_lds_a = lds_address(sk_lds);
  const uint32_t sk_voff = (uint32_t)lane * 4;
  const uint32_t v_tile_ext = rows_extent(0, BN, p.v_ss, D);
  // K8 tile jj and its key scales (every wave copies the 64 scales).
  auto load_k = [&](int jj, int stage, auto in_block_c) __attribute__((always_inline)) {
    const bool in_cur = decltype(in_block_c)::value || jj < c_J;
    const bool live = in_cur || r_cur + 1 < rounds;
    const int j = in_cur ? jj : jj - c_J;
    const int64_t kb = in_cur ? c_k : n_k;
    const int64_t sb = in_cur ? c_s : n_s;
    const u32x4 rk = make_rsrc_words(k8g + kb + (int64_t)(j * BN) * D, live ? (uint32_t)(BN * D) : 0u);
    const uint32_t dst = k_lds_a + stage * KTILEB;
#pragma unroll
    for (int i = 0; i < KIPW; ++i) buf_load16_lds(rk, dst + i * 1024, k_off[i]);
    const u32x4 rs = make_rsrc_words(skg + sb + j * BN, live ? (uint32_t)(BN * 4) : 0u);
    buf_load4_lds(rs, sk_lds_a + stage * SKB, sk_voff);
  };
  auto load_v = [&](int jj, int stage, auto in_block_c) __attribute__((always_inline)) {
    const bool in_cur = decltype(in_block_c)::value || jj < c_J;
    const bool live = in_cur || r_cur + 1 < rounds;
    const int j = in_cur ? jj : jj - c_J;
    const int64_t vb = in_cur ? c_v : n_v;
    const u32x4 rs = make_rsrc_words(vg + vb + (int64_t)(j * BN) * p.v_ss, live ? v_tile_ext : 0u);
    const uint32_t dst = v_lds_a + stage * VTILEB;
#pragma unroll
    for (int i = 0; i < VIPW; ++i) buf_load16_lds(rs, dst + i * 1024, v_off[i]);
  };

  // LDS read offsets: K8 (A operand, 16 B per lane: key row kb*32 + c32,
  // logical chunk 2 kc + g) and V^T (transposing reads, as the fp16 kernels).
  uint32_t k_ofs[NKC], v_ofs[NDB];
#pragma unroll
  for (int kc = 0; kc < NKC; ++kc)
    k_ofs[kc] = (uint32_t)c32 * KROWB + (((uint32_t)(2 * kc + g)) ^ (uint32_t)((c32 >> 1) & 7)) * 16;
  {
    const int j16 = lane & 15;
    const uint32_t v_rd = (uint32_t)(4 * g + (j16 >> 2)) * VROWB + (uint32_t)((j16 & 1) * 8);
    const int v_cx = 2 * (c32 >> 4) + ((j16 & 3) >> 1);
    const int v_sw = j16 >> 2;
#pragma unroll
    for (int db = 0; db < NDB; ++db)
      v_ofs[db] = v_rd + ((((uint32_t)db ^ (uint32_t)v_sw) << 2) + (uint32_t)v_cx) * 16;
  }
  auto v_read = [&](const uint8_t* Vs, int db, int cc) __attribute__((always_inline)) {
    const uint16_t* vp = reinterpret_cast<const uint16_t*>(Vs + v_ofs[db] + cc * 16 * VROWB);
    const u32x2 lo = lds_read_tr16(vp);
    const u32x2 hi = lds_read_tr16(vp + 8 * D);
    return u32x4{lo[0], lo[1], hi[0], hi[1]};
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

  constexpr int NQK = NKC * NKB;
  constexpr int NPV = NDB * NCC;
  // One GEMM phase (int8_pp_kernel's): S^T = K8 Q8^T from K stage kst and
  // the score coefficients s_k[key] * row scale as fp32 outer products,
  // then O^T += V^T P^T from V stage vst with the conversion of the S^T
  // scores into exponents under the PV products.
  auto gemm = [&](int kst, int vst, auto do_qk_c, auto do_pv_c) __attribute__((always_inline)) {
    constexpr bool DO_QK = decltype(do_qk_c)::value;
    constexpr bool DO_PV = decltype(do_pv_c)::value;
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
    if constexpr (DO_QK) {
#pragma unroll
      for (int i = 0; i < NQK; ++i)
        ka[i] = *reinterpret_cast<const u32x4*>(Ks + k_ofs[i / NKB] + (i % NKB) * 32 * KROWB);
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
#pragma unroll
      for (int kb = 0; kb < NKB; ++kb)
        coef[kb] = __builtin_amdgcn_mfma_f32_32x32x2f32(ska[kb], coef_b, f32x16{}, 0, 0, 0);
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
      constexpr int NRDG = DO_QK ? NRD2 : NRD2 - 8;
#pragma unroll
      for (int i = 0; i < NPV; ++i) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        if (i * 2 < NRDG) __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
        if (NVALU > 0 && i >= 1)
          __builtin_amdgcn_sched_group_barrier(0x002, (NVALU + NPV - 2) / (NPV - 1), 0);
      }
    }
    __builtin_amdgcn_sched_barrier(0);
    __builtin_amdgcn_s_setprio(0);
  };
  using yes = std::true_type;
  using no = std::false_type;

  // Softmax of the current block's tile j: causal mask on the diagonal tiles,
  // lazy max / O rescale (the exponents move with m_c), P = exp2(s) packed as
  // the B operand of the next O^T product, row sums over the rounded P.
  auto softmax_tile = [&](int j) __attribute__((always_inline)) {
    const int n0 = j * BN;
    if (CAUSAL && n0 + BN - 1 > qpos_w_min) {
      const int hi0 = key_hi - n0 - 4 * g;
#pragma unroll
      for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          const int ko = kb * 32 + 8 * (v >> 2) + (v & 3);
          const float sv = s[kb][v];
          s[kb][v] = ko > hi0 ? -INFINITY : sv;
        }
    }
    float mq[4] = {-INFINITY, -INFINITY, -INFINITY, -INFINITY};
#pragma unroll
    for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
      for (int v = 0; v < 16; v += 8)
#pragma unroll
        for (int q = 0; q < 4; ++q)
          mq[q] = fmaxf(fmaxf(mq[q], s[kb][v + 2 * q]), s[kb][v + 2 * q + 1]);
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
      for (int j2 = 0; j2 < 4; ++j2) {
        const float e0 = __builtin_amdgcn_exp2f(sv[o8 + 2 * j2]);
        const float e1 = __builtin_amdgcn_exp2f(sv[o8 + 2 * j2 + 1]);
        pbuf[cc][j2] = F16::pack2(e0, e1);
        lq[j2] = F16::sum2(pbuf[cc][j2], lq[j2]);
      }
    }
    l_run += (lq[0] + lq[1]) + (lq[2] + lq[3]);
  };

  // The next block's Q rows into L2 (one 4-byte load per 128-byte line, 64
  // lines per wave, written as a throwaway at the end of LDS).
  auto prefetch_q = [&]() __attribute__((always_inline)) {
    int gi, r0, j0;
    make_blk(r_cur + 1, gi, r0, j0);
    const uint16_t* q0 = qg + q_base_of(gi) + (int64_t)(r0 + 32 * rb) * p.q_ss;
    const u32x4 rs = make_rsrc_words(q0, rows_extent(0, 32, p.q_ss, D));
    const uint32_t voff = (uint32_t)(lane >> 1) * (uint32_t)(p.q_ss * 2) + (uint32_t)(lane & 1) * 128;
    buf_load4_lds(rs, lds_address(smem_ip + Tile::PF_OFF + w * 256), voff);
  };

  // The wait that ends a softmax step.  Tile t's rows are loaded by both
  // groups in their softmax step t - 3, and the first GEMM to read them,
  // group 0's GEMM(t), follows group 0's softmax step t - 1 and group 1's
  // softmax step t - 2: group 0 waits for its loads of two steps back,
  // group 1 for those of one step back.  E loads issued after those (a Q
  // prefetch, the next block's Q rows) stay in flight too.
  auto step_wait = [&](auto e_c) __attribute__((always_inline)) {
    constexpr int E = decltype(e_c)::value;
    if (grp == 0)
      __builtin_amdgcn_s_waitcnt(vmcnt_imm(2 * LPS + E));
    else
      __builtin_amdgcn_s_waitcnt(vmcnt_imm(LPS + E));
  };
  using e0c = std::integral_constant<int, 0>;
  using e1c = std::integral_constant<int, 1>;

  // Softmax phase of the current block's tile j: the loads of K8_{j+3} (with
  // its key scales) and V_{j+2}, the softmax, the step wait.
  auto softmax_step = [&](int j) __attribute__((always_inline)) {
    load_k(j + NS - 1, (j + NS - 1) % NS, no{});
    load_v(j + NS - 2, (j + NS - 2) % NS, no{});
    const bool more = r_cur + 1 < rounds;
    const bool pre = j == c_J - 4 && more;
    if (pre) prefetch_q();
    softmax_tile(j);
    if ((pre || (j > 0 && j == c_J - 3)) && more)
      step_wait(e1c{});
    else
      step_wait(e0c{});
  };
  // A phase j < J - 4: both tiles are this block's, no Q prefetch around.
  auto softmax_step_plain = [&](int j) __attribute__((always_inline)) {
    load_k(j + NS - 1, (j + NS - 1) % NS, yes{});
    load_v(j + NS - 2, (j + NS - 2) % NS, yes{});
    softmax_tile(j);
    step_wait(e0c{});
  };
  // The block's last softmax phase: the next block's Q rows load first (the
  // last S^T product is done), ahead of the phase's tile loads.
  auto softmax_step_last = [&](int j, bool more) __attribute__((always_inline)) {
    if (more) {
      int gi, r0, j0;
      make_blk(r_cur + 1, gi, r0, j0);
      load_q_raw(gi, r0);
    }
    load_k(j + NS - 1, (j + NS - 1) % NS, no{});
    load_v(j + NS - 2, (j + NS - 2) % NS, no{});
    softmax_tile(j);
    if (more)
      step_wait(std::integral_constant<int, NQL>{});
    else
      step_wait(e0c{});
  };

  // ------------------------------------------------------------ prologue
  load_q_raw(c_gi, c_row0);
#pragma unroll
  for (int r = 0; r < NS - 1; ++r) load_k(r, r, no{});
#pragma unroll
  for (int r = 0; r < NS - 2; ++r) load_v(r, r, no{});
  quantize_q();
  __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));
  pp_barrier();

  uint16_t* const og = static_cast<uint16_t*>(p.o);
  // Output of block r (its state is still in acc / l_run / m_run), staged
  // through st_o and stored as whole rows, with the block's LSE.
  auto opaque = [](int x) __attribute__((always_inline)) {
    asm volatile("" : "+v"(x));
    return x;
  };
  auto finish_block = [&](int r, uint8_t* st_o) __attribute__((always_inline)) {
    const float l_tot = halves_sum(l_run);
    const float inv_l = l_tot > 0.f ? 1.f / l_tot : 0.f;
    const float lse_val = l_tot > 0.f ? (m_run + __log2f(l_tot)) * kLn2 : -INFINITY;
    int gi, r0, j0;
    make_blk(r, gi, r0, j0);
    const int lane_s = opaque(lane);
    u32x4 orows[8];
    stage_rows_gather<F16, NDB>(acc, inv_l, st_o, lane_s & 31, lane_s >> 5, lane_s, orows);
    const int row_w = r0 + 32 * rb;
    stage_rows_put(orows, og + o_base_of(gi) + (int64_t)row_w * p.o_ss, p.o_ss, lane_s);
    if (p.lse != nullptr && g == 0) p.lse[(int64_t)gi * S + row_w + c32] = lse_val;
  };
  auto reset_state = [&]() __attribute__((always_inline)) {
#pragma unroll
    for (int db = 0; db < NDB; ++db) acc[db] = f32x16{};
    m_run = -INFINITY;
    l_run = 0.f;
    m_c = 0.f;
  };
  // Output staging: group 0 past the rings (its phase's loads fill K8 stage 2
  // and V stage 1), group 1 one phase later in V stage 3 (its own last O^T
  // operand, next loaded two phases later) and past group 0's areas.
  uint8_t* const past = smem_ip + Tile::PAST_OFF;
  uint8_t* const st_own = grp == 0 ? past + sid * kStageOutBytes
                                   : (sid == 0 ? v_lds + 3 * VTILEB : past + (3 + sid) * kStageOutBytes);

  // The block loop (prefill_persist_kernel's): per block and group GEMM(0)
  // (S^T only), softmax(0), ..., softmax(J-1), GEMM(J) (O^T only), one
  // barrier after each; group 1 runs one phase behind throughout.
  if (grp == 1) pp_barrier();
  for (;;) {
    const int J = c_J;
    const int j_tail = J - 4;
    const bool more = r_cur + 1 < rounds;
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
    if (grp == 1) pp_barrier();
    finish_block(r_cur, st_own);
    reset_state();
    if (grp == 0) pp_barrier();
    if (!more) break;
    quantize_q();
    ++r_cur;
    make_blk(r_cur, c_gi, c_row0, c_J);
    set_bases();
    set_rows();
  }
  if (grp == 0) pp_barrier();
}

}  // namespace fa
