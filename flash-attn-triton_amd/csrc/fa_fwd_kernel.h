// FlashAttention-2 forward kernel for gfx950, fp16 / bf16 inputs, fp32 softmax.
//
// Behaviour follows the reference's dense and varlen forward kernels
// (/root/reference/flash_attn_triton/triton_kernel/attention_kernel.py:424-533
// `_attn_fwd`, :275-372 `_attn_fwd_inner`, :27-104 `_varlen_fwd`) and the
// materialized semantics of flash_attn_interface.py:15-49; the data layout
// and schedule are CDNA4-specific:
//
// * A workgroup owns BM = 32*NW query rows; wave w owns rows [32w, 32w+32).
// * Scores are produced transposed, S^T = K Q^T, with
//   v_mfma_f32_32x32x16_{f16,bf16}: A = K tile from LDS, B = Q^T held in
//   VGPRs for the whole kernel.  The accumulator layout of S^T puts query
//   row (lane % 32) in every lane, so row max / row sum need only the
//   lane^32 exchange (v_permlane32_swap), and the exponentiated scores are
//   already laid out as the B operand of the next product.
// * Output is produced transposed, O^T += V^T P^T, with the same MFMA:
//   A = V^T read from an LDS copy of the V tile stored transposed ([d][key]),
//   B = P^T straight from registers.  The O^T accumulator again holds query
//   row (lane % 32), so the online-softmax rescale is a per-lane scalar.
//   The order of keys inside one MFMA's reduction is a permutation shared by
//   both operands (key = 16c + 8(s/4) + 4(lane/32) + s%4 for slot s of
//   chunk c), which is exactly the order S^T's accumulator delivers them in.
// * K/V tiles of BN keys are double-buffered in LDS; the next tile's global
//   loads are issued before the current tile's math and written to LDS after
//   it, one barrier per tile.
// * Scores stay in fp32.  The softmax scale is folded into the exp2 argument
//   (one FMA per score) instead of pre-scaling and re-rounding Q as the
//   reference does (attention_kernel.py:491-495).
// * Mask order per score: scale -> ALiBi -> softcap -> mask (-inf), as in
//   attention_kernel.py:306-338 and :80-86.  Rows with no visible key produce
//   out = 0 and LSE = -inf (attention_kernel.py:522-532).
#pragma once

#include "fa_common.h"

namespace fa {

enum { kModePrefill = 0, kModeKvcache = 1 };

// All strides are in elements.  Layouts:
//   prefill, dense : q[b*q_sb + i*q_ss + h*q_sh + d]
//   prefill, varlen: q[(cu_q[b] + i)*q_ss + h*q_sh + d]   (cu_q != nullptr)
//   kvcache        : q as dense; keys through block_table (paged) or
//                    cache row / leftpad (batched cache)
struct FwdParams {
  const void* q; const void* k; const void* v; void* o; float* lse;
  int64_t q_sb, q_ss, q_sh;
  int64_t k_sb, k_ss, k_sh;
  int64_t v_sb, v_ss, v_sh;
  int64_t o_sb, o_ss, o_sh;
  int64_t lse_sb, lse_ss, lse_sh;
  int batch, seqlen_q, seqlen_k, heads_q, heads_k, group;
  float scale, scale_log2, softcap, softcap_k;   // softcap_k = 2 log2(e) / softcap
  const float* alibi; int64_t alibi_sb;
  // Optional fp32 additive bias on the scaled scores (after ALiBi, before
  // softcap), bias[b*bias_sb + h*bias_sh + i*bias_sq + j*bias_sk]; broadcast
  // dimensions have stride 0.  Dense prefill only.
  const float* bias; int64_t bias_sb, bias_sh, bias_sq, bias_sk;
  int causal, window_left, window_right;
  int64_t q_offset;
  const int* cu_q; const int* cu_k;
  // Varlen extras (nullable): seqused_q/k[b] limit sequence b to its first
  // queries / keys (0 <= used <= length, checked by the caller); cu_o[b] is the
  // first output (and LSE) row of sequence b when the outputs are packed by
  // the used query counts instead of cu_q.
  const int* seqused_q; const int* seqused_k; const int* cu_o;
  const int* seqlens_k;
  const int* block_table; int64_t bt_stride; int page_size;
  // Leading extent of a paged / batched cache (pages or cache rows) and the
  // block table's columns (0: bounded by seqlen_k): pages outside the cache
  // read as zeros and key counts are clamped to what the table and the cache
  // hold, so no read leaves them whatever the device arrays contain.
  int cache_blocks, bt_cols;
  const int* cache_rows;
  const int* leftpad;
  int kv_causal_offset;
  int num_splits, split_tiles;
  float* o_part; float* lse_part;
  int n_mblocks, total_blocks, heavy_first;
  // prefill_persist_kernel: row blocks per workgroup, and divisions by the
  // row blocks (causal: pairs of row blocks) per group, the query heads and
  // the GQA group size (set by the persistent launchers).
  int persist_rounds;
  FastDiv fd_blk, fd_heads, fd_group;
  // Dropout of the probabilities (prefill, GENERIC instantiations only).
  DropoutCfg drop;
};

template <int D, int NW, int BN>
struct FwdTile {
  static constexpr int DP = D < 32 ? 32 : D;   // head dim padded to one 32-wide MFMA block
  static constexpr int BM = NW * 32;
  static constexpr int NT = NW * 64;
  static constexpr int KSTR = DP + 8;          // K row pitch in LDS (halfs): 16 B pad
  static constexpr int VSTR = BN + 4;          // V^T row pitch in LDS (halfs): 8 B pad
  static constexpr int KTILE = BN * KSTR;
  static constexpr int VTILE = DP * VSTR;
  static constexpr int LDS_BYTES = 2 * (KTILE + VTILE) * 2;
};

template <class T, int D, int NW, int BN, int MODE, bool GENERIC>
__global__ __launch_bounds__(NW * 64) __attribute__((amdgpu_waves_per_eu(2, 2)))
void fwd_kernel(const FwdParams p) {
  using Tile = FwdTile<D, NW, BN>;
  constexpr int DP = Tile::DP;
  constexpr int BM = Tile::BM;
  constexpr int NT = Tile::NT;
  constexpr int KSTR = Tile::KSTR;
  constexpr int VSTR = Tile::VSTR;
  constexpr int KTILE = Tile::KTILE;
  constexpr int VTILE = Tile::VTILE;
  constexpr int NKC = DP / 16;
  constexpr int NDB = DP / 32;
  constexpr int NKB = BN / 32;
  constexpr int NCC = BN / 16;
  constexpr int CPR = DP / 8;                 // 16-byte chunks per row
  constexpr int KCH = BN * CPR;
  constexpr int KPT = (KCH + NT - 1) / NT;
  constexpr int VGR = (BN / 4) * CPR;          // 4-key x 8-dim groups per V tile
  constexpr int VPT = (VGR + NT - 1) / NT;
  static_assert(BN % 32 == 0, "tile must hold whole 32-key MFMA blocks");

  extern __shared__ __attribute__((aligned(16))) uint16_t smem[];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int w = tid >> 6;
  const int c32 = lane & 31;
  const int g = lane >> 5;

  // ---------------------------------------------------------------- work item
  int id = xcd_remap(blockIdx.x, p.total_blocks);
  int mb = id % p.n_mblocks;
  id /= p.n_mblocks;
  int split = 0;
  if (MODE == kModeKvcache) {
    split = id % p.num_splits;
    id /= p.num_splits;
  }
  const int nh = MODE == kModePrefill ? p.heads_q : p.heads_k;
  const int hh = id % nh;
  const int b = id / nh;
  if (p.heavy_first) mb = p.n_mblocks - 1 - mb;

  const uint16_t* qg = static_cast<const uint16_t*>(p.q);
  const uint16_t* kg = static_cast<const uint16_t*>(p.k);
  const uint16_t* vg = static_cast<const uint16_t*>(p.v);
  uint16_t* og = static_cast<uint16_t*>(p.o);

  int Sq, Sk;
  int64_t qoff = 0;
  int64_t q_base, o_base, lse_base;
  int64_t k_base = 0, v_base = 0;
  const int* bt_row = nullptr;
  int kvh;
  if (MODE == kModePrefill) {
    kvh = hh / p.group;
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
      if (p.block_table != nullptr) {
        // Paged varlen: key j of sequence b is slot j % page_size of page
        // block_table[b][j / page_size].
        bt_row = p.block_table + (int64_t)b * p.bt_stride;
        if (p.bt_cols > 0) Sk = min(Sk, (int)min((int64_t)p.bt_cols * p.page_size, (int64_t)1 << 30));
      } else {
        k_base = (int64_t)ks * p.k_ss;
        v_base = (int64_t)ks * p.v_ss;
      }
    } else {
      Sq = p.seqlen_q;
      Sk = p.seqlen_k;
      q_base = (int64_t)b * p.q_sb;
      o_base = (int64_t)b * p.o_sb;
      lse_base = (int64_t)b * p.lse_sb;
      k_base = (int64_t)b * p.k_sb;
      v_base = (int64_t)b * p.v_sb;
    }
    qoff = p.q_offset;
    q_base += (int64_t)hh * p.q_sh;
    o_base += (int64_t)hh * p.o_sh;
    lse_base += (int64_t)hh * p.lse_sh;
  } else {
    kvh = hh;
    Sq = p.seqlen_q;
    Sk = p.seqlen_k;
    if (p.seqlens_k != nullptr) Sk = p.seqlens_k[b];
    // Keys within the cache: seqlen_k (the capacity, for a paged cache at
    // most the table's columns times page_size) less the left padding; a
    // batched-cache row outside the cache holds none.
    int lp = 0;
    if (p.block_table != nullptr) {
      bt_row = p.block_table + (int64_t)b * p.bt_stride;
    } else {
      const int row = p.cache_rows != nullptr ? p.cache_rows[b] : b;
      lp = p.leftpad != nullptr ? p.leftpad[b] : 0;
      lp = max(0, min(lp, p.seqlen_k));
      if (row < 0 || row >= p.cache_blocks) Sk = 0;
      k_base = (int64_t)row * p.k_sb + (int64_t)lp * p.k_ss;
      v_base = (int64_t)row * p.v_sb + (int64_t)lp * p.v_ss;
    }
    Sk = max(0, min(Sk, p.seqlen_k - lp));
    if (p.kv_causal_offset) qoff = (int64_t)Sk - Sq;
    q_base = (int64_t)b * p.q_sb;
    o_base = (int64_t)b * p.o_sb;
    lse_base = (int64_t)b * p.lse_sb;
  }
  k_base += (int64_t)kvh * p.k_sh;
  v_base += (int64_t)kvh * p.v_sh;

  const int G = p.group;
  const int rows_total = MODE == kModePrefill ? Sq : Sq * G;
  const int row0 = mb * BM;
  if (row0 >= rows_total) return;   // varlen blocks past this sequence's queries
  const int row_last = min(row0 + BM, rows_total) - 1;

  auto row_query = [&](int gr) -> int { return MODE == kModePrefill ? gr : gr / G; };

  // Rows of this lane.
  const int gr = row0 + w * 32 + c32;
  const bool row_valid = gr < rows_total;
  const int qi = row_query(gr);
  const int head = MODE == kModePrefill ? hh : hh * G + gr % G;
  const int64_t qpos = (int64_t)qi + qoff;
  float slope = 0.f;
  if (GENERIC && p.alibi != nullptr && row_valid) slope = p.alibi[(int64_t)b * p.alibi_sb + head];

  // Query-position extents of the workgroup and of this wave.
  const int64_t qpos_blk_min = (int64_t)row_query(row0) + qoff;
  const int64_t qpos_blk_max = (int64_t)row_query(row_last) + qoff;
  const int wrow0 = row0 + w * 32;
  const bool wave_active = wrow0 <= row_last;
  const int64_t qpos_w_min = (int64_t)row_query(wrow0) + qoff;
  const int64_t qpos_w_max = (int64_t)row_query(min(wrow0 + 31, row_last)) + qoff;

  const int wl = p.window_left, wr = p.window_right;
  const bool causal = p.causal != 0;

  // Key range [k_lo, k_hi) any row of the workgroup can see.
  int64_t k_hi = Sk;
  if (causal) k_hi = min(k_hi, qpos_blk_max + 1);
  if (wr >= 0) k_hi = min(k_hi, qpos_blk_max + wr + 1);
  int64_t k_lo = 0;
  if (wl >= 0) k_lo = max((int64_t)0, qpos_blk_min - wl);
  int t_begin = (int)(k_lo / BN);
  int t_end = k_hi > k_lo ? (int)((k_hi + BN - 1) / BN) : t_begin;
  if (MODE == kModeKvcache) {
    t_begin = max(t_begin, split * p.split_tiles);
    t_end = min(t_end, (split + 1) * p.split_tiles);
    if (t_end < t_begin) t_end = t_begin;
  }

  // ---------------------------------------------------------------- Q in VGPRs
  u32x4 qreg[NKC];
  {
    const uint16_t* qrow = qg + q_base + (int64_t)qi * p.q_ss +
                           (MODE == kModePrefill ? 0 : (int64_t)head * p.q_sh);
#pragma unroll
    for (int kc = 0; kc < NKC; ++kc) {
      const int d0 = kc * 16 + g * 8;
      qreg[kc] = (row_valid && d0 < D) ? load16(qrow + d0) : u32x4{0, 0, 0, 0};
    }
  }

  // ---------------------------------------------------------------- tile I/O
  // Element offset of key j's row, or -1 for a page outside the cache (the
  // key then reads as zeros).
  auto key_offset = [&](int j, int64_t base, int64_t sb, int64_t ss) -> int64_t {
    if (bt_row != nullptr) {
      const int page = bt_row[j / p.page_size];
      if (page < 0 || page >= p.cache_blocks) return -1;
      return base + (int64_t)page * sb + (int64_t)(j % p.page_size) * ss;
    }
    return base + (int64_t)j * ss;
  };

  u32x4 kreg[KPT];
  u32x4 vreg[VPT][4];
  auto load_tile = [&](int t) {
    const int n0 = t * BN;
#pragma unroll
    for (int i = 0; i < KPT; ++i) {
      const int c = tid + i * NT;
      kreg[i] = u32x4{0, 0, 0, 0};
      if (c < KCH) {
        const int n = c / CPR, d = (c % CPR) * 8;
        const int j = n0 + n;
        if (j < Sk && d < D) {
          const int64_t off = key_offset(j, k_base, p.k_sb, p.k_ss);
          if (off >= 0) kreg[i] = load16(kg + off + d);
        }
      }
    }
#pragma unroll
    for (int i = 0; i < VPT; ++i) {
      const int gi = tid + i * NT;
#pragma unroll
      for (int u = 0; u < 4; ++u) vreg[i][u] = u32x4{0, 0, 0, 0};
      if (gi < VGR) {
        const int ng = gi / CPR, d = (gi % CPR) * 8;
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          const int j = n0 + ng * 4 + u;
          if (j < Sk && d < D) {
            const int64_t off = key_offset(j, v_base, p.v_sb, p.v_ss);
            if (off >= 0) vreg[i][u] = load16(vg + off + d);
          }
        }
      }
    }
  };
  auto store_tile = [&](int buf) {
    uint16_t* Ks = smem + buf * (KTILE + VTILE);
    uint16_t* Vt = Ks + KTILE;
#pragma unroll
    for (int i = 0; i < KPT; ++i) {
      const int c = tid + i * NT;
      if (c < KCH) store16(Ks + (c / CPR) * KSTR + (c % CPR) * 8, kreg[i]);
    }
#pragma unroll
    for (int i = 0; i < VPT; ++i) {
      const int gi = tid + i * NT;
      if (gi < VGR) {
        const int ng = gi / CPR, d0 = (gi % CPR) * 8;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const uint32_t sel = (e & 1) ? 0x07060302u : 0x05040100u;
          const int wd = e >> 1;
          u32x2 pr;
          pr[0] = __builtin_amdgcn_perm(vreg[i][1][wd], vreg[i][0][wd], sel);
          pr[1] = __builtin_amdgcn_perm(vreg[i][3][wd], vreg[i][2][wd], sel);
          *reinterpret_cast<u32x2*>(Vt + (d0 + e) * VSTR + ng * 4) = pr;
        }
      }
    }
  };

  // ---------------------------------------------------------------- main loop
  f32x16 acc[NDB];
#pragma unroll
  for (int db = 0; db < NDB; ++db) acc[db] = f32x16{};
  float m_run = -INFINITY;   // running max in log2 units
  float l_run = 0.f;         // this lane's partial row sum (keys with lane/32 == g)

  if (t_begin < t_end) {
    load_tile(t_begin);
    store_tile(0);
  }
  for (int t = t_begin; t < t_end; ++t) {
    const int buf = (t - t_begin) & 1;
    __syncthreads();
    const bool has_next = t + 1 < t_end;
    if (has_next) load_tile(t + 1);

    const int n0 = t * BN;
    const int n1 = n0 + BN;   // exclusive
    bool skip = !wave_active || n0 >= Sk;
    if (causal) skip = skip || n0 > qpos_w_max;
    if (wr >= 0) skip = skip || n0 > qpos_w_max + wr;
    if (wl >= 0) skip = skip || n1 - 1 < qpos_w_min - wl;
    if (!skip) {
      bool need_mask = n1 > Sk;
      if (causal) need_mask = need_mask || n1 - 1 > qpos_w_min;
      if (wr >= 0) need_mask = need_mask || n1 - 1 > qpos_w_min + wr;
      if (wl >= 0) need_mask = need_mask || n0 < qpos_w_max - wl;

      const uint16_t* Ks = smem + buf * (KTILE + VTILE);
      const uint16_t* Vt = Ks + KTILE;

      f32x16 s[NKB];
#pragma unroll
      for (int kb = 0; kb < NKB; ++kb) {
        s[kb] = f32x16{};
#pragma unroll
        for (int kc = 0; kc < NKC; ++kc) {
          const u32x4 a = load16(Ks + (kb * 32 + c32) * KSTR + kc * 16 + g * 8);
          s[kb] = T::mfma32(a, qreg[kc], s[kb]);
        }
      }

      float mx = -INFINITY;
#pragma unroll
      for (int kb = 0; kb < NKB; ++kb) {
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          const int key = n0 + kb * 32 + 8 * (v >> 2) + 4 * g + (v & 3);
          float x = s[kb][v];
          if (GENERIC) {
            x *= p.scale;
            if (p.alibi != nullptr) x -= slope * fabsf((float)(qpos - key));
            if (MODE == kModePrefill && p.bias != nullptr && row_valid && key < Sk)
              x += p.bias[(int64_t)b * p.bias_sb + (int64_t)head * p.bias_sh +
                          (int64_t)qi * p.bias_sq + (int64_t)key * p.bias_sk];
            if (p.softcap > 0.f) x = p.softcap * tanhf(x / p.softcap);
            x *= kLog2e;
          }
          if (need_mask) {
            bool ok = key < Sk;
            if (causal) ok = ok && key <= qpos;
            if (wl >= 0) ok = ok && key >= qpos - wl;
            if (wr >= 0) ok = ok && key <= qpos + wr;
            if (!ok) x = -INFINITY;
          }
          s[kb][v] = x;
          mx = fmaxf(mx, x);
        }
      }
      mx = halves_max(mx);
      const float m_tile = GENERIC ? mx : mx * p.scale_log2;
      const float m_new = fmaxf(m_run, m_tile);
      const float m_use = m_new == -INFINITY ? 0.f : m_new;
      const float alpha = exp2f(m_run - m_use);
      float rs = 0.f;
#pragma unroll
      for (int kb = 0; kb < NKB; ++kb) {
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          const float e = GENERIC ? exp2f(s[kb][v] - m_use)
                                  : exp2f(fmaf(s[kb][v], p.scale_log2, -m_use));
          s[kb][v] = e;
          rs += e;
        }
      }
      l_run = l_run * alpha + rs;
      m_run = m_new;
#pragma unroll
      for (int db = 0; db < NDB; ++db) acc[db] *= alpha;

#pragma unroll
      for (int cc = 0; cc < NCC; ++cc) {
        const f32x16& sv = s[cc >> 1];
        const int o8 = (cc & 1) * 8;
        u32x4 pb;
        if (MODE == kModePrefill && GENERIC && p.drop.enabled) {
          // Row sums above use the undropped P; the product takes the dropped one.
          const u32x4 r = dropout_draws(p.drop, (n0 >> 4) + cc, g, qi, head, b);
#pragma unroll
          for (int j = 0; j < 4; ++j)
            pb[j] = T::pack2(sv[o8 + 2 * j] * dropout_factor(p.drop, r, 2 * j),
                             sv[o8 + 2 * j + 1] * dropout_factor(p.drop, r, 2 * j + 1));
        } else {
          pb[0] = T::pack2(sv[o8 + 0], sv[o8 + 1]);
          pb[1] = T::pack2(sv[o8 + 2], sv[o8 + 3]);
          pb[2] = T::pack2(sv[o8 + 4], sv[o8 + 5]);
          pb[3] = T::pack2(sv[o8 + 6], sv[o8 + 7]);
        }
#pragma unroll
        for (int db = 0; db < NDB; ++db) {
          const uint16_t* vrow = Vt + (db * 32 + c32) * VSTR + cc * 16 + g * 4;
          const u32x2 lo = *reinterpret_cast<const u32x2*>(vrow);
          const u32x2 hi = *reinterpret_cast<const u32x2*>(vrow + 8);
          const u32x4 a = {lo[0], lo[1], hi[0], hi[1]};
          acc[db] = T::mfma32(a, pb, acc[db]);
        }
      }
    }
    if (has_next) store_tile(buf ^ 1);
  }

  // ---------------------------------------------------------------- epilogue
  const float l_tot = halves_sum(l_run);
  const float inv_l = l_tot > 0.f ? 1.f / l_tot : 0.f;
  const float lse_val = l_tot > 0.f ? (m_run + __log2f(l_tot)) * kLn2 : -INFINITY;
  if (!row_valid) return;

  const bool to_partials = MODE == kModeKvcache && p.num_splits > 1;
  if (to_partials) {
    const int64_t prow = (((int64_t)split * p.batch + b) * Sq + qi) * p.heads_q + head;
    float* orow = p.o_part + prow * D;
#pragma unroll
    for (int db = 0; db < NDB; ++db) {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int d = db * 32 + r * 8 + g * 4;
        if (d < D) {
          f32x4 val = {acc[db][4 * r] * inv_l, acc[db][4 * r + 1] * inv_l,
                       acc[db][4 * r + 2] * inv_l, acc[db][4 * r + 3] * inv_l};
          *reinterpret_cast<f32x4*>(orow + d) = val;
        }
      }
    }
    if (g == 0) p.lse_part[prow] = lse_val;
    return;
  }

  uint16_t* orow = og + o_base + (int64_t)qi * p.o_ss +
                   (MODE == kModePrefill ? 0 : (int64_t)head * p.o_sh);
#pragma unroll
  for (int db = 0; db < NDB; ++db) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int d = db * 32 + r * 8 + g * 4;
      if (d < D) {
        u32x2 val;
        val[0] = T::pack2(acc[db][4 * r] * inv_l, acc[db][4 * r + 1] * inv_l);
        val[1] = T::pack2(acc[db][4 * r + 2] * inv_l, acc[db][4 * r + 3] * inv_l);
        *reinterpret_cast<u32x2*>(orow + d) = val;
      }
    }
  }
  if (p.lse != nullptr && g == 0) {
    const int64_t li = lse_base + (int64_t)qi * p.lse_ss +
                       (MODE == kModePrefill ? 0 : (int64_t)head * p.lse_sh);
    p.lse[li] = lse_val;
  }
}

// Merge split-KV partials: out = sum_s exp(lse_s - lse) * o_s, lse = log sum exp(lse_s).
// One thread per (row, 4 head-dim values); rows enumerate (b, i, h).
template <class T>
__global__ __launch_bounds__(256) void combine_kernel(const float* __restrict__ o_part,
                                                      const float* __restrict__ lse_part,
                                                      void* out, float* lse_out, int num_splits,
                                                      int batch, int seqlen_q, int heads, int D,
                                                      int64_t o_sb, int64_t o_ss, int64_t o_sh,
                                                      int64_t lse_sb, int64_t lse_ss,
                                                      int64_t lse_sh) {
  const int quads = D / 4;
  const int64_t rows = (int64_t)batch * seqlen_q * heads;
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= rows * quads) return;
  const int64_t row = idx / quads;
  const int qd = (int)(idx % quads);
  const int h = (int)(row % heads);
  const int i = (int)((row / heads) % seqlen_q);
  const int b = (int)(row / ((int64_t)heads * seqlen_q));
  float m = -INFINITY;
  for (int s = 0; s < num_splits; ++s) m = fmaxf(m, lse_part[(int64_t)s * rows + row]);
  f32x4 acc = {0.f, 0.f, 0.f, 0.f};
  float tot = 0.f;
  if (m != -INFINITY) {
    for (int s = 0; s < num_splits; ++s) {
      const float ls = lse_part[(int64_t)s * rows + row];
      if (ls == -INFINITY) continue;
      const float wgt = __expf(ls - m);
      tot += wgt;
      const f32x4 o = *reinterpret_cast<const f32x4*>(o_part + ((int64_t)s * rows + row) * D + qd * 4);
      acc += wgt * o;
    }
  }
  const float inv = tot > 0.f ? 1.f / tot : 0.f;
  uint16_t* orow = static_cast<uint16_t*>(out) + (int64_t)b * o_sb + (int64_t)i * o_ss + (int64_t)h * o_sh;
  u32x2 val;
  val[0] = T::pack2(acc[0] * inv, acc[1] * inv);
  val[1] = T::pack2(acc[2] * inv, acc[3] * inv);
  *reinterpret_cast<u32x2*>(orow + qd * 4) = val;
  if (lse_out != nullptr && qd == 0)
    lse_out[(int64_t)b * lse_sb + (int64_t)i * lse_ss + (int64_t)h * lse_sh] =
        tot > 0.f ? m + __logf(tot) : -INFINITY;
}

}  // namespace fa
