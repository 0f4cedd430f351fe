// fp32 attention forward for gfx950: dense / cross / varlen prefill and the
// KV-cache path, for fp32 q/k/v (flash_attn_interface.py:95-96 accepts fp16 and
// fp32; BASELINE config 1 is fp32).
//
// The reference runs its Triton kernels on fp32 tensors with fp32 dot products
// and keeps P in the input dtype for the PV product
// (/root/reference/flash_attn_triton/triton_kernel/attention_kernel.py:366-367),
// i.e. the whole computation stays fp32.  Here both products run on the CDNA4
// fp32 matrix core, v_mfma_f32_32x32x2_f32, which multiplies and accumulates
// in fp32: the results agree with a float64 evaluation to ~1e-6.
//
// Layout per workgroup: four waves, one per SIMD, each owning 32 query rows
// (kernel-wide 128), 32-key tiles of K and V staged in LDS.  The 32x32x2 MFMA
// takes one A and one B value per lane and reduces over k = lane / 32; lane
// half g owns dims [g D/2, (g + 1) D/2), so call j pairs dims j and D/2 + j and
// every operand read is a run of consecutive floats:
//   S^T = K Q^T : call j, A = K[key c32][g D/2 + j], B = Q[row c32][g D/2 + j]
//                 (Q^T held in VGPRs for the whole kernel, D/2 per lane);
//   O^T += V^T P^T: for 32-dim block db, call jj pairs the keys the S^T
//                 accumulator holds in slot jj of the two halves
//                 (key(g, jj) = 8 (jj / 4) + 4 g + jj % 4), so B = P[jj]
//                 straight from the softmax and A = V[key(g, jj)][32 db + c32].
// The score epilogue (scale, ALiBi, bias, softcap, mask), online softmax,
// empty-row rule (out 0, LSE -inf) and alignments are those of fwd_kernel
// (fa_fwd_kernel.h).  P stays fp32.
#include "fa_fwd_launch.h"

namespace fa {

template <int D>
struct F32Tile {
  static constexpr int NW = 4;
  static constexpr int NT = NW * 64;
  static constexpr int BM = NW * 32;
  static constexpr int BN = 32;
  static constexpr int DP = D < 32 ? 32 : D;     // V rows padded to one 32-dim block
  static constexpr int KSTR = D + 4;             // K row pitch in LDS (floats): 16 B pad
  static constexpr int VSTR = DP + 4;            // V row pitch in LDS (floats)
  static constexpr int LDS_BYTES = BN * (KSTR + VSTR) * 4;
  static constexpr int KCH = BN * D / 4;         // 16-byte chunks per K tile
  static constexpr int VCH = BN * D / 4;
  static constexpr int KPT = (KCH + NT - 1) / NT;
};

template <int D, int MODE, bool GENERIC>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, 1)))
void fwd_f32_kernel(const FwdParams p) {
  using Tile = F32Tile<D>;
  constexpr int BM = Tile::BM, BN = Tile::BN, NT = Tile::NT;
  constexpr int DP = Tile::DP, KSTR = Tile::KSTR, VSTR = Tile::VSTR;
  constexpr int KCH = Tile::KCH, KPT = Tile::KPT;
  constexpr int DH = D / 2;          // dims per lane half
  constexpr int NDB = DP / 32;       // 32-dim output blocks
  constexpr int CPR = D / 4;         // 16-byte chunks per row

  extern __shared__ __attribute__((aligned(16))) float smf[];
  float* Ks = smf;
  float* Vs = smf + BN * KSTR;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int w = tid >> 6;
  const int c32 = lane & 31;
  const int g = lane >> 5;

  // ---------------------------------------------------------------- work item
  int id = xcd_remap(blockIdx.x, p.total_blocks);
  int mb = id % p.n_mblocks;
  id /= p.n_mblocks;
  const int nh = MODE == kModePrefill ? p.heads_q : p.heads_k;
  const int hh = id % nh;
  const int b = id / nh;
  if (p.heavy_first) mb = p.n_mblocks - 1 - mb;

  const float* qg = static_cast<const float*>(p.q);
  const float* kg = static_cast<const float*>(p.k);
  const float* vg = static_cast<const float*>(p.v);
  float* og = static_cast<float*>(p.o);

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
        bt_row = p.block_table + (int64_t)b * p.bt_stride;   // paged varlen
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
    // Keys within the cache (see FwdParams::cache_blocks).
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
  if (row0 >= rows_total) return;   // whole workgroup: past this sequence's rows
  const int row_last = min(row0 + BM, rows_total) - 1;
  auto row_query = [&](int gr) -> int { return MODE == kModePrefill ? gr : gr / G; };

  const int gr = row0 + w * 32 + c32;
  const bool row_valid = gr < rows_total;
  const int qi = row_query(row_valid ? gr : row_last);
  const int head = MODE == kModePrefill ? hh : hh * G + (row_valid ? gr : row_last) % G;
  const int64_t qpos = (int64_t)qi + qoff;
  float slope = 0.f;
  if (GENERIC && p.alibi != nullptr && row_valid) slope = p.alibi[(int64_t)b * p.alibi_sb + head];
  const float* bias_row = nullptr;
  if (GENERIC && p.bias != nullptr)
    bias_row = p.bias + (int64_t)b * p.bias_sb + (int64_t)head * p.bias_sh + (int64_t)qi * p.bias_sq;

  const int64_t qpos_blk_min = (int64_t)row_query(row0) + qoff;
  const int64_t qpos_blk_max = (int64_t)row_query(row_last) + qoff;
  const int wl = p.window_left, wr = p.window_right;
  const bool causal = p.causal != 0;
  int64_t key_hi = Sk - 1;
  if (causal) key_hi = min(key_hi, qpos);
  if (wr >= 0) key_hi = min(key_hi, qpos + wr);
  const int64_t key_lo = wl >= 0 ? qpos - wl : INT64_MIN / 2;

  int64_t k_hi = Sk;
  if (causal) k_hi = min(k_hi, qpos_blk_max + 1);
  if (wr >= 0) k_hi = min(k_hi, qpos_blk_max + wr + 1);
  int64_t k_lo = 0;
  if (wl >= 0) k_lo = max((int64_t)0, qpos_blk_min - wl);
  const int t_begin = (int)(k_lo / BN);
  const int t_end = k_hi > k_lo ? (int)((k_hi + BN - 1) / BN) : t_begin;

  // ---------------------------------------------------------------- Q^T in VGPRs
  float qv[DH];
  {
    const float* qrow = qg + q_base + (int64_t)qi * p.q_ss +
                        (MODE == kModePrefill ? 0 : (int64_t)head * p.q_sh) + g * DH;
#pragma unroll
    for (int j = 0; j < DH; j += 4) {
      const f32x4 x = row_valid ? *reinterpret_cast<const f32x4*>(qrow + j) : f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int e = 0; e < 4; ++e) qv[j + e] = x[e];
    }
  }

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

  f32x16 acc[NDB];
#pragma unroll
  for (int db = 0; db < NDB; ++db) acc[db] = f32x16{};
  float m_run = -INFINITY;
  float l_run = 0.f;

  // V rows past D (D = 16) stay zero for the whole kernel.
  if (D < DP) {
    for (int i = tid; i < BN * VSTR; i += NT) Vs[i] = 0.f;
  }

  for (int t = t_begin; t < t_end; ++t) {
    const int n0 = t * BN;
    __syncthreads();   // previous tile's LDS reads are done
#pragma unroll
    for (int i = 0; i < KPT; ++i) {
      const int c = tid + i * NT;
      if (c < KCH) {
        const int n = c / CPR, d = (c % CPR) * 4;
        const int j = n0 + n;
        f32x4 kx = {0.f, 0.f, 0.f, 0.f}, vx = {0.f, 0.f, 0.f, 0.f};
        if (j < Sk) {
          const int64_t ko = key_offset(j, k_base, p.k_sb, p.k_ss);
          const int64_t vo = key_offset(j, v_base, p.v_sb, p.v_ss);
          if (ko >= 0) kx = *reinterpret_cast<const f32x4*>(kg + ko + d);
          if (vo >= 0) vx = *reinterpret_cast<const f32x4*>(vg + vo + d);
        }
        *reinterpret_cast<f32x4*>(Ks + n * KSTR + d) = kx;
        *reinterpret_cast<f32x4*>(Vs + n * VSTR + d) = vx;
      }
    }
    __syncthreads();

    // S^T = K Q^T.
    f32x16 s = f32x16{};
    const float* krow = Ks + c32 * KSTR + g * DH;
#pragma unroll
    for (int j = 0; j < DH; j += 4) {
      const f32x4 kx = *reinterpret_cast<const f32x4*>(krow + j);
#pragma unroll
      for (int e = 0; e < 4; ++e) s = __builtin_amdgcn_mfma_f32_32x32x2f32(kx[e], qv[j + e], s, 0, 0, 0);
    }

    // Score epilogue and mask (keys outside [key_lo, key_hi] -> -inf).
    const float sl = GENERIC ? 1.f : p.scale_log2;
#pragma unroll
    for (int v = 0; v < 16; ++v) {
      const int key = n0 + 8 * (v >> 2) + 4 * g + (v & 3);
      float x = s[v];
      if (GENERIC) {
        x *= p.scale;
        if (p.alibi != nullptr) x = fmaf(-slope, fabsf((float)(qpos - key)), x);
        if (bias_row != nullptr && row_valid && key < Sk) x += bias_row[(int64_t)key * p.bias_sk];
        if (p.softcap > 0.f) x = p.softcap * tanhf(x / p.softcap);
        x *= kLog2e;
      }
      if (key < key_lo || key > key_hi) x = -INFINITY;
      s[v] = x;
    }
    float mx = -INFINITY;
#pragma unroll
    for (int v = 0; v < 16; ++v) mx = fmaxf(mx, s[v]);
    mx = halves_max(mx) * sl;
    const float m_new = fmaxf(m_run, mx);
    const float alpha = m_new == -INFINITY ? 1.f : exp2f(m_run - m_new);
    l_run *= alpha;
#pragma unroll
    for (int db = 0; db < NDB; ++db) acc[db] *= alpha;
    m_run = m_new;
    const float m_use = m_run == -INFINITY ? 0.f : m_run;
    float pv[16];
#pragma unroll
    for (int v = 0; v < 16; ++v) {
      pv[v] = exp2f(fmaf(s[v], sl, -m_use));
      l_run += pv[v];
    }
    if (MODE == kModePrefill && GENERIC && p.drop.enabled) {
      // The row sum above is of the undropped P; the product takes the dropped one.
#pragma unroll
      for (int cc = 0; cc < 2; ++cc) {
        const u32x4 r = dropout_draws(p.drop, (n0 >> 4) + cc, g, qi, hh, b);
#pragma unroll
        for (int e = 0; e < 8; ++e) pv[8 * cc + e] *= dropout_factor(p.drop, r, e);
      }
    }

    // O^T += V^T P^T.
#pragma unroll
    for (int db = 0; db < NDB; ++db) {
#pragma unroll
      for (int jj = 0; jj < 16; ++jj) {
        const int key = 8 * (jj >> 2) + 4 * g + (jj & 3);
        acc[db] = __builtin_amdgcn_mfma_f32_32x32x2f32(Vs[key * VSTR + db * 32 + c32], pv[jj], acc[db], 0, 0, 0);
      }
    }
  }

  // ---------------------------------------------------------------- epilogue
  const float l_tot = halves_sum(l_run);
  const float inv_l = l_tot > 0.f ? 1.f / l_tot : 0.f;
  const float lse_val = l_tot > 0.f ? (m_run + __log2f(l_tot)) * kLn2 : -INFINITY;
  if (!row_valid) return;
  float* orow = og + o_base + (int64_t)qi * p.o_ss + (MODE == kModePrefill ? 0 : (int64_t)head * p.o_sh);
#pragma unroll
  for (int db = 0; db < NDB; ++db) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int d = db * 32 + r * 8 + g * 4;
      if (d < D)
        *reinterpret_cast<f32x4*>(orow + d) =
            f32x4{acc[db][4 * r] * inv_l, acc[db][4 * r + 1] * inv_l, acc[db][4 * r + 2] * inv_l,
                  acc[db][4 * r + 3] * inv_l};
    }
  }
  if (p.lse != nullptr && g == 0) {
    const int64_t li = lse_base + (int64_t)qi * p.lse_ss + (MODE == kModePrefill ? 0 : (int64_t)head * p.lse_sh);
    p.lse[li] = lse_val;
  }
}

template <int D, int MODE, bool GEN>
hipError_t launch_f32_d(FwdParams p, hipStream_t st) {
  using Tile = F32Tile<D>;
  auto kern = fwd_f32_kernel<D, MODE, GEN>;
  static std::atomic<uint64_t> lds_devices{0};
  if (hipError_t e = set_lds_limit(lds_devices, kern, Tile::LDS_BYTES); e != hipSuccess) return e;
  const int rows = MODE == kModePrefill ? p.seqlen_q : p.seqlen_q * p.group;
  p.n_mblocks = (rows + Tile::BM - 1) / Tile::BM;
  const int64_t outer = (int64_t)(MODE == kModePrefill ? p.heads_q : p.heads_k) * p.batch;
  const int64_t total = (int64_t)p.n_mblocks * outer;
  if (total <= 0) return hipSuccess;
  if (total > 0x7fffffff) return hipErrorInvalidConfiguration;
  p.total_blocks = (int)total;
  hipLaunchKernelGGL(kern, dim3((unsigned)total), dim3(Tile::NT), Tile::LDS_BYTES, st, p);
  return hipGetLastError();
}

template <int MODE>
hipError_t launch_f32_mode(const FwdParams& p, int head_dim, bool generic, hipStream_t st) {
#define FA_F32_CASE(DD) \
  case DD: return generic ? launch_f32_d<DD, MODE, true>(p, st) : launch_f32_d<DD, MODE, false>(p, st);
  switch (head_dim) {
    FA_F32_CASE(16)
    FA_F32_CASE(32)
    FA_F32_CASE(64)
    FA_F32_CASE(128)
    FA_F32_CASE(256)
    default:
      return hipErrorInvalidValue;
  }
#undef FA_F32_CASE
}

}  // namespace fa

// fp32 forward: every key of a row in one workgroup (no split-KV).
hipError_t fa_launch_fwd_f32(const fa::FwdParams& p, int mode, int head_dim, bool generic,
                             hipStream_t st) {
  if (mode == fa::kModePrefill) return fa::launch_f32_mode<fa::kModePrefill>(p, head_dim, generic, st);
  return fa::launch_f32_mode<fa::kModeKvcache>(p, head_dim, generic, st);
}
