// fp32 attention backward for gfx950 (dense and varlen), the gradients of
// fwd_f32_kernel (fa_fwd_f32.hip).
//
// The reference's backward is dtype-generic Triton
// (/root/reference/flash_attn_triton/triton_kernel/attention_kernel.py:
// 1104-1155 `_dense_backward`, :1185-1198, varlen :1322-1361), so fp32 inputs
// get fp32 gradients.  The math is that of fa_bwd_kernel.h:
//   P  = exp(x - lse)     x = scale * q.k -> ALiBi -> attn_bias -> softcap -> mask
//   dV = P^T dO           dP = dO V^T        delta = rowsum(dO * O)
//   dS = P (F dP - delta) softcap'           (F: the forward's dropout multipliers)
//   dQ = scale * dS K     dK = scale * dS^T Q   (dV uses F P)
// with every product on the fp32 matrix core, v_mfma_f32_32x32x2_f32, so the
// gradients are fp32 throughout.
//
// Layouts follow the fp32 forward: the 32x32x2 product takes one A and one B
// value per lane and reduces over k = lane / 32, so lane half g owns dims
// [g D/2, (g + 1) D/2) and call j pairs dims j and D/2 + j.
// * bwd_f32_dq_kernel: four waves of 32 query rows; Q^T and dO^T of the
//   wave's rows stay in VGPRs, 32-key tiles of K and V stream through LDS.
//   S^T = K Q^T and dP^T = V dO^T put one query row in each lane (keys
//   8 (v / 4) + 4 g + v % 4 in slot v), so dS^T is already the B operand of
//   dQ^T += K^T dS^T (A = K[key of slot jj][32 db + lane % 32]), as P^T is in
//   the forward's O^T product.  It also writes delta.
// * bwd_f32_dkdv_kernel: four waves of 32 keys; K^T and V^T stay in VGPRs,
//   32-row tiles of Q and dO (with their LSE and delta) stream through LDS for
//   every query head of the K/V head's group.  S = Q K^T and dP = dO V^T put
//   one key in each lane, so F P and dS are the B operands of dV^T += dO^T (F P)
//   and dK^T += Q^T dS.
// No atomics except for the attn_bias gradient (broadcast dims sum).  Head
// dims 32, 64, 128 and 256 (16 is run at 32 by the caller).  At 256 the
// resident Q^T / dO^T (or K^T / V^T) rows take 256 registers per lane, and
// the full-width accumulators another 128 (dQ) or 256 (dK and dV): each
// kernel then makes two passes over its tiles, accumulating and storing
// output dims [0, 128) in the first and [128, 256) in the second, and
// recomputes S and dP in each (one wave per SIMD, 512 registers).
#include "fa_bwd.h"

namespace fa {

template <int D>
struct F32BwdTile {
  static constexpr int NW = 4;
  static constexpr int NT = NW * 64;
  static constexpr int BB = NW * 32;           // query rows (dQ) or keys (dK/dV) per workgroup
  static constexpr int TN = 32;                // streamed keys (dQ) or rows (dK/dV) per tile
  static constexpr int STR = D + 4;            // LDS row pitch (floats): 16 B pad
  static constexpr int CPR = D / 4;            // 16-byte chunks per row
  static constexpr int CH = TN * CPR;          // chunks per streamed operand tile
  static constexpr int CPT = (CH + NT - 1) / NT;
  static constexpr int LDS_BYTES = 2 * TN * STR * 4 + 2 * TN * 4;
};

// The recomputed probability of one score and the softcap derivative; `dead`
// rows (LSE -inf: no visible key) and masked pairs give 0.
template <bool GENERIC, bool BIAS>
__device__ inline float f32_prob(const BwdParams& p, float s, float lse2, float slope, int64_t qpos,
                                 int key, float bias_v, float& cap_grad) {
  cap_grad = 1.f;
  float x = s * p.scale;
  if (GENERIC) {
    if (p.alibi != nullptr) x = fmaf(-slope, fabsf((float)(qpos - key)), x);
    if (BIAS) x += bias_v;
    if (p.softcap > 0.f) {
      const float th = tanhf(x / p.softcap);
      x = p.softcap * th;
      cap_grad = 1.f - th * th;
    }
  }
  return exp2f(fmaf(x, kLog2e, -lse2));
}

__device__ inline int64_t f32_row_base(const BwdParams& p, int64_t sb, int64_t ss, int64_t sh,
                                       int b, int head, int start) {
  return (p.cu_q != nullptr ? (int64_t)start * ss : (int64_t)b * sb) + (int64_t)head * sh;
}

template <int D, bool GENERIC, bool VARLEN, bool BIAS>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, 1)))
void bwd_f32_dq_kernel(const BwdParams p) {
  static_assert(!BIAS || (GENERIC && !VARLEN), "attn_bias: generic dense kernels only");
  using Tile = F32BwdTile<D>;
  constexpr int BB = Tile::BB, TN = Tile::TN, STR = Tile::STR, NT = Tile::NT;
  constexpr int CPR = Tile::CPR, CH = Tile::CH, CPT = Tile::CPT;
  constexpr int DH = D / 2, NDB = D / 32;
  constexpr int NPASS = D > 128 ? 2 : 1;   // passes over the output dims
  constexpr int NDBP = NDB / NPASS;        // 32-dim output blocks per pass

  extern __shared__ __attribute__((aligned(16))) float smf[];
  float* Ks = smf;
  float* Vs = smf + TN * STR;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int w = tid >> 6;
  const int c32 = lane & 31;
  const int g = lane >> 5;

  int mb, id;
  work_item(blockIdx.x, p.total_blocks, p.n_blocks, p.causal != 0, kCausalSpan, mb, id);
  const int hh = id % p.heads_q;
  const int b = id / p.heads_q;
  const int kvh = hh / p.group;
  int Sq = p.seqlen_q, Sk = p.seqlen_k, qs = 0, ks = 0;
  if (VARLEN) {
    qs = p.cu_q[b];
    ks = p.cu_k[b];
    Sq = p.cu_q[b + 1] - qs;
    Sk = p.cu_k[b + 1] - ks;
  }
  const int row0 = mb * BB;
  if (row0 >= Sq) return;
  const int row_last = min(row0 + BB, Sq) - 1;
  const int qi = row0 + w * 32 + c32;
  const bool row_valid = qi < Sq;
  const int64_t qoff = p.q_offset;
  const int64_t qpos = qi + qoff;
  const bool causal = p.causal != 0;
  const int wl = p.window_left, wr = p.window_right;

  int64_t key_hi = Sk - 1;
  if (causal) key_hi = min(key_hi, qpos);
  if (wr >= 0) key_hi = min(key_hi, qpos + wr);
  const int64_t key_lo = wl >= 0 ? qpos - wl : INT64_MIN / 2;
  int64_t k_hi = Sk;
  if (causal) k_hi = min(k_hi, (int64_t)row_last + qoff + 1);
  if (wr >= 0) k_hi = min(k_hi, (int64_t)row_last + qoff + wr + 1);
  int64_t k_lo = 0;
  if (wl >= 0) k_lo = max((int64_t)0, (int64_t)row0 + qoff - wl);
  const int t_begin = (int)(k_lo / TN);
  const int t_end = k_hi > k_lo ? (int)((k_hi + TN - 1) / TN) : t_begin;

  float slope = 0.f;
  if (GENERIC && p.alibi != nullptr) slope = p.alibi[(int64_t)b * p.alibi_sb + hh];
  const float* bias_row = nullptr;
  float* dbias_row = nullptr;
  if (BIAS && row_valid) {
    if (p.bias != nullptr)
      bias_row = p.bias + (int64_t)b * p.bias_sb + (int64_t)hh * p.bias_sh + (int64_t)qi * p.bias_sq;
    if (p.dbias != nullptr)
      dbias_row = p.dbias + (int64_t)b * p.dbias_sb + (int64_t)hh * p.dbias_sh +
                  (int64_t)qi * p.dbias_sq;
  }

  // Q^T, dO^T of this lane's row (dims [g DH, (g + 1) DH)), delta, LSE.
  float qv[DH], dov[DH];
  float dsum = 0.f;
  {
    const float* qrow = static_cast<const float*>(p.q) +
                        f32_row_base(p, p.q_sb, p.q_ss, p.q_sh, b, hh, qs) + (int64_t)qi * p.q_ss + g * DH;
    const float* drow = static_cast<const float*>(p.dout) +
                        f32_row_base(p, p.do_sb, p.do_ss, p.do_sh, b, hh, qs) + (int64_t)qi * p.do_ss +
                        g * DH;
    const float* orow = static_cast<const float*>(p.o) +
                        f32_row_base(p, p.o_sb, p.o_ss, p.o_sh, b, hh, qs) + (int64_t)qi * p.o_ss + g * DH;
#pragma unroll
    for (int j = 0; j < DH; j += 4) {
      const f32x4 z = {0.f, 0.f, 0.f, 0.f};
      const f32x4 xq = row_valid ? *reinterpret_cast<const f32x4*>(qrow + j) : z;
      const f32x4 xd = row_valid ? *reinterpret_cast<const f32x4*>(drow + j) : z;
      const f32x4 xo = row_valid ? *reinterpret_cast<const f32x4*>(orow + j) : z;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        qv[j + e] = xq[e];
        dov[j + e] = xd[e];
        dsum = fmaf(xd[e], xo[e], dsum);
      }
    }
  }
  const float delta = halves_sum(dsum);
  const int64_t lse_i = f32_row_base(p, p.lse_sb, p.lse_ss, p.lse_sh, b, hh, qs) + (int64_t)qi * p.lse_ss;
  float lse2 = 0.f;
  bool dead = true;
  if (row_valid) {
    const float l = p.lse[lse_i];
    dead = l == -INFINITY;
    lse2 = dead ? 0.f : l * kLog2e;
    if (g == 0) p.delta[lse_i] = delta;
  }

  const float* kg = static_cast<const float*>(p.k) + f32_row_base(p, p.k_sb, p.k_ss, p.k_sh, b, kvh, ks);
  const float* vg = static_cast<const float*>(p.v) + f32_row_base(p, p.v_sb, p.v_ss, p.v_sh, b, kvh, ks);
  float* dqrow = static_cast<float*>(p.dq) + f32_row_base(p, p.dq_sb, p.dq_ss, p.dq_sh, b, hh, qs) +
                 (int64_t)qi * p.dq_ss;

  for (int pass = 0; pass < NPASS; ++pass) {
  f32x16 acc[NDBP];
#pragma unroll
  for (int db = 0; db < NDBP; ++db) acc[db] = f32x16{};

  for (int t = t_begin; t < t_end; ++t) {
    const int n0 = t * TN;
    __syncthreads();   // the previous tile's LDS reads are done
#pragma unroll
    for (int i = 0; i < CPT; ++i) {
      const int c = tid + i * NT;
      if (c < CH) {
        const int n = c / CPR, d = (c % CPR) * 4;
        const int j = n0 + n;
        f32x4 kx = {0.f, 0.f, 0.f, 0.f}, vx = {0.f, 0.f, 0.f, 0.f};
        if (j < Sk) {
          kx = *reinterpret_cast<const f32x4*>(kg + (int64_t)j * p.k_ss + d);
          vx = *reinterpret_cast<const f32x4*>(vg + (int64_t)j * p.v_ss + d);
        }
        *reinterpret_cast<f32x4*>(Ks + n * STR + d) = kx;
        *reinterpret_cast<f32x4*>(Vs + n * STR + d) = vx;
      }
    }
    __syncthreads();

    // S^T = K Q^T and dP^T = V dO^T.
    f32x16 s = f32x16{}, dp = f32x16{};
    const float* krow = Ks + c32 * STR + g * DH;
    const float* vrow = Vs + c32 * STR + g * DH;
#pragma unroll
    for (int j = 0; j < DH; j += 4) {
      const f32x4 kx = *reinterpret_cast<const f32x4*>(krow + j);
      const f32x4 vx = *reinterpret_cast<const f32x4*>(vrow + j);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        s = __builtin_amdgcn_mfma_f32_32x32x2f32(kx[e], qv[j + e], s, 0, 0, 0);
        dp = __builtin_amdgcn_mfma_f32_32x32x2f32(vx[e], dov[j + e], dp, 0, 0, 0);
      }
    }

    float dsv[16];
#pragma unroll
    for (int v = 0; v < 16; ++v) {
      const int key = n0 + 8 * (v >> 2) + 4 * g + (v & 3);
      const bool vis = !dead && key < Sk && key >= key_lo && key <= key_hi;
      const float bv = BIAS && bias_row != nullptr && key < Sk ? bias_row[(int64_t)key * p.bias_sk] : 0.f;
      float cg;
      const float pr = vis ? f32_prob<GENERIC, BIAS>(p, s[v], lse2, slope, qpos, key, bv, cg) : 0.f;
      if (!vis) cg = 0.f;
      float dpv = dp[v];
      if (GENERIC && p.drop.enabled && vis) dpv *= dropout_factor_at(p.drop, qi, key, hh, b);
      const float ds = pr * (dpv - delta) * cg;
      dsv[v] = ds;
      // dS is the same in every pass: the bias gradient takes it once.
      if (BIAS && pass == 0 && dbias_row != nullptr && ds != 0.f)
        atomicAdd(dbias_row + (int64_t)key * p.dbias_sk, ds);
    }

    // dQ^T += K^T dS^T (this pass's output dims).
#pragma unroll
    for (int dbl = 0; dbl < NDBP; ++dbl) {
      const int db = pass * NDBP + dbl;
#pragma unroll
      for (int jj = 0; jj < 16; ++jj) {
        const int key = 8 * (jj >> 2) + 4 * g + (jj & 3);
        acc[dbl] = __builtin_amdgcn_mfma_f32_32x32x2f32(Ks[key * STR + db * 32 + c32], dsv[jj], acc[dbl], 0, 0, 0);
      }
    }
  }

  if (row_valid) {
#pragma unroll
    for (int dbl = 0; dbl < NDBP; ++dbl) {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int d = (pass * NDBP + dbl) * 32 + r * 8 + g * 4;
        *reinterpret_cast<f32x4*>(dqrow + d) =
            f32x4{acc[dbl][4 * r] * p.scale, acc[dbl][4 * r + 1] * p.scale,
                  acc[dbl][4 * r + 2] * p.scale, acc[dbl][4 * r + 3] * p.scale};
      }
    }
  }
  }   // pass
}

template <int D, bool GENERIC, bool VARLEN, bool BIAS>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, 1)))
void bwd_f32_dkdv_kernel(const BwdParams p) {
  static_assert(!BIAS || (GENERIC && !VARLEN), "attn_bias: generic dense kernels only");
  using Tile = F32BwdTile<D>;
  constexpr int BB = Tile::BB, TN = Tile::TN, STR = Tile::STR, NT = Tile::NT;
  constexpr int CPR = Tile::CPR, CH = Tile::CH, CPT = Tile::CPT;
  constexpr int DH = D / 2, NDB = D / 32;
  constexpr int NPASS = D > 128 ? 2 : 1;   // passes over the output dims
  constexpr int NDBP = NDB / NPASS;        // 32-dim output blocks per pass

  extern __shared__ __attribute__((aligned(16))) float smf[];
  float* Qs = smf;
  float* Ds = smf + TN * STR;
  float* Ls = smf + 2 * TN * STR;
  float* Es = Ls + TN;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int w = tid >> 6;
  const int c32 = lane & 31;
  const int g = lane >> 5;

  int nb, id;
  work_item(blockIdx.x, p.total_blocks, p.n_blocks, p.causal != 0, kCausalSpan, nb, id);
  if (p.causal) nb = p.n_blocks - 1 - nb;   // early key blocks (seen by the most rows) first
  const int kvh = id % p.heads_k;
  const int b = id / p.heads_k;
  int Sq = p.seqlen_q, Sk = p.seqlen_k, qs = 0, ks = 0;
  if (VARLEN) {
    qs = p.cu_q[b];
    ks = p.cu_k[b];
    Sq = p.cu_q[b + 1] - qs;
    Sk = p.cu_k[b + 1] - ks;
  }
  const int key0 = nb * BB;
  if (key0 >= Sk) return;
  const int key_last = min(key0 + BB, Sk) - 1;
  const int kj = key0 + w * 32 + c32;
  const bool key_valid = kj < Sk;
  const int64_t qoff = p.q_offset;
  const bool causal = p.causal != 0;
  const int wl = p.window_left, wr = p.window_right;

  // K^T, V^T of this lane's key.  D = 256: only K^T stays in registers; the
  // lane's V row is read again (from L2) in two halves for every query tile
  // (dP = dO V^T is its only use), which keeps K^T, the accumulators of one
  // output half and the tile's S / dP / P / dS within the 512 registers.
  constexpr bool kVres = D <= 128;
  float kv[DH], vv[kVres ? DH : 1];
  const float* vrow = static_cast<const float*>(p.v) +
                      f32_row_base(p, p.v_sb, p.v_ss, p.v_sh, b, kvh, ks) + (int64_t)kj * p.v_ss + g * DH;
  {
    const float* krow = static_cast<const float*>(p.k) +
                        f32_row_base(p, p.k_sb, p.k_ss, p.k_sh, b, kvh, ks) + (int64_t)kj * p.k_ss + g * DH;
#pragma unroll
    for (int j = 0; j < DH; j += 4) {
      const f32x4 z = {0.f, 0.f, 0.f, 0.f};
      const f32x4 xk = key_valid ? *reinterpret_cast<const f32x4*>(krow + j) : z;
#pragma unroll
      for (int e = 0; e < 4; ++e) kv[j + e] = xk[e];
      if constexpr (kVres) {
        const f32x4 xv = key_valid ? *reinterpret_cast<const f32x4*>(vrow + j) : z;
#pragma unroll
        for (int e = 0; e < 4; ++e) vv[j + e] = xv[e];
      }
    }
  }
  const float* bias_col = nullptr;
  if (BIAS && key_valid && p.bias != nullptr)
    bias_col = p.bias + (int64_t)b * p.bias_sb + (int64_t)kj * p.bias_sk;

  // Query rows that see a key of this block: [q_lo, q_hi).
  int64_t q_lo = 0, q_hi = Sq;
  if (causal) q_lo = max(q_lo, (int64_t)key0 - qoff);
  if (wr >= 0) q_lo = max(q_lo, (int64_t)key0 - qoff - wr);
  if (wl >= 0) q_hi = min(q_hi, (int64_t)key_last - qoff + wl + 1);
  const int m_begin = (int)(q_lo / TN);
  const int m_end = q_hi > q_lo ? (int)((q_hi + TN - 1) / TN) : m_begin;

  float* dkrow = static_cast<float*>(p.dk) + f32_row_base(p, p.dk_sb, p.dk_ss, p.dk_sh, b, kvh, ks) +
                 (int64_t)kj * p.dk_ss;
  float* dvrow = static_cast<float*>(p.dv) + f32_row_base(p, p.dv_sb, p.dv_ss, p.dv_sh, b, kvh, ks) +
                 (int64_t)kj * p.dv_ss;

  for (int pass = 0; pass < NPASS; ++pass) {
  f32x16 dk[NDBP], dvacc[NDBP];
#pragma unroll
  for (int db = 0; db < NDBP; ++db) {
    dk[db] = f32x16{};
    dvacc[db] = f32x16{};
  }

  for (int gi = 0; gi < p.group; ++gi) {
    const int hq = kvh * p.group + gi;
    float slope = 0.f;
    if (GENERIC && p.alibi != nullptr) slope = p.alibi[(int64_t)b * p.alibi_sb + hq];
    const float* qg = static_cast<const float*>(p.q) + f32_row_base(p, p.q_sb, p.q_ss, p.q_sh, b, hq, qs);
    const float* dg =
        static_cast<const float*>(p.dout) + f32_row_base(p, p.do_sb, p.do_ss, p.do_sh, b, hq, qs);
    const int64_t lse_base = f32_row_base(p, p.lse_sb, p.lse_ss, p.lse_sh, b, hq, qs);
    for (int mt = m_begin; mt < m_end; ++mt) {
      const int m0 = mt * TN;
      __syncthreads();   // the previous tile's LDS reads are done
#pragma unroll
      for (int i = 0; i < CPT; ++i) {
        const int c = tid + i * NT;
        if (c < CH) {
          const int n = c / CPR, d = (c % CPR) * 4;
          const int row = m0 + n;
          f32x4 qx = {0.f, 0.f, 0.f, 0.f}, dx = {0.f, 0.f, 0.f, 0.f};
          if (row < Sq) {
            qx = *reinterpret_cast<const f32x4*>(qg + (int64_t)row * p.q_ss + d);
            dx = *reinterpret_cast<const f32x4*>(dg + (int64_t)row * p.do_ss + d);
          }
          *reinterpret_cast<f32x4*>(Qs + n * STR + d) = qx;
          *reinterpret_cast<f32x4*>(Ds + n * STR + d) = dx;
        }
      }
      if (tid < 2 * TN) {
        const int n = tid % TN, row = m0 + n;
        // Rows past the sequence read as rows with no visible key.
        float x = tid < TN ? -INFINITY : 0.f;
        if (row < Sq) x = (tid < TN ? p.lse : p.delta)[lse_base + (int64_t)row * p.lse_ss];
        (tid < TN ? Ls : Es)[n] = x;
      }
      __syncthreads();

      // S = Q K^T and dP = dO V^T, one key per lane.
      f32x16 s = f32x16{}, dp = f32x16{};
      const float* qrow = Qs + c32 * STR + g * DH;
      const float* drow = Ds + c32 * STR + g * DH;
      if constexpr (kVres) {
#pragma unroll
        for (int j = 0; j < DH; j += 4) {
          const f32x4 qx = *reinterpret_cast<const f32x4*>(qrow + j);
          const f32x4 dx = *reinterpret_cast<const f32x4*>(drow + j);
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            s = __builtin_amdgcn_mfma_f32_32x32x2f32(qx[e], kv[j + e], s, 0, 0, 0);
            dp = __builtin_amdgcn_mfma_f32_32x32x2f32(dx[e], vv[j + e], dp, 0, 0, 0);
          }
        }
      } else {
#pragma unroll
        for (int j = 0; j < DH; j += 4) {
          const f32x4 qx = *reinterpret_cast<const f32x4*>(qrow + j);
#pragma unroll
          for (int e = 0; e < 4; ++e)
            s = __builtin_amdgcn_mfma_f32_32x32x2f32(qx[e], kv[j + e], s, 0, 0, 0);
        }
        constexpr int VH = DH / 2;
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          float vh[VH];
#pragma unroll
          for (int j = 0; j < VH; j += 4) {
            const f32x4 z = {0.f, 0.f, 0.f, 0.f};
            const f32x4 xv = key_valid ? *reinterpret_cast<const f32x4*>(vrow + h * VH + j) : z;
#pragma unroll
            for (int e = 0; e < 4; ++e) vh[j + e] = xv[e];
          }
#pragma unroll
          for (int j = 0; j < VH; j += 4) {
            const f32x4 dx = *reinterpret_cast<const f32x4*>(drow + h * VH + j);
#pragma unroll
            for (int e = 0; e < 4; ++e)
              dp = __builtin_amdgcn_mfma_f32_32x32x2f32(dx[e], vh[j + e], dp, 0, 0, 0);
          }
        }
      }

      float pv[16], dsv[16];
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int rr = 8 * (v >> 2) + 4 * g + (v & 3);
        const int row = m0 + rr;
        const int64_t qpos = row + qoff;
        const float l = Ls[rr];
        bool vis = key_valid && l != -INFINITY;
        if (causal) vis = vis && kj <= qpos;
        if (wr >= 0) vis = vis && kj <= qpos + wr;
        if (wl >= 0) vis = vis && kj >= qpos - wl;
        const float bv = BIAS && bias_col != nullptr && row < Sq
                             ? bias_col[(int64_t)hq * p.bias_sh + (int64_t)row * p.bias_sq]
                             : 0.f;
        float cg;
        const float pr =
            vis ? f32_prob<GENERIC, BIAS>(p, s[v], l * kLog2e, slope, qpos, kj, bv, cg) : 0.f;
        if (!vis) cg = 0.f;
        float f = 1.f;
        if (GENERIC && p.drop.enabled && vis) f = dropout_factor_at(p.drop, row, kj, hq, b);
        pv[v] = pr * f;
        dsv[v] = pr * (dp[v] * f - Es[rr]) * cg;
      }

      // dV^T += dO^T (F P), dK^T += Q^T dS (this pass's output dims).
#pragma unroll
      for (int dbl = 0; dbl < NDBP; ++dbl) {
        const int db = pass * NDBP + dbl;
#pragma unroll
        for (int jj = 0; jj < 16; ++jj) {
          const int rr = 8 * (jj >> 2) + 4 * g + (jj & 3);
          dvacc[dbl] = __builtin_amdgcn_mfma_f32_32x32x2f32(Ds[rr * STR + db * 32 + c32], pv[jj], dvacc[dbl], 0, 0, 0);
          dk[dbl] = __builtin_amdgcn_mfma_f32_32x32x2f32(Qs[rr * STR + db * 32 + c32], dsv[jj], dk[dbl], 0, 0, 0);
        }
      }
    }
  }

  if (key_valid) {
#pragma unroll
    for (int dbl = 0; dbl < NDBP; ++dbl) {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int d = (pass * NDBP + dbl) * 32 + r * 8 + g * 4;
        *reinterpret_cast<f32x4*>(dkrow + d) =
            f32x4{dk[dbl][4 * r] * p.scale, dk[dbl][4 * r + 1] * p.scale,
                  dk[dbl][4 * r + 2] * p.scale, dk[dbl][4 * r + 3] * p.scale};
        *reinterpret_cast<f32x4*>(dvrow + d) =
            f32x4{dvacc[dbl][4 * r], dvacc[dbl][4 * r + 1], dvacc[dbl][4 * r + 2],
                  dvacc[dbl][4 * r + 3]};
      }
    }
  }
  }   // pass
}

template <int D, bool GEN, bool VARLEN, bool BIAS>
hipError_t launch_bwd_f32_v(BwdParams p, hipStream_t st) {
  using Tile = F32BwdTile<D>;
  {
    auto kern = bwd_f32_dq_kernel<D, GEN, VARLEN, BIAS>;
    p.n_blocks = (p.seqlen_q + Tile::BB - 1) / Tile::BB;
    const int64_t total = (int64_t)p.n_blocks * p.heads_q * p.batch;
    if (total > 0x7fffffff) return hipErrorInvalidConfiguration;
    if (total > 0) {
      p.total_blocks = (int)total;
      hipLaunchKernelGGL(kern, dim3((unsigned)total), dim3(Tile::NT), Tile::LDS_BYTES, st, p);
      if (hipError_t e = hipGetLastError(); e != hipSuccess) return e;
    }
  }
  auto kern = bwd_f32_dkdv_kernel<D, GEN, VARLEN, BIAS>;
  p.n_blocks = (p.seqlen_k + Tile::BB - 1) / Tile::BB;
  const int64_t total = (int64_t)p.n_blocks * p.heads_k * p.batch;
  if (total > 0x7fffffff) return hipErrorInvalidConfiguration;
  if (total <= 0) return hipSuccess;
  p.total_blocks = (int)total;
  hipLaunchKernelGGL(kern, dim3((unsigned)total), dim3(Tile::NT), Tile::LDS_BYTES, st, p);
  return hipGetLastError();
}

template <int D, bool GEN>
hipError_t launch_bwd_f32_d(const BwdParams& p, hipStream_t st) {
  if (p.cu_q != nullptr) return launch_bwd_f32_v<D, GEN, true, false>(p, st);
  if constexpr (GEN) {
    if (p.bias != nullptr || p.dbias != nullptr) return launch_bwd_f32_v<D, true, false, true>(p, st);
  }
  return launch_bwd_f32_v<D, GEN, false, false>(p, st);
}

}  // namespace fa

hipError_t fa_launch_bwd_f32(const fa::BwdParams& p, int head_dim, bool generic, hipStream_t st) {
#define FA_F32B_CASE(DD) \
  case DD: return generic ? fa::launch_bwd_f32_d<DD, true>(p, st) : fa::launch_bwd_f32_d<DD, false>(p, st);
  switch (head_dim) {
    FA_F32B_CASE(32)
    FA_F32B_CASE(64)
    FA_F32B_CASE(128)
    FA_F32B_CASE(256)
    default:
      return hipErrorInvalidValue;
  }
#undef FA_F32B_CASE
}
