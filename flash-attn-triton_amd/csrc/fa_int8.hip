// INT8-QK^T attention forward for gfx950.
//
// Follows /root/reference/flash_attn_triton/triton_kernel/attention_kernel_int8.py:
//   _quantize_k_rows (:58-79)  per-token K quantization prepass  -> quant_k_kernel
//   _attn_fwd_int8   (:167-217) + _attn_fwd_int8_inner (:82-141) -> int8_fwd_kernel
//
// Quantization is bit-exact with the definition (IEEE fp32 throughout):
//   s  = fp32(max(amax, 1)) / 127
//   K: x = fp32(k) * (1 / s)      Q: x = fp32(q) / s
//   x8 = x >= 0 ? floor(x + 0.5) : ceil(x - 0.5)
// Floating-point contraction is switched off in these functions: an FMA of
// (k * r + 0.5) would round once instead of twice and change ties.
//
// The attention kernel follows the schedule of prefill_kernel
// (fa_prefill_kernel.h); see int8_fwd_kernel below.
#include "fa_int8_pp.h"
#include "fa_int8_persist.h"

namespace fa {

// One group of D/8 lanes per K row; each lane owns 8 consecutive values.
// Rows enumerate (b, h, s) of a [B, H, S, D] tensor with arbitrary strides;
// k8 is written as [B*H, S, D] contiguous, s_k as [B*H, S].
template <int D>
__global__ __launch_bounds__(256) void quant_k_kernel(const uint16_t* __restrict__ k,
                                                      int8_t* __restrict__ k8,
                                                      float* __restrict__ s_k, int64_t rows,
                                                      int heads, int seqlen, int64_t k_sb,
                                                      int64_t k_sh, int64_t k_ss) {
#pragma clang fp contract(off)
  constexpr int LPR = D / 8;
  const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t row = gid / LPR;
  const int sub = (int)(gid % LPR);
  const bool valid = row < rows;
  float x[8];
  float amax = 0.f;
  if (valid) {
    const int s = (int)(row % seqlen);
    const int64_t bh = row / seqlen;
    const int h = (int)(bh % heads);
    const int64_t b = bh / heads;
    const u32x4 raw = load16(k + b * k_sb + (int64_t)h * k_sh + (int64_t)s * k_ss + sub * 8);
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const uint16_t hbits = (uint16_t)(raw[e >> 1] >> ((e & 1) * 16));
      x[e] = F16::to_float(hbits);
      amax = fmaxf(amax, fabsf(x[e]));
    }
  }
#pragma unroll
  for (int off = 1; off < LPR; off <<= 1) amax = fmaxf(amax, __shfl_xor(amax, off, LPR));
  if (!valid) return;
  const float scale = fmaxf(amax, 1.0f) / 127.0f;
  const float inv = 1.0f / scale;
  float r[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) r[e] = round_half_away(x[e] * inv);
  u32x2 out;
  out[0] = pack_i8x4(r[0], r[1], r[2], r[3]);
  out[1] = pack_i8x4(r[4], r[5], r[6], r[7]);
  *reinterpret_cast<u32x2*>(k8 + row * D + sub * 8) = out;
  if (sub == 0) s_k[row] = scale;
}

// Max over the LPR lanes of a row group (LPR = 4, 8, 16 or 32 consecutive
// lanes) with DPP lane moves within 16-lane rows: quad swaps (xor 1, xor 2),
// then the half-row and row mirrors; 32-lane groups add one exchange across
// rows.
template <int LPR>
__device__ inline float group_max(float v) {
  auto dpp = [](float x, auto ctrl) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), decltype(ctrl)::value,
                                                      0xf, 0xf, false));
  };
  v = fmaxf(v, dpp(v, std::integral_constant<int, 0xB1>{}));   // quad_perm [1,0,3,2]
  v = fmaxf(v, dpp(v, std::integral_constant<int, 0x4E>{}));   // quad_perm [2,3,0,1]
  if constexpr (LPR >= 8) v = fmaxf(v, dpp(v, std::integral_constant<int, 0x141>{}));   // row_half_mirror
  if constexpr (LPR >= 16) v = fmaxf(v, dpp(v, std::integral_constant<int, 0x140>{}));  // row_mirror
  if constexpr (LPR >= 32) v = fmaxf(v, __shfl_xor(v, 16, 32));
  return v;
}

// The prepass for sequence lengths that are a multiple of 64 (every INT8
// launch of the Python API): a workgroup quantizes 64 consecutive rows of one
// (batch, head), whose addressing it computes once in scalar registers.  Four
// lanes share a row, so the per-row work (the max across lanes, the two
// divisions) is spread over D/4 values per lane; lane `sub` owns the 8-value
// chunks sub, sub + 4, ..., so each load instruction reads 64 contiguous bytes
// of a row and each store writes 32.  Every load is issued before any value
// is converted.  Same arithmetic as quant_k_kernel.
template <int D>
__global__ __launch_bounds__(256) void quant_k64_kernel(const uint16_t* __restrict__ k,
                                                        int8_t* __restrict__ k8,
                                                        float* __restrict__ s_k, int heads,
                                                        int seqlen, int64_t k_sb, int64_t k_sh,
                                                        int64_t k_ss) {
#pragma clang fp contract(off)
  constexpr int NC = D / 32;             // 8-value chunks per lane
  const int blocks_per_bh = seqlen >> 6;
  const int bh = blockIdx.x / blocks_per_bh;
  const int s0 = (blockIdx.x - bh * blocks_per_bh) << 6;
  const int h = bh % heads;
  const int b = bh / heads;
  const int t = threadIdx.x;
  const int sub = t & 3;
  const int r = t >> 2;
  const uint16_t* src =
      k + (int64_t)b * k_sb + (int64_t)h * k_sh + (int64_t)(s0 + r) * k_ss + sub * 8;
  u32x4 raw[NC];
#pragma unroll
  for (int i = 0; i < NC; ++i) raw[i] = load16(src + i * 32);
  float x[NC][8];
  float amax = 0.f;
#pragma unroll
  for (int i = 0; i < NC; ++i) {
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      x[i][e] = F16::to_float((uint16_t)(raw[i][e >> 1] >> ((e & 1) * 16)));
      amax = fmaxf(amax, fabsf(x[i][e]));
    }
  }
  amax = group_max<4>(amax);
  const float scale = fmaxf(amax, 1.0f) / 127.0f;
  const float inv = 1.0f / scale;
  const int64_t row = (int64_t)bh * seqlen + s0 + r;
  int8_t* dst = k8 + row * D + sub * 8;
#pragma unroll
  for (int i = 0; i < NC; ++i) {
    int q[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) q[e] = round_half_away_i(x[i][e] * inv);
    u32x2 out;
    out[0] = pack_i8x4_i(q[0], q[1], q[2], q[3]);
    out[1] = pack_i8x4_i(q[4], q[5], q[6], q[7]);
    *reinterpret_cast<u32x2*>(dst + i * 32) = out;
  }
  if (sub == 0) s_k[row] = scale;
}

template <int D, int NW, int BN>
struct Int8Tile {
  static constexpr int BM = NW * 32;
  static constexpr int NT = NW * 64;
  static constexpr int KSTRB = D + 16;   // K8 row pitch in LDS (bytes): 16 B pad
  static constexpr int VSTR = D + 32;    // V row pitch in LDS (elements), as the fp16 kernel
  static constexpr int KTILE_B = BN * KSTRB;
  static constexpr int SK_B = BN * 4;
  static constexpr int VTILE_B = BN * VSTR * 2;
  static constexpr int BUF_B = KTILE_B + SK_B + VTILE_B;
  static constexpr int LDS_BYTES = 2 * BUF_B;
  static constexpr int KCH = BN * D / 16;   // 16-byte K8 chunks per tile
  static constexpr int VCH = BN * D / 8;    // 16-byte V chunks per tile
  static constexpr int KPT = (KCH + NT - 1) / NT;
  static constexpr int VPT = (VCH + NT - 1) / NT;
  static_assert(KCH % NT == 0 || KCH < NT, "K8 tile must split evenly over threads");
  static_assert(VCH % NT == 0 || VCH < NT, "V tile must split evenly over threads");
};

// INT8-QK^T attention forward (the role of _attn_fwd_int8,
// attention_kernel_int8.py:167-217).  Same schedule as prefill_kernel
// (fa_prefill_kernel.h): a workgroup owns BM = 32 NW query rows, S^T = K8 Q8^T
// on v_mfma_i32_32x32x32_i8 (A = K8 rows from LDS, B = Q8^T quantized once per
// row into VGPRs), scores scaled in fp32 by s_q * s_k[key] * sm_scale * log2(e)
// (the reference's order, :106-107), online softmax with the lazy max, and
// O^T += V^T P^T on fp16 MFMA with P rounded to fp16 (the reference keeps PV
// in fp16, :130-137).  K8 / s_k / V tiles are double-buffered in LDS, read
// with raw buffer loads (rows past seq_len_k read as zero and are masked);
// masking (-inf, with an empty-row guard; the reference adds -1e6, :113,119)
// only runs on boundary tiles.
template <int D, int NW, int BN, int WPE>
__global__ __launch_bounds__(NW * 64) __attribute__((amdgpu_waves_per_eu(WPE, WPE)))
void int8_fwd_kernel(const Int8Params p) {
  using Tile = Int8Tile<D, NW, BN>;
  constexpr int BM = Tile::BM;
  constexpr int NT = Tile::NT;
  constexpr int KSTRB = Tile::KSTRB;
  constexpr int VSTR = Tile::VSTR;
  constexpr int NKC = D / 32;        // int8 MFMA k-steps (32 dims each)
  constexpr int NDB = D / 32;
  constexpr int NKB = BN / 32;
  constexpr int NCC = BN / 16;
  constexpr int KCPR = D / 16;       // 16-byte chunks per K8 row
  constexpr int CPR = D / 8;         // 16-byte chunks per V row
  constexpr int KCH = Tile::KCH, VCH = Tile::VCH, KPT = Tile::KPT, VPT = Tile::VPT;

  extern __shared__ __attribute__((aligned(16))) uint8_t smem8[];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int c32 = lane & 31;
  const int g = lane >> 5;

  int mb, bh;
  work_item(blockIdx.x, p.total_blocks, p.n_mblocks, p.causal != 0, kCausalSpan, mb, bh);
  const int h = bh % p.heads;
  const int b = bh / p.heads;
  const int S = p.seqlen;
  const int qoff = p.seq_len_k - p.seq_len_q;
  const int Sk = p.seq_len_k < S ? p.seq_len_k : S;

  const uint16_t* qg = static_cast<const uint16_t*>(p.q) + (int64_t)b * p.q_sb + (int64_t)h * p.q_sh;
  const uint16_t* vg = static_cast<const uint16_t*>(p.v) + (int64_t)b * p.v_sb + (int64_t)h * p.v_sh;
  const int8_t* k8g = p.k8 + (int64_t)bh * S * D;
  const float* skg = p.s_k + (int64_t)bh * S;

  const int row0 = mb * BM;
  const int row_last = min(row0 + BM, S) - 1;
  const int qi = row0 + w * 32 + c32;
  const bool row_valid = qi < S;
  const int qpos = qi + qoff;
  const int wrow0 = row0 + w * 32;
  const bool wave_active = wrow0 <= row_last;
  const int qpos_w_min = wrow0 + qoff;
  const int qpos_w_max = min(wrow0 + 31, row_last) + qoff;
  const bool causal = p.causal != 0;
  int key_hi = Sk - 1;
  if (causal) key_hi = min(key_hi, qpos);

  int k_hi = Sk;
  if (causal) k_hi = min(k_hi, row_last + qoff + 1);
  const int J = k_hi > 0 ? (k_hi + BN - 1) / BN : 0;

  // ---- quantize this lane's half of its Q row (division form, int8:100).
  // Lane (c32, g) holds dims [32kc + 16g, 32kc + 16g + 16) for kc < NKC: the
  // B-operand layout of v_mfma_i32_32x32x32_i8.
  i32x4 q8[NKC];
  float s_q;
  {
#pragma clang fp contract(off)
    float qf[NKC][16];
    float amax = 0.f;
    const uint16_t* qrow = qg + (int64_t)qi * p.q_ss;
#pragma unroll
    for (int kc = 0; kc < NKC; ++kc) {
#pragma unroll
      for (int half = 0; half < 2; ++half) {
        const u32x4 raw = row_valid ? load16(qrow + kc * 32 + g * 16 + half * 8) : u32x4{0, 0, 0, 0};
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const float f = F16::to_float((uint16_t)(raw[e >> 1] >> ((e & 1) * 16)));
          qf[kc][half * 8 + e] = f;
          amax = fmaxf(amax, fabsf(f));
        }
      }
    }
    amax = halves_max(amax);
    s_q = fmaxf(amax, 1.0f) / 127.0f;
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
    __builtin_amdgcn_s_waitcnt(0x0f70);   // vmcnt(0): retire the Q loads before the loop
  }
  const float row_scale = s_q * p.scale_log2;

  // ---- tile loads: raw buffer resources based at the tile's first key row,
  // ending at key Sk - 1 (rows past it read as zero).  All offsets in VGPRs.
  const uint32_t v_row_b = (uint32_t)(p.v_ss * 2);
  uint32_t k_off[KPT], v_off[VPT];
#pragma unroll
  for (int i = 0; i < KPT; ++i) {
    const int c = tid + i * NT;
    k_off[i] = c < KCH ? (uint32_t)(c / KCPR) * D + (uint32_t)(c % KCPR) * 16 : 0xfffffff0u;
  }
#pragma unroll
  for (int i = 0; i < VPT; ++i) {
    const int c = tid + i * NT;
    v_off[i] = c < VCH ? (uint32_t)(c / CPR) * v_row_b + (uint32_t)(c % CPR) * 16 : 0xfffffff0u;
  }
  u32x4 kreg[KPT], vreg[VPT];
  float skreg = 1.f;
  auto load_tile = [&](int t) {
    const int n0 = t * BN;
    const int left = Sk - n0;
    const auto krs = make_rsrc(k8g + (int64_t)n0 * D, left > 0 ? (uint32_t)left * D : 0u);
#pragma unroll
    for (int i = 0; i < KPT; ++i) kreg[i] = buf_load16(krs, k_off[i], 0);
    const auto vrs = make_rsrc(vg + (int64_t)n0 * p.v_ss, rows_extent(n0, Sk, p.v_ss, D));
#pragma unroll
    for (int i = 0; i < VPT; ++i) vreg[i] = buf_load16(vrs, v_off[i], 0);
    if (tid < BN) skreg = (n0 + tid < Sk) ? skg[n0 + tid] : 1.0f;
  };
  auto store_tile = [&](int buf) {
    uint8_t* base = smem8 + buf * Tile::BUF_B;
    float* Sks = reinterpret_cast<float*>(base + Tile::KTILE_B);
    uint16_t* Vs = reinterpret_cast<uint16_t*>(base + Tile::KTILE_B + Tile::SK_B);
#pragma unroll
    for (int i = 0; i < KPT; ++i) {
      const int c = tid + i * NT;
      if (KCH % NT == 0 || c < KCH) store16(base + (c / KCPR) * KSTRB + (c % KCPR) * 16, kreg[i]);
    }
#pragma unroll
    for (int i = 0; i < VPT; ++i) {
      const int c = tid + i * NT;
      if (VCH % NT == 0 || c < VCH) store16(Vs + (c / CPR) * VSTR + (c % CPR) * 8, vreg[i]);
    }
    if (tid < BN) Sks[tid] = skreg;
  };
  const int vt_lane = (4 * g + (lane & 15) / 4) * VSTR + 16 * (c32 >> 4) + 4 * (lane & 3);

  f32x16 acc[NDB];
#pragma unroll
  for (int db = 0; db < NDB; ++db) acc[db] = f32x16{};
  float m_run = -INFINITY;
  float l_run = 0.f;

  if (J > 0) {
    load_tile(0);
    store_tile(0);
  }
  for (int t = 0; t < J; ++t) {
    const int buf = t & 1;
    __syncthreads();
    const bool has_next = t + 1 < J;
    if (has_next) load_tile(t + 1);
    const int n0 = t * BN;
    const int n1 = n0 + BN;
    bool skip = !wave_active || n0 >= Sk;
    if (causal) skip = skip || n0 > qpos_w_max;
    if (!skip) {
      bool need_mask = n1 > Sk;
      if (causal) need_mask = need_mask || n1 - 1 > qpos_w_min;
      const uint8_t* base = smem8 + buf * Tile::BUF_B;
      const float* Sks = reinterpret_cast<const float*>(base + Tile::KTILE_B);
      const uint16_t* Vs = reinterpret_cast<const uint16_t*>(base + Tile::KTILE_B + Tile::SK_B);

      f32x16 s[NKB];
#pragma unroll
      for (int kb = 0; kb < NKB; ++kb) {
        i32x16 si = i32x16{};
#pragma unroll
        for (int kc = 0; kc < NKC; ++kc) {
          const u32x4 a = load16(base + (kb * 32 + c32) * KSTRB + kc * 32 + g * 16);
          si = __builtin_amdgcn_mfma_i32_32x32x32_i8(__builtin_bit_cast(i32x4, a), q8[kc], si, 0, 0, 0);
        }
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const f32x4 sk4 = *reinterpret_cast<const f32x4*>(Sks + kb * 32 + r * 8 + g * 4);
#pragma unroll
          for (int t4 = 0; t4 < 4; ++t4) s[kb][4 * r + t4] = (float)si[4 * r + t4] * sk4[t4];
        }
      }
      if (need_mask) {
#pragma unroll
        for (int kb = 0; kb < NKB; ++kb) {
#pragma unroll
          for (int v = 0; v < 16; ++v) {
            const int key = n0 + kb * 32 + 8 * (v >> 2) + 4 * g + (v & 3);
            if (key > key_hi) s[kb][v] = -INFINITY;
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
      const float mx = halves_max(fmaxf(fmaxf(mq[0], mq[1]), fmaxf(mq[2], mq[3]))) * row_scale;
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
      u32x4 pb[NCC];
      float lq[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int cc = 0; cc < NCC; ++cc) {
        const f32x16& sv = s[cc >> 1];
        const int o8 = (cc & 1) * 8;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const float e0 = __builtin_amdgcn_exp2f(fmaf(sv[o8 + 2 * j], row_scale, -m_use));
          const float e1 = __builtin_amdgcn_exp2f(fmaf(sv[o8 + 2 * j + 1], row_scale, -m_use));
          pb[cc][j] = F16::pack2(e0, e1);
          lq[j] = F16::sum2(pb[cc][j], lq[j]);
        }
      }
      l_run += (lq[0] + lq[1]) + (lq[2] + lq[3]);
#pragma unroll
      for (int cc = 0; cc < NCC; ++cc) {
#pragma unroll
        for (int db = 0; db < NDB; ++db) {
          const uint16_t* vp = Vs + vt_lane + cc * 16 * VSTR + db * 32;
          const u32x2 lo = lds_read_tr16(vp);
          const u32x2 hi = lds_read_tr16(vp + 8 * VSTR);
          const u32x4 a = {lo[0], lo[1], hi[0], hi[1]};
          acc[db] = F16::mfma32(a, pb[cc], acc[db]);
        }
      }
    }
    if (has_next) store_tile(buf ^ 1);
  }

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

template <int D>
hipError_t launch_quant_k(const void* k, int8_t* k8, float* s_k, int batch, int heads, int seqlen,
                          const int64_t* ks, hipStream_t st) {
  const int64_t rows = (int64_t)batch * heads * seqlen;
  if (seqlen % 64 == 0 && rows / 64 <= 0x7fffffff) {
    if (rows == 0) return hipSuccess;
    hipLaunchKernelGGL(quant_k64_kernel<D>, dim3((unsigned)(rows / 64)), dim3(256), 0, st,
                       static_cast<const uint16_t*>(k), k8, s_k, heads, seqlen, ks[0], ks[1],
                       ks[2]);
    return hipGetLastError();
  }
  const int64_t threads = rows * (D / 8);
  const int64_t blocks = (threads + 255) / 256;
  if (blocks <= 0) return hipSuccess;
  hipLaunchKernelGGL(quant_k_kernel<D>, dim3((unsigned)blocks), dim3(256), 0, st,
                     static_cast<const uint16_t*>(k), k8, s_k, rows, heads, seqlen, ks[0], ks[1],
                     ks[2]);
  return hipGetLastError();
}

template <int D, int NW, int BN, int WPE>
hipError_t launch_int8_cfg(Int8Params p, hipStream_t st) {
  using Tile = Int8Tile<D, NW, BN>;
  auto kern = int8_fwd_kernel<D, NW, BN, WPE>;
  static std::atomic<uint64_t> lds_devices{0};
  if (hipError_t e = set_lds_limit(lds_devices, kern, Tile::LDS_BYTES); e != hipSuccess) return e;
  p.n_mblocks = (p.seqlen + Tile::BM - 1) / Tile::BM;
  const int64_t total = (int64_t)p.n_mblocks * p.batch * p.heads;
  if (total <= 0) return hipSuccess;
  if (total > 0x7fffffff) return hipErrorInvalidConfiguration;
  p.total_blocks = (int)total;
  hipLaunchKernelGGL(kern, dim3((unsigned)total), dim3(Tile::NT), Tile::LDS_BYTES, st, p);
  return hipGetLastError();
}

// Ping-pong kernel (fa_int8_pp.h): 8 waves, 256 query rows per workgroup.
template <int D>
hipError_t launch_int8_pp(Int8Params p, hipStream_t st) {
  using Tile = Int8PingPongTile<D>;
  auto kern = int8_pp_kernel<D>;
  static std::atomic<uint64_t> lds_devices{0};
  if (hipError_t e = set_lds_limit(lds_devices, kern, Tile::LDS_BYTES); e != hipSuccess) return e;
  p.n_mblocks = (p.seqlen + Tile::BM - 1) / Tile::BM;
  const int64_t total = (int64_t)p.n_mblocks * p.batch * p.heads;
  if (total <= 0) return hipSuccess;
  if (total > 0x7fffffff) return hipErrorInvalidConfiguration;
  p.total_blocks = (int)total;
  hipLaunchKernelGGL(kern, dim3((unsigned)total), dim3(Tile::NT), Tile::LDS_BYTES, st, p);
  return hipGetLastError();
}

// Persistent INT8 kernel (fa_int8_persist.h) for the large dense launches it
// covers, with the conditions of prefill_persist_kernel's launch: equal
// query and key lengths in full 256-row blocks (causal: an even number of
// them, paired), (batch, head) groups a multiple of the 8 XCDs, and a work
// list that splits evenly over at least 3/4 of the CUs with at least two row
// blocks per workgroup.  *launched is false (nothing launched) otherwise.
template <int D>
hipError_t launch_int8_persist(Int8Params p, hipStream_t st, bool* launched) {
  using Tile = Int8PersistTile<D>;
  *launched = false;
  const bool causal = p.causal != 0;
  const int64_t S = p.seqlen;
  const int64_t G = (int64_t)p.batch * p.heads;
  if (D != 128 || S <= 0 || p.seq_len_k != S || p.seq_len_q != S ||
      S % (causal ? 2 * Tile::BM : Tile::BM) != 0 || G % 8 != 0 || G > (1 << 24))
    return hipSuccess;
  int cus = 0;
  hipError_t e = device_cus(&cus);
  if (e != hipSuccess) return e;
  const int64_t n_mb = S / Tile::BM;
  const int64_t units = G / 8 * (causal ? n_mb / 2 : n_mb);   // per XCD
  const int64_t max_slots = cus / 8;
  int64_t slots = 0;
  for (int64_t d = max_slots; d >= 1; --d)
    if (units % d == 0) {
      slots = d;
      break;
    }
  const int64_t rounds = units / slots * (causal ? 2 : 1);
  if (slots * 4 < max_slots * 3 || rounds < 2 || n_mb > (1 << 20)) return hipSuccess;
  p.n_mblocks = (int)n_mb;
  p.persist_rounds = (int)rounds;
  p.fd_blk = make_fastdiv((uint32_t)(causal ? n_mb / 2 : n_mb));
  p.fd_heads = make_fastdiv((uint32_t)p.heads);
  auto kern = causal ? int8_persist_kernel<D, true> : int8_persist_kernel<D, false>;
  static std::atomic<uint64_t> lds_devices_c{0}, lds_devices_n{0};
  e = set_lds_limit(causal ? lds_devices_c : lds_devices_n, kern, Tile::LDS_BYTES);
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(kern, dim3((unsigned)(8 * slots)), dim3(Tile::NT), Tile::LDS_BYTES, st, p);
  *launched = true;
  return hipGetLastError();
}

// Tile table: D = 128 -> the persistent kernel where it applies, else the
// ping-pong kernel.  Otherwise causal -> 4 waves,
// 32-key tiles (less work past the diagonal), non-causal 8 waves sharing
// 64-key tiles; D = 256: 8 waves, 32-key tiles.
template <int D>
hipError_t launch_int8_fwd(const Int8Params& p, hipStream_t st) {
  if constexpr (D == 128) {
    bool launched = false;
    hipError_t e = launch_int8_persist<D>(p, st, &launched);
    if (e != hipSuccess || launched) return e;
    return launch_int8_pp<D>(p, st);
  } else if constexpr (D == 256) {
    return launch_int8_cfg<D, 8, 32, 2>(p, st);
  } else {
    if (p.causal) return launch_int8_cfg<D, 4, 32, D == 128 ? 3 : 2>(p, st);
    return launch_int8_cfg<D, 8, 64, 2>(p, st);
  }
}

}  // namespace fa

hipError_t fa_launch_quant_k_int8(const void* k, int8_t* k8, float* s_k, int batch, int heads,
                                  int seqlen, int head_dim, const int64_t* k_stride,
                                  hipStream_t st) {
  switch (head_dim) {
    case 32: return fa::launch_quant_k<32>(k, k8, s_k, batch, heads, seqlen, k_stride, st);
    case 64: return fa::launch_quant_k<64>(k, k8, s_k, batch, heads, seqlen, k_stride, st);
    case 128: return fa::launch_quant_k<128>(k, k8, s_k, batch, heads, seqlen, k_stride, st);
    case 256: return fa::launch_quant_k<256>(k, k8, s_k, batch, heads, seqlen, k_stride, st);
    default: return hipErrorInvalidValue;
  }
}

hipError_t fa_launch_int8_fwd(const void* q, const int8_t* k8, const float* s_k, const void* v,
                              void* o, float* lse, int batch, int heads, int seqlen, int head_dim,
                              const int64_t* q_stride, const int64_t* v_stride,
                              const int64_t* o_stride, float sm_scale, int causal, int seq_len_k,
                              int seq_len_q, hipStream_t st) {
  fa::Int8Params p{};
  p.q = q; p.k8 = k8; p.s_k = s_k; p.v = v; p.o = o; p.lse = lse;
  p.q_sb = q_stride[0]; p.q_sh = q_stride[1]; p.q_ss = q_stride[2];
  p.v_sb = v_stride[0]; p.v_sh = v_stride[1]; p.v_ss = v_stride[2];
  p.o_sb = o_stride[0]; p.o_sh = o_stride[1]; p.o_ss = o_stride[2];
  p.batch = batch; p.heads = heads; p.seqlen = seqlen;
  p.scale_log2 = sm_scale * fa::kLog2e;
  p.causal = causal; p.seq_len_k = seq_len_k; p.seq_len_q = seq_len_q;
  switch (head_dim) {
    case 32: return fa::launch_int8_fwd<32>(p, st);
    case 64: return fa::launch_int8_fwd<64>(p, st);
    case 128: return fa::launch_int8_fwd<128>(p, st);
    case 256: return fa::launch_int8_fwd<256>(p, st);
    default: return hipErrorInvalidValue;
  }
}
