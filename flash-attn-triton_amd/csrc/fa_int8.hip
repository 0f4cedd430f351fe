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
// The attention kernel uses the layout of fwd_kernel (fa_fwd_kernel.h):
// S^T = K8 Q8^T on v_mfma_i32_32x32x32_i8 (A = K8 tile from LDS, B = Q8^T in
// VGPRs, quantized once per workgroup), scores scaled in fp32 by
// s_q * s_k[key] * sm_scale * log2(e), online softmax in fp32, and
// O^T += V^T P^T on v_mfma_f32_32x32x16_f16 with P rounded to fp16, as the
// reference keeps PV in FP16 (attention_kernel_int8.py:130-137).  Masked
// scores are -inf with an empty-row guard (the reference adds -1e6,
// :113,119, which matches whenever every row sees a key).
#include "fa_common.h"

namespace fa {

namespace {

__device__ inline float round_half_away(float x) {
#pragma clang fp contract(off)
  return x >= 0.f ? floorf(x + 0.5f) : ceilf(x - 0.5f);
}

__device__ inline uint32_t pack_i8x4(float a, float b, float c, float d) {
  return ((uint32_t)(uint8_t)(int8_t)(int)a) | ((uint32_t)(uint8_t)(int8_t)(int)b << 8) |
         ((uint32_t)(uint8_t)(int8_t)(int)c << 16) | ((uint32_t)(uint8_t)(int8_t)(int)d << 24);
}

}  // namespace

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

struct Int8Params {
  const void* q; const int8_t* k8; const float* s_k; const void* v; void* o; float* lse;
  int64_t q_sb, q_sh, q_ss;
  int64_t v_sb, v_sh, v_ss;
  int64_t o_sb, o_sh, o_ss;
  int batch, heads, seqlen;
  float scale_log2;
  int causal, seq_len_k, seq_len_q;
  int n_mblocks, total_blocks;
};

template <int D, int NW, int BN>
struct Int8Tile {
  static constexpr int BM = NW * 32;
  static constexpr int NT = NW * 64;
  static constexpr int KSTRB = D + 16;   // K8 row pitch in LDS (bytes)
  static constexpr int VSTR = BN + 4;    // V^T row pitch (halfs)
  static constexpr int KTILE_B = BN * KSTRB;
  static constexpr int SK_B = BN * 4;
  static constexpr int VTILE_B = D * VSTR * 2;
  static constexpr int BUF_B = KTILE_B + SK_B + VTILE_B;
  static constexpr int LDS_BYTES = 2 * BUF_B;
};

template <int D, int NW, int BN>
__global__ __launch_bounds__(NW * 64) __attribute__((amdgpu_waves_per_eu(2, 2)))
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
  constexpr int KCH = BN * KCPR;
  constexpr int KPT = (KCH + NT - 1) / NT;
  constexpr int CPR = D / 8;         // 16-byte chunks per V row
  constexpr int VGR = (BN / 4) * CPR;
  constexpr int VPT = (VGR + NT - 1) / NT;
  static_assert(D % 32 == 0 && BN % 32 == 0, "int8 tiles need 32-multiples");

  extern __shared__ __attribute__((aligned(16))) uint8_t smem8[];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int w = tid >> 6;
  const int c32 = lane & 31;
  const int g = lane >> 5;

  int id = xcd_remap(blockIdx.x, p.total_blocks);
  int mb = id % p.n_mblocks;
  const int bh = id / p.n_mblocks;
  if (p.causal) mb = p.n_mblocks - 1 - mb;
  const int h = bh % p.heads;
  const int b = bh / p.heads;
  const int S = p.seqlen;
  const int64_t qoff = (int64_t)p.seq_len_k - p.seq_len_q;
  const int Sk = p.seq_len_k < S ? p.seq_len_k : S;

  const uint16_t* qg = static_cast<const uint16_t*>(p.q) + (int64_t)b * p.q_sb + (int64_t)h * p.q_sh;
  const uint16_t* vg = static_cast<const uint16_t*>(p.v) + (int64_t)b * p.v_sb + (int64_t)h * p.v_sh;
  const int8_t* k8g = p.k8 + (int64_t)bh * S * D;
  const float* skg = p.s_k + (int64_t)bh * S;

  const int row0 = mb * BM;
  const int row_last = min(row0 + BM, S) - 1;
  const int qi = row0 + w * 32 + c32;
  const bool row_valid = qi < S;
  const int64_t qpos = qi + qoff;
  const int wrow0 = row0 + w * 32;
  const bool wave_active = wrow0 <= row_last;
  const int64_t qpos_w_min = wrow0 + qoff;
  const int64_t qpos_w_max = min(wrow0 + 31, row_last) + qoff;
  const bool causal = p.causal != 0;

  int64_t k_hi = Sk;
  if (causal) k_hi = min(k_hi, (int64_t)row_last + qoff + 1);
  const int t_end = k_hi > 0 ? (int)((k_hi + BN - 1) / BN) : 0;

  // ---- quantize this lane's half of its Q row (division form, int8:100)
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
#pragma unroll
    for (int kc = 0; kc < NKC; ++kc) {
#pragma unroll
      for (int wd = 0; wd < 4; ++wd) {
        q8[kc][wd] = (int)pack_i8x4(round_half_away(qf[kc][4 * wd + 0] / s_q),
                                    round_half_away(qf[kc][4 * wd + 1] / s_q),
                                    round_half_away(qf[kc][4 * wd + 2] / s_q),
                                    round_half_away(qf[kc][4 * wd + 3] / s_q));
      }
    }
  }
  const float row_scale = s_q * p.scale_log2;

  u32x4 kreg[KPT];
  float skreg = 0.f;
  u32x4 vreg[VPT][4];
  auto load_tile = [&](int t) {
    const int n0 = t * BN;
#pragma unroll
    for (int i = 0; i < KPT; ++i) {
      const int c = tid + i * NT;
      kreg[i] = u32x4{0, 0, 0, 0};
      if (c < KCH) {
        const int n = c / KCPR, cb = (c % KCPR) * 16;
        if (n0 + n < Sk) kreg[i] = load16(k8g + (int64_t)(n0 + n) * D + cb);
      }
    }
    if (tid < BN) skreg = (n0 + tid < Sk) ? skg[n0 + tid] : 1.0f;
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
          if (j < Sk) vreg[i][u] = load16(vg + (int64_t)j * p.v_ss + d);
        }
      }
    }
  };
  auto store_tile = [&](int buf) {
    uint8_t* base = smem8 + buf * Tile::BUF_B;
    uint8_t* Ks = base;
    float* Sks = reinterpret_cast<float*>(base + Tile::KTILE_B);
    uint16_t* Vt = reinterpret_cast<uint16_t*>(base + Tile::KTILE_B + Tile::SK_B);
#pragma unroll
    for (int i = 0; i < KPT; ++i) {
      const int c = tid + i * NT;
      if (c < KCH) store16(Ks + (c / KCPR) * KSTRB + (c % KCPR) * 16, kreg[i]);
    }
    if (tid < BN) Sks[tid] = skreg;
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

  f32x16 acc[NDB];
#pragma unroll
  for (int db = 0; db < NDB; ++db) acc[db] = f32x16{};
  float m_run = -INFINITY;
  float l_run = 0.f;

  if (t_end > 0) {
    load_tile(0);
    store_tile(0);
  }
  for (int t = 0; t < t_end; ++t) {
    const int buf = t & 1;
    __syncthreads();
    const bool has_next = t + 1 < t_end;
    if (has_next) load_tile(t + 1);
    const int n0 = t * BN;
    const int n1 = n0 + BN;
    bool skip = !wave_active || n0 >= Sk;
    if (causal) skip = skip || n0 > qpos_w_max;
    if (!skip) {
      bool need_mask = n1 > Sk;
      if (causal) need_mask = need_mask || n1 - 1 > qpos_w_min;
      const uint8_t* base = smem8 + buf * Tile::BUF_B;
      const uint8_t* Ks = base;
      const float* Sks = reinterpret_cast<const float*>(base + Tile::KTILE_B);
      const uint16_t* Vt = reinterpret_cast<const uint16_t*>(base + Tile::KTILE_B + Tile::SK_B);

      f32x16 s[NKB];
#pragma unroll
      for (int kb = 0; kb < NKB; ++kb) {
        i32x16 si = i32x16{};
#pragma unroll
        for (int kc = 0; kc < NKC; ++kc) {
          const u32x4 a = load16(Ks + (kb * 32 + c32) * KSTRB + kc * 32 + g * 16);
          si = __builtin_amdgcn_mfma_i32_32x32x32_i8(__builtin_bit_cast(i32x4, a), q8[kc], si, 0, 0, 0);
        }
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const f32x4 sk4 = *reinterpret_cast<const f32x4*>(Sks + kb * 32 + r * 8 + g * 4);
#pragma unroll
          for (int t4 = 0; t4 < 4; ++t4) s[kb][4 * r + t4] = (float)si[4 * r + t4] * sk4[t4];
        }
      }

      float mx = -INFINITY;
#pragma unroll
      for (int kb = 0; kb < NKB; ++kb) {
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          float x = s[kb][v];
          if (need_mask) {
            const int key = n0 + kb * 32 + 8 * (v >> 2) + 4 * g + (v & 3);
            bool ok = key < Sk;
            if (causal) ok = ok && key <= qpos;
            if (!ok) x = -INFINITY;
          }
          s[kb][v] = x;
          mx = fmaxf(mx, x);
        }
      }
      mx = halves_max(mx);
      const float m_tile = mx * row_scale;
      const float m_new = fmaxf(m_run, m_tile);
      const float m_use = m_new == -INFINITY ? 0.f : m_new;
      const float alpha = exp2f(m_run - m_use);
      float rs = 0.f;
#pragma unroll
      for (int kb = 0; kb < NKB; ++kb) {
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          const float e = exp2f(fmaf(s[kb][v], row_scale, -m_use));
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
        pb[0] = F16::pack2(sv[o8 + 0], sv[o8 + 1]);
        pb[1] = F16::pack2(sv[o8 + 2], sv[o8 + 3]);
        pb[2] = F16::pack2(sv[o8 + 4], sv[o8 + 5]);
        pb[3] = F16::pack2(sv[o8 + 6], sv[o8 + 7]);
#pragma unroll
        for (int db = 0; db < NDB; ++db) {
          const uint16_t* vrow = Vt + (db * 32 + c32) * VSTR + cc * 16 + g * 4;
          const u32x2 lo = *reinterpret_cast<const u32x2*>(vrow);
          const u32x2 hi = *reinterpret_cast<const u32x2*>(vrow + 8);
          const u32x4 a = {lo[0], lo[1], hi[0], hi[1]};
          acc[db] = F16::mfma32(a, pb, acc[db]);
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
  const int64_t threads = rows * (D / 8);
  const int64_t blocks = (threads + 255) / 256;
  if (blocks <= 0) return hipSuccess;
  hipLaunchKernelGGL(quant_k_kernel<D>, dim3((unsigned)blocks), dim3(256), 0, st,
                     static_cast<const uint16_t*>(k), k8, s_k, rows, heads, seqlen, ks[0], ks[1],
                     ks[2]);
  return hipGetLastError();
}

template <int D>
hipError_t launch_int8_fwd(Int8Params p, hipStream_t st) {
  constexpr int NW = 4, BN = 64;
  using Tile = Int8Tile<D, NW, BN>;
  auto kern = int8_fwd_kernel<D, NW, BN>;
  static bool lds_attr_set = false;
  if (!lds_attr_set) {
    hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                                       hipFuncAttributeMaxDynamicSharedMemorySize, Tile::LDS_BYTES);
    if (e != hipSuccess) return e;
    lds_attr_set = true;
  }
  p.n_mblocks = (p.seqlen + Tile::BM - 1) / Tile::BM;
  const int64_t total = (int64_t)p.n_mblocks * p.batch * p.heads;
  if (total <= 0) return hipSuccess;
  p.total_blocks = (int)total;
  hipLaunchKernelGGL(kern, dim3((unsigned)total), dim3(Tile::NT), Tile::LDS_BYTES, st, p);
  return hipGetLastError();
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
