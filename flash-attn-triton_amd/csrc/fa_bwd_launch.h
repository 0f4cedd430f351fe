// Host-side launch helpers for the backward kernels (fa_bwd_kernel.h): tile
// choice per head dim and the grids.  Instantiated once per element type
// (fa_bwd_f16.hip, fa_bwd_bf16.hip).
#pragma once

#include "fa_bwd_kernel.h"
#include "fa_bwd_split.h"

namespace fa {

// dQ: 4 waves x 32 query rows, 64-key tiles (32 from D = 128, where Q, dO and
// the dQ^T accumulators take 128 registers; 256 at D = 256).  dK/dV up to
// D = 128: launch_dkdv_split below.  At D = 256: 4 waves x 32 keys, 32 query
// rows per tile in 3 LDS stages, one wave per SIMD, dV and dK in two passes.
template <int D> struct BwdCfg {
  static constexpr int DQ_NW = 4, DQ_BN = D >= 128 ? 32 : 64, DQ_NS = 3, DQ_WPE = D >= 256 ? 1 : 2;
  static constexpr int KV_NW = 4, KV_BM = D >= 128 ? 32 : 64, KV_NS = 3, KV_WPE = 1;
};

template <class T, int D, bool GEN, int PASS, bool VARLEN, bool BIAS>
hipError_t launch_dkdv(BwdParams p, hipStream_t st) {
  using C = BwdCfg<D>;
  using Tile = BwdDkvTile<T, D, C::KV_NW, C::KV_BM, C::KV_NS>;
  auto kern =
      bwd_dkdv_kernel<T, D, C::KV_NW, C::KV_BM, C::KV_NS, GEN, C::KV_WPE, PASS, VARLEN, BIAS>;
  // The ALiBi slope table (one float per query head of the group) follows the
  // stages; the attribute allows the largest table that still fits.
  constexpr int kMaxLds = 160 * 1024;
  static std::atomic<uint64_t> lds_devices{0};
  hipError_t e = set_lds_limit(lds_devices, kern, kMaxLds);
  if (e != hipSuccess) return e;
  const int64_t lds = Tile::LDS_BYTES + (GEN && p.alibi != nullptr ? 4 * (int64_t)p.group : 0);
  if (lds > kMaxLds) return hipErrorInvalidConfiguration;
  p.n_blocks = (p.seqlen_k + Tile::BN - 1) / Tile::BN;
  const int64_t total = (int64_t)p.n_blocks * p.heads_k * p.batch;
  if (total > 0x7fffffff) return hipErrorInvalidConfiguration;
  if (total <= 0) return hipSuccess;
  p.total_blocks = (int)total;
  hipLaunchKernelGGL(kern, dim3((unsigned)total), dim3(Tile::NT), (unsigned)lds, st, p);
  return hipGetLastError();
}

// dK/dV for D <= 128: a P-wave and a dS-wave per group of 32 keys, 128 keys
// per workgroup, 4 LDS stages.
template <class T, int D, bool GEN, bool VARLEN, bool BIAS>
hipError_t launch_dkdv_split(BwdParams p, hipStream_t st) {
  // 32 query rows per tile from D = 128, and for the generic D = 64 kernels
  // (whose elementwise step needs the registers); 64 below.
  constexpr int BM = D >= 128 || (GEN && D >= 64) ? 32 : 64;
  using Tile = BwdDkvSplitTile<T, D, BM, 4>;
  auto kern = bwd_dkdv_split_kernel<T, D, BM, 4, GEN, VARLEN, BIAS>;
  constexpr int kMaxLds = 160 * 1024;
  static std::atomic<uint64_t> lds_devices{0};
  hipError_t e = set_lds_limit(lds_devices, kern, kMaxLds);
  if (e != hipSuccess) return e;
  const int64_t lds = Tile::LDS_BYTES + (GEN && p.alibi != nullptr ? 4 * (int64_t)p.group : 0);
  if (lds > kMaxLds) return hipErrorInvalidConfiguration;
  p.n_blocks = (p.seqlen_k + Tile::BN - 1) / Tile::BN;
  const int64_t total = (int64_t)p.n_blocks * p.heads_k * p.batch;
  if (total > 0x7fffffff) return hipErrorInvalidConfiguration;
  if (total <= 0) return hipSuccess;
  p.total_blocks = (int)total;
  hipLaunchKernelGGL(kern, dim3((unsigned)total), dim3(Tile::NT), (unsigned)lds, st, p);
  return hipGetLastError();
}

template <class T, int D, bool GEN, bool VARLEN, bool BIAS>
hipError_t launch_bwd_v(BwdParams p, hipStream_t st) {
  using C = BwdCfg<D>;
  {
    using Tile = BwdDqTile<T, D, C::DQ_NW, C::DQ_BN, C::DQ_NS>;
    auto kern = bwd_dq_kernel<T, D, C::DQ_NW, C::DQ_BN, C::DQ_NS, GEN, C::DQ_WPE, VARLEN, BIAS>;
    static std::atomic<uint64_t> lds_devices{0};
    hipError_t e = set_lds_limit(lds_devices, kern, Tile::LDS_BYTES);
    if (e != hipSuccess) return e;
    p.n_blocks = (p.seqlen_q + Tile::BM - 1) / Tile::BM;
    const int64_t total = (int64_t)p.n_blocks * p.heads_q * p.batch;
    if (total > 0x7fffffff) return hipErrorInvalidConfiguration;
    if (total > 0) {
      p.total_blocks = (int)total;
      hipLaunchKernelGGL(kern, dim3((unsigned)total), dim3(Tile::NT), Tile::LDS_BYTES, st, p);
      e = hipGetLastError();
      if (e != hipSuccess) return e;
    }
  }
  if constexpr (D >= 256) {
    hipError_t e = launch_dkdv<T, D, GEN, 1, VARLEN, BIAS>(p, st);
    if (e != hipSuccess) return e;
    return launch_dkdv<T, D, GEN, 2, VARLEN, BIAS>(p, st);
  } else {
    return launch_dkdv_split<T, D, GEN, VARLEN, BIAS>(p, st);
  }
}

// attn_bias (dense only) selects the BIAS instantiations of the generic kernels.
template <class T, int D, bool GEN>
hipError_t launch_bwd_d(const BwdParams& p, hipStream_t st) {
  if (p.cu_q != nullptr) return launch_bwd_v<T, D, GEN, true, false>(p, st);
  if constexpr (GEN) {
    if (p.bias != nullptr || p.dbias != nullptr) return launch_bwd_v<T, D, true, false, true>(p, st);
  }
  return launch_bwd_v<T, D, GEN, false, false>(p, st);
}

template <class T>
hipError_t launch_bwd(const BwdParams& p, int head_dim, bool generic, hipStream_t st) {
#define FA_CASE(DD)                                                              \
  case DD:                                                                       \
    return generic ? launch_bwd_d<T, DD, true>(p, st) : launch_bwd_d<T, DD, false>(p, st);
  switch (head_dim) {
    FA_CASE(32)
    FA_CASE(64)
    FA_CASE(128)
    FA_CASE(256)
    default:
      return hipErrorInvalidValue;
  }
#undef FA_CASE
}

}  // namespace fa
