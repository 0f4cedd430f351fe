// Host-side launch helpers for fwd_kernel: tile choice per head dim and the
// grid decomposition.  Instantiated once per element type (fa_fwd_f16.hip,
// fa_fwd_bf16.hip) so the two halves compile in parallel.
#pragma once

#include "fa_prefill_kernel.h"
#include "fa_prefill_pp.h"
#include "fa_prefill_persist.h"

namespace fa {

// Tile shape per head dim (prefill): 4 waves x 32 rows; 64-key tiles except
// D=256, where 32-key tiles keep the double-buffered K/V^T tiles and the
// 128-register O accumulator within budget.
template <int D> struct PrefillCfg { static constexpr int NW = 4, BN = D >= 256 ? 32 : 64; };
// KV-cache: one wave owns up to 32 (query, head-in-group) rows; more rows use
// four waves.  32-key tiles keep the single wave's prefetch registers small.
template <int D> struct KvCfg1 { static constexpr int NW = 1, BN = 32; };
template <int D> struct KvCfg4 { static constexpr int NW = 4, BN = D >= 256 ? 32 : 64; };

template <class T, int D, int NW, int BN, int MODE, bool GEN>
hipError_t launch_fwd_cfg(FwdParams p, int rows_for_grid, int outer_blocks, hipStream_t st) {
  using Tile = FwdTile<D, NW, BN>;
  auto kern = fwd_kernel<T, D, NW, BN, MODE, GEN>;
  static std::atomic<uint64_t> lds_devices{0};
  if (hipError_t e = set_lds_limit(lds_devices, kern, Tile::LDS_BYTES); e != hipSuccess) return e;
  p.n_mblocks = (rows_for_grid + Tile::BM - 1) / Tile::BM;
  const int64_t total = (int64_t)p.n_mblocks * outer_blocks;
  if (total <= 0) return hipSuccess;
  if (total > 0x7fffffff) return hipErrorInvalidConfiguration;
  p.total_blocks = (int)total;
  hipLaunchKernelGGL(kern, dim3((unsigned)total), dim3(Tile::NT), Tile::LDS_BYTES, st, p);
  return hipGetLastError();
}

// Prefill tile table (fa_prefill_kernel.h), keyed by head dim and by whether
// the problem is masked (causal, window or varlen):
//   D = 128, masked  : 4 waves, 32-key tiles, 3 waves per SIMD (165 VGPRs);
//                      with the generic epilogue 2 waves, 2 per SIMD, tiles
//                      by LDS-DMA through a 3 K / 2 V stage ring (KS = 3)
//   D = 128, unmasked: 8 waves (256 query rows share each K/V tile), 64-key tiles
//   D = 256          : 8 waves, 32-key tiles (the O^T accumulators take 128 VGPRs)
//   D = 32 / 64      : 4 waves, 64-key tiles
// Measured on MI355X at B4 H32 S4096 D128: the masked choice is ahead on
// causal and varlen (less work past the diagonal / sequence end), the
// unmasked one on non-causal.
template <class T, int D, int NW, int BN, bool GEN, int WPE, bool BIAS = false, int KS = 0>
hipError_t launch_prefill_cfg(FwdParams p, hipStream_t st) {
  using Tile = PrefillTile<D, NW, BN>;
  constexpr int kLds = prefill_lds_bytes<D, NW, BN, KS>();
  auto kern = prefill_kernel<T, D, NW, BN, GEN, WPE, BIAS, KS>;
  static std::atomic<uint64_t> lds_devices{0};
  if (hipError_t e = set_lds_limit(lds_devices, kern, kLds); e != hipSuccess) return e;
  p.n_mblocks = (p.seqlen_q + Tile::BM - 1) / Tile::BM;
  const int64_t total = (int64_t)p.n_mblocks * p.heads_q * p.batch;
  if (total <= 0) return hipSuccess;
  if (total > 0x7fffffff) return hipErrorInvalidConfiguration;
  p.total_blocks = (int)total;
  hipLaunchKernelGGL(kern, dim3((unsigned)total), dim3(Tile::NT), kLds, st, p);
  return hipGetLastError();
}

// Ping-pong prefill (fa_prefill_pp.h): 8 waves, 256 query rows per workgroup.
template <class T, int D, bool VARLEN>
hipError_t launch_prefill_pp(FwdParams p, hipStream_t st) {
  using Tile = PingPongTile<D>;
  auto kern = prefill_pp_kernel<T, D, VARLEN>;
  static std::atomic<uint64_t> lds_devices{0};
  if (hipError_t e = set_lds_limit(lds_devices, kern, Tile::LDS_BYTES); e != hipSuccess) return e;
  p.n_mblocks = (p.seqlen_q + Tile::BM - 1) / Tile::BM;
  const int64_t total = (int64_t)p.n_mblocks * p.heads_q * p.batch;
  if (total <= 0) return hipSuccess;
  if (total > 0x7fffffff) return hipErrorInvalidConfiguration;
  p.total_blocks = (int)total;
  hipLaunchKernelGGL(kern, dim3((unsigned)total), dim3(Tile::NT), Tile::LDS_BYTES, st, p);
  return hipGetLastError();
}

// Persistent ping-pong prefill (fa_prefill_persist.h) when the launch is a
// large dense one it covers: equal query and key lengths with full 256-row
// blocks (causal: an even number of them, paired), no window or offset, the
// (batch, head) groups a multiple of the 8 XCDs, and a work list that splits
// evenly over at least 3/4 of the CUs with at least two row blocks per
// workgroup.  *launched is false (and nothing is launched) otherwise.
template <class T, int D>
hipError_t launch_prefill_persist(FwdParams p, hipStream_t st, bool* launched) {
  using Tile = PingPongTile<D>;
  *launched = false;
  const bool causal = p.causal != 0;
  const int64_t S = p.seqlen_q;
  const int64_t G = (int64_t)p.batch * p.heads_q;
  if (D != 128 || p.cu_q != nullptr || p.block_table != nullptr || S != p.seqlen_k ||
      p.q_offset != 0 || p.window_left >= 0 || p.window_right >= 0 || S <= 0 ||
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
  p.fd_heads = make_fastdiv((uint32_t)p.heads_q);
  p.fd_group = make_fastdiv((uint32_t)p.group);
  auto kern = causal ? prefill_persist_kernel<T, D, true> : prefill_persist_kernel<T, D, false>;
  static std::atomic<uint64_t> lds_devices_c{0}, lds_devices_n{0};
  e = set_lds_limit(causal ? lds_devices_c : lds_devices_n, kern, Tile::LDS_BYTES);
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(kern, dim3((unsigned)(8 * slots)), dim3(Tile::NT), Tile::LDS_BYTES, st, p);
  *launched = true;
  return hipGetLastError();
}

template <class T, int D, bool GEN>
hipError_t launch_prefill(const FwdParams& p, hipStream_t st) {
  if constexpr (GEN) {
    // attn_bias (the materialized-probabilities option): 2 waves per SIMD
    // leave room for the bias loads.
    if (p.bias != nullptr) {
      if constexpr (D == 256) return launch_prefill_cfg<T, D, 8, 32, true, 2, true>(p, st);
      else return launch_prefill_cfg<T, D, 4, (D == 128 ? 32 : 64), true, 2, true>(p, st);
    }
  }
  const bool masked = p.causal || p.window_left >= 0 || p.window_right >= 0 || p.cu_q != nullptr;
  if constexpr (D == 128) {
    // The generic epilogue stays on prefill_kernel: measured at BASELINE
    // config 5 (varlen, causal + window 1024, ALiBi, softcap) the ping-pong
    // kernel is 1.22x slower there (its 256-row blocks visit every key tile
    // of the block's window for all rows, and the softmax phase outgrows the
    // GEMM phase).
    if constexpr (!GEN) {
      if (p.cu_q != nullptr) return launch_prefill_pp<T, D, true>(p, st);
      bool launched = false;
      hipError_t e = launch_prefill_persist<T, D>(p, st, &launched);
      if (e != hipSuccess || launched) return e;
      return launch_prefill_pp<T, D, false>(p, st);
    }
    // The generic epilogue (varlen, ALiBi, softcap, window) does not fit the
    // 168-VGPR budget of 3 waves per SIMD without spilling: 2 waves, in
    // workgroups of 2 (64 rows; measured at BASELINE config 5 with the tiles
    // staged through VGPRs: 4 % faster than 4-wave workgroups, which visit
    // more key tiles per row at a window edge; 3 waves per SIMD spill and
    // were 3.3x slower, 64-key tiles 1.6x).
    // The tiles go global -> LDS by LDS-DMA in a ring of 3 K and 2 V stages
    // (40 KiB: four workgroups per CU).  Measured at BASELINE config 5 on one
    // MI355X: 884 us against 927 us with the tiles staged through VGPRs; the
    // 4-wave form with 5 + 4 stages measured 927 us.
    if (masked) {
      if constexpr (GEN) return launch_prefill_cfg<T, D, 2, 32, GEN, 2, false, 3>(p, st);
      else return launch_prefill_cfg<T, D, 4, 32, GEN, 3>(p, st);
    }
    return launch_prefill_cfg<T, D, 8, 64, GEN, 2>(p, st);
  } else if constexpr (D == 256) {
    return launch_prefill_cfg<T, D, 8, 32, GEN, 2>(p, st);
  } else {
    return launch_prefill_cfg<T, D, 4, 64, GEN, 2>(p, st);
  }
}

template <class T, int D, int MODE, bool GEN>
hipError_t launch_fwd_d(const FwdParams& p, hipStream_t st) {
  if (MODE == kModePrefill) {
    // Paged varlen keys need a page lookup per key: the general kernel.
    if (p.block_table != nullptr) {
      using C = PrefillCfg<D>;
      return launch_fwd_cfg<T, D, C::NW, C::BN, MODE, GEN>(p, p.seqlen_q, p.heads_q * p.batch, st);
    }
    if constexpr (D % 32 == 0) {
      return launch_prefill<T, D, GEN>(p, st);
    } else {
      using C = PrefillCfg<D>;
      return launch_fwd_cfg<T, D, C::NW, C::BN, MODE, GEN>(p, p.seqlen_q, p.heads_q * p.batch, st);
    }
  }
  const int rows = p.seqlen_q * p.group;
  const int outer = p.heads_k * p.batch * p.num_splits;
  if (rows <= 32 && D <= 128) {
    using C = KvCfg1<D>;
    return launch_fwd_cfg<T, D, C::NW, C::BN, MODE, GEN>(p, rows, outer, st);
  }
  using C = KvCfg4<D>;
  return launch_fwd_cfg<T, D, C::NW, C::BN, MODE, GEN>(p, rows, outer, st);
}

template <class T, int MODE>
hipError_t launch_fwd_mode(const FwdParams& p, int head_dim, bool generic, hipStream_t st) {
#define FA_CASE(DD)                                                         \
  case DD:                                                                  \
    return generic ? launch_fwd_d<T, DD, MODE, true>(p, st)                 \
                   : launch_fwd_d<T, DD, MODE, false>(p, st);
  switch (head_dim) {
    FA_CASE(16)
    FA_CASE(32)
    FA_CASE(64)
    FA_CASE(128)
    FA_CASE(256)
    default:
      return hipErrorInvalidValue;
  }
#undef FA_CASE
}

// Key-tile width the KV-cache launch will use (needed to size split-KV work).
inline int kvcache_tile_keys(int rows, int head_dim) {
  if (rows <= 32 && head_dim <= 128) return 32;
  return head_dim >= 256 ? 32 : 64;
}

}  // namespace fa

// Launch entry points shared by the C ABI (fa_api.hip): forward kernels are
// defined per element type in fa_fwd_f16.hip / fa_fwd_bf16.hip, the INT8 path
// in fa_int8.hip and the split-KV merge in fa_api.hip.
hipError_t fa_launch_fwd_f16(const fa::FwdParams& p, int mode, int head_dim, bool generic,
                             hipStream_t st);
hipError_t fa_launch_fwd_bf16(const fa::FwdParams& p, int mode, int head_dim, bool generic,
                              hipStream_t st);
hipError_t fa_launch_fwd_f32(const fa::FwdParams& p, int mode, int head_dim, bool generic,
                             hipStream_t st);
hipError_t fa_launch_combine(int dtype, const float* o_part, const float* lse_part, void* out,
                             float* lse, int num_splits, int batch, int seqlen_q, int heads,
                             int head_dim, const int64_t* o_stride, const int64_t* lse_stride,
                             hipStream_t st);
#include "fa_decode.h"
bool fa_decode_eligible(int64_t rows, int64_t head_dim, int64_t page_size);
int fa_decode_split_keys(int64_t batch, int64_t heads_k, int64_t max_keys);
hipError_t fa_launch_decode(int dtype, const fa::DecodeParams& p, int head_dim, bool generic,
                            hipStream_t st);
hipError_t fa_launch_quant_k_int8(const void* k, int8_t* k8, float* s_k, int batch, int heads,
                                  int seqlen, int head_dim, const int64_t* k_stride,
                                  hipStream_t st);
hipError_t fa_launch_int8_fwd(const void* q, const int8_t* k8, const float* s_k, const void* v,
                              void* o, float* lse, int batch, int heads, int seqlen, int head_dim,
                              const int64_t* q_stride, const int64_t* v_stride,
                              const int64_t* o_stride, float sm_scale, int causal, int seq_len_k,
                              int seq_len_q, hipStream_t st);
