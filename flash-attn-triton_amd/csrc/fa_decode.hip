// Attention of a few query rows against a (paged or batched) KV cache: the
// decode path of flash_attn_with_kvcache.
//
// The reference runs a Python loop over the batch that gathers each
// sequence's pages into a contiguous copy and launches a padded O(L^2)
// prefill per sequence (/root/reference/flash_attn_triton/flash_attn_interface.py:494-525).
// Here one launch reads every page in place through the block table and a
// second one merges the per-split results; the semantics (bottom-right causal
// alignment for causal, window, ALiBi, empty rows -> 0 / -inf) are those of
// fwd_kernel's KV-cache mode (fa_fwd_kernel.h).
//
// decode_kernel is bandwidth-bound by design: every K/V byte is read once.
//  * A workgroup owns (batch b, KV head, split of split_keys keys); its four
//    waves stream disjoint 32-key tiles of the split (tile w, w+4, ...) with
//    no barrier inside the loop.
//  * Query rows r = i * G + (h % G) (query i, the G query heads of the KV
//    head) form the B operand Q^T of S^T = K Q^T on v_mfma_f32_32x32x16, so up
//    to 32 rows share every K/V byte.  K and V tiles are loaded row-coalesced
//    into registers and pass through per-wave LDS slots: K comes back in the
//    A-operand layout (ds_read_b128 from a swizzled slot), V as the V^T
//    operand of O^T += V^T P^T through ds_read_b64_tr_b16.
//  * Two K register sets alternate and V's next load starts as soon as the
//    current V tile is in LDS, so every wave keeps about two tiles of loads in
//    flight (the bandwidth a wave sustains is its bytes in flight over memory
//    latency).
//  * Tiles never straddle a page (page_size % 32 == 0): the block table is
//    read once per tile, and the tile's loads are raw buffer loads from a
//    scalar base with 32-bit lane offsets; rows past the sequence end read
//    as zero and are masked.  The kernel must not spill: a scratch reload
//    shares the load counter with the prefetches and would wait for all of
//    them.
//  * The four waves merge their (max, sum, O) through LDS at the end; the
//    workgroup writes the final row (one split) or a partial for
//    decode_combine_kernel.
#include "fa_decode.h"
#include "fa_fwd_launch.h"

namespace fa {

constexpr int kDecodeWaves = 4;
constexpr int kDecodeBN = 32;

template <int D>
struct DecodeTile {
  static constexpr int VSTR = D + 32;                       // V row pitch in LDS (elements)
  static constexpr int VSLOT = kDecodeBN * VSTR;            // one wave's V tile (elements)
  static constexpr int KSLOT = kDecodeBN * D;               // one wave's K tile (elements, swizzled)
  static constexpr int KV_BYTES = kDecodeWaves * (VSLOT + KSLOT) * 2;
  static constexpr int MERGE_BYTES = kDecodeWaves * 32 * (D + 2) * 4;   // O rows + (m, l)
  static constexpr int LDS_BYTES = KV_BYTES > MERGE_BYTES ? KV_BYTES : MERGE_BYTES;
};

template <class T, int D, bool GENERIC>
__global__ __launch_bounds__(kDecodeWaves * 64) __attribute__((amdgpu_waves_per_eu(2, 2)))
void decode_kernel(const DecodeParams p) {
  using Tile = DecodeTile<D>;
  constexpr int BN = kDecodeBN;
  constexpr int NKC = D / 16;
  constexpr int NDB = D / 32;
  constexpr int NCC = BN / 16;
  constexpr int VSTR = Tile::VSTR;
  constexpr int CPR = D / 8;                   // 16-byte chunks per row
  constexpr int VCH = BN * CPR / 64;           // V chunks per lane per tile
  static_assert((BN * CPR) % 64 == 0, "V tile must split evenly over a wave");

  extern __shared__ __attribute__((aligned(16))) uint16_t smem[];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int c32 = lane & 31;
  const int g = lane >> 5;

  // KV heads vary fastest across workgroups: the heads of one (sequence,
  // split) run together and read the same token rows of the cache (each row
  // holds all heads), which keeps DRAM pages open.  The split index varies
  // slowest: every sequence's full leading splits are dispatched first and
  // the short or empty trailing ones last, which trims the tail of the grid
  // (measured 5 % at config 4).
  int id = blockIdx.x;
  const int kvh = id % p.heads_k;
  id /= p.heads_k;
  const int b = id % p.batch;
  const int split = id / p.batch;

  int crow, lpad;
  const int L = decode_keys(p, b, &crow, &lpad);
  const int k_begin = split * p.split_keys;
  // Splits past the cache end hold no keys (the combine skips them).  Split
  // 0 always runs, so that an empty cache still writes its rows (0 and LSE
  // -inf) when there is no combine.
  if (k_begin >= L && split > 0) return;
  const int k_end = min(L, k_begin + p.split_keys);

  const int G = p.group;
  const int Sq = p.seqlen_q;
  const int rows = Sq * G;
  const int r = c32;                           // this lane's query row
  const bool row_valid = r < rows;
  const int qi = row_valid ? r / G : 0;
  const int head = kvh * G + (row_valid ? r % G : 0);
  const int qpos = qi + (p.causal ? L - Sq : 0);
  // Keys of this split only: tiles past the split end (processed with zero
  // data to keep the load order fixed) must not contribute.
  int key_hi = k_end - 1;
  if (p.causal) key_hi = min(key_hi, qpos);
  if (p.window_right >= 0) key_hi = min(key_hi, qpos + p.window_right);
  const int key_lo = p.window_left >= 0 ? qpos - p.window_left : INT32_MIN;
  float slope = 0.f;
  if (GENERIC && p.alibi != nullptr && row_valid) slope = p.alibi[(int64_t)b * p.alibi_sb + head];

  // Q^T in VGPRs (rows past `rows` are zero).
  u32x4 qreg[NKC];
  {
    const uint16_t* qrow = static_cast<const uint16_t*>(p.q) + (int64_t)b * p.q_sb +
                           (int64_t)qi * p.q_ss + (int64_t)head * p.q_sh;
#pragma unroll
    for (int kc = 0; kc < NKC; ++kc)
      qreg[kc] = row_valid ? load16(qrow + kc * 16 + g * 8) : u32x4{0, 0, 0, 0};
  }

  // Element offset of key j's row for this KV head (j < L).  Paged caches
  // hold key j at slot j % page_size of page block_table[b][j / page_size];
  // batched caches at slot leftpad + j of cache row cache_rows[b].
  const int* bt_row = p.block_table != nullptr ? p.block_table + (int64_t)b * p.bt_stride : nullptr;
  int64_t row_k0 = 0, row_v0 = 0;
  if (bt_row == nullptr && L > 0) {
    row_k0 = (int64_t)crow * p.k_sb + (int64_t)lpad * p.k_ss;
    row_v0 = (int64_t)crow * p.v_sb + (int64_t)lpad * p.v_ss;
  }
  row_k0 += (int64_t)kvh * p.k_sh;
  row_v0 += (int64_t)kvh * p.v_sh;
  // Offsets of the first key of the tile starting at n0 (a tile never
  // straddles a page: the host only routes page_size % 32 == 0 here), or -1
  // when the block table names a page outside the cache: that tile reads as
  // zeros (an empty buffer resource) instead of leaving the cache.
  auto tile_k = [&](int n0) -> int64_t {
    if (bt_row == nullptr) return row_k0 + (int64_t)n0 * p.k_ss;
    const int page = bt_row[n0 / p.page_size];
    if (page < 0 || page >= p.cache_blocks) return -1;
    return row_k0 + (int64_t)page * p.k_sb + (int64_t)(n0 % p.page_size) * p.k_ss;
  };
  auto tile_v = [&](int n0) -> int64_t {
    if (bt_row == nullptr) return row_v0 + (int64_t)n0 * p.v_ss;
    const int page = bt_row[n0 / p.page_size];
    if (page < 0 || page >= p.cache_blocks) return -1;
    return row_v0 + (int64_t)page * p.v_sb + (int64_t)(n0 % p.page_size) * p.v_ss;
  };

  const uint16_t* kg = static_cast<const uint16_t*>(p.k);
  const uint16_t* vg = static_cast<const uint16_t*>(p.v);
  uint16_t* vslot = smem + w * Tile::VSLOT;
  uint16_t* kslot = smem + kDecodeWaves * Tile::VSLOT + w * Tile::KSLOT;
  const int vt_lane = (4 * g + (lane & 15) / 4) * VSTR + 16 * (c32 >> 4) + 4 * (lane & 3);
  // K tile in LDS: rows of D halfs without padding, 16-byte chunk c of row r
  // at chunk position c ^ (r % 16) (D = 128) or c ^ (r % 8) (D = 64), so the
  // 16 rows one quarter-wave reads for an MFMA step land on distinct banks.
  constexpr int KSW = CPR >= 16 ? 15 : CPR - 1;
  auto k_lds_ofs = [&](int row, int chunk) { return row * D + ((chunk ^ (row & KSW)) << 3); };

  const int n_tiles = (k_end - k_begin + BN - 1) / BN;
  // Loads of tile tt through raw buffer resources based at the tile's first
  // key row and ending at key L - 1: rows past the sequence end read as zero
  // (they are masked anyway), and every per-lane offset is a 32-bit VGPR
  // (a tile spans 32 rows of at most a page).
  const uint32_t k_row_b = (uint32_t)(p.k_ss * 2);
  const uint32_t v_row_b = (uint32_t)(p.v_ss * 2);
  // K and V tiles are both read row-coalesced: one load instruction covers
  // 64 / CPR whole rows (a row is D * 2 contiguous bytes), which the memory
  // pipeline serves as whole cache lines.  (Loading K straight in the MFMA
  // operand layout touches 32 rows per instruction, 32 bytes each, and
  // measured 11-20 % slower on this access pattern.)
  const uint32_t k_voff = (uint32_t)(lane / CPR) * k_row_b + (uint32_t)(lane % CPR) * 16;
  const uint32_t v_voff = (uint32_t)(lane / CPR) * v_row_b + (uint32_t)(lane % CPR) * 16;
  // A tile past the split's end gets an empty resource: its loads return
  // zeros without touching memory or the block table.  Issuing every load
  // unconditionally keeps the order of outstanding loads the same on every
  // path, so each wait names only the tile it needs.
  auto load_k = [&](int tt, u32x4* kr_) {
    const int n0 = k_begin + tt * BN;
    const int64_t off = n0 < k_end ? tile_k(n0) : -1;
    const bool live = off >= 0;
    const auto rs = make_rsrc(live ? kg + off : kg,
                              live ? rows_extent(0, L - n0, p.k_ss, D) : 0u);
#pragma unroll
    for (int m = 0; m < VCH; ++m)
      kr_[m] = buf_load16_nt(rs, k_voff + (uint32_t)(m * (64 / CPR)) * k_row_b, 0);
  };
  u32x4 vreg[VCH];
  auto load_v = [&](int tt) {
    const int n0 = k_begin + tt * BN;
    const int64_t off = n0 < k_end ? tile_v(n0) : -1;
    const bool live = off >= 0;
    const auto rs = make_rsrc(live ? vg + off : vg,
                              live ? rows_extent(0, L - n0, p.v_ss, D) : 0u);
#pragma unroll
    for (int m = 0; m < VCH; ++m)
      vreg[m] = buf_load16_nt(rs, v_voff + (uint32_t)(m * (64 / CPR)) * v_row_b, 0);
  };

  f32x16 acc[NDB];
#pragma unroll
  for (int db = 0; db < NDB; ++db) acc[db] = f32x16{};
  float m_run = -INFINITY;
  float l_run = 0.f;

  // One tile: the K and V registers (loaded one tile ahead) go to this
  // wave's LDS slots, the next tile's loads are issued into the same
  // registers, and the products run from LDS while those loads are in flight.
  u32x4 kreg[VCH];
  auto process = [&](int tt) {
    const int n0 = k_begin + tt * BN;
    // V tile -> this wave's LDS slot.  LDS executes one wave's instructions in
    // order, so the previous tile's transpose reads finished before these
    // writes; the fences below order the writes against this tile's reads.
#pragma unroll
    for (int m = 0; m < VCH; ++m) {
      const int c = lane + 64 * m;
      store16(vslot + (c / CPR) * VSTR + (c % CPR) * 8, vreg[m]);
      store16(kslot + k_lds_ofs(c / CPR, c % CPR), kreg[m]);
    }
    load_v(tt + kDecodeWaves);
    load_k(tt + kDecodeWaves, kreg);
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");

    // S^T = K Q^T: A = K rows from this wave's LDS slot (lane (c32, g) reads
    // row c32, 16-dim step kc, half g).
    f32x16 s = f32x16{};
#pragma unroll
    for (int kc = 0; kc < NKC; ++kc)
      s = T::mfma32(load16(kslot + k_lds_ofs(c32, 2 * kc + g)), qreg[kc], s);

    // Scores -> log2 units (GENERIC applies ALiBi first); mask keys outside
    // [key_lo, key_hi] (including rows past the sequence end).
    const float sl = GENERIC ? 1.f : p.scale_log2;
    float mx = -INFINITY;
#pragma unroll
    for (int v = 0; v < 16; ++v) {
      const int key = n0 + 8 * (v >> 2) + 4 * g + (v & 3);
      float x = s[v];
      if (GENERIC) {
        x *= p.scale;
        if (p.alibi != nullptr) x = fmaf(-slope, fabsf((float)(qpos - key)), x);
        x *= kLog2e;
      }
      if (key < key_lo || key > key_hi) x = -INFINITY;
      s[v] = x;
      mx = fmaxf(mx, x);
    }
    mx = halves_max(mx) * sl;
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
#pragma unroll
    for (int cc = 0; cc < NCC; ++cc) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const float e0 = __builtin_amdgcn_exp2f(fmaf(s[cc * 8 + 2 * j], sl, -m_use));
        const float e1 = __builtin_amdgcn_exp2f(fmaf(s[cc * 8 + 2 * j + 1], sl, -m_use));
        pb[cc][j] = T::pack2(e0, e1);
        l_run += e0 + e1;
      }
    }
#pragma unroll
    for (int cc = 0; cc < NCC; ++cc) {
#pragma unroll
      for (int db = 0; db < NDB; ++db) {
        const uint16_t* vp = vslot + vt_lane + cc * 16 * VSTR + db * 32;
        const u32x2 lo = lds_read_tr16(vp);
        const u32x2 hi = lds_read_tr16(vp + 8 * VSTR);
        const u32x4 a = {lo[0], lo[1], hi[0], hi[1]};
        acc[db] = T::mfma32(a, pb[cc], acc[db]);
      }
    }
  };

  // Tiles w, w + 4, ... of the split.
  load_k(w, kreg);
  load_v(w);
  for (int tt = w; tt < n_tiles; tt += kDecodeWaves) process(tt);

  // ------------------------------------------------------------ merge waves
  // LDS (after every wave's last V read): per wave w and row r, O^T values
  // and (m, l).  Lane (r, g) holds O^T[d][r] for d = 32 db + 8 (v / 4) + 4 g +
  // v % 4.
  __syncthreads();
  float* mo = reinterpret_cast<float*>(smem);
  float* ml = mo + kDecodeWaves * 32 * D;
  const float l_w = halves_sum(l_run);
  if (row_valid) {   // only the real rows are merged
    float* orow = mo + ((w * 32) + r) * D;
#pragma unroll
    for (int db = 0; db < NDB; ++db) {
#pragma unroll
      for (int q4 = 0; q4 < 4; ++q4)
        *reinterpret_cast<f32x4*>(orow + db * 32 + 8 * q4 + 4 * g) =
            f32x4{acc[db][4 * q4], acc[db][4 * q4 + 1], acc[db][4 * q4 + 2], acc[db][4 * q4 + 3]};
    }
    if (g == 0) {
      ml[(w * 32 + r) * 2] = m_run;
      ml[(w * 32 + r) * 2 + 1] = l_w;
    }
  }
  __syncthreads();
  // Thread t handles row t / 8 and dims 16 (t % 8) .. 16 (t % 8) + 15 (D=128;
  // D / 8 per thread in general).
  constexpr int DPT = D / 8;
  const int rr = tid >> 3;
  if (rr >= rows) return;
  const int d0 = (tid & 7) * DPT;
  float mw[kDecodeWaves], lw[kDecodeWaves];
  float M = -INFINITY;
#pragma unroll
  for (int u = 0; u < kDecodeWaves; ++u) {
    mw[u] = ml[(u * 32 + rr) * 2];
    lw[u] = ml[(u * 32 + rr) * 2 + 1];
    M = fmaxf(M, mw[u]);
  }
  float Ltot = 0.f, wt[kDecodeWaves];
#pragma unroll
  for (int u = 0; u < kDecodeWaves; ++u) {
    wt[u] = lw[u] > 0.f ? __builtin_amdgcn_exp2f(mw[u] - M) : 0.f;
    Ltot += lw[u] * wt[u];
  }
  const float inv = Ltot > 0.f ? 1.f / Ltot : 0.f;
  const float lse_val = Ltot > 0.f ? (M + __log2f(Ltot)) * kLn2 : -INFINITY;
  float o[DPT];
#pragma unroll
  for (int e = 0; e < DPT; ++e) o[e] = 0.f;
#pragma unroll
  for (int u = 0; u < kDecodeWaves; ++u) {
    const float* src = mo + (u * 32 + rr) * D + d0;
#pragma unroll
    for (int e = 0; e < DPT; e += 4) {
      const f32x4 x = *reinterpret_cast<const f32x4*>(src + e);
#pragma unroll
      for (int k = 0; k < 4; ++k) o[e + k] = fmaf(x[k], wt[u], o[e + k]);
    }
  }
  const int oi = rr / G;
  const int oh = kvh * G + rr % G;
  if (p.num_splits == 1) {
    uint16_t* dst = static_cast<uint16_t*>(p.o) + (int64_t)b * p.o_sb + (int64_t)oi * p.o_ss +
                    (int64_t)oh * p.o_sh + d0;
#pragma unroll
    for (int e = 0; e < DPT; e += 8) {
      u32x4 val;
#pragma unroll
      for (int k = 0; k < 4; ++k) val[k] = T::pack2(o[e + 2 * k] * inv, o[e + 2 * k + 1] * inv);
      store16(dst + e, val);
    }
    if (p.lse != nullptr && (tid & 7) == 0)
      p.lse[(int64_t)b * p.lse_sb + (int64_t)oi * p.lse_ss + (int64_t)oh * p.lse_sh] = lse_val;
  } else {
    const int64_t prow = (((int64_t)split * p.batch + b) * Sq + oi) * p.heads_q + oh;
    float* dst = p.o_part + prow * D + d0;
#pragma unroll
    for (int e = 0; e < DPT; e += 4)
      *reinterpret_cast<f32x4*>(dst + e) =
          f32x4{o[e] * inv, o[e + 1] * inv, o[e + 2] * inv, o[e + 3] * inv};
    if ((tid & 7) == 0) p.lse_part[prow] = lse_val;
  }
}

// Merge the splits of each (b, query, head) row: out = sum_s exp(lse_s - lse)
// o_s, lse = log sum_s exp(lse_s), over the splits that hold keys of that
// sequence (ceil(L_b / split_keys); none -> out 0, lse -inf).  One thread per
// row and 4 dims.  The split LSEs and partial rows are fetched in batches of
// kCombineBatch independent loads: a loop of dependent loads would pay one
// memory latency per split.
constexpr int kCombineBatch = 8;
template <class T>
__global__ __launch_bounds__(256) void decode_combine_kernel(const DecodeParams p, int head_dim) {
  const int quads = head_dim / 4;
  const int64_t nrows = (int64_t)p.batch * p.seqlen_q * p.heads_q;
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= nrows * quads) return;
  const int64_t row = idx / quads;
  const int qd = (int)(idx % quads);
  const int h = (int)(row % p.heads_q);
  const int i = (int)((row / p.heads_q) % p.seqlen_q);
  const int b = (int)(row / ((int64_t)p.heads_q * p.seqlen_q));
  const int L = decode_keys(p, b, nullptr, nullptr);
  const int n = min(p.num_splits, (L + p.split_keys - 1) / p.split_keys);
  // Running (max, sum, weighted rows) over batches of splits.
  float m = -INFINITY, tot = 0.f;
  f32x4 acc = {0.f, 0.f, 0.f, 0.f};
  for (int s0 = 0; s0 < n; s0 += kCombineBatch) {
    float ls[kCombineBatch];
    f32x4 o[kCombineBatch];
#pragma unroll
    for (int u = 0; u < kCombineBatch; ++u) {
      const int s = s0 + u;
      ls[u] = s < n ? p.lse_part[(int64_t)s * nrows + row] : -INFINITY;
      o[u] = s < n ? *reinterpret_cast<const f32x4*>(p.o_part + ((int64_t)s * nrows + row) * head_dim + qd * 4)
                   : f32x4{0.f, 0.f, 0.f, 0.f};
    }
    float mb = m;
#pragma unroll
    for (int u = 0; u < kCombineBatch; ++u) mb = fmaxf(mb, ls[u]);
    if (mb == -INFINITY) continue;
    const float rescale = __expf(m - mb);   // m == -inf -> 0
    tot *= rescale;
    acc *= rescale;
#pragma unroll
    for (int u = 0; u < kCombineBatch; ++u) {
      const float wgt = ls[u] == -INFINITY ? 0.f : __expf(ls[u] - mb);
      tot += wgt;
      acc += wgt * o[u];
    }
    m = mb;
  }
  const float inv = tot > 0.f ? 1.f / tot : 0.f;
  uint16_t* orow = static_cast<uint16_t*>(p.o) + (int64_t)b * p.o_sb + (int64_t)i * p.o_ss +
                   (int64_t)h * p.o_sh;
  u32x2 val;
  val[0] = T::pack2(acc[0] * inv, acc[1] * inv);
  val[1] = T::pack2(acc[2] * inv, acc[3] * inv);
  *reinterpret_cast<u32x2*>(orow + qd * 4) = val;
  if (p.lse != nullptr && qd == 0)
    p.lse[(int64_t)b * p.lse_sb + (int64_t)i * p.lse_ss + (int64_t)h * p.lse_sh] =
        tot > 0.f ? m + __logf(tot) : -INFINITY;
}

template <class T, int D, bool GEN>
hipError_t launch_decode_t(const DecodeParams& p, hipStream_t st) {
  using Tile = DecodeTile<D>;
  auto kern = decode_kernel<T, D, GEN>;
  static std::atomic<uint64_t> lds_devices{0};
  if (hipError_t e = set_lds_limit(lds_devices, kern, Tile::LDS_BYTES); e != hipSuccess) return e;
  const int64_t wgs = (int64_t)p.num_splits * p.heads_k * p.batch;
  if (wgs <= 0) return hipSuccess;
  if (wgs > 0x7fffffff) return hipErrorInvalidConfiguration;
  hipLaunchKernelGGL(kern, dim3((unsigned)wgs), dim3(kDecodeWaves * 64), Tile::LDS_BYTES, st, p);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess || p.num_splits == 1) return e;
  const int64_t threads = (int64_t)p.batch * p.seqlen_q * p.heads_q * (D / 4);
  hipLaunchKernelGGL(decode_combine_kernel<T>, dim3((unsigned)((threads + 255) / 256)), dim3(256),
                     0, st, p, D);
  return hipGetLastError();
}

}  // namespace fa

// Decode path eligibility: up to 32 query rows (seqlen_q * group) per KV head,
// head dim 64 or 128, pages that hold whole 32-key tiles.
bool fa_decode_eligible(int64_t rows, int64_t head_dim, int64_t page_size) {
  return rows >= 1 && rows <= 32 && (head_dim == 64 || head_dim == 128) &&
         (page_size == 0 || page_size % fa::kDecodeBN == 0);
}

// Split size: the largest of 2048 / 1024 / 512 / 256 keys that still gives
// every CU several workgroups (batch * heads_k * splits >= 4096); 128 keys
// (one tile per wave) otherwise.
int fa_decode_split_keys(int64_t batch, int64_t heads_k, int64_t max_keys) {
  const int64_t items = batch * heads_k;
  for (int sk = 2048; sk >= 256; sk /= 2)
    if (items * ((max_keys + sk - 1) / sk) >= 4096) return sk;
  return 128;
}

hipError_t fa_launch_decode(int dtype, const fa::DecodeParams& p, int head_dim, bool generic,
                            hipStream_t st) {
#define FA_DEC(TT, DD)                                                              \
  return generic ? fa::launch_decode_t<TT, DD, true>(p, st) : fa::launch_decode_t<TT, DD, false>(p, st);
  if (dtype == 0) {
    if (head_dim == 64) { FA_DEC(fa::F16, 64) }
    if (head_dim == 128) { FA_DEC(fa::F16, 128) }
  } else {
    if (head_dim == 64) { FA_DEC(fa::BF16, 64) }
    if (head_dim == 128) { FA_DEC(fa::BF16, 128) }
  }
#undef FA_DEC
  return hipErrorInvalidValue;
}
