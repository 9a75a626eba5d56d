// Sparse FT backward for gfx950.
//
// Default algorithm (SFT_BWD_SORTED), deterministic and in the reference's
// summation order (FT/kernel.py:108-138, 167-186):
//   1. stable radix sort (ft_sort.hip) of the flat slots s = b*K + k by key
//      (position chunk, feature); inactive slots sort to the end; values are
//      positions b.
//   2. seg_start[f] = first sorted slot with key >= f, for f = 0..N.
//   3. one lane group per feature row: acc = 0, acc += grad[b] over the
//      feature's positions in ascending order, then one store of the row
//      (dW[f] + acc, or acc when overwriting).  No atomics touch dW.  Long
//      segments (features active in many positions) are summed by whole
//      workgroups in the same order.
// Steps 1-2 need only the indices and run on a side stream beside the bias
// pass, which streams the grad (fork/join by events).
// Alternative (SFT_BWD_ATOMIC): position-major scatter, each active slot adds
// the position's grad row into dW[f] with fp32 atomics.
// Bias grad (FT/kernel.py:269): per-block column partial sums, then a fixed-
// order reduction of the partials; deterministic.
#include <algorithm>
#include <mutex>
#include <optional>
#include <type_traits>
#include <utility>
#include <vector>

#include "common.h"

namespace sft {

size_t index_lds_bytes(int G, int K);
size_t slot_sort_workspace(int64_t M);
// Stable sort of the active slots by (position chunk, feature); also zeroes
// clear[0 .. nclear) before it returns (stream-ordered).
int slot_sort(const int32_t *idx, int64_t M, int K, int64_t N, int chunk_rows, int nchunks, void *ws,
              unsigned **keys_sorted, int **pos_sorted, unsigned **digit_totals, int *digit_count, int *clear,
              int nclear, hipStream_t s);
int *slot_sort_positions(int64_t M, int64_t N, int nchunks, void *ws);
// The same sort with the segment pass folded in (a radix pass on the high key
// bits, then one workgroup per bucket), for key spaces it covers.
bool slot_sort_buckets_supported(int64_t N, int nchunks);
int slot_sort_buckets(const int32_t *idx, int64_t M, int K, int64_t N, int chunk_rows, int nchunks, void *ws,
                      int32_t *seg, int32_t *list, int *count, uint16_t *pos16, int long_period, int **pos_sorted,
                      hipStream_t s);
// Its two halves: the radix pass into ws, then the buckets from ws (only read).
int slot_sort_buckets_high(const int32_t *idx, int64_t M, int K, int64_t N, int chunk_rows, int nchunks, void *ws,
                           int *clear, int nclear, hipStream_t s);
int slot_sort_buckets_low(const void *ws, int64_t M, int64_t N, int chunk_rows, int nchunks, int *vout,
                          int32_t *seg, int32_t *list, int *count, uint16_t *pos16, int long_period, hipStream_t s,
                          int bfirst = 0, int bend = -1);
// Buckets that complete position chunk 0 (0: no such split).
int slot_sort_buckets_chunk0(int64_t N, int nchunks);

namespace {

// Row blocks of the bias pass: up to 512 (B = 65536: 128 rows each; 1024 blocks
// of 64 made the pass slower beside the sort, 120 -> 126 us), and at least 64
// rows each (B = 16384: 256 blocks instead of 128, 56 -> 39 us).
#ifndef SFT_BIAS_ROWS
#define SFT_BIAS_ROWS 64
#endif
#ifndef SFT_BIAS_PARTS
#define SFT_BIAS_PARTS 512
#endif
constexpr int kBiasRowsPerBlock = SFT_BIAS_ROWS;
constexpr int kBiasMaxParts = SFT_BIAS_PARTS;

// ------------------------------------------------------- long segments ----
// On real data a few features are active in a large share of the positions
// (a quarter of them and more); one lane group summing such a segment would
// run for the whole launch.  Long segments are summed by whole workgroups
// (long_segment_sum_wg: reserved workgroups of the same gather launch) and
// skipped by the per-feature lane groups.  Whether segment [s0, s1) of the
// sorted slots is long depends on its bounds alone, so both sides agree: it
// is long when it contains two consecutive multiples of kLongSeg ("samples")
// of the sorted slot index.  Every segment of 2 kLongSeg slots or more is
// long, none of kLongSeg slots or fewer.  seg_offsets_kernel lists them (per
// position chunk) as it finds them at their first sample m:
// keys[m + kLongSeg] == keys[m] != keys[m - kLongSeg].
#ifndef SFT_BWD_LONG_SEG
#define SFT_BWD_LONG_SEG 128
#endif
constexpr int kLongSeg = SFT_BWD_LONG_SEG;
__host__ __device__ inline bool long_segment(int64_t s0, int64_t s1) { return sft::long_segment(s0, s1, kLongSeg); }

// Segment starts and the lists of long segments of one sort: seg[0 .. nc N]
// (nc position chunks of nfeat features), then per chunk c a list of its long
// features (list + c nfeat, count[c] entries; listed in no particular order).
// After them, 16-byte aligned: pos16[i] = the i-th sorted slot's position as an
// offset from its position chunk's first position (M entries), the stream the
// tiled gather stages (half the bytes of the positions themselves).
struct SegBufs {
  int32_t *seg, *list;
  int *count;
  uint16_t *pos16;
};
inline size_t seg_ints(int nc, int64_t nfeat) { return (size_t)(2 * nc * nfeat + 1 + nc); }
inline size_t seg_region_bytes(int nc, int64_t nfeat, int64_t M) {
  return (seg_ints(nc, nfeat) * sizeof(int32_t) + 15) / 16 * 16 + (size_t)M * sizeof(uint16_t) + 16;
}
inline SegBufs seg_bufs(void *base, int nc, int64_t nfeat) {
  int32_t *seg = static_cast<int32_t *>(base);
  char *p16 = static_cast<char *>(base) + (seg_ints(nc, nfeat) * sizeof(int32_t) + 15) / 16 * 16;
  return SegBufs{seg, seg + nc * nfeat + 1, seg + 2 * nc * nfeat + 1, reinterpret_cast<uint16_t *>(p16)};
}

// seg_start[k] for k in [0, N]: index of the first sorted key >= k, N = key
// count; with pos16, also each slot's 16-bit chunk offset (SegBufs).  The sorted array holds the active slots only; their number is the
// sum of the sort's last digit totals (read here, on the device, once per
// workgroup by one wave).  Grid-stride over the sorted slots.  Long segments
// are appended to their chunk's list (key = chunk * nfeat + feature; the
// counts start at zero).
__global__ __launch_bounds__(kBlock) void seg_offsets_kernel(const unsigned *__restrict__ keys, int64_t N,
                                                             const unsigned *__restrict__ totals, int ntot,
                                                             int32_t *__restrict__ seg_start, int64_t nfeat,
                                                             int32_t *__restrict__ long_list,
                                                             int *__restrict__ long_count,
                                                             const int32_t *__restrict__ pos,
                                                             uint16_t *__restrict__ pos16, int chunk_rows) {
  __shared__ unsigned s_active;
  if (threadIdx.x < kWave) {
    unsigned v = 0;
    for (int d = threadIdx.x; d < ntot; d += kWave) v += totals[d];
#pragma unroll
    for (int m = 1; m < kWave; m <<= 1) v += __shfl_xor(v, m);
    if (threadIdx.x == 0) s_active = v;
  }
  __syncthreads();
  const int64_t M = s_active;
  for (int64_t i = (int64_t)blockIdx.x * kBlock + threadIdx.x; i <= M; i += (int64_t)gridDim.x * kBlock) {
    const int64_t cur = i < M ? (int64_t)keys[i] : N + 1;
    const int64_t prev = i > 0 ? (int64_t)keys[i - 1] : -1;
    if (pos16 != nullptr && i < M) pos16[i] = (uint16_t)(pos[i] - (int)(cur / nfeat) * chunk_rows);
    const int64_t hi = cur < N ? cur : N;
    for (int64_t f = prev + 1; f <= hi; ++f) seg_start[f] = (int32_t)i;
    if (long_listed_at(keys, M, i, kLongSeg)) {
      const int64_t c = cur / nfeat;
      const int at = atomicAdd(long_count + c, 1);
      long_list[c * nfeat + at] = (int32_t)(cur - c * nfeat);
    }
  }
}

constexpr int kSegBlocks = 2048;

template <int G>
__device__ __forceinline__ void group_minmax(int v, int &vmin, int &vmax) {
  vmin = v;
  vmax = v;
#pragma unroll
  for (int off = G; off < kWave; off <<= 1) {
    vmin = min(vmin, __shfl_xor(vmin, off));
    vmax = max(vmax, __shfl_xor(vmax, off));
  }
  vmin = uniform(vmin);
  vmax = uniform(vmax);
}

// Where a launch starts and leaves each feature's sum:
//   src_mode kSrcZero: acc = 0;  kSrcTmp: acc = tmp row
//   dst_mode kDstOut: dst row = acc;  kDstTmp: tmp row = acc;
//            kDstOutPlus: dst row = dst row + acc.
// One perspective: (zero, tmp), (tmp, tmp) ..., (tmp, out) over its position
// chunks; (zero, out) with one chunk.  A second perspective ends with
// kDstOutPlus instead: dW = dW_0 + dW_1, the sum autograd forms for the
// composed table (FEAT/composed.py:52-53).  dst rows are split into blocks
// (RowDst).
enum { kSrcZero = 0, kSrcTmp = 2 };
enum { kDstOut = 0, kDstTmp = 1, kDstOutPlus = 2 };

// The sums carried from one position chunk to the next are kept tile-major:
// the 8 chunks (32 columns) of tile t for feature f at tmp + tmp_row(t, f, N),
// so a row is one aligned 128-byte line and a workgroup's 32 features are 4 KB
// of consecutive lines.  (A row-major [N, L] row puts tile t at byte 4L f + 128 t,
// which for L % 32 != 0 straddles two lines three times in four -- lines that
// the neighbouring tiles, gathered on other XCDs, also touch.)
__host__ __device__ inline int64_t tmp_row(int tile, int64_t f, int64_t nfeat) {
  return ((int64_t)tile * nfeat + f) * 8;
}

// Rows of column block cb for position p: 8 chunks at base + cb * blk_stride
// + p * pos_stride (grad tiles: blk_stride = B * 8, pos_stride = 8; row-major
// grad: blk_stride = 8, pos_stride = cols4); chunk q of block cb is column
// chunk tile_col(map, cb, q) of dW.
struct LongRows {
  const f32x4 *base;
  int64_t blk_stride, pos_stride;
};

// Where a long segment's sum for block cb starts and goes (lanes 0-31 of the
// calling wave; lane l owns float l of the block row); ccol < 0: no column.
struct LongEnds {
  float *dp, *tp;
  int ccol;
};
__device__ __forceinline__ LongEnds long_ends(int64_t f, int cb, int lane, const ColMap &map, const RowDst &dst,
                                              f32x4 *tmp, int64_t nfeat) {
  LongEnds e{nullptr, nullptr, lane < 32 ? tile_col(map, cb, lane >> 2) : -1};
  if (e.ccol >= 0) {
    const int blk = block_of(f, dst.n, dst.start);
    e.dp = reinterpret_cast<float *>(pick(dst.p, blk) + (f - pick(dst.start, blk)) * map.cols4 + e.ccol) + (lane & 3);
    if (tmp != nullptr) e.tp = reinterpret_cast<float *>(tmp + tmp_row(cb, f, nfeat) + (lane >> 2)) + (lane & 3);
  }
  return e;
}
__device__ __forceinline__ float long_start(const LongEnds &e, int src_mode) {
  if (e.ccol < 0) return 0.f;
  if (src_mode == kSrcTmp) return *e.tp;
  return 0.f;
}
__device__ __forceinline__ void long_store(const LongEnds &e, int dst_mode, float acc) {
  if (e.ccol < 0) return;
  if (dst_mode == kDstTmp) *e.tp = acc;
  else if (dst_mode == kDstOutPlus) *e.dp = *e.dp + acc;
  else *e.dp = acc;
}

// A long segment (see long_segment) summed for one column block by a whole
// workgroup: its 256 threads stage kWgLongRows rows at a time into LDS (the
// next batch's loads in flight meanwhile) and lanes 0-31 of wave 0 add them in
// order: acc = start value, acc += row for the positions ascending -- the
// gather's own sequence, so a feature's result does not depend on the path.
// Threads kBlock and above of a larger workgroup take part in the barriers only.
constexpr int kWgLongRows = 128;  // 128 x 128 B = 16 KB of LDS
__device__ __forceinline__ void long_segment_sum_wg(const int32_t *__restrict__ sorted_pos, int64_t f, int s0, int n,
                                                    int cb, const LongRows &rows, const ColMap &map,
                                                    const RowDst &dst, f32x4 *__restrict__ tmp, int64_t nfeat,
                                                    int src_mode, int dst_mode, f32x4 *buf) {
  constexpr int kRowsPerPass = kBlock / 8;
  constexpr int kPass = kWgLongRows / kRowsPerPass;
  const bool stager = threadIdx.x < kBlock;
  const LongEnds ends = long_ends(f, cb, (int)threadIdx.x, map, dst, tmp, nfeat);
  float acc = long_start(ends, src_mode);
  const int q = threadIdx.x & 7, r0 = threadIdx.x >> 3;  // staging: chunk q of rows r0 + 32 u
  const bool qok = tile_col(map, cb, q) >= 0;
  const f32x4 *src = rows.base + cb * rows.blk_stride + q;
  const int nb = (n + kWgLongRows - 1) / kWgLongRows;
  int p[kPass];
  f32x4 v[kPass];
  auto load_pos = [&](int b) {
#pragma unroll
    for (int u = 0; u < kPass; ++u) {
      const int r = b * kWgLongRows + r0 + kRowsPerPass * u;
      p[u] = (stager && r < n) ? sorted_pos[s0 + r] : -1;
    }
  };
  auto load_rows = [&]() {
#pragma unroll
    for (int u = 0; u < kPass; ++u)
      v[u] = (p[u] >= 0 && qok) ? src[(int64_t)p[u] * rows.pos_stride] : f32x4{0.f, 0.f, 0.f, 0.f};
  };
  auto stage = [&]() {
    if (!stager) return;
#pragma unroll
    for (int u = 0; u < kPass; ++u) buf[(r0 + kRowsPerPass * u) * 8 + q] = v[u];
  };
  load_pos(0);
  load_rows();
  if (nb > 1) load_pos(1);
  stage();
  __syncthreads();
  for (int b = 0; b < nb; ++b) {  // nb is workgroup-uniform
    const bool more = b + 1 < nb;
    if (more) {
      load_rows();
      if (b + 2 < nb) load_pos(b + 2);
    }
    if (ends.ccol >= 0) {
      const float *row = reinterpret_cast<const float *>(buf) + threadIdx.x;
      const int nrows = min(kWgLongRows, n - b * kWgLongRows);
#pragma unroll 16
      for (int r = 0; r < nrows; ++r) acc += row[r * 32];
    }
    __syncthreads();
    if (more) stage();
    __syncthreads();
  }
  long_store(ends, dst_mode, acc);
}

// Row gather: the first nlong workgroups (column slab 0) sum the listed long
// segments in 32-column blocks (items e * nblk + cb dealt round-robin; the
// float4 instantiation only); the others are feature blocks.
template <typename T, int G, int CPL, int U>
__global__ __launch_bounds__(kBlock) void gather_rows_kernel(const int32_t *__restrict__ seg_start,
                                                             const int32_t *__restrict__ sorted_pos, int64_t N,
                                                             const T *__restrict__ grad, int64_t cols,
                                                             T *__restrict__ dW, int overwrite,
                                                             const int32_t *__restrict__ long_list,
                                                             const int *__restrict__ long_count, int nlong) {
  if ((int)blockIdx.x < nlong) {  // whole block: uniform
    if constexpr (std::is_same<T, f32x4>::value) {
      __shared__ f32x4 lbuf[kWgLongRows * 8];
      if (blockIdx.y != 0) return;
      const ColMap map = plain_map((int)cols, 8);
      const int nblk = map_tiles(map);
      RowDst dst{};
      dst.n = 1;
      dst.start[1] = N;
      dst.p[0] = dW;
      const int64_t items = (int64_t)*long_count * nblk;
      for (int64_t k = blockIdx.x; k < items; k += nlong) {
        const int64_t f = long_list[k / nblk];
        const int s0 = seg_start[f];
        long_segment_sum_wg(sorted_pos, f, s0, seg_start[f + 1] - s0, (int)(k % nblk), LongRows{grad, 8, cols}, map,
                            dst, nullptr, N, kSrcZero, overwrite ? kDstOut : kDstOutPlus, lbuf);
      }
    }
    return;
  }
  const bool skip_long = nlong > 0;
  constexpr int PPW = kWave / G;
  const int wave = uniform(threadIdx.x / kWave);
  const int lane = threadIdx.x % kWave;
  const int g = lane / G, t = lane % G;
  const int64_t f = ((int64_t)(blockIdx.x - nlong) * kWavesPerBlock + wave) * PPW + g;
  const bool live = f < N;
  int s0 = 0, s1 = 0;
  if (live) {
    s0 = seg_start[f];
    s1 = seg_start[f + 1];
  }
  if (G == kWave) {
    s0 = uniform(s0);
    s1 = uniform(s1);
  }
  const bool is_long = skip_long && live && long_segment(s0, s1);  // summed by the long-segment blocks
  const int n = is_long ? 0 : s1 - s0;
  int nmin, nmax;
  group_minmax<G>(n, nmin, nmax);

  const int64_t c0 = (int64_t)blockIdx.y * (G * CPL) + t;
  bool colok[CPL];
  T acc[CPL];
#pragma unroll
  for (int j = 0; j < CPL; ++j) {
    colok[j] = (c0 + G * j) < cols;
    acc[j] = T(0);
  }
  const int32_t *plist = sorted_pos + s0;

  int k = 0;
  for (; k + U <= nmin; k += U) {
    T w[U][CPL];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      int b = plist[k + u];
      if (G == kWave) b = uniform(b);
      const T *row = grad + (int64_t)b * cols + c0;
#pragma unroll
      for (int j = 0; j < CPL; ++j)
        if (colok[j]) w[u][j] = row[G * j];
    }
#pragma unroll
    for (int u = 0; u < U; ++u)
#pragma unroll
      for (int j = 0; j < CPL; ++j)
        if (colok[j]) acc[j] += w[u][j];
  }
  for (; k < nmax; k += U) {
    T w[U][CPL];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const bool v = k + u < n;
      int b = v ? plist[k + u] : 0;
      if (G == kWave) b = uniform(b);
      const T *row = grad + (int64_t)b * cols + c0;
#pragma unroll
      for (int j = 0; j < CPL; ++j) {
        w[u][j] = T(0);
        if (v && colok[j]) w[u][j] = row[G * j];
      }
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const bool v = k + u < n;
#pragma unroll
      for (int j = 0; j < CPL; ++j)
        if (v && colok[j]) acc[j] += w[u][j];
    }
  }

  if (live && !is_long && (n > 0 || overwrite)) {
    T *d = dW + f * cols + c0;
#pragma unroll
    for (int j = 0; j < CPL; ++j) {
      if (!colok[j]) continue;
      if (overwrite)
        __builtin_nontemporal_store(acc[j], d + G * j);
      else
        d[G * j] = d[G * j] + acc[j];
    }
  }
}

// ---------------------------------------------------- tiled feature gather ----
// dW[f, tile] for one 32-column tile, from the grad re-laid out as column
// tiles (Gt: tile t holds columns [32t, 32t + 32) of every position, 128 B per
// position).  The slots are sorted by (position half, feature), and the batch
// is done in two launches: half 0 stores its sum for (f, tile) to a tile-major
// buffer (tmp_row), half 1 loads that value and keeps adding.  Either way a feature's sum is acc = 0,
// acc += grad[b] over its positions ascending: the reference order
// (FT/kernel.py:122, 178-181), bit for bit.  A lane group of 8 lanes x 16 B
// owns one feature's tile row; tiles go to XCDs whole (tile_sched_item), so an
// XCD reads one tile-half of Gt at a time: 32768 x 128 B = 4 MB, its L2.
// The summed tile rows are written once per launch and read back, if at all,
// by the next launch.  When a tile-half of the grad tiles takes half of an
// XCD's L2 or more, non-temporal stores keep them from evicting it (220 -> 215
// us per launch at B = 65536); with smaller batches the grad tile fits anyway
// and the read-back is cheaper from the cache (B = 16384: 90 vs 99 us), so the
// host picks per launch (kNtStoreTileBytes; a template parameter, as the
// compiler merges a runtime choice between the two stores into a plain one).
// The carried sums are read back with the same policy (207.3 -> 204.8 us).
constexpr int64_t kNtStoreTileBytes = 2 << 20;
template <bool NT>
__device__ __forceinline__ void store_row(f32x4 *p, f32x4 v) {
  if constexpr (NT) __builtin_nontemporal_store(v, p);
  else *p = v;
}
template <bool NT>
__device__ __forceinline__ f32x4 load_row(const f32x4 *p) {
  if constexpr (NT) return __builtin_nontemporal_load(p);
  else return *p;
}
constexpr int kBwdTileCh = 8;  // float4 chunks per 32-column tile row (grad tiles and weight-grad blocks)
static_assert(kBwdTileCh == 8, "tmp_row and the long-segment lanes hold 8 chunks per tile");
// Features per workgroup of the tiled gather: one per 8-lane group.
constexpr int bwd_feat_per_block() { return kWavesPerBlock * (kWave / kBwdTileCh); }
// Long segments are summed in 32-column blocks by the tiled gather's
// long-segment slots.
#ifndef SFT_BWD_LONG_SLOTS
#define SFT_BWD_LONG_SLOTS 128
#endif
constexpr int kLongSlots = SFT_BWD_LONG_SLOTS;  // long-segment workgroups per tile
#ifndef SFT_BWD_ROW_LONG_BLOCKS
#define SFT_BWD_ROW_LONG_BLOCKS 1024
#endif
constexpr int kRowLongBlocks = SFT_BWD_ROW_LONG_BLOCKS;  // long-segment workgroups of the row gather

#ifndef SFT_BWD_POS_LDS
#define SFT_BWD_POS_LDS 4096
#endif
constexpr int kBwdPosLds = SFT_BWD_POS_LDS;  // staged positions per workgroup

#ifndef SFT_BWD_ROLL
#define SFT_BWD_ROLL 1
#endif
// Sums one lane group's positions from `list` (LDS or global) into acc.  A
// lane group has TCH lanes (one 16-byte chunk of the tile row each) and keeps
// TCH row loads in flight.  Rows are 32-bit byte offsets from the grad tile's
// wave-uniform base (a tile is B x 16 TCH bytes, B < 2^31 / K).  Every lane
// loads, padding lanes of the last tile included (a tile holds all TCH chunks
// of each row; the caller does not store a padding lane's sum), so the loads
// carry no execution masks.
//
// The sum starts from *from when `use` (the sum an earlier position chunk
// left), else from acc.  *from is loaded by every lane with the first rows,
// in the same block of code (from must point at readable memory whatever
// `use` is): a load whose value merges from a branch is waited for at the
// merge, before the row loads are issued.
template <bool FROM_LDS, int TCH, bool NT, typename P>
__device__ __forceinline__ void bwd_tile_sum(const P *list, int n, int nmin, int nmax, int t,
                                             const char *__restrict__ gtile, f32x4 &acc, const f32x4 *from,
                                             bool use) {
  const uint32_t lane_off = (uint32_t)t * (uint32_t)sizeof(f32x4);
  auto row = [&](int b) {
    return *reinterpret_cast<const f32x4 *>(gtile + ((uint32_t)b * (uint32_t)(TCH * sizeof(f32x4)) + lane_off));
  };
  constexpr int U = TCH;  // one position per lane of the group when read from global memory
  int k = 0;
  if (SFT_BWD_ROLL && FROM_LDS && nmin >= 2 * U) {
    // A rolling window of U rows in flight over the rows every lane group of
    // the wave has: each add frees the oldest row's registers, which take the
    // row U places further at once, so the loads in flight do not drain to
    // zero between steps.  Same adds, same order.  (Workload 1: 206.5 ->
    // 204.2 us per launch, step 1.719 -> 1.712 ms; L = 136 and Full_Threats
    // 0.5-1% per step.)
    f32x4 w[U];
    // Issued in the order the loop consumes them (no reordering across the
    // barriers), so the loads in flight at the loop head are in the same
    // order on both of its edges and each add waits for its own row only.
    // (an opaque zero offset keeps this load here: the same load in both
    // branches would be hoisted above them and waited for there)
    int z = 0;
    asm volatile("" : "+v"(z));
    const f32x4 c = load_row<NT>(from + z);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int u = 0; u < U; ++u) {
      w[u] = row((int)list[u]);
      __builtin_amdgcn_sched_barrier(0);
    }
    acc = use ? c : acc;
    for (k = U; k + U <= nmin; k += U) {
      int b[U];
#pragma unroll
      for (int u = 0; u < U; ++u) b[u] = (int)list[k + u];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        acc += w[u];
        w[u] = row(b[u]);
      }
    }
#pragma unroll
    for (int u = 0; u < U; ++u) acc += w[u];
  } else {
    const f32x4 c = load_row<NT>(from);
    acc = use ? c : acc;
  }
  for (; k + U <= nmin; k += U) {
    int b[U];
    if (FROM_LDS) {
#pragma unroll
      for (int u = 0; u < U; ++u) b[u] = (int)list[k + u];
    } else {
      const int mine = (int)list[k + t];
#pragma unroll
      for (int u = 0; u < U; ++u) b[u] = __shfl(mine, u, TCH);
    }
    f32x4 w[U];
#pragma unroll
    for (int u = 0; u < U; ++u) w[u] = row(b[u]);
#pragma unroll
    for (int u = 0; u < U; ++u) acc += w[u];
  }
  for (; k < nmax; k += U) {
    int b[U];
    if (FROM_LDS) {
#pragma unroll
      for (int u = 0; u < U; ++u) b[u] = (k + u < n) ? (int)list[k + u] : 0;
    } else {
      const int mine = (k + t < n) ? (int)list[k + t] : 0;
#pragma unroll
      for (int u = 0; u < U; ++u) b[u] = __shfl(mine, u, TCH);
    }
    f32x4 w[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      w[u] = f32x4{0.f, 0.f, 0.f, 0.f};
      if (k + u < n) w[u] = row(b[u]);
    }
#pragma unroll
    for (int u = 0; u < U; ++u)
      if (k + u < n) acc += w[u];
  }
}

// The 32 features of a workgroup are consecutive, so their position lists
// form one contiguous range of the sorted array; it is copied to LDS and read
// from there, which keeps the position reads off the in-order vector-memory
// counter the row loads wait on.  Ranges longer than kBwdPosLds entries read
// their positions from global memory instead.
//
// In front of the gather a workgroup makes two rounds of global loads, each
// issued whole before anything waits on it: (1) the segment bounds; (2) the
// positions (8 loads per thread in flight) together with, for kDstOutPlus, the
// rows the sums add onto -- thread i loads chunk i % 8 of feature i / 8 into
// LDS.  Meanwhile wave 0 ranks the 32 features by segment length with
// cross-lane reads.  One barrier, then each lane group sums one feature,
// starting from the sum the previous position chunk left, which the lane
// loads itself beside its first row loads.  (Staging one position per thread
// per round trip, reading the segment bounds again after the ranking barrier
// and loading the start row after it, each waited for on its own, made a chain
// of about ten dependent round trips that took half of a launch at
// B = 65536.)
//
// The launch starts with nlong long-segment slots per tile (every tile of an
// XCD, in its tile order): slot j sums the chunk's listed long segments j,
// j + nlong, ... for its tile with the whole workgroup (long_segment_sum_wg);
// the feature blocks follow, tile by tile.  A long segment is a chain of
// dependent adds, so the chains of an XCD's tiles run side by side instead of
// one tile after another (Zipf alpha = 1.0, B = 65536: 415.6 -> 365.3 us per
// launch at 128 slots, uniform features 204.1 -> 205.7 us).
//
// Dynamic LDS: positions (kBwdPosLds ints) | plus rows (256 chunks, present
// for kDstOutPlus); at least the long-segment row buffer.
constexpr int kBwdFeat = bwd_feat_per_block();  // 32
struct GatherLds {
  int plus, bytes;  // byte offset (-1: absent) and size
};
__host__ __device__ inline GatherLds gather_lds(int dst_mode) {
  GatherLds l;
  int off = kBwdPosLds * 4;
  l.plus = dst_mode == kDstOutPlus ? off : -1;
  off += dst_mode == kDstOutPlus ? kBlock * 16 : 0;
  const int long_buf = kWgLongRows * 8 * (int)sizeof(f32x4);
  l.bytes = off > long_buf ? off : long_buf;
  return l;
}

template <typename T>
__device__ __forceinline__ T shfl_xor_t(T v, int m);
template <>
__device__ __forceinline__ float shfl_xor_t<float>(float v, int m) {
  return __shfl_xor(v, m);
}
template <>
__device__ __forceinline__ f32x4 shfl_xor_t<f32x4>(f32x4 v, int m) {
  return f32x4{__shfl_xor(v.x, m), __shfl_xor(v.y, m), __shfl_xor(v.z, m), __shfl_xor(v.w, m)};
}

// db[c] (+)= sum over parts of partial[p, c].  One wave per column chunk: lane
// l sums parts l, l+64, ..., then a fixed xor-shuffle tree.  Deterministic.
template <typename T>
__device__ __forceinline__ void bias_final_block(int64_t block, const T *__restrict__ partial, int nparts,
                                                 int64_t cols, T *__restrict__ db, int overwrite) {
  const int wave = uniform(threadIdx.x / kWave), lane = threadIdx.x % kWave;
  const int64_t c = block * kWavesPerBlock + wave;
  if (c >= cols) return;
  // a lane's partials p = lane, lane + 64, ... in that order, 8 at a time, the
  // 8 loaded first (from rows clamped into range) and then added (a pair of
  // grads reduces 2 x 512 partials)
  constexpr int kPer = 8;
  T s = T(0);
  for (int p0 = 0; p0 < nparts; p0 += kPer * kWave) {
    T v[kPer];
#pragma unroll
    for (int i = 0; i < kPer; ++i) v[i] = partial[(int64_t)min(p0 + lane + i * kWave, nparts - 1) * cols + c];
#pragma unroll
    for (int i = 0; i < kPer; ++i)
      if (p0 + lane + i * kWave < nparts) s += v[i];
  }
#pragma unroll
  for (int m = 1; m < kWave; m <<= 1) s += shfl_xor_t(s, m);
  if (lane == 0) db[c] = overwrite ? s : db[c] + s;
}
// Workgroups of the bias reduction over cols columns (one wave per column).
int64_t bias_final_blocks(int64_t cols) { return ceil_div(cols, (int64_t)kWavesPerBlock); }

// The arguments of one tiled gather launch.
struct TiledArgs {
  const int32_t *seg, *sorted_pos;
  const uint16_t *pos16;
  int chunk_base;
  int64_t N;
  const f32x4 *gt;
  int64_t B;
  ColMap map;
  RowDst dst;
  f32x4 *tmp;
  int src_mode, dst_mode, ntiles, ngroups;
  const int32_t *long_list;
  const int *long_count;
  int nlong;
  // workgroups from gblocks on reduce the bias partials instead (bias_final_block)
  int64_t gblocks;
  const f32x4 *bpart;
  int bparts;
  int64_t bcols;
  f32x4 *db;
  int boverwrite;
};

// Long-segment slot it.chunk of tile it.tile (whole workgroup).
__device__ __forceinline__ void tiled_long_item(const TiledArgs &a, TileItem it, char *gsm) {
  constexpr int TCH = kBwdTileCh;
  const int cnt = *a.long_count;
  for (int e = it.chunk; e < cnt; e += a.nlong) {
    const int64_t f = a.long_list[e];
    const int s0 = a.seg[f];
    long_segment_sum_wg(a.sorted_pos, f, s0, a.seg[f + 1] - s0, it.tile, LongRows{a.gt, a.B * TCH, TCH}, a.map,
                        a.dst, a.tmp, a.N, a.src_mode, a.dst_mode, reinterpret_cast<f32x4 *>(gsm));
  }
}

// Feature block it.chunk of tile it.tile (whole workgroup; one barrier inside).
template <bool NT, bool P16>
__device__ __forceinline__ void tiled_feature_item(const TiledArgs &a, TileItem it, char *gsm, int *s_seg,
                                                   int *s_perm) {
  constexpr int TCH = kBwdTileCh;
  const int32_t *__restrict__ seg = a.seg;
  const int32_t *__restrict__ sorted_pos = a.sorted_pos;
  const uint16_t *__restrict__ pos16 = a.pos16;
  const int64_t N = a.N, B = a.B;
  const ColMap &map = a.map;
  const RowDst &dst = a.dst;
  f32x4 *__restrict__ tmp = a.tmp;
  const int src_mode = a.src_mode, dst_mode = a.dst_mode, chunk_base = a.chunk_base;
  const f32x4 *__restrict__ gt = a.gt;
  const GatherLds lay = gather_lds(dst_mode);
  int *spos = reinterpret_cast<int *>(gsm);
  const int64_t cols4 = map.cols4;
  const int tid = threadIdx.x;
  const int wave = uniform(tid / kWave);
  const int lane = tid % kWave;
  const int64_t fb = (int64_t)it.chunk * kBwdFeat;
  const int nf = (int)(N - fb < kBwdFeat ? N - fb : kBwdFeat);  // features of this block, >= 1

  // load round 1: segment bounds -- the range (uniform), this thread's feature for
  // the start rows, and one feature per lane of wave 0 for the ranking
  const int r0 = seg[fb], r1 = seg[fb + nf];
  const int64_t fs = fb + tid / TCH;  // start-row feature of this thread
  const int cs = tid % TCH;
  int as = 0, es = 0;
  if (fs < N) {
    as = seg[fs];
    es = seg[fs + 1];
  }
  int la = 0;
  if (wave == 0) la = seg[fb + (lane < nf ? lane : nf)];

  // load round 2: positions, start rows, plus rows.  The range is copied in
  // 16-byte pieces from r0 rounded down to a piece boundary (the position
  // streams are 16-byte aligned and padded by 16 bytes), so spos[j] holds
  // entry ra + j: from the 16-bit chunk offsets (P16: eight per piece, widened
  // to ints in LDS), else from the positions (four per piece).
  constexpr int PER = P16 ? 8 : 4;  // entries per 16-byte piece
  const int ra = r0 & ~(PER - 1);
  const int cnt4 = (r1 - ra + PER - 1) / PER;           // 16-byte pieces
  const bool staged = cnt4 * PER <= kBwdPosLds;         // block-uniform
  if (staged) {
    constexpr int U = 4;
    const i32x4 *src = P16 ? reinterpret_cast<const i32x4 *>(pos16 + ra)
                           : reinterpret_cast<const i32x4 *>(sorted_pos + ra);
    i32x4 *dst4 = reinterpret_cast<i32x4 *>(spos);
    for (int b0 = 0; b0 < cnt4; b0 += U * kBlock) {
      i32x4 v[U];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int i = b0 + u * kBlock + tid;
        v[u] = i < cnt4 ? SFT_STREAM_LOAD(src + i) : i32x4{0, 0, 0, 0};
      }
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int i = b0 + u * kBlock + tid;
        if (i >= cnt4) continue;
        if (P16) {
          const uint32_t w0 = (uint32_t)v[u][0], w1 = (uint32_t)v[u][1], w2 = (uint32_t)v[u][2], w3 = (uint32_t)v[u][3];
          dst4[2 * i] = i32x4{(int)(w0 & 0xffffu), (int)(w0 >> 16), (int)(w1 & 0xffffu), (int)(w1 >> 16)};
          dst4[2 * i + 1] = i32x4{(int)(w2 & 0xffffu), (int)(w2 >> 16), (int)(w3 & 0xffffu), (int)(w3 >> 16)};
        } else {
          dst4[i] = v[u];
        }
      }
    }
  }
  if (lay.plus >= 0) {
    const int colm = tile_col(map, it.tile, cs);
    f32x4 vp = f32x4{0.f, 0.f, 0.f, 0.f};
    if (fs < N && colm >= 0 && !long_segment(as, es)) {
      const int blk = block_of(fs, dst.n, dst.start);
      vp = load_row<NT>(pick(dst.p, blk) + (fs - pick(dst.start, blk)) * cols4 + colm);
    }
    reinterpret_cast<f32x4 *>(gsm + lay.plus)[tid] = vp;
  }
  if (wave == 0) {
    // A wave runs as long as its longest segment: rank the features by segment
    // length (ties by index, long segments as 0) and give each wave 8
    // consecutive ranks.
    const int le = __shfl_down(la, 1);
    const bool live = lane < nf;
    const int len = (live && !long_segment(la, le)) ? le - la : 0;
    int rank = 0;
    for (int j = 0; j < kBwdFeat; ++j) {
      const int o = __builtin_amdgcn_readlane(len, j);
      rank += (o > len || (o == len && j < lane)) ? 1 : 0;
    }
    if (lane < kBwdFeat) s_perm[rank] = lane;
    if (lane <= kBwdFeat) s_seg[lane] = la;
  }
  __syncthreads();

  const int g = lane / TCH, t = lane % TCH;
  const int p = s_perm[wave * (kWave / TCH) + g];
  const int64_t f = fb + p;
  const int s0 = s_seg[p], s1 = s_seg[p + 1];
  const bool live = p < nf;
  const bool is_long = live && long_segment(s0, s1);  // summed by the long-segment slots
  const int n = (live && !is_long) ? s1 - s0 : 0;
  int nmin, nmax;
  group_minmax<TCH>(n, nmin, nmax);
  const int colm = tile_col(map, it.tile, t);
  const bool colok = colm >= 0;
  const char *gtile = reinterpret_cast<const char *>(gt + (int64_t)it.tile * B * TCH);
  // The sum the previous position chunk left, loaded by the lane itself with
  // its first row loads so that its latency overlaps theirs (staging it
  // through LDS put it in front of the workgroup's barrier); still the first
  // operand of the adds.  Lanes without one load a grad line instead.
  f32x4 acc = f32x4{0.f, 0.f, 0.f, 0.f};
  const bool cont = src_mode == kSrcTmp && live && !is_long && colok;
  const f32x4 *from = src_mode == kSrcTmp ? tmp + tmp_row(it.tile, live ? f : fb, N) + t  // stored with NT too
                                          : reinterpret_cast<const f32x4 *>(gtile) + t;
  if (staged)  // P16: offsets from the chunk's first grad row
    bwd_tile_sum<true, TCH, NT>(spos + (s0 - ra), n, nmin, nmax, t,
                                P16 ? gtile + (size_t)chunk_base * (TCH * sizeof(f32x4)) : gtile, acc, from, cont);
  else
    bwd_tile_sum<false, TCH, NT>(sorted_pos + s0, n, nmin, nmax, t, gtile, acc, from, cont);
  if (!live || !colok || is_long) return;
  const int blk = block_of(f, dst.n, dst.start);
  f32x4 *d = pick(dst.p, blk) + (f - pick(dst.start, blk)) * cols4 + colm;
  if (dst_mode == kDstTmp) {
    store_row<NT>(tmp + tmp_row(it.tile, f, N) + t, acc);
  } else if (dst_mode == kDstOutPlus) {
    store_row<NT>(d, reinterpret_cast<const f32x4 *>(gsm + lay.plus)[p * TCH + t] + acc);
  } else {
    store_row<NT>(d, acc);
  }
}

// One item per workgroup: workgroup i serves item i / 8 of XCD i % 8 (the
// long-segment slots first, then the feature blocks); workgroups after the
// items, when the launch carries them, reduce the bias partials (the bias
// pass's second step, which then needs no launch of its own).
template <bool NT, bool P16>
__global__ __launch_bounds__(kBlock) void bwd_tiled_gather_kernel(TiledArgs a) {
  extern __shared__ __align__(16) char gsm[];
  __shared__ int s_seg[kBwdFeat + 1], s_perm[kBwdFeat];
  if ((int64_t)blockIdx.x >= a.gblocks) {  // whole block: uniform
    bias_final_block<f32x4>((int64_t)blockIdx.x - a.gblocks, a.bpart, a.bparts, a.bcols, a.db, a.boverwrite);
    return;
  }
  const int64_t nl_items = tile_sched_items_per_xcd(a.ntiles, a.nlong) * kXcds;
  const bool long_item = (int64_t)blockIdx.x < nl_items;  // whole block: uniform
  const TileItem it = long_item ? tile_sched_item(blockIdx.x, a.ntiles, a.nlong)
                                : tile_sched_item(blockIdx.x - nl_items, a.ntiles, a.ngroups);
  if (it.tile >= a.ntiles) return;  // whole block: uniform
  if (long_item)
    tiled_long_item(a, it, gsm);
  else
    tiled_feature_item<NT, P16>(a, it, gsm, s_seg, s_perm);
}


// One position chunk's tiled weight-grad gather.
// pos16: the slots' 16-bit chunk offsets (null when a chunk has more than
// 65536 positions), chunk_base the first position of this launch's chunk.
// The bias reduction a tiled gather launch may carry: db (+)= the sum of
// nparts partial rows of cols 16-byte chunks.
struct BiasFinal {
  const f32x4 *partial;
  int nparts;
  int64_t cols;
  f32x4 *db;
  int overwrite;
};
int launch_tiled_gather(bool nt, const int32_t *seg, const int32_t *pos, const uint16_t *pos16, int64_t chunk_base,
                        int64_t N, const f32x4 *gt, int64_t B, const ColMap &map, const RowDst &dst, f32x4 *tmp,
                        int src_mode, int dst_mode, int ntiles, int ngroups, const int32_t *long_list,
                        const int *long_count, int nlong, hipStream_t s, const BiasFinal *bias = nullptr) {
  const int64_t items = tile_sched_items_per_xcd(ntiles, nlong) + tile_sched_items_per_xcd(ntiles, ngroups);
  const size_t lds = (size_t)gather_lds(dst_mode).bytes;
  if ((uintptr_t)pos % 16 != 0 || (uintptr_t)pos16 % 16 != 0)  // 256-byte / 16-byte aligned workspace regions
    return fail(SFT_EINVAL, "tiled feature gather: sorted positions not 16-byte aligned");
  const int64_t gblocks = items * kXcds;
  const TiledArgs a{seg, pos, pos16, (int)chunk_base, N, gt, B, map, dst, tmp, src_mode, dst_mode, ntiles, ngroups,
                    long_list, long_count, nlong, gblocks, bias ? bias->partial : nullptr, bias ? bias->nparts : 0,
                    bias ? bias->cols : 0, bias ? bias->db : nullptr, bias ? bias->overwrite : 0};
  const bool p16 = pos16 != nullptr;
  const dim3 grid((unsigned)(gblocks + (bias ? bias_final_blocks(bias->cols) : 0)));
  hipLaunchKernelGGL((nt ? (p16 ? bwd_tiled_gather_kernel<true, true> : bwd_tiled_gather_kernel<true, false>)
                         : (p16 ? bwd_tiled_gather_kernel<false, true> : bwd_tiled_gather_kernel<false, false>)),
                     grid, dim3(kBlock), lds, s, a);
  return check_launch("tiled feature gather");
}

// dV[j, :] = sum over i < reps of dWb[i * period + j, :], i ascending (the
// reduction behind virtual_weight.repeat(32, 1), FEAT/halfka_v2_hm.py:69-70).
// One thread per 16-byte chunk of dV; rows of consecutive threads are
// consecutive, so every step reads contiguous memory.
__global__ __launch_bounds__(kBlock) void virtual_reduce_kernel(const f32x4 *__restrict__ dWb, int64_t period,
                                                                int reps, int64_t cols4, f32x4 *__restrict__ dV) {
  constexpr int U = 8;
  const int64_t total = period * cols4;
  for (int64_t i = (int64_t)blockIdx.x * kBlock + threadIdx.x; i < total; i += (int64_t)gridDim.x * kBlock) {
    f32x4 acc = f32x4{0.f, 0.f, 0.f, 0.f};
    int r = 0;
    for (; r + U <= reps; r += U) {
      f32x4 x[U];
#pragma unroll
      for (int u = 0; u < U; ++u) x[u] = dWb[(int64_t)(r + u) * total + i];
#pragma unroll
      for (int u = 0; u < U; ++u) acc += x[u];
    }
    for (; r < reps; ++r) acc += dWb[(int64_t)r * total + i];
    dV[i] = acc;
  }
}

// Backward of the post-FT epilogue (src/model/model.py:93-115), elementwise
// and in the order autograd evaluates it, so every grad is bit-identical:
//   d_sel  = g_l0[b, half + j] * (127/128)         half chosen by us[b] and the perspective
//   d_pw   = d_sel + 0        (the two where() grads are summed; one is +0)
//   d_c    = d_pw * clamp(partner) + 0   (mul backward; the two select() grads summed)
//   d_raw  = (0 <= raw <= 1) ? d_c : 0   (clamp backward)
//   PSQT column k: (k == psqt_idx[b]) ? 0 + (+/-)(g_psqt[b] * (us[b] - 0.5)) : 0
//                  (mul, sub and gather backward; + for white, - for black)
// The grads go straight to the grad tiles of the weight-grad gather (paired
// map), and their column sums over the block's positions of both perspectives
// to partial[blockIdx.x] for the bias grad.
//
// Mapping: wave w of a workgroup takes rows r0 + w, r0 + w + 4, ...; lane
// group g of the wave takes tiles g, g + 8, ... (kEpiIt per pass), so the
// eight lane groups of a wave read 8 consecutive 64-byte chunks of each half
// of the row's l0 grad (512 contiguous bytes) and each lane group one whole
// 128-byte line of the pre-activation and grad tiles.  All loads of a row are
// issued before any arithmetic.
struct BwdEpilogue {
  const float *g_l0;         // [B, L1]
  const float *g_psqt;       // [B]
  const float *us;           // [B]
  const int64_t *psqt_idx;   // [B]
  const f32x4 *raw0, *raw1;  // pre-activations, [B][ntiles][8] paired-tile chunks
  f32x4 *gt0, *gt1;          // grad tiles out
  f32x4 *partial;            // [gridDim.x][cols4]
  int P;
};
// 80 rows: 820 workgroups at B = 65536, leaving the two sorts beside the pass
// more of the CUs' slots (epilogue op 1.955 -> 1.915 ms per step, Full_Threats
// 7.091 -> 7.048 ms against 64 rows; 96 rows: 1.918 / 7.049 ms).
#ifndef SFT_EPI_ROWS
#define SFT_EPI_ROWS 80
#endif
constexpr int kEpiRows = SFT_EPI_ROWS;  // positions per workgroup
#ifndef SFT_EPI_IT
#define SFT_EPI_IT 3
#endif
constexpr int kEpiIt = SFT_EPI_IT;  // tile slots per lane group and pass (8 kEpiIt tiles per pass)
__device__ __forceinline__ float clamp01f(float x) { return x < 0.f ? 0.f : (x > 1.f ? 1.f : x); }
__device__ __forceinline__ f32x4 shfl_xor4(f32x4 v, int m) {
  return f32x4{__shfl_xor(v.x, m), __shfl_xor(v.y, m), __shfl_xor(v.z, m), __shfl_xor(v.w, m)};
}

__global__ __launch_bounds__(kBlock) void bwd_epilogue_kernel(BwdEpilogue e, ColMap map, int64_t B, int ntiles) {
  __shared__ f32x4 red[kWavesPerBlock][kEpiIt][kWave];
  const int wave = uniform(threadIdx.x / kWave);
  const int lane = threadIdx.x % kWave;
  const int g = lane / kBwdTileCh, q = lane % kBwdTileCh;
  const int64_t l0_row = 2 * (int64_t)map.half4;
  const float k127 = 127.0f / 128.0f;
  const int64_t r0 = (int64_t)blockIdx.x * kEpiRows;
  for (int t0 = 0; t0 < ntiles; t0 += kBwdTileCh * kEpiIt) {
    int tile[kEpiIt], colm[kEpiIt];
#pragma unroll
    for (int i = 0; i < kEpiIt; ++i) {
      tile[i] = t0 + g + kBwdTileCh * i;
      colm[i] = tile[i] < ntiles ? tile_col(map, tile[i], q) : -1;
    }
    f32x4 bsum[kEpiIt];
#pragma unroll
    for (int i = 0; i < kEpiIt; ++i) bsum[i] = f32x4{0.f, 0.f, 0.f, 0.f};
    for (int r = wave; r < kEpiRows; r += kWavesPerBlock) {
      const int64_t b = r0 + r;
      if (b >= B) break;  // wave-uniform
      const bool wtm = e.us[b] != 0.f;
      const int64_t k = e.psqt_idx[b];
      const float dp = e.g_psqt[b] * (e.us[b] - 0.5f);
      // One perspective at a time: its loads for all kEpiIt tile slots are
      // issued together, which bounds the live registers to one perspective.
#pragma unroll 1
      for (int p = 0; p < 2; ++p) {
        const int64_t half = ((p == 1) ? wtm : !wtm) ? map.half4 : 0;
        const f32x4 *__restrict__ raw = p == 0 ? e.raw0 : e.raw1;
        f32x4 *__restrict__ gt = p == 0 ? e.gt0 : e.gt1;
        f32x4 a[kEpiIt], gs[kEpiIt];
#pragma unroll
        for (int i = 0; i < kEpiIt; ++i) {
          const bool ok = colm[i] >= 0;
          const bool paired = tile[i] < map.t1;
          const int64_t j = 4 * (int64_t)tile[i] + (q & 3);
          const f32x4 zero = f32x4{0.f, 0.f, 0.f, 0.f};
          a[i] = ok ? raw[(b * ntiles + tile[i]) * kBwdTileCh + q] : zero;
          gs[i] = (ok && paired) ? reinterpret_cast<const f32x4 *>(e.g_l0)[b * l0_row + half + j] : zero;
        }
#pragma unroll
        for (int i = 0; i < kEpiIt; ++i) {
          const bool paired = tile[i] < map.t1;
          const f32x4 av = a[i];
          const f32x4 partner = shfl_xor4(av, 4);
          f32x4 d = f32x4{0.f, 0.f, 0.f, 0.f};
          if (colm[i] >= 0) {
            if (paired) {
              const f32x4 dpw = gs[i] * k127 + 0.0f;
              const f32x4 cp = f32x4{clamp01f(partner.x), clamp01f(partner.y), clamp01f(partner.z),
                                     clamp01f(partner.w)};
              const f32x4 dc = dpw * cp + 0.0f;
              d.x = (av.x >= 0.f && av.x <= 1.f) ? dc.x : 0.f;
              d.y = (av.y >= 0.f && av.y <= 1.f) ? dc.y : 0.f;
              d.z = (av.z >= 0.f && av.z <= 1.f) ? dc.z : 0.f;
              d.w = (av.w >= 0.f && av.w <= 1.f) ? dc.w : 0.f;
            } else {
              const int64_t kq = 4 * (int64_t)(colm[i] - 2 * map.half4);  // PSQT column of element 0
              if (k >= kq && k < kq + 4) d[(int)(k - kq)] = 0.0f + (p == 0 ? dp : -dp);
            }
            gt[((int64_t)tile[i] * B + b) * kBwdTileCh + q] = d;
          }
          bsum[i] += d;
        }
      }
    }
#pragma unroll
    for (int i = 0; i < kEpiIt; ++i) red[wave][i][lane] = bsum[i];
    __syncthreads();
    for (int x = threadIdx.x; x < kEpiIt * kWave; x += kBlock) {
      const int i = x / kWave, l = x % kWave;
      const int t = t0 + l / kBwdTileCh + kBwdTileCh * i;
      const int c = t < ntiles ? tile_col(map, t, l % kBwdTileCh) : -1;
      if (c >= 0)
        e.partial[(int64_t)blockIdx.x * map.cols4 + c] = (red[0][i][l] + red[1][i][l]) + (red[2][i][l] + red[3][i][l]);
    }
    __syncthreads();
  }
}

// Position-major fp32 atomic scatter.  One wave per position (lanes over
// consecutive floats, so each atomic instruction covers 256 contiguous bytes);
// FPL floats per lane per slab.
template <int FPL>
__global__ __launch_bounds__(kBlock) void scatter_atomic_kernel(const int32_t *__restrict__ idx, int64_t B, int K,
                                                                int N, const float *__restrict__ grad, int64_t L,
                                                                float *__restrict__ dW, int kpad) {
  extern __shared__ int smem[];
  const int wave = uniform(threadIdx.x / kWave);
  const int lane = threadIdx.x % kWave;
  int *list = smem + wave * kpad;
  int *count = smem + kWavesPerBlock * kpad + wave;
  const int64_t pos = (int64_t)blockIdx.x * kWavesPerBlock + wave;
  compact_rows(idx, B, K, N, pos, 1, list, kpad, count);
  wave_lds_barrier();
  if (pos >= B) return;
  const int n = uniform(count[0]);
  const int64_t c0 = (int64_t)blockIdx.y * (kWave * FPL) + lane;
  float g[FPL];
  const float *grow = grad + pos * L + c0;
#pragma unroll
  for (int j = 0; j < FPL; ++j) g[j] = (c0 + kWave * j < L) ? grow[kWave * j] : 0.0f;
  for (int k = 0; k < n; ++k) {
    const int f = uniform(list[k]);
    float *drow = dW + (int64_t)f * L + c0;
#pragma unroll
    for (int j = 0; j < FPL; ++j)
      if (c0 + kWave * j < L) unsafeAtomicAdd(drow + kWave * j, g[j]);
  }
}

__global__ __launch_bounds__(kBlock) void zero_kernel(float *__restrict__ p, int64_t n) {
  for (int64_t i = (int64_t)blockIdx.x * kBlock + threadIdx.x; i < n; i += (int64_t)gridDim.x * kBlock) p[i] = 0.0f;
}

// partial[blk, c] = sum of grad[r, c] over the block's rows.  Wave w of the
// block takes rows r0 + w, r0 + w + 4, ... (U rows per step, loads first),
// lane l owns chunks c0 + l + 64 j like the row gathers; the four wave sums
// are combined in a fixed order.  Deterministic.
//
// When gt is not null, each grad element read (a 16-byte chunk for T = f32x4,
// a float for T = float) is also stored to the column-tile layout of the tiled
// gather, tiles of 2^gt_shift elements: gt[(c >> gt_shift) * B + r][c mod
// 2^gt_shift] -- the same bytes for a float4 c with shift s as for its floats
// with shift s + 2 -- so the grad crosses HBM once for both the bias sum and
// the re-layout.
template <typename T, int CPL>
__global__ __launch_bounds__(kBlock) void bias_partial_kernel(const T *__restrict__ grad, int64_t B, int64_t cols,
                                                              int64_t rows_per_block, T *__restrict__ partial,
                                                              T *__restrict__ gt, int gt_shift) {
  constexpr int U = 4;
  __shared__ T red[kWavesPerBlock][kWave * CPL];
  const int wave = uniform(threadIdx.x / kWave);
  const int lane = threadIdx.x % kWave;
  const int64_t c0 = (int64_t)blockIdx.y * (kWave * CPL) + lane;
  const int64_t r0 = (int64_t)blockIdx.x * rows_per_block;
  const int64_t r1 = std::min<int64_t>(B, r0 + rows_per_block);
  bool colok[CPL];
  T acc[CPL];
#pragma unroll
  for (int j = 0; j < CPL; ++j) {
    colok[j] = c0 + kWave * j < cols;
    acc[j] = T(0);
  }
  for (int64_t r = r0 + wave; r < r1; r += kWavesPerBlock * U) {
    T v[U][CPL];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t rr = r + (int64_t)kWavesPerBlock * u;
      const T *row = grad + rr * cols + c0;
#pragma unroll
      for (int j = 0; j < CPL; ++j) {
        v[u][j] = T(0);
        if (rr < r1 && colok[j]) v[u][j] = __builtin_nontemporal_load(row + kWave * j);  // read once
      }
    }
    if (gt != nullptr) {
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int64_t rr = r + (int64_t)kWavesPerBlock * u;
#pragma unroll
        for (int j = 0; j < CPL; ++j) {
          const int64_t c = c0 + kWave * j;
          if (rr < r1 && colok[j]) gt[(((c >> gt_shift) * B + rr) << gt_shift) + (c & ((1 << gt_shift) - 1))] = v[u][j];
        }
      }
    }
#pragma unroll
    for (int u = 0; u < U; ++u)
#pragma unroll
      for (int j = 0; j < CPL; ++j) acc[j] += v[u][j];
  }
#pragma unroll
  for (int j = 0; j < CPL; ++j) red[wave][lane + kWave * j] = acc[j];
  __syncthreads();
  for (int i = threadIdx.x; i < kWave * CPL; i += kBlock) {
    const int64_t c = (int64_t)blockIdx.y * (kWave * CPL) + i;
    if (c < cols) partial[(int64_t)blockIdx.x * cols + c] = (red[0][i] + red[1][i]) + (red[2][i] + red[3][i]);
  }
}

template <typename T>
__global__ __launch_bounds__(kBlock) void bias_final_kernel(const T *__restrict__ partial, int nparts, int64_t cols,
                                                            T *__restrict__ db, int overwrite) {
  bias_final_block<T>(blockIdx.x, partial, nparts, cols, db, overwrite);
}

template <typename T, int G, int CPL>
void launch_gather(dim3 grid, hipStream_t s, const int32_t *seg_start, const int32_t *pos, int64_t N, const void *grad,
                   int64_t cols, void *dW, int overwrite, const SegBufs &sb, int nlong) {
  hipLaunchKernelGGL((gather_rows_kernel<T, G, CPL, 4>), grid, dim3(kBlock), 0, s, seg_start, pos, N,
                     static_cast<const T *>(grad), cols, static_cast<T *>(dW), overwrite, sb.list, sb.count, nlong);
}

#define SFT_CPL_CASES(FN, T, G, ...) \
  switch (m.cpl) {                   \
    case 1: FN<T, G, 1>(__VA_ARGS__); break; \
    case 2: FN<T, G, 2>(__VA_ARGS__); break; \
    case 3: FN<T, G, 3>(__VA_ARGS__); break; \
    case 4: FN<T, G, 4>(__VA_ARGS__); break; \
    case 5: FN<T, G, 5>(__VA_ARGS__); break; \
    case 6: FN<T, G, 6>(__VA_ARGS__); break; \
    case 7: FN<T, G, 7>(__VA_ARGS__); break; \
    default: FN<T, G, 8>(__VA_ARGS__); break; \
  }

#define SFT_G_CASES(FN, T, ...)                          \
  switch (m.G) {                                         \
    case 64: SFT_CPL_CASES(FN, T, 64, __VA_ARGS__) break; \
    case 32: SFT_CPL_CASES(FN, T, 32, __VA_ARGS__) break; \
    case 16: SFT_CPL_CASES(FN, T, 16, __VA_ARGS__) break; \
    default: SFT_CPL_CASES(FN, T, 8, __VA_ARGS__) break;  \
  }

size_t align256(size_t v) { return (v + 255) & ~(size_t)255; }

struct BwdLayout {
  size_t sort, seg, spos, partial, gt, tmp, total;
  int nparts;
};

// Beside the whole sort (radix pass and buckets on the side stream, which
// outlasts the bias pass at B = 65536), the pass takes 7/8 of the row blocks:
// 448 instead of 512 at B = 65536, L = 1048, step 1.706-1.712 -> 1.670-1.678 ms
// (A/B builds on three boxes; 384: 1.680, 320: 1.693, 256: 1.693 ms); the
// composed pair op, whose two sorts run beside both bias passes, 1.700 ->
// 1.693 ms (Full_Threats+HalfKAv2_hm^ 6.634 -> 6.620 ms).  At B = 16384 (256 ->
// 224 blocks) fewer blocks were even; with the prepared sort (nothing or only
// the buckets beside the pass) the pass keeps them all (L = 136, 384 blocks:
// 0.377 -> 0.383 ms).  13/16 and 15/16 of the blocks were even or slower.
#ifndef SFT_BIAS_BESIDE_SORT_16THS
#define SFT_BIAS_BESIDE_SORT_16THS 14
#endif
int bias_parts(int64_t B, bool beside_sort) {
  const int64_t p = std::max<int64_t>(1, std::min<int64_t>(kBiasMaxParts, ceil_div(B, kBiasRowsPerBlock)));
  return (int)(beside_sort ? std::max<int64_t>(1, p * SFT_BIAS_BESIDE_SORT_16THS / 16) : p);
}

bool tiled_shape(int64_t B, int L, uint32_t flags) {
  return !(flags & (SFT_BWD_ATOMIC | SFT_BWD_ROWS)) && (flags & SFT_BWD_OVERWRITE) && L % 4 == 0 &&
         ceil_div(L, 32) >= kBwdMinTiles && B * 16 * kBwdTileCh <= (int64_t)UINT32_MAX;  // 32-bit grad row offsets
}

// Position chunks of the tiled gather (one launch each).
#ifndef SFT_BWD_CHUNKS
#define SFT_BWD_CHUNKS 2
#endif
constexpr int kBwdHalves = SFT_BWD_CHUNKS;
// A batch whose whole grad tile fits an XCD's L2 (4 MB: B <= 32768) is gathered
// in one position chunk: no partial weight grads to store and reload (B = 16384:
// 0.768 -> 0.619 ms per step, B = 32768: 1.139 -> 0.998 ms).  At B = 65536 one
// chunk of 8.4 MB thrashes the L2 (1.84 -> 2.03 ms).
#ifndef SFT_BWD_ONE_CHUNK_BYTES
#define SFT_BWD_ONE_CHUNK_BYTES (4 << 20)
#endif
int sort_chunks(int64_t B, int L, uint32_t flags) {
  if (!tiled_shape(B, L, flags) || B < kBwdHalves) return 1;
  return B * 16 * kBwdTileCh <= (int64_t)(SFT_BWD_ONE_CHUNK_BYTES) ? 1 : kBwdHalves;
}
int64_t half_rows(int64_t B) { return ceil_div(B, kBwdHalves); }

// The sort and offsets buffers are sized for the tiled (chunked) key space,
// which also covers the one-chunk key space of the row gather, so the choice
// between the two can wait for the pointers' alignment at call time.  With
// SFT_BWD_PREPARED they live in the caller's prepared buffer instead
// (make_prep_layout) and the workspace holds the rest.
bool prep_pays(int64_t B, int K, int L, uint32_t flags);
bool prep_split(int64_t B, int K, int64_t N, int L, uint32_t flags);
int make_layout(int64_t B, int K, int64_t N, int L, uint32_t flags, BwdLayout &lay) {
  const int64_t M = B * K;
  lay.nparts = bias_parts(B, !(flags & SFT_BWD_ATOMIC) && M > 0 &&
                                 !((flags & SFT_BWD_PREPARED) && prep_pays(B, K, L, flags)));
  size_t off = 0;
  lay.partial = off;
  off = align256(off + (size_t)lay.nparts * (size_t)L * sizeof(float));
  lay.sort = lay.seg = lay.spos = lay.gt = lay.tmp = off;
  if (!(flags & SFT_BWD_ATOMIC) && M > 0) {
    const int nc = sort_chunks(B, L, flags);
    const bool prepared = (flags & SFT_BWD_PREPARED) && prep_pays(B, K, L, flags);
    if (!prepared) {
      lay.sort = off;
      off = align256(off + slot_sort_workspace(M));
      lay.seg = off;
      off = align256(off + seg_region_bytes(nc, N, M));
    } else if (prep_split(B, K, N, L, flags)) {  // the buckets' outputs: sorted positions and segments
      lay.spos = off;
      off = align256(off + (size_t)M * 4);
      lay.seg = off;
      off = align256(off + seg_region_bytes(nc, N, M));
    }
    lay.gt = off;
    if (tiled_shape(B, L, flags)) {  // the grad tiles the bias pass writes, whatever the chunk count
      const int64_t ntiles = ceil_div(L / 4, kBwdTileCh);
      off = align256(off + (size_t)(ntiles * B * kBwdTileCh) * 16);
      lay.tmp = off;
      if (nc > 1) off = align256(off + (size_t)(ntiles * N * kBwdTileCh) * 16);  // sums between chunks
    }
  }
  lay.total = off;
  return SFT_OK;
}

int launch_bias_partial(const float *grad, int64_t B, int L, int nparts, float *partial, f32x4 *gt, bool vec,
                        hipStream_t s, int gt_tch = 8) {
  // tile width in the kernel's element type: gt_tch 16-byte chunks, or 4 x as many floats
  const int gt_shift = (gt_tch == 4 ? 2 : gt_tch == 16 ? 4 : 3) + (vec ? 0 : 2);
  const int64_t cols = vec ? L / 4 : L;
  const int64_t rows = ceil_div(std::max<int64_t>(B, 1), nparts);
  const int cpl = (int)std::min<int64_t>(ceil_div(cols, kWave), kMaxCpl);
  const dim3 pgrid((unsigned)nparts, (unsigned)ceil_div(cols, (int64_t)kWave * cpl));
  ProfScope prof(kProfBwdBiasPartial, s);
#define SFT_BIAS_CASE(T, C)                                                                                  \
  hipLaunchKernelGGL((bias_partial_kernel<T, C>), pgrid, dim3(kBlock), 0, s, reinterpret_cast<const T *>(grad), \
                     B, cols, rows, reinterpret_cast<T *>(partial), reinterpret_cast<T *>(gt), gt_shift)
#define SFT_BIAS_SWITCH(T)               \
  switch (cpl) {                         \
    case 1: SFT_BIAS_CASE(T, 1); break;  \
    case 2: SFT_BIAS_CASE(T, 2); break;  \
    case 3: SFT_BIAS_CASE(T, 3); break;  \
    case 4: SFT_BIAS_CASE(T, 4); break;  \
    case 5: SFT_BIAS_CASE(T, 5); break;  \
    case 6: SFT_BIAS_CASE(T, 6); break;  \
    case 7: SFT_BIAS_CASE(T, 7); break;  \
    default: SFT_BIAS_CASE(T, 8); break; \
  }
  if (vec) {
    SFT_BIAS_SWITCH(f32x4)
  } else {
    SFT_BIAS_SWITCH(float)
  }
#undef SFT_BIAS_SWITCH
#undef SFT_BIAS_CASE
  return check_launch("bias partial sums");
}

int launch_bias_final(const float *partial, int nparts, int L, float *db, int overwrite, bool vec, hipStream_t s) {
  const int64_t cols = vec ? L / 4 : L;
  ProfScope prof(kProfBwdBiasFinal, s);
  const dim3 grid((unsigned)ceil_div(cols, kWavesPerBlock));
  if (vec)
    hipLaunchKernelGGL(bias_final_kernel<f32x4>, grid, dim3(kBlock), 0, s, reinterpret_cast<const f32x4 *>(partial),
                       nparts, cols, reinterpret_cast<f32x4 *>(db), overwrite);
  else
    hipLaunchKernelGGL(bias_final_kernel<float>, grid, dim3(kBlock), 0, s, partial, nparts, cols, db, overwrite);
  return check_launch("bias reduction");
}

// Segment starts of one sort and its lists of long segments (the counts
// were zeroed by the sort).
int launch_segments(const unsigned *keys, int64_t M, int nc, int64_t nfeat, const unsigned *totals, int ntot,
                    const SegBufs &sb, const int32_t *pos, int64_t chunk_rows, hipStream_t s) {
  ProfScope prof(kProfBwdOffsets, s);
  uint16_t *p16 = chunk_rows <= 65536 ? sb.pos16 : nullptr;
  hipLaunchKernelGGL(seg_offsets_kernel, dim3((unsigned)std::min<int64_t>(ceil_div(M + 1, kBlock), kSegBlocks)),
                     dim3(kBlock), 0, s, keys, (int64_t)nc * nfeat, totals, ntot, sb.seg, nfeat, sb.list, sb.count,
                     pos, p16, (int)std::min<int64_t>(chunk_rows, 65536));
  return check_launch("segment offsets");
}

// The prepared buffer: the sort's workspace, then the segment region of the
// tiled key space (nc chunks); empty when the backward sorts nothing or when
// sorting under the forward does not pay.  Beside the backward's bias pass the
// sort costs only what it outlasts that pass; beside the forward's gather it
// slows the gather (workload 1, K = 32, L = 1048: the forward +17 us, the
// backward -12 us per perspective).  The sort grows with the slots, the bias
// pass with the columns: the sort is prepared from K >= L / 20 (L = 136:
// step 0.530 -> 0.504 ms; L = 1048, K = 160: the K = 160 sort outlasts the
// bias pass by ~180 us).
#ifndef SFT_BWD_PREP_K_PER_L
#define SFT_BWD_PREP_K_PER_L 20
#endif
bool prep_pays(int64_t B, int K, int L, uint32_t flags) {
  return !(flags & SFT_BWD_ATOMIC) && B * K > 0 && (int64_t)K * SFT_BWD_PREP_K_PER_L >= L;
}
// Split prepared sort: the forward runs only the bucket sort's radix pass,
// the backward its buckets beside the bias pass, for shapes where the whole
// sort outlasts the forward's gather it hides behind (rows narrow for their
// slot count: K >= L / SFT_BWD_SPLIT_K_PER_L).
#ifndef SFT_BWD_SPLIT_K_PER_L
#define SFT_BWD_SPLIT_K_PER_L 5
#endif
// The bias reduction in the first tiled gather launch instead of a launch of
// its own.
#ifndef SFT_BWD_FUSE_BIAS_FINAL
#define SFT_BWD_FUSE_BIAS_FINAL 1
#endif
// With the split prepared sort and the gather in position chunks, the
// backward's buckets in two launches: those that complete chunk 0 first, so
// that chunk 0's gather waits for them only and the rest run beside it
// (L = 136: 0.3805-0.3816 -> 0.3778-0.3802 ms per step, A/B builds on two boxes).  The whole sort in the
// backward (radix pass and buckets beside the bias pass) split the same way
// was slower (workload 1: 1.7072-1.7089 -> 1.7099-1.7118 ms): there the
// buckets are a smaller part of the sort the bias pass hides.
#ifndef SFT_BWD_SPLIT_BUCKETS
#define SFT_BWD_SPLIT_BUCKETS 1
#endif
constexpr int kChunk0Mark = 1;  // side-stream mark after chunk 0's buckets
bool prep_split(int64_t B, int K, int64_t N, int L, uint32_t flags) {
  return prep_pays(B, K, L, flags) && (int64_t)K * SFT_BWD_SPLIT_K_PER_L >= L &&
         slot_sort_buckets_supported(N, sort_chunks(B, L, flags));
}
struct PrepLayout {
  size_t sort, seg, total;
  int nc;
};
void make_prep_layout(int64_t B, int K, int64_t N, int L, uint32_t flags, PrepLayout &p) {
  const int64_t M = B * K;
  p.nc = sort_chunks(B, L, flags);
  p.sort = p.seg = p.total = 0;
  if (!prep_pays(B, K, L, flags)) return;
  p.seg = align256(slot_sort_workspace(M));
  p.total = p.seg + align256(seg_region_bytes(p.nc, N, M));
}

// Sort of the slots into nc position chunks and their segment starts, on s.
int sort_and_segments(const int32_t *idx, int64_t B, int K, int64_t N, int nc, void *sort_ws, int32_t *seg,
                      int32_t **pos, hipStream_t s) {
  const int64_t M = B * K;
  const SegBufs sb = seg_bufs(seg, nc, N);
  const int64_t crow = nc > 1 ? half_rows(B) : B;
  if (slot_sort_buckets_supported(N, nc)) {
    ProfScope prof(kProfBwdSort, s);
    return slot_sort_buckets(idx, M, K, N, (int)crow, nc, sort_ws, sb.seg, sb.list, sb.count,
                             crow <= 65536 ? sb.pos16 : nullptr, kLongSeg, pos, s);
  }
  unsigned *keys = nullptr, *totals = nullptr;
  int ntot = 0, rc;
  {
    ProfScope prof(kProfBwdSort, s);
    if ((rc = slot_sort(idx, M, K, N, (int)crow, nc, sort_ws, &keys, pos, &totals, &ntot, sb.count, nc, s)) != SFT_OK)
      return rc;
  }
  return launch_segments(keys, M, nc, N, totals, ntot, sb, *pos, crow, s);
}

}  // namespace

int bwd_prep_bytes(int64_t B, int K, int64_t N, int L, uint32_t flags, size_t *bytes) {
  PrepLayout p;
  make_prep_layout(B, K, N, L, flags, p);
  *bytes = p.total;
  return SFT_OK;
}

// Fills a prepared buffer for a later bwd_f32 with SFT_BWD_PREPARED and the
// same indices, sizes and flags.
int bwd_prepare(const int32_t *idx, int64_t B, int K, int64_t N, int L, uint32_t flags, void *prep,
                size_t prep_bytes, hipStream_t s) {
  PrepLayout p;
  make_prep_layout(B, K, N, L, flags, p);
  if (p.total == 0) return SFT_OK;
  if (prep == nullptr || prep_bytes < p.total || (uintptr_t)prep % 256 != 0)
    return fail(SFT_EWORKSPACE, "prepared buffer smaller than sft_ft_bwd_f32_prep_size() or not 256-byte aligned");
  char *w = static_cast<char *>(prep);
  if (prep_split(B, K, N, L, flags)) {  // the radix pass only; the backward runs the buckets
    ProfScope prof(kProfBwdSort, s);
    return slot_sort_buckets_high(idx, B * K, K, N, (int)(p.nc > 1 ? half_rows(B) : B), p.nc, w + p.sort, nullptr, 0,
                                  s);
  }
  int32_t *pos = nullptr;
  return sort_and_segments(idx, B, K, N, p.nc, w + p.sort, reinterpret_cast<int32_t *>(w + p.seg), &pos, s);
}

int bwd_workspace(int64_t B, int K, int64_t N, int L, uint32_t flags, size_t *bytes) {
  BwdLayout lay;
  int rc = make_layout(B, K, N, L, flags, lay);
  if (rc != SFT_OK) return rc;
  *bytes = lay.total;
  return SFT_OK;
}

int bwd_f32(const int32_t *idx, int64_t B, int K, const float *grad, int64_t N, int L, float *dW, float *db,
            void *ws, size_t ws_bytes, uint32_t flags, hipStream_t s, void *prep, size_t prep_bytes) {
  BwdLayout lay;
  int rc = make_layout(B, K, N, L, flags, lay);
  if (rc != SFT_OK) return rc;
  if (ws_bytes < lay.total || (lay.total > 0 && ws == nullptr))
    return fail(SFT_EWORKSPACE, "workspace smaller than sft_ft_bwd_f32_workspace_size()");
  if ((uintptr_t)ws % 256 != 0) return fail(SFT_EWORKSPACE, "workspace must be 256-byte aligned");
  char *w = static_cast<char *>(ws);
  const int overwrite = (flags & SFT_BWD_OVERWRITE) ? 1 : 0;
  const int64_t M = B * K;

  // The tiled weight-grad gather reads the grad in column tiles; the bias pass
  // writes that layout while it streams the grad (16-byte loads when the grad
  // allows them, 4-byte loads otherwise), and stores 16-byte weight-grad chunks.
  const bool tiled = !(flags & SFT_BWD_ATOMIC) && M > 0 && tiled_shape(B, L, flags) && (uintptr_t)dW % 16 == 0;
  f32x4 *gt = tiled ? reinterpret_cast<f32x4 *>(w + lay.gt) : nullptr;

  // ---- sort of the slots and their segments: they need only the indices, so
  // they run on the side stream while the bias pass streams the grad ----
  const bool sorted = !(flags & SFT_BWD_ATOMIC) && M > 0;
  const bool prepared = (flags & SFT_BWD_PREPARED) && prep_pays(B, K, L, flags);
  const int nc = tiled ? sort_chunks(B, L, flags) : 1;
  int32_t *seg = reinterpret_cast<int32_t *>(w + lay.seg);
  int32_t *pos = nullptr;
  std::optional<SideJoinGuard> side_join;  // joins the side stream on every early return
  // chunk 0's gather waits for the buckets of chunk 0 only (kChunk0Mark)
  const bool chunk0_split = SFT_BWD_SPLIT_BUCKETS && sorted && prepared && tiled && nc > 1 &&
                            prep_split(B, K, N, L, flags) && slot_sort_buckets_chunk0(N, nc) > 0;
  bool chunk0_marked = false;
  if (sorted && prepared) {
    PrepLayout pl;
    make_prep_layout(B, K, N, L, flags, pl);
    if (prep == nullptr || prep_bytes < pl.total || (uintptr_t)prep % 256 != 0)
      return fail(SFT_EWORKSPACE, "prepared buffer smaller than sft_ft_bwd_f32_prep_size() or not 256-byte aligned");
    // The prepared buffer is only read: a later backward over the same buffer
    // (a graph backward run twice) finds it as the forward left it.  Its sort
    // was made for the chunks of the tiled gather, which only a weight grad
    // that is not 16-byte aligned rules out.
    if (nc != pl.nc)
      return fail(SFT_EINVAL, "sft_ft_bwd_f32_prepared: weight_grad must be 16-byte aligned when the prepared sort "
                              "is in position chunks (batch above 32768 with the tiled gather)");
    char *pw = static_cast<char *>(prep);
    if (prep_split(B, K, N, L, flags)) {
      // the buckets on the side stream, beside the bias pass, from the radix
      // pass the forward left in the prepared buffer, into the workspace
      hipStream_t side;
      if ((rc = fork_side(s, &side)) != SFT_OK) return rc;
      side_join.emplace(s);
      const SegBufs sbs = seg_bufs(seg, nc, N);
      const int64_t crow = nc > 1 ? half_rows(B) : B;
      pos = reinterpret_cast<int32_t *>(w + lay.spos);
      ProfScope prof(kProfBwdSort, side);
      hipLaunchKernelGGL(zero_kernel, dim3(1), dim3(kBlock), 0, side, reinterpret_cast<float *>(sbs.count),
                         (int64_t)nc);  // the long-segment counts (the forward's radix pass left them alone)
      if ((rc = check_launch("long-segment count clear")) != SFT_OK) return rc;
      const int nb0 = chunk0_split ? slot_sort_buckets_chunk0(N, nc) : 0;
      if ((rc = slot_sort_buckets_low(pw + pl.sort, M, N, (int)crow, nc, pos, sbs.seg, sbs.list, sbs.count,
                                      crow <= 65536 ? sbs.pos16 : nullptr, kLongSeg, side, 0,
                                      nb0 > 0 ? nb0 : -1)) != SFT_OK)
        return rc;
      if (nb0 > 0) {
        if ((rc = mark_side(kChunk0Mark)) != SFT_OK) return rc;
        chunk0_marked = true;
        if ((rc = slot_sort_buckets_low(pw + pl.sort, M, N, (int)crow, nc, pos, sbs.seg, sbs.list, sbs.count,
                                        crow <= 65536 ? sbs.pos16 : nullptr, kLongSeg, side, nb0, -1)) != SFT_OK)
          return rc;
      }
    } else {
      seg = reinterpret_cast<int32_t *>(pw + pl.seg);
      pos = slot_sort_positions(M, N, nc, pw + pl.sort);
    }
  } else if (sorted) {
    hipStream_t side;
    if ((rc = fork_side(s, &side)) != SFT_OK) return rc;
    side_join.emplace(s);
    if ((rc = sort_and_segments(idx, B, K, N, nc, w + lay.sort, seg, &pos, side)) != SFT_OK) return rc;
  }
  const SegBufs sb = seg_bufs(seg, nc, N);

  // ---- bias grad ----
  const bool fuse_bias_final = tiled && M > 0 && (L % 4 == 0) && ((uintptr_t)grad % 16 == 0) && ((uintptr_t)db % 16 == 0);
  {
    const bool vec = (L % 4 == 0) && ((uintptr_t)grad % 16 == 0) && ((uintptr_t)db % 16 == 0);
    if ((rc = launch_bias_partial(grad, B, L, lay.nparts, reinterpret_cast<float *>(w + lay.partial), gt, vec, s,
                                  kBwdTileCh)) != SFT_OK)
      return rc;
    // with the tiled gather, its first launch reduces the partials too
    if (!(fuse_bias_final && SFT_BWD_FUSE_BIAS_FINAL) &&
        (rc = launch_bias_final(reinterpret_cast<const float *>(w + lay.partial), lay.nparts, L, db, overwrite, vec,
                                s)) != SFT_OK)
      return rc;
  }
  if (chunk0_marked) {
    // the rest of the buckets still run: joined before chunk 1's gather
    if ((rc = wait_side(s, kChunk0Mark)) != SFT_OK) return rc;
  } else if (side_join) {
    if ((rc = join_side(s)) != SFT_OK) return rc;
    side_join->release();
  }

  if (flags & SFT_BWD_ATOMIC) {
    if (overwrite) {
      const int64_t n = N * (int64_t)L;
      ProfScope prof(kProfBwdZero, s);
      hipLaunchKernelGGL(zero_kernel, dim3((unsigned)std::min<int64_t>(ceil_div(n, kBlock), 1 << 16)), dim3(kBlock),
                         0, s, dW, n);
      if ((rc = check_launch("weight grad zero fill")) != SFT_OK) return rc;
    }
    if (B == 0) return SFT_OK;
    const int kpad = round_up4(K);
    const size_t lds = (size_t)(kWavesPerBlock * kpad + kWavesPerBlock) * sizeof(int);
    if (lds > kMaxIndexLds) return fail(SFT_EUNSUPPORTED, "sft_ft_bwd_f32: max_active too large for the LDS index lists");
    int fpl = (int)std::min<int64_t>(ceil_div(L, kWave), 32);
    const unsigned slabs = (unsigned)ceil_div(L, (int64_t)kWave * fpl);
    const dim3 grid((unsigned)ceil_div(B, kWavesPerBlock), slabs);
    ProfScope prof(kProfBwdAtomic, s);
#define SFT_ATOMIC_CASE(F) \
  hipLaunchKernelGGL(scatter_atomic_kernel<F>, grid, dim3(kBlock), lds, s, idx, B, K, (int)N, grad, (int64_t)L, dW, kpad)
    if (fpl <= 1) SFT_ATOMIC_CASE(1);
    else if (fpl <= 2) SFT_ATOMIC_CASE(2);
    else if (fpl <= 4) SFT_ATOMIC_CASE(4);
    else if (fpl <= 8) SFT_ATOMIC_CASE(8);
    else if (fpl <= 12) SFT_ATOMIC_CASE(12);
    else if (fpl <= 17) SFT_ATOMIC_CASE(17);
    else if (fpl <= 24) SFT_ATOMIC_CASE(24);
    else SFT_ATOMIC_CASE(32);
#undef SFT_ATOMIC_CASE
    return check_launch("atomic scatter");
  }

  // ---- sorted (deterministic) weight grad ----
  if (M == 0) {
    if (!overwrite) return SFT_OK;  // nothing active: dW untouched
    const int64_t n = N * (int64_t)L;  // overwrite with no slots at all: every row is zero
    ProfScope prof(kProfBwdZero, s);
    hipLaunchKernelGGL(zero_kernel, dim3((unsigned)std::min<int64_t>(ceil_div(n, kBlock), 1 << 16)), dim3(kBlock), 0,
                       s, dW, n);
    return check_launch("weight grad zero fill");
  }
  if (tiled) {
    const int64_t cols4 = L / 4;
    const ColMap map = plain_map((int)cols4, kBwdTileCh);
    const int ntiles = map_tiles(map);
    const int ngroups = (int)ceil_div(N, bwd_feat_per_block());
    RowDst dst{};
    dst.n = 1;
    dst.start[1] = N;
    dst.p[0] = reinterpret_cast<f32x4 *>(dW);
    f32x4 *tmp = reinterpret_cast<f32x4 *>(w + lay.tmp);
    const BiasFinal bf{reinterpret_cast<const f32x4 *>(w + lay.partial), lay.nparts, cols4,
                       reinterpret_cast<f32x4 *>(db), overwrite};
    for (int h = 0; h < nc; ++h) {
      if (h == 1 && chunk0_marked) {
        if ((rc = join_side(s)) != SFT_OK) return rc;
        side_join->release();
      }
      ProfScope prof(kProfBwdTiled, s);
      const bool nt = (nc > 1 ? half_rows(B) : B) * kBwdTileCh * 16 >= kNtStoreTileBytes;
      const int64_t crow = nc > 1 ? half_rows(B) : B;
      rc = launch_tiled_gather(nt, seg + (int64_t)h * N, pos, crow <= 65536 ? sb.pos16 : nullptr, h * crow, N, gt, B,
                               map, dst, tmp, h == 0 ? kSrcZero : kSrcTmp, h == nc - 1 ? kDstOut : kDstTmp, ntiles,
                               ngroups, sb.list + h * N, sb.count + h, kLongSlots, s,
                               h == 0 && fuse_bias_final && SFT_BWD_FUSE_BIAS_FINAL ? &bf : nullptr);
      if (rc != SFT_OK) return rc;
    }
    return SFT_OK;
  }
  {
    const bool vec = (L % 4 == 0) && ((uintptr_t)grad % 16 == 0) && ((uintptr_t)dW % 16 == 0);
    const int64_t cols = vec ? L / 4 : L;
    const Mapping m = choose_mapping(cols);
    const int fpb = kWavesPerBlock * (kWave / m.G);
    const int nlong = vec ? kRowLongBlocks : 0;
    const dim3 grid((unsigned)(nlong + ceil_div(N, fpb)), (unsigned)m.slabs);
    ProfScope prof(kProfBwdGather, s);
    if (vec) {
      SFT_G_CASES(launch_gather, f32x4, grid, s, seg, pos, N, grad, cols, dW, overwrite, sb, nlong)
    } else {
      SFT_G_CASES(launch_gather, float, grid, s, seg, pos, N, grad, cols, dW, overwrite, sb, 0)
    }
  }
  return check_launch("feature row gather");
}


// ------------------------------------------- composed table, two perspectives ----
// Workspace: bias partials of both grads | sort buffers | segment starts |
// grad tiles (one perspective at a time) | tmp (sums between position chunks,
// tile-major).
struct PairLayout {
  size_t partial, sort[2], seg[2], gt, tmp, total;
  int nparts, nc;
};

void make_pair_layout(int64_t B, int K, int64_t N, int L, PairLayout &lay) {
  const int64_t M = B * K;
  lay.nparts = bias_parts(B, M > 0);  // both sorts run on the side stream
  lay.nc = sort_chunks(B, L, SFT_BWD_OVERWRITE);
  size_t off = 0;
  lay.partial = off;
  off = align256(off + (size_t)2 * lay.nparts * (size_t)L * sizeof(float));
  for (int p = 0; p < 2; ++p) {  // each perspective sorts into its own buffers
    lay.sort[p] = off;
    off = align256(off + slot_sort_workspace(std::max<int64_t>(M, 1)));
    lay.seg[p] = off;
    off = align256(off + seg_region_bytes(lay.nc, N, M));
  }
  // grad tiles, one perspective at a time: perspective 1's bias pass writes
  // them after perspective 0's gathers have read theirs (same stream)
  lay.gt = off;
  off = align256(off + (size_t)(ceil_div(L, 32) * B * 32) * sizeof(float));
  lay.tmp = off;
  off = align256(off + (size_t)(ceil_div(L, 32) * N * 32) * sizeof(float));
  lay.total = off;
}

size_t bwd_pair_workspace(int64_t B, int K, int64_t N, int L) {
  PairLayout lay;
  make_pair_layout(B, K, N, L, lay);
  return lay.total;
}

// One perspective's slots sorted, with their segments (on the side stream).
struct SortedSlots {
  SegBufs sb;
  int32_t *pos;
};
static int pair_sort_perspective(const int32_t *idx, int64_t B, int K, int64_t N, int nc, char *sort_ws,
                                 int32_t *seg, SortedSlots &out, hipStream_t s) {
  const int64_t M = B * K;
  unsigned *keys = nullptr, *totals = nullptr;
  int ntot = 0, rc;
  out.sb = seg_bufs(seg, nc, N);
  const int64_t crow = nc > 1 ? half_rows(B) : B;
  if (slot_sort_buckets_supported(N, nc)) {
    ProfScope prof(kProfBwdSort, s);
    return slot_sort_buckets(idx, M, K, N, (int)crow, nc, sort_ws, out.sb.seg, out.sb.list, out.sb.count,
                             crow <= 65536 ? out.sb.pos16 : nullptr, kLongSeg, &out.pos, s);
  }
  {
    ProfScope prof(kProfBwdSort, s);
    if ((rc = slot_sort(idx, M, K, N, (int)crow, nc, sort_ws, &keys, &out.pos, &totals, &ntot, out.sb.count, nc,
                        s)) != SFT_OK)
      return rc;
  }
  return launch_segments(keys, M, nc, N, totals, ntot, out.sb, out.pos, crow, s);
}

// One perspective's position-chunk launches of the tiled gather, the sums
// carried between chunks in tmp: perspective 0's last launch stores its sums to
// dst, perspective 1's adds them to dst.
static int pair_gather_perspective(int p, const SortedSlots &ss, int64_t B, int64_t N, const ColMap &map,
                                   const f32x4 *gt, const RowDst &dst, f32x4 *tmp, int nc, hipStream_t s,
                                   const BiasFinal *bias = nullptr) {  // reduced by the first launch
  const int ntiles = map_tiles(map);
  const int ngroups = (int)ceil_div(N, bwd_feat_per_block());
  for (int h = 0; h < nc; ++h) {
    int src_mode, dst_mode;
    src_mode = h == 0 ? kSrcZero : kSrcTmp;
    dst_mode = h < nc - 1 ? kDstTmp : p == 0 ? kDstOut : kDstOutPlus;
    ProfScope prof(kProfBwdTiled, s);
    const bool nt = (nc > 1 ? half_rows(B) : B) * kBwdTileCh * 16 >= kNtStoreTileBytes;
    const int64_t crow = nc > 1 ? half_rows(B) : B;
    const int rc = launch_tiled_gather(nt, ss.sb.seg + (int64_t)h * N, ss.pos, crow <= 65536 ? ss.sb.pos16 : nullptr,
                                       h * crow, N, gt, B, map, dst, tmp, src_mode,
                                       dst_mode, ntiles, ngroups, ss.sb.list + h * N, ss.sb.count + h, kLongSlots, s,
                                       h == 0 ? bias : nullptr);
    if (rc != SFT_OK) return rc;
  }
  return SFT_OK;
}

// Both perspectives' sorts on the side stream, into their own buffers; mark p
// follows perspective p's sort, so its gathers wait for that sort only.
static int pair_sort_both(const int32_t *idx0, const int32_t *idx1, int64_t B, int K, int64_t N, int nc,
                          char *w, const size_t (&sort_off)[2], const size_t (&seg_off)[2], SortedSlots (&ss)[2],
                          hipStream_t s) {
  static_assert(kSideMarks >= 2, "one mark per perspective");
  hipStream_t side;
  int rc = fork_side(s, &side);
  if (rc != SFT_OK) return rc;
  SideJoinGuard side_join(s);
  for (int p = 0; p < 2; ++p) {
    if ((rc = pair_sort_perspective(p == 0 ? idx0 : idx1, B, K, N, nc, w + sort_off[p],
                                    reinterpret_cast<int32_t *>(w + seg_off[p]), ss[p], side)) != SFT_OK)
      return rc;
    if ((rc = mark_side(p)) != SFT_OK) return rc;
  }
  side_join.release();  // the caller waits for each mark before that perspective's gathers
  return SFT_OK;
}

static int virtual_reduce(const float *const *vgrad_src, float *const *vgrad, const int64_t *vperiod,
                          const int64_t *vreps, int nvirt, int64_t cols4, hipStream_t s) {
  for (int v = 0; v < nvirt; ++v) {
    const int64_t total = vperiod[v] * cols4;
    ProfScope prof(kProfBwdVirtual, s);
    hipLaunchKernelGGL(virtual_reduce_kernel, dim3((unsigned)std::min<int64_t>(ceil_div(total, kBlock), 1 << 16)),
                       dim3(kBlock), 0, s, reinterpret_cast<const f32x4 *>(vgrad_src[v]), vperiod[v], (int)vreps[v],
                       cols4, reinterpret_cast<f32x4 *>(vgrad[v]));
    int rc = check_launch("virtual row reduction");
    if (rc != SFT_OK) return rc;
  }
  return SFT_OK;
}

int bwd_pair_f32(const int32_t *idx0, const int32_t *idx1, int64_t B, int K, const float *grad0, const float *grad1,
                 int64_t N, int L, const RowDst &dst, const float *const *vgrad_src, float *const *vgrad,
                 const int64_t *vperiod, const int64_t *vreps, int nvirt, float *db, void *ws, size_t ws_bytes,
                 hipStream_t s) {
  PairLayout lay;
  make_pair_layout(B, K, N, L, lay);
  if (ws_bytes < lay.total || ws == nullptr || (uintptr_t)ws % 256 != 0)
    return fail(SFT_EWORKSPACE, "sft_ft_bwd_pair_f32: workspace smaller than sft_ft_pair_workspace_size() "
                                "or not 256-byte aligned");
  char *w = static_cast<char *>(ws);
  const ColMap map = plain_map(L / 4);
  float *partial = reinterpret_cast<float *>(w + lay.partial);
  f32x4 *gt = reinterpret_cast<f32x4 *>(w + lay.gt);
  f32x4 *tmp = reinterpret_cast<f32x4 *>(w + lay.tmp);
  SortedSlots ss[2];
  int rc = pair_sort_both(idx0, idx1, B, K, N, lay.nc, w, lay.sort, lay.seg, ss, s);
  if (rc != SFT_OK) return rc;
  SideJoinGuard side_join(s);  // until both marks are waited for
  // Each perspective's bias pass (which also writes its grad tiles) right
  // before its gathers, the sorts on the side stream meanwhile: both bias
  // passes first, beside both sorts, took 133 against 107 us each (composed
  // HalfKAv2_hm^ step 1.752 -> 1.740 ms, Full_Threats+HalfKAv2_hm^ 6.988 ->
  // 6.951 ms).
  // the bias reduction over both perspectives' partials rides in perspective
  // 1's first gather launch
  const BiasFinal bf{reinterpret_cast<const f32x4 *>(partial), 2 * lay.nparts, L / 4, reinterpret_cast<f32x4 *>(db), 1};
  for (int p = 0; p < 2; ++p) {
    const float *grad = p == 0 ? grad0 : grad1;
    if ((rc = launch_bias_partial(grad, B, L, lay.nparts, partial + (size_t)p * lay.nparts * L, gt, true, s)) !=
        SFT_OK)
      return rc;
    if ((rc = wait_side(s, p)) != SFT_OK) return rc;
    if ((rc = pair_gather_perspective(p, ss[p], B, N, map, gt, dst, tmp, lay.nc, s,
                                      p == 1 && SFT_BWD_FUSE_BIAS_FINAL ? &bf : nullptr)) != SFT_OK)
      return rc;
  }
  side_join.release();
  if (!SFT_BWD_FUSE_BIAS_FINAL && (rc = launch_bias_final(partial, 2 * lay.nparts, L, db, 1, true, s)) != SFT_OK)
    return rc;
  return virtual_reduce(vgrad_src, vgrad, vperiod, vreps, nvirt, L / 4, s);
}

// ------------------------------------------- composed table + post-FT epilogue ----
// Workspace: bias partials | sort buffers | segment starts | grad tiles of both
// perspectives (paired map) | tmp (tile-major, paired map).
struct TransformLayout {
  size_t partial, sort[2], seg[2], gt0, gt1, tmp, total;
  int nparts, nc;
};

void make_transform_layout(int64_t B, int K, int64_t N, int L, int L1, TransformLayout &lay) {
  const ColMap map = paired_map(L / 4, L1 / 8);
  const int64_t M = B * K;
  lay.nparts = (int)std::max<int64_t>(1, ceil_div(B, kEpiRows));
  lay.nc = sort_chunks(B, L, SFT_BWD_OVERWRITE);
  const size_t gtb = (size_t)map_tiles(map) * (size_t)B * 128;
  size_t off = 0;
  lay.partial = off;
  off = align256(off + (size_t)lay.nparts * (size_t)L * sizeof(float));
  for (int p = 0; p < 2; ++p) {
    lay.sort[p] = off;
    off = align256(off + slot_sort_workspace(std::max<int64_t>(M, 1)));
    lay.seg[p] = off;
    off = align256(off + seg_region_bytes(lay.nc, N, M));
  }
  lay.gt0 = off;
  off = align256(off + gtb);
  lay.gt1 = off;
  off = align256(off + gtb);
  lay.tmp = off;
  off = align256(off + (size_t)map_tiles(map) * (size_t)N * 128);
  lay.total = off;
}

size_t bwd_transform_workspace(int64_t B, int K, int64_t N, int L, int L1) {
  TransformLayout lay;
  make_transform_layout(B, K, N, L, L1, lay);
  return lay.total;
}

int bwd_transform_f32(const int32_t *idx0, const int32_t *idx1, int64_t B, int K, const float *g_l0,
                      const float *g_psqt, const float *us, const int64_t *psqt_idx, const void *saved,
                      size_t saved_bytes, int64_t N, int L, int L1, const RowDst &dst, const float *const *vgrad_src,
                      float *const *vgrad, const int64_t *vperiod, const int64_t *vreps, int nvirt, float *db,
                      void *ws, size_t ws_bytes, hipStream_t s) {
  TransformLayout lay;
  make_transform_layout(B, K, N, L, L1, lay);
  const ColMap map = paired_map(L / 4, L1 / 8);
  const size_t raw_bytes = (size_t)map_tiles(map) * (size_t)B * 128;
  if (ws_bytes < lay.total || ws == nullptr || (uintptr_t)ws % 256 != 0 || saved == nullptr ||
      saved_bytes < 2 * raw_bytes || (uintptr_t)saved % 256 != 0)
    return fail(SFT_EWORKSPACE, "sft_ft_bwd_transform_f32: saved or workspace buffer smaller than "
                                "sft_ft_transform_workspace_size() or not 256-byte aligned");
  char *w = static_cast<char *>(ws);
  f32x4 *gt0 = reinterpret_cast<f32x4 *>(w + lay.gt0), *gt1 = reinterpret_cast<f32x4 *>(w + lay.gt1);
  BwdEpilogue e;
  e.g_l0 = g_l0;
  e.g_psqt = g_psqt;
  e.us = us;
  e.psqt_idx = psqt_idx;
  e.raw0 = static_cast<const f32x4 *>(saved);
  e.raw1 = reinterpret_cast<const f32x4 *>(static_cast<const char *>(saved) + raw_bytes);
  e.gt0 = gt0;
  e.gt1 = gt1;
  e.partial = reinterpret_cast<f32x4 *>(w + lay.partial);
  e.P = L - L1;
  SortedSlots ss[2];  // sorted on the side stream while the epilogue runs
  int rc = pair_sort_both(idx0, idx1, B, K, N, lay.nc, w, lay.sort, lay.seg, ss, s);
  if (rc != SFT_OK) return rc;
  SideJoinGuard side_join(s);  // until both marks are waited for
  {
    ProfScope prof(kProfBwdEpilogue, s);
    hipLaunchKernelGGL(bwd_epilogue_kernel, dim3((unsigned)lay.nparts), dim3(kBlock), 0, s, e, map, B,
                       map_tiles(map));
    if ((rc = check_launch("epilogue backward")) != SFT_OK) return rc;
  }
  // the bias reduction rides in perspective 0's first gather launch
  const BiasFinal bf{reinterpret_cast<const f32x4 *>(w + lay.partial), lay.nparts, L / 4,
                     reinterpret_cast<f32x4 *>(db), 1};
  if (!SFT_BWD_FUSE_BIAS_FINAL &&
      (rc = launch_bias_final(reinterpret_cast<const float *>(w + lay.partial), lay.nparts, L, db, 1, true, s)) !=
          SFT_OK)
    return rc;
  f32x4 *tmp = reinterpret_cast<f32x4 *>(w + lay.tmp);
  for (int p = 0; p < 2; ++p) {
    if ((rc = wait_side(s, p)) != SFT_OK) return rc;
    if ((rc = pair_gather_perspective(p, ss[p], B, N, map, p == 0 ? gt0 : gt1, dst, tmp, lay.nc, s,
                                      p == 0 && SFT_BWD_FUSE_BIAS_FINAL ? &bf : nullptr)) != SFT_OK)
      return rc;
  }
  side_join.release();
  return virtual_reduce(vgrad_src, vgrad, vperiod, vreps, nvirt, L / 4, s);
}

void zero_f32(float *p, int64_t n, hipStream_t s) {
  if (n <= 0) return;
  ProfScope prof(kProfBwdZero, s);
  hipLaunchKernelGGL(zero_kernel, dim3((unsigned)std::min<int64_t>(ceil_div(n, kBlock), 1 << 16)), dim3(kBlock), 0, s,
                     p, n);
}

}  // namespace sft
