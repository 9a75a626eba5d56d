// Stable LSD radix sort of the backward's flat index slots, for gfx950.
//
// Sorts the active slots s = b*K + k (0 <= idx[s] < N) by key
// chunk(b) * N + feature, carrying the slot's position b, stably, so each
// key's positions come out in ascending order; inactive slots are dropped by
// the first pass.  RB-bit digits (8, or 9 when two 9-bit passes cover a key
// that 8-bit digits would need three for), least significant first; each pass:
//   upsweep:   per 2048-slot tile, a 2^RB-bin digit histogram;
//   scan:      per digit, an exclusive scan of its tile counts and the digit
//              total; a digit's base is the scan of the totals (done in the
//              downsweep), so (digit, tile) starts at base + its tile prefix;
//   downsweep: per tile, stable ranks (digit-major, then slot order) from
//              wave-wide match masks (RB ballots) and per-wave digit counts,
//              the tile reordered in LDS, then written out as contiguous runs.
// The first pass reads the keys straight from the index matrix.  Passes after
// the first, and the segment-offset kernel, take the number of active slots
// from the previous scan's digit totals, on the device.
#include <algorithm>

#include "common.h"

namespace sft {

namespace {

// Slots per thread of a sort tile: 8 (2048-slot tiles) for up to kBigSort
// slots, 16 above, where fewer tiles shrink the per-tile digit counts the
// scans walk (10.5 M slots: 278 -> 226 us per sort).  Alone, a 2.1 M-slot sort
// was faster with 8 (65 vs 72 us), but beside the kernels it shares the GPU
// with the steps are faster with 16 at every batch: B = 65536, L = 1048 1.671
// -> 1.666 ms, L = 136 0.378 -> 0.376 ms, B = 16384 0.575 -> 0.574 ms (A/B
// builds, same box), so the threshold is 0.
constexpr int kSortItems = 8;
constexpr int kSortItemsBig = 16;
#ifndef SFT_SORT_BIG_SLOTS
#define SFT_SORT_BIG_SLOTS 0
#endif
constexpr int64_t kBigSort = SFT_SORT_BIG_SLOTS;
constexpr int kSortTile = kBlock * kSortItems;  // the smaller tile: sizes the count buffer
constexpr int kMaxRadix = 1024;  // 10-bit digits (the bucket sort's first pass)
#ifndef SFT_SORT_BUCKETS
#define SFT_SORT_BUCKETS 1
#endif

// FastDiv (index_math.h): n / d by a divisor fixed at launch.

// Key of slot s (s < 2^31): chunk(b) * N + feature for an active slot, the
// sentinel (>= every real key) for an inactive one; the value is b = s / K.
struct SlotKey {
  const int32_t *idx;
  unsigned N;
  FastDiv divK, divChunk;
  unsigned sentinel;
  __device__ __forceinline__ unsigned key(int64_t s) const { return key_of(s, (unsigned)idx[s]); }
  // The key of slot s from its loaded index value v (loads issued apart from
  // the arithmetic, whose divisor checks are branches the loads do not cross).
  __device__ __forceinline__ unsigned key_of(int64_t s, unsigned v) const {
    return v < N ? divChunk(divK((uint32_t)s)) * N + v : sentinel;
  }
  __device__ __forceinline__ int pos(int64_t s) const { return (int)divK((uint32_t)s); }
};

// Number of elements a pass reads: all slots for the first pass, else the
// active count = sum of the previous scan's digit totals (block-wide sum).
template <int R>
__device__ __forceinline__ int64_t pass_count(bool first, int64_t M, const unsigned *__restrict__ totals,
                                              unsigned *red) {
  if (first) return M;
  const int tid = threadIdx.x;
  unsigned v = 0;
  for (int d = tid; d < R; d += kBlock) v += totals[d];
  red[tid] = v;
  __syncthreads();
  for (int off = kBlock / 2; off > 0; off >>= 1) {
    if (tid < off) red[tid] += red[tid + off];
    __syncthreads();
  }
  const int64_t n = red[0];
  __syncthreads();
  return n;
}

// Lanes of the wave holding the same digit as this lane (among `valid` lanes).
template <int RB>
__device__ __forceinline__ uint64_t match_digit(unsigned d, bool valid) {
  uint64_t peers = ballot(valid);
#pragma unroll
  for (int b = 0; b < RB; ++b) {
    const bool bit = (d >> b) & 1u;
    const uint64_t m = ballot(bit);
    peers &= bit ? m : ~m;
  }
  return peers;
}

template <int RB, bool FIRST, int IT>
__global__ __launch_bounds__(kBlock) void radix_upsweep(SlotKey sk, const unsigned *__restrict__ kin, int64_t M,
                                                        const unsigned *__restrict__ prev_totals, int ntiles,
                                                        int shift, unsigned *__restrict__ hist) {
  constexpr int R = 1 << RB;
  __shared__ unsigned hw[kWavesPerBlock][R];
  __shared__ unsigned red[kBlock];
  const int tid = threadIdx.x, wave = tid / kWave;
  for (int d = tid; d < R; d += kBlock)
#pragma unroll
    for (int w = 0; w < kWavesPerBlock; ++w) hw[w][d] = 0;
  const int64_t count = pass_count<R>(FIRST, M, prev_totals, red);
  __syncthreads();
  const int64_t base = (int64_t)blockIdx.x * (kBlock * IT);
  if (count > 0) {  // block-uniform
    // Every load first, from indices clamped into range (an out-of-range
    // element loads a real one and is not counted): guarded loads compile to a
    // branch and a full wait per load, a memory round trip per element.
    unsigned k[IT];
#pragma unroll
    for (int i = 0; i < IT; ++i) {
      const int64_t e = std::min<int64_t>(base + (int64_t)i * kBlock + tid, count - 1);
      k[i] = FIRST ? (unsigned)sk.idx[e] : kin[e];
    }
#pragma unroll
    for (int i = 0; i < IT; ++i) {
      const int64_t e = base + (int64_t)i * kBlock + tid;
      if (FIRST) k[i] = sk.key_of(std::min<int64_t>(e, count - 1), k[i]);
      if (e < count && (!FIRST || k[i] < sk.sentinel)) atomicAdd(&hw[wave][(k[i] >> shift) & (R - 1)], 1u);
    }
  }
  __syncthreads();
  for (int d = tid; d < R; d += kBlock)
    hist[(int64_t)d * ntiles + blockIdx.x] = hw[0][d] + hw[1][d] + hw[2][d] + hw[3][d];
}

// Per digit d (one block each): exclusive scan of hist[d][0 .. ntiles) in
// place, and the digit's total into totals[d].
__global__ __launch_bounds__(kBlock) void radix_scan_digits(unsigned *__restrict__ hist, int ntiles,
                                                            unsigned *__restrict__ totals, int *__restrict__ clear,
                                                            int nclear) {
  __shared__ unsigned part[kBlock];
  const int tid = threadIdx.x;
  if (blockIdx.x == 0)  // the caller's counters, zeroed here to save a launch
    for (int i = tid; i < nclear; i += kBlock) clear[i] = 0;
  unsigned *h = hist + (int64_t)blockIdx.x * ntiles;
  const int per = (ntiles + kBlock - 1) / kBlock;
  const int lo = std::min(ntiles, tid * per), hi = std::min(ntiles, lo + per);
  unsigned s = 0;
  for (int i = lo; i < hi; ++i) s += h[i];
  part[tid] = s;
  __syncthreads();
  for (int off = 1; off < kBlock; off <<= 1) {  // Hillis-Steele inclusive scan
    const unsigned v = tid >= off ? part[tid - off] : 0u;
    __syncthreads();
    part[tid] += v;
    __syncthreads();
  }
  unsigned run = part[tid] - s;
  for (int i = lo; i < hi; ++i) {
    const unsigned v = h[i];
    h[i] = run;
    run += v;
  }
  if (tid == kBlock - 1) totals[blockIdx.x] = part[tid];
}

// The same scan for up to kBlock * PER tiles: thread t holds the counts of
// tiles t, t + 256, ... (coalesced, all loaded before any is used), a row of
// 256 tiles is scanned with wave shuffles and one exchange of the wave totals,
// and row j starts after the totals of rows 0 .. j-1.  (The loop above reads
// each thread's run of counts one load after another and scans with 16
// barriers: 16 us per call beside the bias pass at 1 024 tiles.)
template <int PER>
__global__ __launch_bounds__(kBlock) void radix_scan_digits_rows(unsigned *__restrict__ hist, int ntiles,
                                                                 unsigned *__restrict__ totals,
                                                                 int *__restrict__ clear, int nclear) {
  __shared__ unsigned wsum[PER][kWavesPerBlock];
  const int tid = threadIdx.x, lane = tid % kWave, wave = tid / kWave;
  if (blockIdx.x == 0)  // the caller's counters, zeroed here to save a launch
    for (int i = tid; i < nclear; i += kBlock) clear[i] = 0;
  unsigned *h = hist + (int64_t)blockIdx.x * ntiles;
  unsigned v[PER], incl[PER];
#pragma unroll
  for (int j = 0; j < PER; ++j) v[j] = h[std::min(j * kBlock + tid, ntiles - 1)];
#pragma unroll
  for (int j = 0; j < PER; ++j) {
    if (j * kBlock + tid >= ntiles) v[j] = 0u;
    incl[j] = v[j];
#pragma unroll
    for (int off = 1; off < kWave; off <<= 1) {
      const unsigned o = __shfl_up(incl[j], off);
      if (lane >= off) incl[j] += o;
    }
    if (lane == kWave - 1) wsum[j][wave] = incl[j];
  }
  __syncthreads();
  unsigned rowbase = 0;
#pragma unroll
  for (int j = 0; j < PER; ++j) {
    unsigned before = 0, row = 0;
#pragma unroll
    for (int w = 0; w < kWavesPerBlock; ++w) {
      const unsigned x = wsum[j][w];
      row += x;
      before += w < wave ? x : 0u;
    }
    const int i = j * kBlock + tid;
    if (i < ntiles) h[i] = rowbase + before + incl[j] - v[j];
    rowbase += row;
  }
  if (tid == 0) totals[blockIdx.x] = rowbase;
}

// Exclusive scan of the per-tile counts of each of the nr digits, their totals.
static void launch_scan_digits(int nr, unsigned *hist, int ntiles, unsigned *totals, int *clear, int nclear,
                               hipStream_t s) {
  const int per = (ntiles + kBlock - 1) / kBlock;
#define SFT_SCAN_ROWS(P) \
  hipLaunchKernelGGL(radix_scan_digits_rows<P>, dim3(nr), dim3(kBlock), 0, s, hist, ntiles, totals, clear, nclear)
  if (per <= 2) SFT_SCAN_ROWS(2);
  else if (per <= 4) SFT_SCAN_ROWS(4);
  else if (per <= 8) SFT_SCAN_ROWS(8);
  else if (per <= 16) SFT_SCAN_ROWS(16);
  else hipLaunchKernelGGL(radix_scan_digits, dim3(nr), dim3(kBlock), 0, s, hist, ntiles, totals, clear, nclear);
#undef SFT_SCAN_ROWS
}

// Exclusive scan of R per-digit values by one wave (R / 64 digits per lane).
template <int R>
__device__ __forceinline__ void wave_scan_digits(const unsigned *in, unsigned *out, int lane) {
  constexpr int PER = R / kWave;
  unsigned c[PER];
  unsigned s = 0;
#pragma unroll
  for (int j = 0; j < PER; ++j) {
    c[j] = in[lane * PER + j];
    s += c[j];
  }
  unsigned incl = s;
#pragma unroll
  for (int off = 1; off < kWave; off <<= 1) {
    const unsigned v = __shfl_up(incl, off);
    if (lane >= off) incl += v;
  }
  unsigned run = incl - s;
#pragma unroll
  for (int j = 0; j < PER; ++j) {
    out[lane * PER + j] = run;
    run += c[j];
  }
}

// Tile layout: wave w owns the contiguous quarter [w * PER_WAVE, (w + 1) *
// PER_WAVE) of the tile and walks it in 64-slot rounds, so (wave, round, lane) is slot
// order.  Each wave ranks its elements with its own digit counters (no block
// barrier inside the loop); afterwards a digit's rank base for wave w is the
// count of that digit in waves 0 .. w-1.
template <int RB, bool FIRST, int IT>
__global__ __launch_bounds__(kBlock) void radix_downsweep(SlotKey sk, const unsigned *__restrict__ kin,
                                                          const int *__restrict__ vin, unsigned *__restrict__ kout,
                                                          int *__restrict__ vout, const unsigned *__restrict__ offs,
                                                          const unsigned *__restrict__ totals, int64_t M, int ntiles,
                                                          int shift) {
  constexpr int R = 1 << RB;
  constexpr int TILE = kBlock * IT;
  constexpr int PER_WAVE = TILE / kWavesPerBlock;
  __shared__ unsigned s_keys[TILE];
  __shared__ int s_vals[TILE];
  __shared__ unsigned wrun[kWavesPerBlock][R];
  __shared__ unsigned dstart[R];
  __shared__ unsigned dtot[R];
  __shared__ unsigned dbase[R];
  const int tid = threadIdx.x, lane = tid % kWave, wave = tid / kWave;
  for (int d = tid; d < R; d += kBlock) {
    dtot[d] = totals[d];
#pragma unroll
    for (int w = 0; w < kWavesPerBlock; ++w) wrun[w][d] = 0;
  }
  __syncthreads();
  if (wave == 1) wave_scan_digits<R>(dtot, dbase, lane);  // digit bases in the whole output
  __syncthreads();
  // Elements read by this pass: all slots (first pass) or the active ones,
  // whose count is the sum of this pass's digit totals.
  const int64_t n_in = FIRST ? M : (int64_t)dbase[R - 1] + dtot[R - 1];
  const int64_t base = (int64_t)blockIdx.x * TILE + (int64_t)wave * PER_WAVE;

  unsigned key[IT];
  int val[IT];
  unsigned rank[IT];
  bool act[IT];
  // loads from clamped indices, all issued before any is used (see the upsweep)
  const int64_t last = n_in > 0 ? n_in - 1 : 0;
#pragma unroll
  for (int i = 0; i < IT; ++i) {
    const int64_t ec = std::min<int64_t>(base + (int64_t)i * kWave + lane, last);
    key[i] = FIRST ? (unsigned)sk.idx[ec] : kin[ec];
    if (!FIRST) val[i] = vin[ec];
  }
#pragma unroll
  for (int i = 0; i < IT; ++i) {
    const int64_t e = base + (int64_t)i * kWave + lane;
    const int64_t ec = std::min<int64_t>(e, last);
    if (FIRST) {
      key[i] = sk.key_of(ec, key[i]);
      val[i] = sk.pos(ec);
    }
    act[i] = e < n_in && (!FIRST || key[i] < sk.sentinel);
  }
  unsigned *my = wrun[wave];
#pragma unroll
  for (int i = 0; i < IT; ++i) {
    const unsigned d = (key[i] >> shift) & (R - 1);
    const uint64_t peers = match_digit<RB>(d, act[i]);
    if (act[i]) rank[i] = my[d] + (unsigned)popc_below(peers);
    __builtin_amdgcn_wave_barrier();
    if (act[i] && (int)(__ffsll((unsigned long long)peers) - 1) == lane) my[d] += (unsigned)__popcll(peers);
    __builtin_amdgcn_wave_barrier();
  }
  __syncthreads();
  // Per digit: counts of earlier waves (rank bases) and the tile total.
  for (int d = tid; d < R; d += kBlock) {
    unsigned run = 0;
#pragma unroll
    for (int w = 0; w < kWavesPerBlock; ++w) {
      const unsigned c = wrun[w][d];
      wrun[w][d] = run;
      run += c;
    }
    dtot[d] = run;  // reuse: digit count of this tile
  }
  __syncthreads();
  if (wave == 0) wave_scan_digits<R>(dtot, dstart, lane);
  __syncthreads();
#pragma unroll
  for (int i = 0; i < IT; ++i) {
    if (act[i]) {
      const unsigned d = (key[i] >> shift) & (R - 1);
      const unsigned p = dstart[d] + my[d] + rank[i];
      s_keys[p] = key[i];
      s_vals[p] = val[i];
    }
  }
  const int kept = (int)(dstart[R - 1] + dtot[R - 1]);  // active elements of the tile
  __syncthreads();

  for (int j = tid; j < kept; j += kBlock) {
    const unsigned k = s_keys[j];
    const unsigned d = (k >> shift) & (R - 1);
    const int64_t dst = (int64_t)dbase[d] + offs[(int64_t)d * ntiles + blockIdx.x] + (j - dstart[d]);
    kout[dst] = k;
    vout[dst] = s_vals[j];
  }
}

size_t align256(size_t v) { return (v + 255) & ~(size_t)255; }

unsigned key_bits(int64_t maxkey) {
  unsigned bits = 1;
  while (((int64_t)1 << bits) <= maxkey) ++bits;  // keys lie in [0, maxkey]
  return bits;
}

template <int RB, int IT>
int run_passes(const SlotKey &sk, int64_t M, int passes, unsigned *kbuf[2], int *vbuf[2], unsigned *hist,
               unsigned *totals, int ntiles, int *clear, int nclear, hipStream_t s) {
  for (int p = 0; p < passes; ++p) {
    const int shift = p * RB;
    const unsigned *kin = p == 0 ? nullptr : kbuf[(p - 1) & 1];
    const int *vin = p == 0 ? nullptr : vbuf[(p - 1) & 1];
    unsigned *kout = kbuf[p & 1];
    int *vout = vbuf[p & 1];
    if (p == 0)
      hipLaunchKernelGGL((radix_upsweep<RB, true, IT>), dim3(ntiles), dim3(kBlock), 0, s, sk, kin, M, totals, ntiles,
                         shift, hist);
    else
      hipLaunchKernelGGL((radix_upsweep<RB, false, IT>), dim3(ntiles), dim3(kBlock), 0, s, sk, kin, M, totals, ntiles,
                         shift, hist);
    launch_scan_digits(1 << RB, hist, ntiles, totals, clear, p == 0 ? nclear : 0, s);
    if (p == 0)
      hipLaunchKernelGGL((radix_downsweep<RB, true, IT>), dim3(ntiles), dim3(kBlock), 0, s, sk, kin, vin, kout, vout,
                         hist, totals, M, ntiles, shift);
    else
      hipLaunchKernelGGL((radix_downsweep<RB, false, IT>), dim3(ntiles), dim3(kBlock), 0, s, sk, kin, vin, kout, vout,
                         hist, totals, M, ntiles, shift);
    const int rc = check_launch("slot radix sort");
    if (rc != SFT_OK) return rc;
  }
  return SFT_OK;
}

// ---- bucket sort: one radix pass on the high key bits, then each bucket in one workgroup ----
// Pass 1 (the radix kernels above, one pass, digit = key >> SB) leaves the
// active slots grouped by bucket b = key >> SB, in slot order within a bucket.
// Pass 2 sorts each bucket by its low SB bits with one workgroup: a digit
// histogram gives the bucket's segment starts seg[key] = bucket start + the
// count of smaller low digits (no neighbour comparisons), its long segments,
// and then, tile by tile in slot order, stable ranks (per-wave match masks, as
// the downsweep) place each slot's position and its 16-bit chunk offset.  The
// order is the same as the LSD passes' (stable by key), so the backward that
// reads it is bit-identical.  Buckets hold ~4-10 K slots at the FT's shapes.
constexpr int kBucketBlock = 512;
constexpr int kBucketWaves = kBucketBlock / kWave;
// (8 per thread, tiles of 4096 and half the LDS: steps 1.665 -> 1.670 ms at
// L = 1048 and 0.375 -> 0.379 ms at L = 136, B = 65536; even at B = 16384.)
#ifndef SFT_BUCKET_ITEMS
#define SFT_BUCKET_ITEMS 16
#endif
constexpr int kBucketItems = SFT_BUCKET_ITEMS;  // slots per thread per tile: tiles of 8192
template <int SB>
__global__ __launch_bounds__(kBucketBlock) void bucket_sort_kernel(
    const unsigned *__restrict__ kin, const int *__restrict__ vin, const unsigned *__restrict__ totals, int ntot,
    unsigned nkeys, FastDiv div_feat, unsigned nfeat, int *__restrict__ vout, uint16_t *__restrict__ pos16,
    int chunk_rows, int32_t *__restrict__ seg, int32_t *__restrict__ long_list, int *__restrict__ long_count,
    int long_period, int b0) {
  constexpr int D = 1 << SB;
  constexpr int TILE = kBucketBlock * kBucketItems;
  constexpr int PER_WAVE = TILE / kBucketWaves;
  __shared__ unsigned red[2][kBucketWaves];
  __shared__ unsigned s_cnt[D], s_run[D], s_tile[D], s_trun[D];
  __shared__ unsigned wrun[kBucketWaves][D];
  __shared__ int s_val[TILE];  // a tile in sorted order: positions, digits, chunk offsets
  __shared__ uint8_t s_dig[TILE];
  __shared__ uint16_t s_p16[TILE];
  const int tid = threadIdx.x, lane = tid % kWave, wave = tid / kWave;
  const int b = (int)blockIdx.x + b0;  // bucket
  // bucket start (digit totals of the buckets before b) and the active total
  unsigned before = 0, all = 0;
  for (int i = tid; i < ntot; i += kBucketBlock) {
    const unsigned v = totals[i];
    all += v;
    before += i < b ? v : 0u;
  }
#pragma unroll
  for (int m = 1; m < kWave; m <<= 1) {
    all += __shfl_xor(all, m);
    before += __shfl_xor(before, m);
  }
  if (lane == 0) {
    red[0][wave] = before;
    red[1][wave] = all;
  }
  for (int d = tid; d < D; d += kBucketBlock) s_cnt[d] = 0;
  __syncthreads();
  unsigned bs = 0, total = 0;
#pragma unroll
  for (int w = 0; w < kBucketWaves; ++w) {
    bs += red[0][w];
    total += red[1][w];
  }
  const unsigned S = totals[b];
  // A tile's slots: wave w owns the w-th contiguous eighth, walked in 64-slot
  // rounds, so (wave, round, lane) is slot order.
  unsigned key[kBucketItems], rank[kBucketItems];
  int val[kBucketItems];
  bool act[kBucketItems];
  unsigned *my = wrun[wave];
  // loads from clamped indices, all issued before any is used (see the
  // upsweep); an empty bucket loads nothing
  auto load_tile = [&](unsigned t0, bool vals) {
#pragma unroll
    for (int i = 0; i < kBucketItems; ++i) {
      const unsigned e = t0 + (unsigned)(wave * PER_WAVE + i * kWave + lane);
      act[i] = e < S;
      const unsigned ec = bs + (e < S ? e : S - 1);
      key[i] = S > 0 ? kin[ec] : 0u;
      if (vals) val[i] = S > 0 ? vin[ec] : 0;
    }
  };
  // Stable ranks of the tile in registers among its equal low digits, per
  // wave (match masks), the wave's digit counts left in wrun[wave].
  auto rank_tile = [&]() {
#pragma unroll
    for (int i = 0; i < kBucketItems; ++i) {
      const unsigned d = key[i] & (D - 1);
      const uint64_t peers = match_digit<SB>(d, act[i]);
      if (act[i]) rank[i] = my[d] + (unsigned)popc_below(peers);
      __builtin_amdgcn_wave_barrier();
      if (act[i] && (int)(__ffsll((unsigned long long)peers) - 1) == lane) my[d] += (unsigned)__popcll(peers);
      __builtin_amdgcn_wave_barrier();
    }
  };
  // Per digit: wrun becomes the earlier waves' counts, s_tile the tile's count.
  auto wave_bases = [&]() {
    for (int d = tid; d < D; d += kBucketBlock) {
      unsigned run = 0;
#pragma unroll
      for (int w = 0; w < kBucketWaves; ++w) {
        const unsigned c = wrun[w][d];
        wrun[w][d] = run;
        run += c;
      }
      s_tile[d] = run;
    }
  };
  // The tile in sorted order in LDS (j = the digit's start in the tile + the
  // earlier waves' count + the rank), then copied out: slot j of digit d goes
  // to bs + s_run[d] + (j - s_trun[d]), so runs of one digit are stored by
  // consecutive lanes (a one-tile bucket is one contiguous stretch) instead of
  // each lane storing to a line of its own.
  auto place_tile = [&](unsigned n) {
#pragma unroll
    for (int i = 0; i < kBucketItems; ++i) {
      if (!act[i]) continue;
      const unsigned d = key[i] & (D - 1);
      const unsigned j = s_trun[d] + my[d] + rank[i];
      s_val[j] = val[i];
      s_dig[j] = (uint8_t)d;
      if (pos16 != nullptr) s_p16[j] = (uint16_t)(val[i] - (int)div_feat(key[i]) * chunk_rows);
    }
    __syncthreads();
    for (unsigned j = tid; j < n; j += kBucketBlock) {
      const unsigned d = s_dig[j];
      const unsigned o = bs + s_run[d] + (j - s_trun[d]);
      vout[o] = s_val[j];
      if (pos16 != nullptr) pos16[o] = s_p16[j];
    }
  };
  for (int d = tid; d < D; d += kBucketBlock)
#pragma unroll
    for (int w = 0; w < kBucketWaves; ++w) wrun[w][d] = 0;
  // the digit counts of tiles after the first (buckets of more than one tile):
  // their keys loaded whole, then counted
  for (unsigned t0 = TILE; t0 < S; t0 += TILE) {  // block-uniform
    load_tile(t0, false);
#pragma unroll
    for (int i = 0; i < kBucketItems; ++i)
      if (act[i]) atomicAdd(&s_cnt[key[i] & (D - 1)], 1u);
  }
  // the first tile: ranked at once, its counts from the ranking
  load_tile(0, true);
  __syncthreads();
  rank_tile();
  __syncthreads();
  wave_bases();
  __syncthreads();
  for (int d = tid; d < D; d += kBucketBlock) s_cnt[d] += s_tile[d];
  __syncthreads();
  if (wave == 0) wave_scan_digits<D>(s_cnt, s_run, lane);
  if (wave == 1) wave_scan_digits<D>(s_tile, s_trun, lane);
  __syncthreads();
  // segment starts and long segments of the bucket's keys
  for (int d = tid; d < D; d += kBucketBlock) {
    const unsigned k = (unsigned)b * D + d;
    if (k >= nkeys) continue;
    const int64_t s0 = (int64_t)bs + s_run[d], s1 = s0 + s_cnt[d];
    seg[k] = (int32_t)s0;
    if (long_segment(s0, s1, long_period)) {
      const unsigned c = div_feat(k);
      const int at = atomicAdd(long_count + c, 1);
      long_list[(int64_t)c * nfeat + at] = (int32_t)(k - c * nfeat);
    }
  }
  if (b == 0 && tid == 0) seg[nkeys] = (int32_t)total;
  place_tile(S < (unsigned)TILE ? S : (unsigned)TILE);
  // the other tiles, in order
  for (unsigned t0 = TILE; t0 < S; t0 += TILE) {  // block-uniform
    __syncthreads();
    for (int d = tid; d < D; d += kBucketBlock) {
      s_run[d] += s_tile[d];
#pragma unroll
      for (int w = 0; w < kBucketWaves; ++w) wrun[w][d] = 0;
    }
    load_tile(t0, true);
    __syncthreads();
    rank_tile();
    __syncthreads();
    wave_bases();
    __syncthreads();
    if (wave == 0) wave_scan_digits<D>(s_tile, s_trun, lane);
    __syncthreads();
    place_tile(S - t0 < (unsigned)TILE ? S - t0 : (unsigned)TILE);
  }
}

// One radix pass on bits [shift, shift + RB) of the keys built from the index
// matrix (the first pass of run_passes).
template <int RB, int IT>
int run_high_pass(const SlotKey &sk, int64_t M, int shift, unsigned *kout, int *vout, unsigned *hist,
                  unsigned *totals, int ntiles, int *clear, int nclear, hipStream_t s) {
  hipLaunchKernelGGL((radix_upsweep<RB, true, IT>), dim3(ntiles), dim3(kBlock), 0, s, sk, nullptr, M, totals, ntiles,
                     shift, hist);
  launch_scan_digits(1 << RB, hist, ntiles, totals, clear, nclear, s);
  hipLaunchKernelGGL((radix_downsweep<RB, true, IT>), dim3(ntiles), dim3(kBlock), 0, s, sk, nullptr, nullptr, kout,
                     vout, hist, totals, M, ntiles, shift);
  return check_launch("slot bucket sort (first pass)");
}

}  // namespace

// Workspace: two key/position buffer pairs (ping-pong), the histograms and
// the digit totals (the active-slot count is their sum).
size_t slot_sort_workspace(int64_t M) {
  const int64_t ntiles = ceil_div(std::max<int64_t>(M, 1), kSortTile);
  return 4 * align256((size_t)M * 4) + align256((size_t)(kMaxRadix * ntiles) * 4) + align256(kMaxRadix * 4);
}

// Digit width and pass count for keys below nkeys: 9-bit digits when they
// save a pass.
static void sort_passes(int64_t nkeys, int &rb, int &passes) {
  const unsigned bits = key_bits(nkeys - 1 > 0 ? nkeys - 1 : 1);  // real keys < nkeys
  rb = 8;
  passes = (int)ceil_div(bits, 8);
  if (passes > 1 && ceil_div(bits, 9) < passes) {
    rb = 9;
    passes = (int)ceil_div(bits, 9);
  }
}

bool slot_sort_buckets_supported(int64_t N, int nchunks);
// Where slot_sort (or slot_sort_buckets) leaves the sorted positions in its workspace.
int *slot_sort_positions(int64_t M, int64_t N, int nchunks, void *ws) {
  const size_t a = align256((size_t)M * 4);
  int rb, passes;
  if (slot_sort_buckets_supported(N, nchunks)) passes = 2;  // the buckets' positions: the fourth buffer
  else sort_passes((int64_t)nchunks * N, rb, passes);
  return reinterpret_cast<int *>(static_cast<char *>(ws) + (((passes - 1) & 1) ? 3 * a : a));
}

int slot_sort(const int32_t *idx, int64_t M, int K, int64_t N, int chunk_rows, int nchunks, void *ws,
              unsigned **keys_sorted, int **pos_sorted, unsigned **digit_totals, int *digit_count, int *clear,
              int nclear, hipStream_t s) {
  char *w = static_cast<char *>(ws);
  const size_t a = align256((size_t)M * 4);
  unsigned *kbuf[2] = {reinterpret_cast<unsigned *>(w), reinterpret_cast<unsigned *>(w + 2 * a)};
  int *vbuf[2] = {reinterpret_cast<int *>(w + a), reinterpret_cast<int *>(w + 3 * a)};
  const int max_tiles = (int)ceil_div(std::max<int64_t>(M, 1), kSortTile);
  const bool big = M > kBigSort;
  const int ntiles = (int)ceil_div(std::max<int64_t>(M, 1), (int64_t)kBlock * (big ? kSortItemsBig : kSortItems));
  unsigned *hist = reinterpret_cast<unsigned *>(w + 4 * a);
  unsigned *totals = reinterpret_cast<unsigned *>(w + 4 * a + align256((size_t)(kMaxRadix * max_tiles) * 4));
  const unsigned nkeys = (unsigned)((int64_t)nchunks * N);
  const SlotKey sk{idx, (unsigned)N, FastDiv((uint32_t)K), FastDiv((uint32_t)chunk_rows), nkeys};
  int rb, passes;
  sort_passes(nkeys, rb, passes);
  int rc;
  if (big)
    rc = rb == 9 ? run_passes<9, kSortItemsBig>(sk, M, passes, kbuf, vbuf, hist, totals, ntiles, clear, nclear, s)
                 : run_passes<8, kSortItemsBig>(sk, M, passes, kbuf, vbuf, hist, totals, ntiles, clear, nclear, s);
  else
    rc = rb == 9 ? run_passes<9, kSortItems>(sk, M, passes, kbuf, vbuf, hist, totals, ntiles, clear, nclear, s)
                 : run_passes<8, kSortItems>(sk, M, passes, kbuf, vbuf, hist, totals, ntiles, clear, nclear, s);
  if (rc != SFT_OK) return rc;
  *keys_sorted = kbuf[(passes - 1) & 1];
  *pos_sorted = vbuf[(passes - 1) & 1];
  *digit_totals = totals;
  *digit_count = 1 << rb;
  return SFT_OK;
}

// Bucket-sort plan for keys below nkeys: low bits SB (7 or 8) sorted inside a
// bucket, high bits RB (8-10) by the radix pass; false when the key space
// needs more (then the LSD passes and the segment kernel run instead).
// 8-bit buckets from 18-bit keys on; from 16-bit keys (a 2 x 23 232-key
// space: an 8-bit radix pass, buckets twice as large) the steps were slower
// (1.707 -> 1.713 ms at L = 1048, 0.377 -> 0.389 ms at L = 136).
#ifndef SFT_SORT_SB8_BITS
#define SFT_SORT_SB8_BITS 18
#endif
static bool bucket_plan(int64_t nkeys, int &sb, int &rb) {
  const int kb = (int)key_bits(nkeys - 1 > 0 ? nkeys - 1 : 1);
  sb = kb >= SFT_SORT_SB8_BITS ? 8 : 7;
  rb = std::max(8, kb - sb);
  return rb <= 10;
}
bool slot_sort_buckets_supported(int64_t N, int nchunks) {
  int sb, rb;
  return SFT_SORT_BUCKETS && bucket_plan((int64_t)nchunks * N, sb, rb);
}

// The bucket sort's buffers in a slot_sort workspace: the high pass's keys and
// positions (k1, v1), its per-tile digit counts and digit totals, and the
// buckets' sorted positions (v2, the fourth buffer).
struct BucketBufs {
  unsigned *k1;
  int *v1, *v2;
  unsigned *hist, *totals;
  int ntiles, sb, rb;
  bool big;
};
static int bucket_bufs(void *ws, int64_t M, int64_t N, int nchunks, BucketBufs &bb) {
  char *w = static_cast<char *>(ws);
  const size_t a = align256((size_t)M * 4);
  const int max_tiles = (int)ceil_div(std::max<int64_t>(M, 1), kSortTile);
  bb.k1 = reinterpret_cast<unsigned *>(w);
  bb.v1 = reinterpret_cast<int *>(w + a);
  bb.v2 = reinterpret_cast<int *>(w + 3 * a);
  bb.hist = reinterpret_cast<unsigned *>(w + 4 * a);
  bb.totals = reinterpret_cast<unsigned *>(w + 4 * a + align256((size_t)(kMaxRadix * max_tiles) * 4));
  bb.big = M > kBigSort;
  bb.ntiles = (int)ceil_div(std::max<int64_t>(M, 1), (int64_t)kBlock * (bb.big ? kSortItemsBig : kSortItems));
  if (!bucket_plan((int64_t)nchunks * N, bb.sb, bb.rb)) return fail(SFT_EINVAL, "slot bucket sort: key space too large");
  return SFT_OK;
}

// First half of the bucket sort: the radix pass on the high key bits, into
// the workspace; zeroes clear[0 .. nclear) (stream-ordered).
int slot_sort_buckets_high(const int32_t *idx, int64_t M, int K, int64_t N, int chunk_rows, int nchunks, void *ws,
                           int *clear, int nclear, hipStream_t s) {
  BucketBufs bb;
  int rc = bucket_bufs(ws, M, N, nchunks, bb);
  if (rc != SFT_OK) return rc;
  const unsigned nkeys = (unsigned)((int64_t)nchunks * N);
  const SlotKey sk{idx, (unsigned)N, FastDiv((uint32_t)K), FastDiv((uint32_t)chunk_rows), nkeys};
#define SFT_HIGH_PASS(RB)                                                                                          \
  rc = bb.big ? run_high_pass<RB, kSortItemsBig>(sk, M, bb.sb, bb.k1, bb.v1, bb.hist, bb.totals, bb.ntiles, clear, \
                                                 nclear, s)                                                        \
              : run_high_pass<RB, kSortItems>(sk, M, bb.sb, bb.k1, bb.v1, bb.hist, bb.totals, bb.ntiles, clear,    \
                                              nclear, s)
  if (bb.rb == 8) SFT_HIGH_PASS(8);
  else if (bb.rb == 9) SFT_HIGH_PASS(9);
  else SFT_HIGH_PASS(10);
#undef SFT_HIGH_PASS
  return rc;
}

// Second half: one workgroup per bucket over the high pass's output in ws
// (only read), writing the sorted positions to vout, their 16-bit chunk
// offsets (pos16, when not null), segment starts seg[0 .. nchunks N] and per
// chunk the list of long segments (list + c N, count[c], which must be zero).
// Buckets [bfirst, bend) only (bend < 0: to the last); split launches must
// together cover every bucket once, bucket 0 (which also stores seg[nchunks N])
// included.
int slot_sort_buckets_low(const void *ws, int64_t M, int64_t N, int chunk_rows, int nchunks, int *vout,
                          int32_t *seg, int32_t *list, int *count, uint16_t *pos16, int long_period, hipStream_t s,
                          int bfirst, int bend) {
  BucketBufs bb;
  int rc = bucket_bufs(const_cast<void *>(ws), M, N, nchunks, bb);
  if (rc != SFT_OK) return rc;
  const unsigned nkeys = (unsigned)((int64_t)nchunks * N);
  const int nb = (int)ceil_div(std::max<int64_t>(nkeys, 1), (int64_t)1 << bb.sb);
  if (bend < 0 || bend > nb) bend = nb;
  if (bfirst < 0 || bfirst > bend) return fail(SFT_EINVAL, "slot bucket sort: bucket range out of order");
  if (bfirst == bend) return SFT_OK;
  const FastDiv div_feat((uint32_t)N);
  const dim3 grid((unsigned)(bend - bfirst));
  if (bb.sb == 8)
    hipLaunchKernelGGL(bucket_sort_kernel<8>, grid, dim3(kBucketBlock), 0, s, bb.k1, bb.v1, bb.totals, 1 << bb.rb,
                       nkeys, div_feat, (unsigned)N, vout, pos16, chunk_rows, seg, list, count, long_period, bfirst);
  else
    hipLaunchKernelGGL(bucket_sort_kernel<7>, grid, dim3(kBucketBlock), 0, s, bb.k1, bb.v1, bb.totals, 1 << bb.rb,
                       nkeys, div_feat, (unsigned)N, vout, pos16, chunk_rows, seg, list, count, long_period, bfirst);
  return check_launch("slot bucket sort (buckets)");
}

// Buckets [0, n) hold every key of position chunk 0 and the first key of
// chunk 1 (key N: its segment start ends chunk 0's last segment), so after
// them chunk 0's positions, segment starts and long-segment list are final;
// 0 when there is one chunk or no bucket plan.
int slot_sort_buckets_chunk0(int64_t N, int nchunks) {
  int sb, rb;
  if (nchunks < 2 || N <= 0 || !bucket_plan((int64_t)nchunks * N, sb, rb)) return 0;
  return buckets_through_chunk0(N, nchunks, sb);
}

// The bucket sort with the segment pass folded in: both halves, the sorted
// positions in the workspace's fourth buffer (returned), the long-segment
// counts zeroed by the first half.  Same results as slot_sort + the segment kernel.
int slot_sort_buckets(const int32_t *idx, int64_t M, int K, int64_t N, int chunk_rows, int nchunks, void *ws,
                      int32_t *seg, int32_t *list, int *count, uint16_t *pos16, int long_period, int **pos_sorted,
                      hipStream_t s) {
  BucketBufs bb;
  int rc = bucket_bufs(ws, M, N, nchunks, bb);
  if (rc != SFT_OK) return rc;
  if ((rc = slot_sort_buckets_high(idx, M, K, N, chunk_rows, nchunks, ws, count, nchunks, s)) != SFT_OK) return rc;
  if ((rc = slot_sort_buckets_low(ws, M, N, chunk_rows, nchunks, bb.v2, seg, list, count, pos16, long_period, s, 0,
                                  -1)) != SFT_OK)
    return rc;
  *pos_sorted = bb.v2;
  return SFT_OK;
}

}  // namespace sft
