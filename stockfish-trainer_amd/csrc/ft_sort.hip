// Stable LSD radix sort of the backward's flat index slots, for gfx950.
//
// Sorts the B*K slots s = b*K + k by key (SlotKey: chunk(b) * N + feature for
// an active slot, a sentinel past every real key otherwise) carrying the slot's
// position b, stably, so each key's positions come out in ascending order.
// 8-bit digits, least significant first; each pass is
//   upsweep:   per 2048-slot tile, a 256-bin digit histogram;
//   scan:      per digit, an exclusive scan of its tile counts and the digit
//              total; a digit's base is the scan of the totals (done in the
//              downsweep), so (digit, tile) starts at base + its tile prefix;
//   downsweep: per tile, stable ranks (digit-major, then slot order) from
//              wave-wide match masks (8 ballots) and per-wave digit counts,
//              the tile reordered in LDS, then written out as contiguous runs.
// The first pass reads the keys straight from the index matrix.
#include <algorithm>

#include "common.h"

namespace sft {

namespace {

constexpr int kRadixBits = 8;
constexpr int kRadix = 1 << kRadixBits;
constexpr int kSortItems = 8;
constexpr int kSortTile = kBlock * kSortItems;  // 2048 slots per tile

// n / d for 32-bit n by a divisor fixed at launch: multiply-high by a magic
// number (Granlund & Montgomery 1994, round-up variant): with l = ceil(log2 d)
// and m = floor(2^32 (2^l - d) / d) + 1, n / d = (t + ((n - t) >> 1)) >> (l - 1)
// where t = mulhi(m, n), for d >= 2.
struct FastDiv {
  uint32_t d, mul, shift;
  FastDiv() = default;
  __host__ explicit FastDiv(uint32_t div) : d(div), mul(0), shift(0) {
    uint32_t l = 0;
    while (((uint64_t)1 << l) < div) ++l;
    shift = l;
    mul = (uint32_t)((((uint64_t)1 << 32) * (((uint64_t)1 << l) - div)) / div + 1);
  }
  __device__ __forceinline__ uint32_t operator()(uint32_t n) const {
    if (d == 1) return n;
    const uint32_t t = __umulhi(mul, n);
    return (t + ((n - t) >> 1)) >> (shift - 1);
  }
};

// Key of slot s (s < 2^31): chunk(b) * N + feature for an active slot, the
// sentinel for an inactive one; the carried value is the position b = s / K.
struct SlotKey {
  const int32_t *idx;
  unsigned N;
  FastDiv divK, divChunk;
  unsigned sentinel;
  __device__ __forceinline__ unsigned key(int64_t s) const {
    const unsigned v = (unsigned)idx[s];
    return v < N ? divChunk(divK((uint32_t)s)) * N + v : sentinel;
  }
  __device__ __forceinline__ int pos(int64_t s) const { return (int)divK((uint32_t)s); }
};

// Lanes of the wave holding the same digit as this lane (among `valid` lanes).
__device__ __forceinline__ uint64_t match_digit(unsigned d, bool valid) {
  uint64_t peers = ballot(valid);
#pragma unroll
  for (int b = 0; b < kRadixBits; ++b) {
    const bool bit = (d >> b) & 1u;
    const uint64_t m = ballot(bit);
    peers &= bit ? m : ~m;
  }
  return peers;
}

template <bool FIRST>
__global__ __launch_bounds__(kBlock) void radix_upsweep(SlotKey sk, const unsigned *__restrict__ kin, int64_t M,
                                                        int ntiles, int shift, unsigned *__restrict__ hist) {
  __shared__ unsigned hw[kWavesPerBlock][kRadix];
  const int tid = threadIdx.x, wave = tid / kWave;
#pragma unroll
  for (int w = 0; w < kWavesPerBlock; ++w) hw[w][tid] = 0;
  __syncthreads();
  const int64_t base = (int64_t)blockIdx.x * kSortTile;
#pragma unroll
  for (int i = 0; i < kSortItems; ++i) {
    const int64_t e = base + (int64_t)i * kBlock + tid;
    if (e < M) atomicAdd(&hw[wave][((FIRST ? sk.key(e) : kin[e]) >> shift) & (kRadix - 1)], 1u);
  }
  __syncthreads();
  hist[(int64_t)tid * ntiles + blockIdx.x] = hw[0][tid] + hw[1][tid] + hw[2][tid] + hw[3][tid];
}

// Per digit d (one block each): exclusive scan of hist[d][0 .. ntiles) in
// place, and the digit's total into totals[d].
__global__ __launch_bounds__(kBlock) void radix_scan_digits(unsigned *__restrict__ hist, int ntiles,
                                                            unsigned *__restrict__ totals) {
  __shared__ unsigned part[kBlock];
  const int tid = threadIdx.x;
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

// Exclusive scan of 256 per-digit values by one wave (4 digits per lane).
__device__ __forceinline__ void wave_scan_256(const unsigned *in, unsigned *out, int lane) {
  unsigned c[kRadix / kWave];
  unsigned s = 0;
#pragma unroll
  for (int j = 0; j < kRadix / kWave; ++j) {
    c[j] = in[lane * (kRadix / kWave) + j];
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
  for (int j = 0; j < kRadix / kWave; ++j) {
    out[lane * (kRadix / kWave) + j] = run;
    run += c[j];
  }
}

template <bool FIRST>
__global__ __launch_bounds__(kBlock) void radix_downsweep(SlotKey sk, const unsigned *__restrict__ kin,
                                                          const int *__restrict__ vin, unsigned *__restrict__ kout,
                                                          int *__restrict__ vout, const unsigned *__restrict__ offs,
                                                          const unsigned *__restrict__ totals, int64_t M, int ntiles,
                                                          int shift) {
  __shared__ unsigned s_keys[kSortTile];
  __shared__ int s_vals[kSortTile];
  __shared__ unsigned running[kRadix];
  __shared__ unsigned wcnt[kWavesPerBlock][kRadix];
  __shared__ unsigned dstart[kRadix];
  __shared__ unsigned dtot[kRadix];
  __shared__ unsigned dbase[kRadix];
  const int tid = threadIdx.x, lane = tid % kWave, wave = tid / kWave;
  const int64_t base = (int64_t)blockIdx.x * kSortTile;
  const int count = (int)std::min<int64_t>(kSortTile, M - base);

  running[tid] = 0;
  dtot[tid] = totals[tid];
#pragma unroll
  for (int w = 0; w < kWavesPerBlock; ++w) wcnt[w][tid] = 0;

  unsigned key[kSortItems];
  int val[kSortItems];
  unsigned rank[kSortItems];
#pragma unroll
  for (int i = 0; i < kSortItems; ++i) {
    const int64_t e = base + (int64_t)i * kBlock + tid;
    key[i] = 0;
    val[i] = 0;
    if (e < M) {
      key[i] = FIRST ? sk.key(e) : kin[e];
      val[i] = FIRST ? sk.pos(e) : vin[e];
    }
  }
  __syncthreads();

  // Stable ranks within the tile: slot order is (round i, wave, lane).
#pragma unroll
  for (int i = 0; i < kSortItems; ++i) {
    const bool valid = i * kBlock + tid < count;
    const unsigned d = (key[i] >> shift) & (kRadix - 1);
    const uint64_t peers = match_digit(d, valid);
    if (valid && (int)(__ffsll((unsigned long long)peers) - 1) == lane) wcnt[wave][d] = (unsigned)__popcll(peers);
    __syncthreads();
    if (valid) {
      unsigned r = running[d] + (unsigned)popc_below(peers);
      for (int w = 0; w < wave; ++w) r += wcnt[w][d];
      rank[i] = r;
    }
    __syncthreads();
    unsigned tot = 0;
#pragma unroll
    for (int w = 0; w < kWavesPerBlock; ++w) {
      tot += wcnt[w][tid];
      wcnt[w][tid] = 0;
    }
    running[tid] += tot;
    __syncthreads();
  }

  // Digit starts inside the tile, and of each digit in the whole output.
  if (wave == 0) wave_scan_256(running, dstart, lane);
  if (wave == 1) wave_scan_256(dtot, dbase, lane);
  __syncthreads();

#pragma unroll
  for (int i = 0; i < kSortItems; ++i) {
    if (i * kBlock + tid < count) {
      const unsigned d = (key[i] >> shift) & (kRadix - 1);
      const unsigned p = dstart[d] + rank[i];
      s_keys[p] = key[i];
      s_vals[p] = val[i];
    }
  }
  __syncthreads();

  for (int j = tid; j < count; j += kBlock) {
    const unsigned k = s_keys[j];
    const unsigned d = (k >> shift) & (kRadix - 1);
    const int64_t dst = (int64_t)dbase[d] + offs[(int64_t)d * ntiles + blockIdx.x] + (j - dstart[d]);
    kout[dst] = k;
    vout[dst] = s_vals[j];
  }
}

size_t align256(size_t v) { return (v + 255) & ~(size_t)255; }

}  // namespace

unsigned sort_key_bits(int64_t maxkey) {
  unsigned bits = 1;
  while (((int64_t)1 << bits) <= maxkey) ++bits;  // keys lie in [0, maxkey]
  return bits;
}

// Workspace: two key/position buffer pairs (ping-pong), the histograms and
// the digit totals.
size_t slot_sort_workspace(int64_t M) {
  const int64_t ntiles = ceil_div(std::max<int64_t>(M, 1), kSortTile);
  return 4 * align256((size_t)M * 4) + align256((size_t)(kRadix * ntiles) * 4) + align256(kRadix * 4);
}

int slot_sort(const int32_t *idx, int64_t M, int K, int64_t N, int chunk_rows, int nchunks, void *ws,
              unsigned **keys_sorted, int **pos_sorted, hipStream_t s) {
  char *w = static_cast<char *>(ws);
  const size_t a = align256((size_t)M * 4);
  unsigned *kbuf[2] = {reinterpret_cast<unsigned *>(w), reinterpret_cast<unsigned *>(w + 2 * a)};
  int *vbuf[2] = {reinterpret_cast<int *>(w + a), reinterpret_cast<int *>(w + 3 * a)};
  const int ntiles = (int)ceil_div(std::max<int64_t>(M, 1), kSortTile);
  unsigned *hist = reinterpret_cast<unsigned *>(w + 4 * a);
  unsigned *totals = reinterpret_cast<unsigned *>(w + 4 * a + align256((size_t)(kRadix * ntiles) * 4));
  const unsigned sentinel = (unsigned)((int64_t)nchunks * N);
  const SlotKey sk{idx, (unsigned)N, FastDiv((uint32_t)K), FastDiv((uint32_t)chunk_rows), sentinel};
  const int passes = (int)ceil_div(sort_key_bits(sentinel), kRadixBits);
  for (int p = 0; p < passes; ++p) {
    const int shift = p * kRadixBits;
    const unsigned *kin = p == 0 ? nullptr : kbuf[(p - 1) & 1];
    const int *vin = p == 0 ? nullptr : vbuf[(p - 1) & 1];
    unsigned *kout = kbuf[p & 1];
    int *vout = vbuf[p & 1];
    if (p == 0)
      hipLaunchKernelGGL(radix_upsweep<true>, dim3(ntiles), dim3(kBlock), 0, s, sk, kin, M, ntiles, shift, hist);
    else
      hipLaunchKernelGGL(radix_upsweep<false>, dim3(ntiles), dim3(kBlock), 0, s, sk, kin, M, ntiles, shift, hist);
    hipLaunchKernelGGL(radix_scan_digits, dim3(kRadix), dim3(kBlock), 0, s, hist, ntiles, totals);
    if (p == 0)
      hipLaunchKernelGGL(radix_downsweep<true>, dim3(ntiles), dim3(kBlock), 0, s, sk, kin, vin, kout, vout, hist,
                         totals, M, ntiles, shift);
    else
      hipLaunchKernelGGL(radix_downsweep<false>, dim3(ntiles), dim3(kBlock), 0, s, sk, kin, vin, kout, vout, hist,
                         totals, M, ntiles, shift);
    const int rc = check_launch("slot radix sort");
    if (rc != SFT_OK) return rc;
  }
  *keys_sorted = kbuf[(passes - 1) & 1];
  *pos_sorted = vbuf[(passes - 1) & 1];
  return SFT_OK;
}

}  // namespace sft
