// Sparse FT forward kernels for gfx950: fp32 gather-sum and int16 quantized
// gather-sum.
//
// Mapping (see Mapping in common.h): a 256-thread workgroup is 4 waves; each
// wave serves 64/G positions, one lane group of G lanes per position.  The wave
// first compacts its positions' index rows into LDS (active slots only, slot
// order kept), then every lane accumulates its 16-byte column chunks over the
// compacted list, U rows at a time: the U*CPL row loads of a step are issued
// before any add, then the adds run in slot order.  For G == 64 the index is
// wave-uniform and is moved to an SGPR, so the row base address is scalar.
//
// fp32: acc = bias, then acc += W[idx[k]] for active k ascending; every add is
// a binary32 add in the reference order (FT/kernel.py:93-100), so the result
// is bit-identical to that order.
// int16: exact int32 accumulation (order-free), optional wrap to int16, clamp.
#include <algorithm>

#include "common.h"

namespace sft {

namespace {


template <typename T>
__device__ __forceinline__ T zero_of() {
  return T(0);
}

// Reads compacted slots k..k+3 of a list (kpad is a multiple of 4 and k % 4 == 0).
__device__ __forceinline__ i32x4 read4(const int *list, int k) { return *reinterpret_cast<const i32x4 *>(list + k); }

// Wave-wide min and max of a value that is constant within each lane group.
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

// ------------------------------------------------------------------ fp32 ----
template <typename T, int G, int CPL, int U>
__global__ __launch_bounds__(kBlock) void fwd_f32_kernel(const int32_t *__restrict__ idx, int64_t B, int K, int N,
                                                         const T *__restrict__ W, int64_t cols,
                                                         const T *__restrict__ bias, T *__restrict__ out, int kpad) {
  static_assert(U == 4, "index reads are 4-wide");
  constexpr int PPW = kWave / G;
  static_assert(PPW <= kCompactRows, "compact_rows takes at most kCompactRows rows");
  extern __shared__ int smem[];
  const int wave = uniform(threadIdx.x / kWave);
  const int lane = threadIdx.x % kWave;
  int *list = smem + wave * PPW * kpad;
  int *count = smem + kWavesPerBlock * PPW * kpad + wave * PPW;
  const int64_t pos0 = ((int64_t)blockIdx.x * kWavesPerBlock + wave) * PPW;
  compact_rows(idx, B, K, N, pos0, PPW, list, kpad, count);
  wave_lds_barrier();

  const int g = lane / G, t = lane % G;
  const int64_t pos = pos0 + g;
  const int n = count[g];
  int nmin, nmax;
  group_minmax<G>(n, nmin, nmax);
  const int *mylist = list + g * kpad;

  const int64_t c0 = (int64_t)blockIdx.y * (G * CPL) + t;
  bool colok[CPL];
  T acc[CPL];
#pragma unroll
  for (int j = 0; j < CPL; ++j) {
    colok[j] = (c0 + G * j) < cols;
    acc[j] = colok[j] ? bias[c0 + G * j] : zero_of<T>();
  }

  int k = 0;
  for (; k + U <= nmin; k += U) {
    i32x4 f4 = read4(mylist, k);
    T w[U][CPL];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      int f = f4[u];
      if (G == kWave) f = uniform(f);
      const T *row = W + (int64_t)f * cols + c0;
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
    i32x4 f4 = read4(mylist, k);
    T w[U][CPL];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const bool v = k + u < n;
      int f = v ? f4[u] : 0;
      if (G == kWave) f = uniform(f);
      const T *row = W + (int64_t)f * cols + c0;
#pragma unroll
      for (int j = 0; j < CPL; ++j) {
        w[u][j] = zero_of<T>();
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

  if (pos < B) {
    T *o = out + pos * cols + c0;
#pragma unroll
    for (int j = 0; j < CPL; ++j)
      if (colok[j]) __builtin_nontemporal_store(acc[j], o + G * j);
  }
}

// ----------------------------------------------------------------- int16 ----
template <typename T>
struct Q16;
template <>
struct Q16<i16x8> {
  typedef i32x8 Acc;
  static __device__ __forceinline__ Acc widen(i16x8 v) { return __builtin_convertvector(v, i32x8); }
  static __device__ __forceinline__ i16x8 finish(Acc a, int lo, int hi, int wrap16) {
    if (wrap16) a = __builtin_convertvector(__builtin_convertvector(a, i16x8), i32x8);  // low 16 bits, sign-extended
    a = a < lo ? (Acc)lo : a;
    a = a > hi ? (Acc)hi : a;
    return __builtin_convertvector(a, i16x8);
  }
};
template <>
struct Q16<short> {
  typedef int Acc;
  static __device__ __forceinline__ Acc widen(short v) { return (int)v; }
  static __device__ __forceinline__ short finish(Acc a, int lo, int hi, int wrap16) {
    if (wrap16) a = (int)(short)(unsigned short)(unsigned)a;
    a = a < lo ? lo : a;
    a = a > hi ? hi : a;
    return (short)a;
  }
};

template <typename T, int G, int CPL, int U>
__global__ __launch_bounds__(kBlock) void fwd_i16_kernel(const int32_t *__restrict__ idx, int64_t B, int K, int N,
                                                         const T *__restrict__ W, int64_t cols,
                                                         const T *__restrict__ bias,
                                                         const int32_t *__restrict__ psqt, int P,
                                                         T *__restrict__ out, int32_t *__restrict__ psqt_out,
                                                         int clip_lo, int clip_hi, int wrap16, int kpad) {
  static_assert(U == 4, "index reads are 4-wide");
  typedef typename Q16<T>::Acc Acc;
  constexpr int PPW = kWave / G;
  static_assert(PPW <= kCompactRows, "compact_rows takes at most kCompactRows rows");
  extern __shared__ int smem[];
  const int wave = uniform(threadIdx.x / kWave);
  const int lane = threadIdx.x % kWave;
  int *list = smem + wave * PPW * kpad;
  int *count = smem + kWavesPerBlock * PPW * kpad + wave * PPW;
  const int64_t pos0 = ((int64_t)blockIdx.x * kWavesPerBlock + wave) * PPW;
  compact_rows(idx, B, K, N, pos0, PPW, list, kpad, count);
  wave_lds_barrier();

  const int g = lane / G, t = lane % G;
  const int64_t pos = pos0 + g;
  const int n = count[g];
  int nmin, nmax;
  group_minmax<G>(n, nmin, nmax);
  const int *mylist = list + g * kpad;
  // PSQT columns: lane t < P of the group, slab 0 only (host guarantees P <= G).
  const bool do_psqt = psqt != nullptr && blockIdx.y == 0 && t < P;
  int pacc = 0;

  const int64_t c0 = (int64_t)blockIdx.y * (G * CPL) + t;
  bool colok[CPL];
  Acc acc[CPL];
#pragma unroll
  for (int j = 0; j < CPL; ++j) {
    colok[j] = (c0 + G * j) < cols;
    acc[j] = colok[j] ? Q16<T>::widen(bias[c0 + G * j]) : (Acc)0;
  }

  for (int k = 0; k < nmax; k += U) {
    i32x4 f4 = read4(mylist, k);
    T w[U][CPL];
    int pw[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const bool v = k + u < n;
      int f = v ? f4[u] : 0;
      if (G == kWave) f = uniform(f);
      const T *row = W + (int64_t)f * cols + c0;
#pragma unroll
      for (int j = 0; j < CPL; ++j) {
        w[u][j] = T(0);
        if (v && colok[j]) w[u][j] = row[G * j];
      }
      pw[u] = 0;
      if (v && do_psqt) pw[u] = psqt[(int64_t)f * P + t];
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
#pragma unroll
      for (int j = 0; j < CPL; ++j) acc[j] += Q16<T>::widen(w[u][j]);
      pacc += pw[u];
    }
  }
  (void)nmin;

  if (pos < B) {
    T *o = out + pos * cols + c0;
#pragma unroll
    for (int j = 0; j < CPL; ++j)
      if (colok[j]) __builtin_nontemporal_store(Q16<T>::finish(acc[j], clip_lo, clip_hi, wrap16), o + G * j);
    if (do_psqt) psqt_out[pos * P + t] = pacc;
  }
}

// ------------------------------------------------------ tiled fp32 gather ----
// The table is first re-laid out as column tiles: tile t holds columns
// [32t, 32t + 32) of every row, 128 bytes per row, rows contiguous, so one
// tile is N * 128 B (2.97 MB for N = 23 232) and fits one XCD's 4 MB L2.
// The gather then runs tile by tile on each XCD (tile_sched_item), lane
// groups of 8 lanes x 16 B covering one tile row per position, so every
// table read after the first touch of a tile is an L2 hit.
//
// Each tile ends with a pad row (row N) of -0.0 in every column.  A
// position's LDS list holds its active rows and then N up to the wave's
// longest list, so all lanes load and add a row at every step with no
// execution masks: x + (-0.0) == x for every x in round-to-nearest (-0.0 and
// +0.0 included, NaN stays NaN), and the sum is the one over the active rows
// in list order.
constexpr int kTileF = 32;                 // floats per tile row
constexpr int kTileCh = kTileF / 4;        // float4 chunks per tile row (= lane group size)
#ifndef SFT_TILED_ROUNDS
#define SFT_TILED_ROUNDS 1
#endif
constexpr int kTiledRounds = SFT_TILED_ROUNDS;                        // position rounds per block
constexpr int kTiledPosPerRound = kWavesPerBlock * (kWave / kTileCh);  // 32
constexpr int kTiledPosPerBlock = kTiledPosPerRound * kTiledRounds;

// Post-FT epilogue of the forward (src/model/model.py:93-115), applied in
// registers by the EPI instantiation over the paired column map: the
// pre-activations are stored to raw0/raw1 position-major (kept for the
// backward), and for the paired tiles lane q < 4 multiplies its clamped chunk
// with the partner chunk of the other half (lane q + 4), scales by 127/128 and
// stores it to the half of l0 the side to move selects:
//   l0 = cat(where(us, pw_white, pw_black), where(us, pw_black, pw_white)) * 127/128.
struct FwdEpilogue {
  const float *us;     // [B]; nonzero: white to move
  f32x4 *l0;           // [B, 2 * half4] chunks
  f32x4 *raw0, *raw1;  // [B][ntiles][8] chunks per perspective (position-major)
};

// torch.clamp(x, 0, 1): NaN passes through.
__device__ __forceinline__ float clamp01(float x) { return x < 0.f ? 0.f : (x > 1.f ? 1.f : x); }
__device__ __forceinline__ f32x4 clamp01(f32x4 v) {
  return f32x4{clamp01(v.x), clamp01(v.y), clamp01(v.z), clamp01(v.w)};
}
__device__ __forceinline__ f32x4 shfl_xor4(f32x4 v, int m) {
  return f32x4{__shfl_xor(v.x, m), __shfl_xor(v.y, m), __shfl_xor(v.z, m), __shfl_xor(v.w, m)};
}

constexpr uint32_t kTileRowBytes = kTileCh * sizeof(f32x4);  // 128
// Rows per fp32 table tile: the N table rows and the pad row.
__host__ __device__ inline int64_t tile_rows(int64_t N) { return N + 1; }

__device__ __forceinline__ f32x4 f32_row(const char *tbase, uint32_t lane_off, int f) {
  return *reinterpret_cast<const f32x4 *>(tbase + ((uint32_t)f * kTileRowBytes + lane_off));
}

// Rows [0, nmax) of one position's list in one tile, added onto acc in list
// order: the position's active rows, then the pad row (see above) up to the
// wave's longest list.  Padding lanes of the last tile load their chunk too
// (it is allocated; their sums are not stored).  Row addresses are 32-bit
// offsets from the tile's base (a tile is (N + 1) x 128 B).
#ifndef SFT_FWD_TILED_U
#define SFT_FWD_TILED_U 8
#endif
__device__ __forceinline__ f32x4 f32_tile_rows(const int *mylist, int nmax, const char *tbase, uint32_t lane_off,
                                               f32x4 acc) {
  constexpr int U = SFT_FWD_TILED_U;  // rows in flight per step (a multiple of 4)
  static_assert(U % 4 == 0, "rows are read from the LDS list four at a time");
  int k = 0;
  for (; k + U <= nmax; k += U) {
    int fi[U];
#pragma unroll
    for (int u = 0; u < U; u += 4) {
      const i32x4 f4 = read4(mylist, k + u);
      fi[u] = f4[0], fi[u + 1] = f4[1], fi[u + 2] = f4[2], fi[u + 3] = f4[3];
    }
    f32x4 w[U];
#pragma unroll
    for (int u = 0; u < U; ++u) w[u] = f32_row(tbase, lane_off, fi[u]);
#pragma unroll
    for (int u = 0; u < U; ++u) acc += w[u];
  }
  for (; k + 4 <= nmax; k += 4) {
    const i32x4 f4 = read4(mylist, k);
    f32x4 w[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) w[u] = f32_row(tbase, lane_off, f4[u]);
#pragma unroll
    for (int u = 0; u < 4; ++u) acc += w[u];
  }
  for (; k < nmax; ++k) acc += f32_row(tbase, lane_off, mylist[k]);
  return acc;
}

// ------------------------------------------------ rank lists of the gather ----
// Before the tiled fp32 gather, each perspective's index rows become lists in
// rank order: rank r holds position pos[r], its active slots (0 <= v < N) in
// slot order and then N (the pad row) up to kpad entries.  Within each block
// of 256 consecutive positions the ranks run through the positions by active
// count, largest first, so the 8 consecutive ranks a wave sums have nearly
// the same count: the wave steps as many rows as its longest list, and a step
// costs one vector-memory instruction whatever the number of lanes with a
// row.  The lists are built once per call instead of compacted again for
// every column tile, and a wave loads its 8 lists with 16-byte loads (one per
// lane at K = 32).  Ranks B .. Bpad - 1 are padding: position -1, count 0,
// list all N.  Positions of one count are ranked in the order LDS atomics
// hand out; a position's sum does not depend on its rank.
// Narrow lists (`narrow`: tables of at most 65 535 rows gathered in one pass,
// kpad a multiple of 8 and the lists staged in LDS) hold 16-bit entries, eight
// per 16-byte piece, widened to ints in the gather's LDS: every column tile
// pass streams the lists through the L2 that holds the table tile, and this
// halves them.
constexpr int kRanksPerBlock = kWavesPerBlock * (kWave / kTileCh);  // 32: 8 per wave
constexpr int kRankSortBlock = kBlock;                               // positions ranked together
struct RankLists {
  int32_t *list;   // [Bpad][kpad] (narrow: uint16_t entries); table parts: the packed runs
  int32_t *pos;    // [Bpad] rank -> position, -1 for padding
  int32_t *count;  // [Bpad] active slots of the rank's position, non-increasing within each 256 ranks
  i32x4 *cut;      // [Bpad] table parts (nparts > 1): see "Table parts" below
  i32x4 *roff;     // [Bpad] table parts: where each pass's run of the rank starts in `list`
  int narrow;      // 16-bit list entries (STAGE builds only, nparts == 1)
};
struct RankArgs {
  const int32_t *idx[2];
  RankLists L[2];
  int nparts, part_rows;
  FastDiv part_of;  // v / part_rows
};

// ---- table parts ----
// A table whose 32-column tile (N + 1 rows of 128 B) is larger than an XCD's
// L2 is gathered in nparts passes, pass p reading table rows [p part_rows,
// (p + 1) part_rows).  For each position its list is cut into nparts runs,
// in list (= slot) order: slot k goes to pass max(part of slots 0 .. k) (the
// running maximum), so pass p adds list[lo_p, hi_p) onto the sum the previous
// passes left and the position's adds keep the reference order.  For a list
// whose parts never decrease (sorted rows) that is each slot's own part; a
// list that goes back to an earlier part (the encoders emit threats by colour
// and piece: about a fifth of the rows of random positions, most going back
// once near a part boundary) reads those few rows in a later pass, from beyond
// that pass's L2 working set, and keeps every other slot in its own part's
// pass.  cut[r] = {start of pass 1's run, of pass 2's, of pass 3's, final
// pass}; lo_p = (p == 0 ? 0 : cut[p - 1]), hi_p = (p == final ? count : cut[p]).
// The runs are stored packed instead of the lists: within each block of 256
// ranks, the runs of pass 0 for the ranks in rank order, then those of pass 1,
// and so on (at most 256 kpad entries in all), and roff[r][p] gives where the
// run of rank r for pass p starts -- so a pass reads only its runs, and a
// wave's 8 runs lie together, instead of a stretch from the middle of each of
// 8 padded list rows (Full_Threats: most of a pass's list bytes).
constexpr int kMaxParts = 4;

// One workgroup per 256 positions of one perspective (grid.y).  STAGE: the
// lists are assembled in LDS (row stride kpad + 1, free of bank conflicts)
// and stored with coalesced 16-byte stores; else each thread stores its own.
template <bool STAGE>
__device__ __forceinline__ void rank_lists_block(const RankArgs &a, int bx, int by, int64_t B, int64_t Bpad, int K,
                                                 int N, int kpad, int vec) {
  extern __shared__ int sm[];  // bins[K + 1] | offsets[K + 1] | (STAGE) 256 rows of kpad + 1 | (parts) run scans
  unsigned *bin = reinterpret_cast<unsigned *>(sm), *off = bin + (K + 1);
  int *rows = sm + 2 * (K + 1);
  const RankLists &L = a.L[by];
  const int32_t *__restrict__ idx = a.idx[by];
  const int tid = threadIdx.x;
  const int64_t base = (int64_t)bx * kRankSortBlock;
  const int64_t b = base + tid;
  const bool real = b < B;
  const int32_t *row = idx + (real ? b : 0) * K;
  auto slot = [&](int k) { return row[k]; };
  for (int i = tid; i <= K; i += kBlock) bin[i] = 0u;
  __syncthreads();
  // Rows of up to 32 slots (staged, 16-byte aligned) are loaded once, into
  // registers, for both the count and the list.
  constexpr int kRegRow = 8;  // 16-byte pieces: the staged kpad <= 32
  const bool regrow = STAGE && vec && K <= 4 * kRegRow;
  i32x4 rv[kRegRow];
  int c = 0;
  // With table parts the same pass also finds the runs: cut[p] = the number of
  // active slots before the first slot whose running maximum of parts exceeds
  // p.  (A second pass over the row for them took 49 of 156 us per call at
  // K = 160; with it folded in here and 8 row loads in flight per thread in
  // both passes, the call takes 128 us.)
  int cut[kMaxParts - 1], part = 0;  // part: the running maximum
  auto count_slot = [&](int v) {
    if ((unsigned)v >= (unsigned)N) return;
    if (a.nparts > 1) {  // launch-uniform
      const int pv = (int)a.part_of((uint32_t)v);
      for (; part < pv; ++part)
        if (part < kMaxParts - 1) cut[part] = c;
    }
    ++c;
  };
  if (regrow) {
#pragma unroll
    for (int u = 0; u < kRegRow; ++u)
      rv[u] = (real && 4 * u < K) ? *reinterpret_cast<const i32x4 *>(row + 4 * u) : i32x4{-1, -1, -1, -1};
    if (a.nparts > 1) {
#pragma unroll
      for (int u = 0; u < kRegRow; ++u)
#pragma unroll
        for (int e = 0; e < 4; ++e) count_slot(rv[u][e]);
    } else {
#pragma unroll
      for (int u = 0; u < kRegRow; ++u)
        c += ((unsigned)rv[u][0] < (unsigned)N) + ((unsigned)rv[u][1] < (unsigned)N) +
             ((unsigned)rv[u][2] < (unsigned)N) + ((unsigned)rv[u][3] < (unsigned)N);
    }
  } else if (real) {
    if (vec && a.nparts > 1) {
#pragma unroll 8
      for (int k = 0; k < K; k += 4) {
        const i32x4 v = *reinterpret_cast<const i32x4 *>(row + k);
#pragma unroll
        for (int e = 0; e < 4; ++e) count_slot(v[e]);
      }
    } else if (vec) {
      for (int k = 0; k < K; k += 4) {
        const i32x4 v = *reinterpret_cast<const i32x4 *>(row + k);
        c += ((unsigned)v[0] < (unsigned)N) + ((unsigned)v[1] < (unsigned)N) + ((unsigned)v[2] < (unsigned)N) +
             ((unsigned)v[3] < (unsigned)N);
      }
    } else {
      for (int k = 0; k < K; ++k) count_slot(slot(k));
    }
  }
  for (; part < kMaxParts - 1; ++part) cut[part] = c;  // parts after the row's last
  const unsigned mine = real ? atomicAdd(&bin[c], 1u) : 0u;
  __syncthreads();
  if (tid < kWave) {  // off[cc] = sum of bin[cc + 1 .. K]: wave 0, 64 bins per step, largest count first
    unsigned carry = 0u;
    for (int top = K; top >= 0; top -= kWave) {
      const int cc = top - tid;
      const unsigned v = cc >= 0 ? bin[cc] : 0u;
      unsigned incl = v;  // inclusive scan over lanes 0 .. tid (bins top .. cc)
#pragma unroll
      for (int d = 1; d < kWave; d <<= 1) {
        const unsigned o = __shfl_up(incl, d);
        if (tid >= d) incl += o;
      }
      if (cc >= 0) off[cc] = carry + incl - v;
      carry += __shfl(incl, kWave - 1);
    }
  }
  __syncthreads();
  const int rl = real ? (int)(off[c] + mine) : tid;  // positions past B are the block's last (padding) ranks
  const int64_t r = base + rl;
  if (r < Bpad) {
    L.pos[r] = real ? (int32_t)b : -1;
    L.count[r] = real ? c : 0;
  }
  if (a.nparts > 1) {  // launch-uniform: packed runs (see "Table parts")
    // fn(v) for the row's active slots in slot order (16-byte loads, several in flight)
    auto each_active = [&](auto &&fn) {
      if (!real) return;
      if (vec) {
        constexpr int U = 8;  // row loads issued before the batch's stores
        for (int k0 = 0; k0 < K; k0 += 4 * U) {
          i32x4 v4[U];
#pragma unroll
          for (int u = 0; u < U; ++u)
            v4[u] = k0 + 4 * u < K ? *reinterpret_cast<const i32x4 *>(row + k0 + 4 * u) : i32x4{-1, -1, -1, -1};
#pragma unroll
          for (int u = 0; u < U; ++u)
#pragma unroll
            for (int e = 0; e < 4; ++e)
              if ((unsigned)v4[u][e] < (unsigned)N) fn(v4[u][e]);
        }
      } else {
        for (int k = 0; k < K; ++k) {
          const int v = slot(k);
          if ((unsigned)v < (unsigned)N) fn(v);
        }
      }
    };
    const i32x4 cv = i32x4{cut[0], cut[1], cut[2], a.nparts - 1};
    int len[kMaxParts];
#pragma unroll
    for (int p = 0; p < kMaxParts; ++p) {
      const int lo = p == 0 ? 0 : cv[p - 1];
      const int hi = p == cv[3] ? c : (p < kMaxParts - 1 ? cv[p] : c);
      len[p] = (p < a.nparts && p <= cv[3]) ? hi - lo : 0;
    }
    // exclusive scans of the run lengths in rank order, one per pass
    int *scan = rows;  // [kMaxParts][kRankSortBlock]
#pragma unroll
    for (int p = 0; p < kMaxParts; ++p) scan[p * kRankSortBlock + rl] = len[p];
    __syncthreads();
    for (int d = 1; d < kRankSortBlock; d <<= 1) {
      int v[kMaxParts];
#pragma unroll
      for (int p = 0; p < kMaxParts; ++p)
        v[p] = scan[p * kRankSortBlock + tid] + (tid >= d ? scan[p * kRankSortBlock + tid - d] : 0);
      __syncthreads();
#pragma unroll
      for (int p = 0; p < kMaxParts; ++p) scan[p * kRankSortBlock + tid] = v[p];
      __syncthreads();
    }
    int start[kMaxParts];
    int64_t pbase = base * kpad;  // this block's region of the runs
#pragma unroll
    for (int p = 0; p < kMaxParts; ++p) {
      start[p] = (int)(pbase + scan[p * kRankSortBlock + rl] - len[p]);
      pbase += scan[p * kRankSortBlock + kRankSortBlock - 1];
    }
    if (r < Bpad) {
      L.cut[r] = cv;
      L.roff[r] = i32x4{start[0], start[1], start[2], start[3]};
    }
    int w[kMaxParts] = {0, 0, 0, 0};
    int rmax = 0;  // the running maximum of parts: the pass of this slot
    each_active([&](int v) {
      const int pv = (int)a.part_of((uint32_t)v);
      rmax = pv > rmax ? pv : rmax;
      const int p = rmax;
      const int at = p == 0 ? start[0] + w[0]++ : p == 1 ? start[1] + w[1]++ : p == 2 ? start[2] + w[2]++ : start[3] + w[3]++;
      L.list[at] = v;
    });
    return;
  }
  int *dst = STAGE ? rows + rl * (kpad + 1) : L.list + r * kpad;
  if (STAGE || r < Bpad) {
    int j = 0;
    if (regrow) {
#pragma unroll
      for (int u = 0; u < kRegRow; ++u)
#pragma unroll
        for (int e = 0; e < 4; ++e)
          if ((unsigned)rv[u][e] < (unsigned)N) dst[j++] = rv[u][e];
    } else if (real && vec) {
#pragma unroll 4
      for (int k = 0; k < K; k += 4) {
        const i32x4 v4 = *reinterpret_cast<const i32x4 *>(row + k);
#pragma unroll
        for (int e = 0; e < 4; ++e)
          if ((unsigned)v4[e] < (unsigned)N) dst[j++] = v4[e];
      }
    } else if (real) {
      for (int k = 0; k < K; ++k) {
        const int v = slot(k);
        if ((unsigned)v < (unsigned)N) dst[j++] = v;
      }
    }
    for (; j < kpad; ++j) dst[j] = N;
  }
  if (STAGE && L.narrow) {  // entries <= N <= 65535
    __syncthreads();
    const int q8 = kpad / 8;
    i32x4 *out = reinterpret_cast<i32x4 *>(reinterpret_cast<uint16_t *>(L.list) + base * kpad);
    auto pack = [](int lo, int hi) { return (int)(((uint32_t)lo & 0xffffu) | ((uint32_t)hi << 16)); };
    for (int i = tid; i < kRankSortBlock * q8; i += kBlock) {
      const int rr = i / q8, q = i - rr * q8;
      if (base + rr >= Bpad) break;  // i ascending: every later piece is past Bpad too
      const int *src = rows + rr * (kpad + 1) + 8 * q;
      out[i] = i32x4{pack(src[0], src[1]), pack(src[2], src[3]), pack(src[4], src[5]), pack(src[6], src[7])};
    }
  } else if (STAGE) {
    __syncthreads();
    const int q4 = kpad / 4;
    i32x4 *out = reinterpret_cast<i32x4 *>(L.list + base * kpad);
    for (int i = tid; i < kRankSortBlock * q4; i += kBlock) {
      const int rr = i / q4, q = i - rr * q4;
      if (base + rr >= Bpad) break;  // i ascending: every later piece is past Bpad too
      const int *src = rows + rr * (kpad + 1) + 4 * q;
      out[i] = i32x4{src[0], src[1], src[2], src[3]};
    }
  }
}

template <bool STAGE>
__global__ __launch_bounds__(kBlock) void rank_lists_kernel(RankArgs a, int64_t B, int64_t Bpad, int K, int N,
                                                            int kpad, int vec) {
  rank_lists_block<STAGE>(a, (int)blockIdx.x, (int)blockIdx.y, B, Bpad, K, N, kpad, vec);
}

// Lists longer than the staged ones (K > 32, rows of 16-byte pieces): four
// threads per position, each holding a quarter of the row in registers from
// one batch of loads (nothing read twice), so a workgroup of 256 positions
// runs 16 waves instead of 4 and each thread walks a quarter of the slots.
// The quarters are combined across their four lanes with shuffles: the
// running maximum of parts enters quarter q as the maximum over quarters
// before it, and each pass's run takes the quarters' entries in quarter
// order.  Same outputs as rank_lists_kernel (pos, count, list; with table
// parts cut, roff and the packed runs).
constexpr int kWideSubs = 4;
constexpr int kWideBlock = kRankSortBlock * kWideSubs;  // 1024 threads
constexpr int kWideWindow = 12288;                      // list entries staged in LDS at once (48 KB)
template <int NL>  // 16-byte pieces per thread (quarters of up to 4 NL slots)
__global__ __launch_bounds__(kWideBlock) void rank_lists_wide_kernel(RankArgs a, int64_t B, int64_t Bpad, int K,
                                                                     int N, int kpad, int S) {
  extern __shared__ int sm[];  // bins[K + 1] | offsets[K + 1] | (parts) run scans [kMaxParts][256] | window
  unsigned *bin = reinterpret_cast<unsigned *>(sm), *off = bin + (K + 1);
  int *scan = sm + round_up4(2 * (K + 1));  // 16-byte aligned: the window after it is read in 16-byte pieces
  const RankLists &L = a.L[blockIdx.y];
  const int32_t *__restrict__ idx = a.idx[blockIdx.y];
  const int tid = threadIdx.x, j = tid % kWideSubs, lp = tid / kWideSubs;
  const int64_t base = (int64_t)blockIdx.x * kRankSortBlock;
  const int64_t b = base + lp;
  const bool real = b < B;
  const int32_t *row = idx + (real ? b : 0) * K;
  for (int i = tid; i <= K; i += kWideBlock) bin[i] = 0u;
  // quarter j = slots [j S, j S + S): every piece loaded first, from offsets
  // clamped into the row; pieces past K or S, and padding positions, read as -1
  i32x4 rv[NL];
#pragma unroll
  for (int u = 0; u < NL; ++u) {
    const int k = j * S + 4 * u;
    rv[u] = *reinterpret_cast<const i32x4 *>(row + (k < K - 4 ? k : K - 4));
  }
#pragma unroll
  for (int u = 0; u < NL; ++u)
    if (!real || 4 * u >= S || j * S + 4 * u >= K) rv[u] = i32x4{-1, -1, -1, -1};
  const bool parts = a.nparts > 1;  // launch-uniform
  auto part_of = [&](int v) { return parts ? (int)a.part_of((uint32_t)v) : 0; };
  // the quarter's highest part; the running maximum entering it (quarters before)
  int ml = 0;
#pragma unroll
  for (int u = 0; u < NL; ++u)
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int v = rv[u][e];
      ml = (unsigned)v < (unsigned)N ? max(ml, part_of(v)) : ml;
    }
  int incl = ml;
#pragma unroll
  for (int d = 1; d < kWideSubs; d <<= 1) {
    const int o = __shfl_up(incl, d, kWideSubs);
    if (j >= d) incl = max(incl, o);
  }
  int enter = __shfl_up(incl, 1, kWideSubs);
  if (j == 0) enter = 0;
  // the quarter's entries per pass (pass = running maximum of parts)
  int cp[kMaxParts] = {0, 0, 0, 0};
  {
    int rm = enter;
#pragma unroll
    for (int u = 0; u < NL; ++u)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int v = rv[u][e];
        const bool act = (unsigned)v < (unsigned)N;
        rm = act ? max(rm, part_of(v)) : rm;
#pragma unroll
        for (int q = 0; q < kMaxParts; ++q) cp[q] += (act && rm == q) ? 1 : 0;
      }
  }
  // per pass: entries of the quarters before this one, and the position's total
  int pre[kMaxParts], tot[kMaxParts];
#pragma unroll
  for (int q = 0; q < kMaxParts; ++q) {
    int s = cp[q];
#pragma unroll
    for (int d = 1; d < kWideSubs; d <<= 1) {
      const int o = __shfl_up(s, d, kWideSubs);
      if (j >= d) s += o;
    }
    pre[q] = s - cp[q];
    tot[q] = __shfl(s, kWideSubs - 1, kWideSubs);
  }
  const int c = tot[0] + tot[1] + tot[2] + tot[3];
  __syncthreads();  // bins cleared
  unsigned mine = 0u;
  if (j == 0 && real) mine = atomicAdd(&bin[c], 1u);
  __syncthreads();
  if (tid < kWave) {  // off[cc] = sum of bin[cc + 1 .. K], largest count first (as rank_lists_kernel)
    unsigned carry = 0u;
    for (int top = K; top >= 0; top -= kWave) {
      const int cc = top - tid;
      const unsigned v = cc >= 0 ? bin[cc] : 0u;
      unsigned sc = v;
#pragma unroll
      for (int d = 1; d < kWave; d <<= 1) {
        const unsigned o = __shfl_up(sc, d);
        if (tid >= d) sc += o;
      }
      if (cc >= 0) off[cc] = carry + sc - v;
      carry += __shfl(sc, kWave - 1);
    }
  }
  __syncthreads();
  mine = __shfl(mine, 0, kWideSubs);
  const int rl = real ? (int)(off[c] + mine) : lp;  // positions past B are the block's last (padding) ranks
  const int64_t r = base + rl;
  if (j == 0 && r < Bpad) {
    L.pos[r] = real ? (int32_t)b : -1;
    L.count[r] = real ? c : 0;
  }
  if (parts) {  // packed runs (see "Table parts"): pass p's run of a rank is tot[p] long
    if (j == 0) {
#pragma unroll
      for (int p = 0; p < kMaxParts; ++p) scan[p * kRankSortBlock + rl] = tot[p];
    }
    __syncthreads();
    {  // inclusive scans of the run lengths in rank order, one per pass: thread = (pass, rank)
      const int sp = tid / kRankSortBlock, si = tid % kRankSortBlock;
      int *col = scan + sp * kRankSortBlock;
      for (int d = 1; d < kRankSortBlock; d <<= 1) {
        const int v = col[si] + (si >= d ? col[si - d] : 0);
        __syncthreads();
        col[si] = v;
        __syncthreads();
      }
    }
    int start[kMaxParts];
    int64_t pbase = base * kpad;  // this block's region of the runs
#pragma unroll
    for (int p = 0; p < kMaxParts; ++p) {
      start[p] = (int)(pbase + scan[p * kRankSortBlock + rl] - tot[p]);
      pbase += scan[p * kRankSortBlock + kRankSortBlock - 1];
    }
    if (j == 0 && r < Bpad) {
      L.cut[r] = i32x4{tot[0], tot[0] + tot[1], tot[0] + tot[1] + tot[2], a.nparts - 1};
      L.roff[r] = i32x4{start[0], start[1], start[2], start[3]};
    }
    // The block's runs fill [base kpad, base kpad + total) of the list: they
    // are placed in LDS a window at a time (each thread walks its quarter
    // again from registers) and stored with coalesced 16-byte stores, instead
    // of a 4-byte store per entry scattered over the block's region.
    int *win = scan + kMaxParts * kRankSortBlock;
    const int total = (int)(pbase - base * kpad);
    int32_t *region = L.list + base * kpad;  // 16-byte aligned: kpad is a multiple of 4
    for (int w0 = 0; w0 < total; w0 += kWideWindow) {  // block-uniform
      int w[kMaxParts];
#pragma unroll
      for (int p = 0; p < kMaxParts; ++p) w[p] = start[p] - (int)(base * kpad) + pre[p] - w0;
      int rm = enter;
#pragma unroll
      for (int u = 0; u < NL; ++u)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int v = rv[u][e];
          if ((unsigned)v >= (unsigned)N) continue;
          rm = max(rm, part_of(v));
          const int at = rm == 0 ? w[0]++ : rm == 1 ? w[1]++ : rm == 2 ? w[2]++ : w[3]++;
          if ((unsigned)at < (unsigned)kWideWindow) win[at] = v;
        }
      __syncthreads();
      const int n = min(kWideWindow, total - w0);
      i32x4 *dst4 = reinterpret_cast<i32x4 *>(region + w0);
      const i32x4 *src4 = reinterpret_cast<const i32x4 *>(win);
      for (int i = tid; i < n / 4; i += kWideBlock) dst4[i] = src4[i];
      for (int i = (n & ~3) + tid; i < n; i += kWideBlock) region[w0 + i] = win[i];
      __syncthreads();
    }
    return;
  }
  if (r < Bpad) {
    int32_t *dst = L.list + r * kpad;
    int at = pre[0];
#pragma unroll
    for (int u = 0; u < NL; ++u)
#pragma unroll
      for (int e = 0; e < 4; ++e)
        if ((unsigned)rv[u][e] < (unsigned)N) dst[at++] = rv[u][e];
    for (int i = c + j; i < kpad; i += kWideSubs) dst[i] = N;
  }
}

// Chunk c (of 32 ranks) of a tile pass -> rank chunk: the longest lists
// first across all sort blocks -- chunk 0 of every block, then chunk 1 of
// every block, and so on (the last block may hold fewer chunks) -- so a tile
// pass starts with its longest items and ends with its shortest.
constexpr int kChunksPerSortBlock = kRankSortBlock / kRanksPerBlock;  // 8
__device__ __forceinline__ int64_t rank_chunk(int64_t c, int64_t nchunks) {
  const int64_t nb = (nchunks + kChunksPerSortBlock - 1) / kChunksPerSortBlock;  // sort blocks
  const int64_t last = nchunks - (nb - 1) * kChunksPerSortBlock;                 // chunks of the last block
  if (c < last * nb) return (c % nb) * kChunksPerSortBlock + c / nb;
  const int64_t c2 = c - last * nb;
  return (c2 % (nb - 1)) * kChunksPerSortBlock + last + c2 / (nb - 1);
}

// The whole lists of ranks r0 .. r0 + 7 (a wave's 8, padded to kpad) into the
// wave's LDS lists, 16-bit entries widened to ints.
__device__ __forceinline__ void stage_rank_lists(const RankLists &R, int64_t r0, int kpad, int *list, int lane) {
  constexpr int PPW = kWave / kTileCh;
  i32x4 *dst = reinterpret_cast<i32x4 *>(list);
  if (R.narrow) {  // launch-uniform
    const i32x4 *__restrict__ src =
        reinterpret_cast<const i32x4 *>(reinterpret_cast<const uint16_t *>(R.list) + r0 * kpad);
    for (int j = lane; j < PPW * kpad / 8; j += kWave) {
      const i32x4 v = src[j];
      const uint32_t w0 = (uint32_t)v[0], w1 = (uint32_t)v[1], w2 = (uint32_t)v[2], w3 = (uint32_t)v[3];
      dst[2 * j] = i32x4{(int)(w0 & 0xffffu), (int)(w0 >> 16), (int)(w1 & 0xffffu), (int)(w1 >> 16)};
      dst[2 * j + 1] = i32x4{(int)(w2 & 0xffffu), (int)(w2 >> 16), (int)(w3 & 0xffffu), (int)(w3 >> 16)};
    }
  } else {
    const i32x4 *__restrict__ src = reinterpret_cast<const i32x4 *>(R.list + r0 * kpad);
    for (int j = lane; j < PPW * kpad / 4; j += kWave) dst[j] = src[j];
  }
}

// Two perspectives share one launch: chunks [0, nchunks_p) read the rank
// lists R0 and write out0, chunks [nchunks_p, 2 nchunks_p) R1 and out1, so an
// XCD gathers both perspectives from a tile while it is in L2.  A
// single-perspective call passes the same lists twice and nchunks_p = nchunks.
// A chunk is 32 ranks, 8 per wave; the waves of a workgroup do not wait for
// each other.  With table parts the sums carried from pass to pass go to
// carry0 / carry1 (tile-major: tile t, position b at (t B + b) 8 chunks, one
// aligned 128-byte line each; the epilogue's raw tiles serve instead under
// EPI), not to the row-major outputs, whose 32-column slices straddle two
// lines three times in four at L = 1048.
template <bool EPI, bool PARTS>  // PARTS: nparts > 1
__global__ __launch_bounds__(kBlock) void fwd_tiled_kernel(RankLists R0, RankLists R1, int N,
                                                           const f32x4 *__restrict__ Wt, ColMap map,
                                                           const f32x4 *__restrict__ bias, f32x4 *__restrict__ out0,
                                                           f32x4 *__restrict__ out1, FwdEpilogue epi, int kpad,
                                                           int ntiles, int nchunks, int nchunks_p, int part,
                                                           int nparts, f32x4 *__restrict__ carry0,
                                                           f32x4 *__restrict__ carry1, int64_t B) {
  constexpr int PPW = kWave / kTileCh;  // 8 ranks per wave
  extern __shared__ int smem[];         // 8 lists of kpad entries per wave
  TileItem it = tile_sched_item(blockIdx.x, ntiles, nchunks);
  if (it.tile >= ntiles) return;  // whole block: uniform
  const bool second = it.chunk >= nchunks_p;
  if (second) it.chunk -= nchunks_p;
  const RankLists R = second ? R1 : R0;
  const int wave = uniform(threadIdx.x / kWave);
  const int lane = threadIdx.x % kWave;
  const int g = lane / kTileCh, t = lane % kTileCh;
  const int col = tile_col(map, it.tile, t);
  const bool colok = col >= 0;
  const int64_t col4 = col;
  const int64_t cols4 = map.cols4;
  const f32x4 b4 = colok ? bias[col4] : f32x4{0.f, 0.f, 0.f, 0.f};
  const char *tbase = reinterpret_cast<const char *>(Wt + (int64_t)it.tile * tile_rows(N) * kTileCh);
  const uint32_t lane_off = (uint32_t)t * (uint32_t)sizeof(f32x4);

  const int64_t r0 = rank_chunk(it.chunk, nchunks_p) * kRanksPerBlock + wave * PPW;  // the wave's first rank
  int *list = smem + wave * PPW * kpad;
  const int32_t *__restrict__ rp = R.pos + r0;
  int pos = rp[0];
#pragma unroll
  for (int u = 1; u < PPW; ++u) pos = g == u ? rp[u] : pos;
  f32x4 *__restrict__ raw = nullptr;
  const int64_t pz = pos < 0 ? 0 : pos;
  if (EPI) raw = (second ? epi.raw1 : epi.raw0) + (pz * ntiles + it.tile) * kTileCh + t;
  else if (PARTS) raw = (second ? carry1 : carry0) + ((int64_t)it.tile * B + pz) * kTileCh + t;
  // After the first pass, the sum earlier passes left, loaded first (every
  // lane: padding ranks load position 0's) and used when a pass did store it
  // (lo > 0 below).  Loaded before the run's bounds and entries instead of
  // beside the first rows: a pass at Full_Threats 541 -> 526 us.
  f32x4 carried = b4;
  if (PARTS && part > 0) carried = EPI ? *raw : __builtin_nontemporal_load(raw);  // launch-uniform
  int nmax, lo = 0;
  bool work = true, final_pass = true;
  if (!PARTS) {  // whole lists
    stage_rank_lists(R, r0, kpad, list, lane);
    nmax = R.count[r0];  // counts fall with rank within each 256 ranks: the wave's longest list
  } else {
    // this pass's run [lo, hi) of each list (table parts, above), padded with
    // the pad row to the wave's longest run
    const int64_t r = r0 + g;
    const i32x4 cv = R.cut[r];
    const int cnt = R.count[r];
    const int fin = cv[3];
    final_pass = part == fin;
    lo = part == 0 ? 0 : (part == 1 ? cv[0] : (part == 2 ? cv[1] : cv[2]));
    const int hi = final_pass ? cnt : (part == 0 ? cv[0] : (part == 1 ? cv[1] : cv[2]));
    work = part <= fin && (hi > lo || final_pass);
    const int len = work ? hi - lo : 0;
    int mx = len;
#pragma unroll
    for (int off = kTileCh; off < kWave; off <<= 1) mx = max(mx, __shfl_xor(mx, off));
    nmax = uniform(mx);
    const i32x4 ro = R.roff[r];
    // The run, four entries per lane per round: the loads of a round issued
    // first from indices clamped into the run (an empty run reads the list's
    // first entry), then the pad row past its end.  (Guarded one-entry loads
    // waited for each load in turn: a memory round trip per entry.)
    const int32_t *__restrict__ src =
        len > 0 ? R.list + (part == 0 ? ro[0] : (part == 1 ? ro[1] : (part == 2 ? ro[2] : ro[3]))) : R.list;
    const int last = len > 0 ? len - 1 : 0;
    int *dst = list + g * kpad;
    const int n4 = round_up4(nmax);
    for (int j0 = t; j0 < n4; j0 += 4 * kTileCh) {
      int v[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) v[u] = src[min(j0 + u * kTileCh, last)];
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int j = j0 + u * kTileCh;
        if (j < n4) dst[j] = j < len ? v[u] : N;
      }
    }
  }
  wave_lds_barrier();
  f32x4 acc = f32_tile_rows(list + g * kpad, nmax, tbase, lane_off, PARTS && lo > 0 && pos >= 0 && work ? carried : b4);
  if (!colok) acc = f32x4{0.f, 0.f, 0.f, 0.f};  // padding lanes read unwritten chunks; their raw rows stay 0
  if (pos < 0 || !work) return;                 // a padding rank, or nothing to do in this pass
  if (PARTS && !final_pass) {
    __builtin_nontemporal_store(acc, raw);
    return;
  }
  if (!EPI) {
    f32x4 *__restrict__ out = second ? out1 : out0;
    if (colok) __builtin_nontemporal_store(acc, out + pos * cols4 + col4);
  } else {
    __builtin_nontemporal_store(acc, raw);
    if (it.tile < map.t1) {  // block-uniform
      const f32x4 partner = shfl_xor4(acc, 4);
      if (t < 4 && colok) {
        const bool white_to_move = epi.us[pos] != 0.f;
        const int64_t half = (second ? white_to_move : !white_to_move) ? map.half4 : 0;
        const f32x4 pw = clamp01(acc) * clamp01(partner);
        const f32x4 v = pw * (127.0f / 128.0f);
        __builtin_nontemporal_store(v, epi.l0 + (int64_t)pos * (2 * (int64_t)map.half4) + half + col4);
      }
    }
  }
}

// psqt[b] = (white[b, L1 + k] - black[b, L1 + k]) * (us[b] - 0.5), k = psqt_idx[b]
// (src/model/model.py:110-114), read from the raw tiles; an index outside
// [0, P) gives 0.
__global__ __launch_bounds__(kBlock) void psqt_out_kernel(const f32x4 *__restrict__ raw0,
                                                          const f32x4 *__restrict__ raw1, ColMap map, int64_t B,
                                                          const float *__restrict__ us,
                                                          const int64_t *__restrict__ psqt_idx, int P,
                                                          float *__restrict__ psqt) {
  const int64_t b = (int64_t)blockIdx.x * kBlock + threadIdx.x;
  if (b >= B) return;
  const int64_t k = psqt_idx[b];
  float v = 0.f;
  if (k >= 0 && k < P) {
    int t, q;
    tile_of_col(map, 2 * map.half4 + (int)(k >> 2), t, q);
    const int64_t at = (b * map_tiles(map) + t) * kTileCh + q;
    const float w = raw0[at][k & 3], bl = raw1[at][k & 3];
    v = (w - bl) * (us[b] - 0.5f);
  }
  psqt[b] = v;
}

// ----------------------------------------------------- tiled int16 gather ----
// Same schedule as the fp32 tiled gather over an int16 table re-laid out in
// 64-column tiles (128 B per row; 2.9 MB per tile at N = 22 528).  Lane t of
// an 8-lane group owns 8 int16 columns accumulated in int32 (exact); the PSQT
// columns (P <= 8 int32 per row) are appended to every packed row as extra
// 16-byte chunks and summed by the lanes that hold them (i16_relayout_kernel).
// A tile is at most 64 MB, so row addresses are 32-bit offsets from the
// tile's (wave-uniform) base.
#ifndef SFT_I16_ROLL
#define SFT_I16_ROLL 1
#endif
#ifndef SFT_I16_TILED_U
#define SFT_I16_TILED_U 8
#endif
constexpr uint32_t kI16RowBytes = kTileCh * sizeof(i16x8);  // 128

typedef short i16x2 __attribute__((ext_vector_type(2)));

// acc[c] += w[c] over one row's 8 int16 columns.  v_dot2c_i32_i16 with the
// weights (1, 0) and (0, 1) adds one sign-extended half of a packed pair into
// an int32 (1·x is exact), two instructions per pair where widening costs an
// extract per half plus the adds.
__device__ __forceinline__ void add_pair_i16(i32x8 &acc, int j, i16x2 p) {
  const i16x2 lo = {1, 0}, hi = {0, 1};
  acc[2 * j] = __builtin_amdgcn_sdot2(p, lo, acc[2 * j], false);
  acc[2 * j + 1] = __builtin_amdgcn_sdot2(p, hi, acc[2 * j + 1], false);
}

__device__ __forceinline__ void add_row_i16(i32x8 &acc, i16x8 w) {
  add_pair_i16(acc, 0, __builtin_shufflevector(w, w, 0, 1));
  add_pair_i16(acc, 1, __builtin_shufflevector(w, w, 2, 3));
  add_pair_i16(acc, 2, __builtin_shufflevector(w, w, 4, 5));
  add_pair_i16(acc, 3, __builtin_shufflevector(w, w, 6, 7));
}

__device__ __forceinline__ i16x8 i16_row(const char *tbase, uint32_t lane_off, int f) {
  return *reinterpret_cast<const i16x8 *>(tbase + ((uint32_t)f * kI16RowBytes + lane_off));
}

// One position's rows of one tile: an unmasked main loop over the rows every
// lane of the 8-lane group has (nmin), then a masked tail up to nmax.  MIXED
// (block-uniform: the tile holds PSQT or padding lanes, see i16_relayout_kernel)
// masks the padding lanes' loads, so that they fetch nothing, and adds the PSQT
// lanes' four int32 columns as int32; in a pure int16 tile every lane loads.
template <bool MIXED>
__device__ __forceinline__ void i16_tile_rows(const int *mylist, int n, int nmin, int nmax, const char *tbase,
                                              uint32_t lane_off, bool live, bool is_psqt, i32x8 &acc) {
  constexpr int U = SFT_I16_TILED_U;
  static_assert(U % 4 == 0, "rows are read from the LDS list four at a time");
  auto add = [&](i16x8 w) {
    if (MIXED && is_psqt) {
      const i32x4 v = __builtin_bit_cast(i32x4, w);
      acc[0] += v[0], acc[1] += v[1], acc[2] += v[2], acc[3] += v[3];
    } else {
      add_row_i16(acc, w);
    }
  };
  int k = 0;
  if (SFT_I16_ROLL && !MIXED && nmin >= 2 * U) {
    // A rolling window of U rows in flight over the rows every lane group of
    // the wave has: each add frees the oldest row's registers, which take the
    // row U places further at once.  The first U loads are issued in the order
    // the loop consumes them, so each add waits for its own row only.  Same
    // adds, same order (integer adds: any order gives the same sums anyway).
    i16x8 w[U];
#pragma unroll
    for (int u = 0; u < U; u += 4) {
      const i32x4 f4 = read4(mylist, u);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        w[u + e] = i16_row(tbase, lane_off, f4[e]);
        __builtin_amdgcn_sched_barrier(0);
      }
    }
    for (k = U; k + U <= nmin; k += U) {
      int fi[U];
#pragma unroll
      for (int u = 0; u < U; u += 4) {
        const i32x4 f4 = read4(mylist, k + u);
        fi[u] = f4[0], fi[u + 1] = f4[1], fi[u + 2] = f4[2], fi[u + 3] = f4[3];
      }
#pragma unroll
      for (int u = 0; u < U; ++u) {
        add(w[u]);
        w[u] = i16_row(tbase, lane_off, fi[u]);
      }
    }
#pragma unroll
    for (int u = 0; u < U; ++u) add(w[u]);
  }
  for (; k + U <= nmin; k += U) {
    int fi[U];
#pragma unroll
    for (int u = 0; u < U; u += 4) {
      const i32x4 f4 = read4(mylist, k + u);
      fi[u] = f4[0], fi[u + 1] = f4[1], fi[u + 2] = f4[2], fi[u + 3] = f4[3];
    }
    i16x8 w[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      w[u] = (i16x8)0;
      if (!MIXED || live) w[u] = i16_row(tbase, lane_off, fi[u]);
    }
#pragma unroll
    for (int u = 0; u < U; ++u) add(w[u]);
  }
  for (; k < nmax; k += 4) {
    const i32x4 f4 = read4(mylist, k);
    i16x8 w[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      w[u] = (i16x8)0;
      if (k + u < n && (!MIXED || live)) w[u] = i16_row(tbase, lane_off, f4[u]);
    }
#pragma unroll
    for (int u = 0; u < 4; ++u) add(w[u]);
  }
}

// Lane chunk c = 8 * tile + t of the extended row: c < cols8 is int16 columns
// 8c .. 8c+7 (plus bias, clamped into out), cols8 <= c < cols8 + pch is PSQT
// columns 4j .. 4j+3 (j = c - cols8; into psqt_out, those < P), the rest is
// padding.  The PSQT columns thus ride in the last tile(s), which the schedule
// spreads over all XCDs, instead of loading every tile-0 workgroup.
// Two perspectives share a launch like the fp32 tiled gather: chunks
// [0, nchunks_p) read idx0 into out0 / psqt_out0, chunks [nchunks_p, nchunks)
// idx1 into out1 / psqt_out1; one perspective passes its arrays twice and
// nchunks_p = nchunks.
__global__ __launch_bounds__(kBlock) void fwd_i16_tiled_kernel(const int32_t *__restrict__ idx0,
                                                               const int32_t *__restrict__ idx1, int64_t B, int K,
                                                               int N, const i16x8 *__restrict__ Wt, int64_t cols8,
                                                               int pch, const i16x8 *__restrict__ bias, int P,
                                                               i16x8 *__restrict__ out0, i16x8 *__restrict__ out1,
                                                               int32_t *__restrict__ psqt_out0,
                                                               int32_t *__restrict__ psqt_out1, int clip_lo,
                                                               int clip_hi, int wrap16, int kpad, int ntiles,
                                                               int nchunks, int nchunks_p) {
  constexpr int PPW = kWave / kTileCh;
  static_assert(PPW <= kCompactRows, "compact_rows takes at most kCompactRows rows");
  extern __shared__ int smem[];
  TileItem it = tile_sched_item(blockIdx.x, ntiles, nchunks);
  if (it.tile >= ntiles) return;
  const bool second = it.chunk >= nchunks_p;  // block-uniform
  if (second) it.chunk -= nchunks_p;
  const int32_t *__restrict__ idx = second ? idx1 : idx0;
  i16x8 *__restrict__ out = second ? out1 : out0;
  int32_t *__restrict__ psqt_out = second ? psqt_out1 : psqt_out0;
  const int wave = uniform(threadIdx.x / kWave);
  const int lane = threadIdx.x % kWave;
  int *list = smem + wave * PPW * kpad;
  int *count = smem + kWavesPerBlock * PPW * kpad + wave * PPW;
  const int g = lane / kTileCh, t = lane % kTileCh;
  const int64_t col = (int64_t)it.tile * kTileCh + t;
  const bool colok = col < cols8;
  const bool is_psqt = !colok && col < cols8 + pch;
  const int pj = (int)(col - cols8) * 4;                     // first PSQT column of a PSQT lane
  const bool mixed = (int64_t)(it.tile + 1) * kTileCh > cols8;  // block-uniform
  const char *tbase = reinterpret_cast<const char *>(Wt + (int64_t)it.tile * N * kTileCh);
  const uint32_t lane_off = (uint32_t)t * (uint32_t)sizeof(i16x8);
  const i32x8 b8 = colok ? Q16<i16x8>::widen(bias[col]) : (i32x8)0;

  for (int round = 0; round < kTiledRounds; ++round) {
    const int64_t pos0 = (int64_t)it.chunk * kTiledPosPerBlock + round * kTiledPosPerRound + wave * PPW;
    compact_rows(idx, B, K, N, pos0, PPW, list, kpad, count);
    wave_lds_barrier();
    const int64_t pos = pos0 + g;
    const int n = count[g];
    int nmin, nmax;
    group_minmax<kTileCh>(n, nmin, nmax);
    const int *mylist = list + g * kpad;
    i32x8 acc = b8;
    if (mixed)
      i16_tile_rows<true>(mylist, n, nmin, nmax, tbase, lane_off, colok || is_psqt, is_psqt, acc);
    else
      i16_tile_rows<false>(mylist, n, nmin, nmax, tbase, lane_off, true, false, acc);
    if (pos < B) {
      if (colok) __builtin_nontemporal_store(Q16<i16x8>::finish(acc, clip_lo, clip_hi, wrap16), out + pos * cols8 + col);
      if (is_psqt) {
#pragma unroll
        for (int e = 0; e < 4; ++e)
          if (pj + e < P) psqt_out[pos * P + pj + e] = acc[e];
      }
    }
    wave_lds_barrier();
  }
}

// The int16 gather over rank lists (sft_ft_fwd_i16_packed_ex): the packed
// 64-column tiles of fwd_i16_tiled_kernel, gathered from the lists the fp32
// tiled gather uses (rank_lists_kernel, built once per call for both
// perspectives, 16-bit entries for tables of up to 65 535 rows) instead of
// compacting every position's index row again for each of the 17 column tiles.
// A wave's 8 ranks hold nearly the same number of rows: it steps its longest
// list with an unmasked loop up to its shortest.  The packed table has no pad
// row, so the entries past a rank's count are masked.
__global__ __launch_bounds__(kBlock) void fwd_i16_ranked_kernel(RankLists R0, RankLists R1, int N,
                                                                const i16x8 *__restrict__ Wt, int64_t cols8, int pch,
                                                                const i16x8 *__restrict__ bias, int P,
                                                                i16x8 *__restrict__ out0, i16x8 *__restrict__ out1,
                                                                int32_t *__restrict__ psqt_out0,
                                                                int32_t *__restrict__ psqt_out1, int clip_lo,
                                                                int clip_hi, int wrap16, int kpad, int ntiles,
                                                                int nchunks, int nchunks_p) {
  constexpr int PPW = kWave / kTileCh;  // 8 ranks per wave
  extern __shared__ int smem[];         // 8 lists of kpad entries per wave
  TileItem it = tile_sched_item(blockIdx.x, ntiles, nchunks);
  if (it.tile >= ntiles) return;  // whole block: uniform
  const bool second = it.chunk >= nchunks_p;  // block-uniform
  if (second) it.chunk -= nchunks_p;
  const RankLists R = second ? R1 : R0;
  i16x8 *__restrict__ out = second ? out1 : out0;
  int32_t *__restrict__ psqt_out = second ? psqt_out1 : psqt_out0;
  const int wave = uniform(threadIdx.x / kWave);
  const int lane = threadIdx.x % kWave;
  const int g = lane / kTileCh, t = lane % kTileCh;
  const int64_t col = (int64_t)it.tile * kTileCh + t;
  const bool colok = col < cols8;
  const bool is_psqt = !colok && col < cols8 + pch;
  const int pj = (int)(col - cols8) * 4;                        // first PSQT column of a PSQT lane
  const bool mixed = (int64_t)(it.tile + 1) * kTileCh > cols8;  // block-uniform
  const char *tbase = reinterpret_cast<const char *>(Wt + (int64_t)it.tile * N * kTileCh);
  const uint32_t lane_off = (uint32_t)t * (uint32_t)sizeof(i16x8);
  const i32x8 b8 = colok ? Q16<i16x8>::widen(bias[col]) : (i32x8)0;

  const int64_t r0 = rank_chunk(it.chunk, nchunks_p) * kRanksPerBlock + wave * PPW;  // the wave's first rank
  int *list = smem + wave * PPW * kpad;
  const int32_t *__restrict__ rp = R.pos + r0;
  const int32_t *__restrict__ rc = R.count + r0;
  int pos = rp[0], n = rc[0];
#pragma unroll
  for (int u = 1; u < PPW; ++u) {
    pos = g == u ? rp[u] : pos;
    n = g == u ? rc[u] : n;
  }
  const int nmax = uniform(rc[0]), nmin = uniform(rc[PPW - 1]);  // counts fall with rank within each 256 ranks
  stage_rank_lists(R, r0, kpad, list, lane);
  wave_lds_barrier();
  const int *mylist = list + g * kpad;
  i32x8 acc = b8;
  if (mixed)
    i16_tile_rows<true>(mylist, n, nmin, nmax, tbase, lane_off, colok || is_psqt, is_psqt, acc);
  else
    i16_tile_rows<false>(mylist, n, nmin, nmax, tbase, lane_off, true, false, acc);
  if (pos < 0) return;  // a padding rank
  if (colok) __builtin_nontemporal_store(Q16<i16x8>::finish(acc, clip_lo, clip_hi, wrap16), out + pos * cols8 + col);
  if (is_psqt) {
#pragma unroll
    for (int e = 0; e < 4; ++e)
      if (pj + e < P) psqt_out[(int64_t)pos * P + pj + e] = acc[e];
  }
}

// Extended int16 table in 64-column tiles: chunk c of row r (c < cols8: int16
// columns 8c .. 8c+7 of weight; else PSQT columns 4j .. 4j+3 of psqt, j =
// c - cols8, zero past P) goes to Wt[(t * N + r) * 8 + q], t = c / 8, q = c % 8.
// total = N * (cols8 + pch) chunks < 2^31.
__global__ __launch_bounds__(kBlock) void i16_relayout_kernel(const i16x8 *__restrict__ W, const int32_t *__restrict__ psqt,
                                                              int P, int64_t N, int cols8, int pch,
                                                              i16x8 *__restrict__ Wt) {
  const int cw = cols8 + pch;
  const int64_t total = N * cw;
  for (int64_t i = (int64_t)blockIdx.x * kBlock + threadIdx.x; i < total; i += (int64_t)gridDim.x * kBlock) {
    const int64_t r = i / cw;
    const int c = (int)(i - r * cw);
    i16x8 v;
    if (c < cols8) {
      v = W[r * cols8 + c];
    } else {
      const int j = 4 * (c - cols8);
      i32x4 p;
#pragma unroll
      for (int e = 0; e < 4; ++e) p[e] = j + e < P ? psqt[r * P + j + e] : 0;
      v = __builtin_bit_cast(i16x8, p);
    }
    Wt[((int64_t)(c / kTileCh) * N + r) * kTileCh + c % kTileCh] = v;
  }
}

// --------------------------------------------------------------- quantize ----
__global__ __launch_bounds__(kBlock) void quantize_i16_kernel(const float *__restrict__ x, int64_t n, float scale,
                                                              int16_t *__restrict__ out) {
  for (int64_t i = (int64_t)blockIdx.x * kBlock + threadIdx.x; i < n; i += (int64_t)gridDim.x * kBlock) {
    float r = __builtin_rintf(x[i] * scale);  // binary32 product, round half to even
    r = fminf(fmaxf(r, -32768.0f), 32767.0f);
    out[i] = (int16_t)r;
  }
}

// ------------------------------------------------------------- dispatch ----
template <typename T, int G, int CPL>
void launch_fwd_f32(dim3 grid, size_t lds, hipStream_t s, const int32_t *idx, int64_t B, int K, int N, const void *W,
                    int64_t cols, const void *bias, void *out, int kpad) {
  hipLaunchKernelGGL((fwd_f32_kernel<T, G, CPL, 4>), grid, dim3(kBlock), lds, s, idx, B, K, N,
                     static_cast<const T *>(W), cols, static_cast<const T *>(bias), static_cast<T *>(out), kpad);
}

template <typename T, int G, int CPL>
void launch_fwd_i16(dim3 grid, size_t lds, hipStream_t s, const int32_t *idx, int64_t B, int K, int N, const void *W,
                    int64_t cols, const void *bias, const int32_t *psqt, int P, void *out, int32_t *psqt_out, int lo,
                    int hi, int wrap16, int kpad) {
  hipLaunchKernelGGL((fwd_i16_kernel<T, G, CPL, 4>), grid, dim3(kBlock), lds, s, idx, B, K, N,
                     static_cast<const T *>(W), cols, static_cast<const T *>(bias), psqt, P, static_cast<T *>(out),
                     psqt_out, lo, hi, wrap16, kpad);
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

}  // namespace

// Wt[(t * (N + 1) + r) * 8 + q] = W[r, 4 * (8 t + q) .. +3], and row N of
// every tile = -0.0 (the pad row); the table's padding chunks of the last
// tile are not written.
// Workgroup b of g re-lays chunks b * kBlock + tid, + g * kBlock, ... out.
__device__ __forceinline__ void tile_relayout_part(int64_t b, int64_t g, const f32x4 *__restrict__ W, int64_t N,
                                                   int64_t cols4, f32x4 *__restrict__ Wt) {
  const int64_t body = N * cols4, total = body + ceil_div(cols4, (int64_t)8) * 8;
  const int64_t rows = tile_rows(N);
  for (int64_t i = b * kBlock + threadIdx.x; i < total; i += g * kBlock) {
    if (i < body) {
      const int64_t r = i / cols4, c = i % cols4;
      const int64_t t = c / 8, q = c % 8;
      Wt[(t * rows + r) * 8 + q] = W[i];
    } else {
      const int64_t t = (i - body) / 8, q = (i - body) % 8;
      Wt[(t * rows + N) * 8 + q] = f32x4{-0.f, -0.f, -0.f, -0.f};
    }
  }
}
static __global__ __launch_bounds__(kBlock) void tile_relayout_kernel(const f32x4 *__restrict__ W, int64_t N, int64_t cols4,
                                                               f32x4 *__restrict__ Wt) {
  tile_relayout_part(blockIdx.x, gridDim.x, W, N, cols4, Wt);
}

// The staged rank lists and the table re-layout in one launch: workgroups
// 0 .. nrank-1 build the rank lists (rank_lists_block, nrx per perspective),
// the others re-lay the table out.  Both only read the indices and the table,
// so they need no order between them, and the gather after them then waits for
// one launch instead of two back to back.
#ifndef SFT_FWD_FUSE_RANKS
#define SFT_FWD_FUSE_RANKS 1
#endif
static __global__ __launch_bounds__(kBlock) void relayout_rank_kernel(RankArgs a, int64_t B, int64_t Bpad, int K,
                                                                      int N, int kpad, int vec, int nrx, int nrank,
                                                                      const f32x4 *__restrict__ W, int64_t cols4,
                                                                      f32x4 *__restrict__ Wt) {
  if ((int)blockIdx.x < nrank) {  // whole block: uniform
    rank_lists_block<true>(a, (int)blockIdx.x % nrx, (int)blockIdx.x / nrx, B, Bpad, K, N, kpad, vec);
    return;
  }
  tile_relayout_part((int64_t)blockIdx.x - nrank, (int64_t)gridDim.x - nrank, W, N, cols4, Wt);
}

void launch_tile_relayout(const f32x4 *src, int64_t rows, int64_t cols4, f32x4 *dst, hipStream_t s) {
  const int64_t total = rows * cols4 + ceil_div(cols4, (int64_t)8) * 8;
  hipLaunchKernelGGL(tile_relayout_kernel, dim3((unsigned)std::min<int64_t>(ceil_div(total, kBlock), 1 << 16)),
                     dim3(kBlock), 0, s, src, rows, cols4, dst);
}

// Composed-table re-layout: merged row r of block s is w_s[r'] (+ v_s[r' %
// period_s] when the block has virtual rows; r' = r - start_s), added in
// binary32 exactly as the table the reference materialises
// (FEAT/halfka_v2_hm.py:69-70, FEAT/composed.py:49-50), and stored straight into
// the 32-column tiles of the tiled gather, each closed by its pad row of
// -0.0.  total = N * cols4 + 8 * ntiles < 2^31.
static __global__ __launch_bounds__(kBlock) void fold_relayout_kernel(FoldSrc src, int N, ColMap map,
                                                                      f32x4 *__restrict__ Wt) {
  const int cols4 = map.cols4;
  const int body = N * cols4, total = body + 8 * map_tiles(map);
  const int64_t rows = tile_rows(N);
  for (int i = blockIdx.x * kBlock + threadIdx.x; i < total; i += gridDim.x * kBlock) {
    if (i >= body) {
      const int t = (i - body) / 8, q = (i - body) % 8;
      Wt[((int64_t)t * rows + N) * 8 + q] = f32x4{-0.f, -0.f, -0.f, -0.f};
      continue;
    }
    const int r = i / cols4, c = i - r * cols4;
    const int s = block_of(r, src.n, src.start);
    const int rl = r - (int)pick(src.start, s);
    f32x4 x = pick(src.w, s)[(int64_t)rl * cols4 + c];
    const f32x4 *v = pick(src.v, s);
    if (v != nullptr) {
      const f32x4 y = v[(int64_t)(rl % (int)pick(src.period, s)) * cols4 + c];
      x += y;
    }
    int t, q;
    tile_of_col(map, c, t, q);
    Wt[((int64_t)t * rows + r) * 8 + q] = x;
  }
}

size_t index_lds_bytes(int G, int K) {
  const int ppw = kWave / G;
  return (size_t)(kWavesPerBlock * ppw * round_up4(K) + kWavesPerBlock * ppw) * sizeof(int);
}

int fwd_f32(const int32_t *idx, int64_t B, int K, const float *W, int64_t N, int L, const float *bias, float *out,
            hipStream_t s) {
  const bool vec = (L % 4 == 0) && ((uintptr_t)W % 16 == 0) && ((uintptr_t)bias % 16 == 0) &&
                   ((uintptr_t)out % 16 == 0);
  const int64_t cols = vec ? L / 4 : L;
  const Mapping m = choose_mapping(cols);
  const int ppb = kWavesPerBlock * (kWave / m.G);
  const dim3 grid((unsigned)ceil_div(B, ppb), (unsigned)m.slabs);
  const size_t lds = index_lds_bytes(m.G, K);
  if (lds > kMaxIndexLds) return fail(SFT_EUNSUPPORTED, "sft_ft_fwd_f32: max_active too large for the LDS index lists");
  const int kpad = round_up4(K);
  ProfScope prof(kProfFwdF32, s);
  if (vec) {
    SFT_G_CASES(launch_fwd_f32, f32x4, grid, lds, s, idx, B, K, (int)N, W, cols, bias, out, kpad)
  } else {
    SFT_G_CASES(launch_fwd_f32, float, grid, lds, s, idx, B, K, (int)N, W, cols, bias, out, kpad)
  }
  return check_launch("sft_ft_fwd_f32");
}

static size_t align256(size_t v) { return (v + 255) & ~(size_t)255; }

// ---- rank lists (host side) ----
static int64_t rank_pad(int64_t B) { return ceil_div(B, (int64_t)kRanksPerBlock) * kRanksPerBlock; }
// One perspective's rank lists, each array 256-byte aligned.
size_t rank_lists_bytes(int64_t B, int K) {
  const int64_t Bp = rank_pad(B);
  return align256((size_t)(Bp * round_up4(K)) * 4) + 2 * align256((size_t)Bp * 4) + 2 * align256((size_t)Bp * 16);
}
static RankLists rank_lists_at(char *p, int64_t B, int K, int narrow) {
  const int64_t Bp = rank_pad(B);
  RankLists r;
  r.narrow = narrow;
  r.list = reinterpret_cast<int32_t *>(p);
  p += align256((size_t)(Bp * round_up4(K)) * 4);
  r.pos = reinterpret_cast<int32_t *>(p);
  p += align256((size_t)Bp * 4);
  r.count = reinterpret_cast<int32_t *>(p);
  p += align256((size_t)Bp * 4);
  r.cut = reinterpret_cast<i32x4 *>(p);
  p += align256((size_t)Bp * 16);
  r.roff = reinterpret_cast<i32x4 *>(p);
  return r;
}

// Table parts of a gather over N rows (see "Table parts"): as many as keep a
// part's tile rows within SFT_FWD_PART_BYTES, at most kMaxParts.
// Rank lists of K > 32 built by four threads per position (rank_lists_wide_kernel).
#ifndef SFT_FWD_WIDE_RANKS
#define SFT_FWD_WIDE_RANKS 1
#endif
#ifndef SFT_FWD_PART_BYTES
#define SFT_FWD_PART_BYTES (7 << 19)
#endif
static int table_parts(int64_t N) {
  const int64_t p = ceil_div(tile_rows(N) * (int64_t)kTileRowBytes, (int64_t)(SFT_FWD_PART_BYTES));
  return (int)std::min<int64_t>(std::max<int64_t>(p, 1), kMaxParts);
}
static int part_rows_of(int64_t N, int nparts) { return (int)ceil_div(std::max<int64_t>(N, 1), nparts); }
// LDS of the tiled gather: the 32 lists of a workgroup.
static size_t rank_lds_bytes(int K) { return (size_t)kRanksPerBlock * round_up4(K) * sizeof(int); }
// Lists staged in LDS up to kpad = 32 (33 KB); longer ones are stored by their threads.
constexpr int kRankStageMaxPad = 32;
static_assert(kRankStageMaxPad == 32, "rank_lists_kernel holds a staged row in 8 16-byte registers");
// 16-bit lists: one table pass, entries up to N <= 65535, staged rows of 8-entry pieces.
static int lists_narrow(int K, int64_t N, int nparts) {
  const int kpad = round_up4(K);
  return nparts == 1 && N <= 65535 && kpad % 8 == 0 && kpad <= kRankStageMaxPad;
}

// Rank lists of np perspectives (idx[p] -> R[p]) in one launch.
// With relay_W, the table re-layout into relay_Wt too: in the same launch as
// the staged rank lists when SFT_FWD_FUSE_RANKS, else launched first.
static int build_rank_lists(const int32_t *idx0, const int32_t *idx1, int np, int64_t B, int K, int N,
                            const RankLists &R0, const RankLists &R1, int nparts, hipStream_t s, const char *who,
                            const f32x4 *relay_W = nullptr, int64_t relay_cols4 = 0, f32x4 *relay_Wt = nullptr) {
  RankArgs a;
  a.idx[0] = idx0;
  a.idx[1] = idx1;
  a.L[0] = R0;
  a.L[1] = R1;
  a.nparts = nparts;
  a.part_rows = part_rows_of(N, nparts);
  a.part_of = FastDiv((uint32_t)a.part_rows);
  const int64_t Bp = rank_pad(B);
  const int kpad = round_up4(K);
  const int vec = K % 4 == 0 && (uintptr_t)idx0 % 16 == 0 && (uintptr_t)idx1 % 16 == 0;
  const bool stage = kpad <= kRankStageMaxPad;
  if (nparts > 1 && Bp * kpad > (int64_t)INT32_MAX)
    return fail(SFT_EUNSUPPORTED, std::string(who) + ": batch x max_active too large for the packed table-part runs");
  if ((R0.narrow || R1.narrow) && (!stage || kpad % 8 != 0 || N > 65535))
    return fail(SFT_EINVAL, std::string(who) + ": 16-bit rank lists need staged lists of 8-entry pieces");
  const size_t rows_lds = stage ? (size_t)kRankSortBlock * (kpad + 1) * 4 : 0;
  const size_t scan_lds = nparts > 1 ? (size_t)kMaxParts * kRankSortBlock * 4 : 0;  // run scans, over the rows
  const size_t lds = (size_t)(2 * (K + 1)) * 4 + std::max(rows_lds, scan_lds);
  const dim3 grid((unsigned)ceil_div(Bp, (int64_t)kRankSortBlock), (unsigned)np);
  if (relay_W != nullptr && SFT_FWD_FUSE_RANKS && stage && lds <= kMaxIndexLds) {
    ProfScope prof(kProfFwdRelayout, s);
    const int64_t total = (int64_t)N * relay_cols4 + ceil_div(relay_cols4, (int64_t)8) * 8;
    const int nrank = (int)(grid.x * grid.y);
    const int64_t nrel = std::min<int64_t>(ceil_div(total, kBlock), 1 << 16);
    hipLaunchKernelGGL(relayout_rank_kernel, dim3((unsigned)(nrank + nrel)), dim3(kBlock), lds, s, a, B, Bp, K, N,
                       kpad, vec, (int)grid.x, nrank, relay_W, relay_cols4, relay_Wt);
    return check_launch((std::string(who) + " (re-layout and rank lists)").c_str());
  }
  if (relay_W != nullptr) {
    {
      ProfScope prof(kProfFwdRelayout, s);
      launch_tile_relayout(relay_W, N, relay_cols4, relay_Wt, s);
    }
    const int rc = check_launch((std::string(who) + " (relayout)").c_str());
    if (rc != SFT_OK) return rc;
  }
  ProfScope prof(kProfFwdRanks, s);
  // longer lists: four threads per position, quarters of S slots (whole 16-byte pieces)
  const int S = round_up4((K + kWideSubs - 1) / kWideSubs);
  if (SFT_FWD_WIDE_RANKS && !stage && vec && S <= 48) {  // up to K = 192 (12 pieces a thread, no spills)
    const size_t wlds =
        (size_t)round_up4(2 * (K + 1)) * 4 + (nparts > 1 ? (size_t)(kMaxParts * kRankSortBlock + kWideWindow) * 4 : 0);
#define SFT_WIDE_RANKS(NL)                                                                                        \
  hipLaunchKernelGGL(rank_lists_wide_kernel<NL>, grid, dim3(kWideBlock), wlds, s, a, B, Bp, K, N, kpad, S)
    const int nl = S / 4;
    if (nl <= 4) SFT_WIDE_RANKS(4);
    else if (nl <= 6) SFT_WIDE_RANKS(6);
    else if (nl <= 8) SFT_WIDE_RANKS(8);
    else if (nl <= 10) SFT_WIDE_RANKS(10);
    else SFT_WIDE_RANKS(12);
#undef SFT_WIDE_RANKS
  } else if (stage)
    hipLaunchKernelGGL(rank_lists_kernel<true>, grid, dim3(kBlock), lds, s, a, B, Bp, K, N, kpad, vec);
  else
    hipLaunchKernelGGL(rank_lists_kernel<false>, grid, dim3(kBlock), lds, s, a, B, Bp, K, N, kpad, vec);
  return check_launch((std::string(who) + " (rank lists)").c_str());
}

// Table tiles (with their pad rows), then the rank lists of one perspective.
// Table tiles, rank lists, then (table parts) the carried sums.
static size_t carry_bytes(int64_t ntiles, int64_t B) { return align256((size_t)(ntiles * B) * kTileRowBytes); }
size_t fwd_tiled_workspace(int64_t B, int K, int64_t N, int L) {
  if (L % 4 != 0) return 0;
  const int64_t ntiles = ceil_div(L, kTileF);
  return align256((size_t)(ntiles * tile_rows(N) * kTileF) * sizeof(float)) + rank_lists_bytes(B, K) +
         (table_parts(N) > 1 ? carry_bytes(ntiles, B) : 0);
}

#ifndef SFT_FWD_TILE_MAX_BYTES
#define SFT_FWD_TILE_MAX_BYTES (64ll << 20)
#endif
// The fp32 forward tiles from 4 column tiles up (L > 96): at L = 136 (5 tiles)
// the tiled gather and its re-layout take 86 us against 95 us for the row
// gather.
#ifndef SFT_FWD_MIN_TILES
#define SFT_FWD_MIN_TILES 4
#endif
bool fwd_tiled_supported(int64_t N, int L, const void *W, const void *bias, const void *out) {
  return L % 4 == 0 && ceil_div(L, kTileF) >= SFT_FWD_MIN_TILES && N * kTileF * 4 <= (int64_t)(SFT_FWD_TILE_MAX_BYTES) &&
         (uintptr_t)W % 16 == 0 && (uintptr_t)bias % 16 == 0 && (uintptr_t)out % 16 == 0;
}

int fwd_f32_tiled(const int32_t *idx, int64_t B, int K, const float *W, int64_t N, int L, const float *bias, float *out,
                  void *ws, size_t ws_bytes, hipStream_t s) {
  const char *who = "sft_ft_fwd_f32_ex";
  if (ws_bytes < fwd_tiled_workspace(B, K, N, L) || ws == nullptr || (uintptr_t)ws % 256 != 0)
    return fail(SFT_EWORKSPACE, "sft_ft_fwd_f32_ex: workspace smaller than sft_ft_fwd_f32_workspace_size() "
                                "or not 256-byte aligned");
  const int64_t cols4 = L / 4;
  const int ntiles = (int)ceil_div(L, kTileF);
  const int kpad = round_up4(K);
  const size_t lds = rank_lds_bytes(K);
  if (lds > kMaxIndexLds) return fail(SFT_EUNSUPPORTED, "sft_ft_fwd_f32_ex: max_active too large for the LDS index lists");
  f32x4 *wt = static_cast<f32x4 *>(ws);
  const int nparts = table_parts(N);
  char *lists = static_cast<char *>(ws) + align256((size_t)(ntiles * tile_rows(N) * kTileF) * 4);
  const RankLists R = rank_lists_at(lists, B, K, lists_narrow(K, N, nparts));
  f32x4 *carry = nparts > 1 ? reinterpret_cast<f32x4 *>(lists + rank_lists_bytes(B, K)) : nullptr;
  int rc = build_rank_lists(idx, idx, 1, B, K, (int)N, R, R, nparts, s, who, reinterpret_cast<const f32x4 *>(W), cols4,
                            wt);
  if (rc != SFT_OK) return rc;
  const int nchunks = (int)(rank_pad(B) / kRanksPerBlock);
  const int64_t blocks = tile_sched_items_per_xcd(ntiles, nchunks) * kXcds;
  for (int part = 0; part < nparts; ++part) {
    ProfScope prof(kProfFwdTiled, s);
    hipLaunchKernelGGL((nparts > 1 ? fwd_tiled_kernel<false, true> : fwd_tiled_kernel<false, false>),
                       dim3((unsigned)blocks), dim3(kBlock), lds, s, R, R, (int)N, wt,
                       plain_map((int)cols4), reinterpret_cast<const f32x4 *>(bias), reinterpret_cast<f32x4 *>(out),
                       reinterpret_cast<f32x4 *>(out), FwdEpilogue{}, kpad, ntiles, nchunks, nchunks, part, nparts,
                       carry, carry, B);
    if ((rc = check_launch("sft_ft_fwd_f32_ex (tiled gather)")) != SFT_OK) return rc;
  }
  return SFT_OK;
}

size_t map_tiles_workspace(const ColMap &m, int64_t rows) { return (size_t)map_tiles(m) * (size_t)rows * 128; }
// The fp32 table tiles of a column map (with their pad rows).
size_t table_tiles_workspace(const ColMap &m, int64_t N) { return map_tiles_workspace(m, tile_rows(N)); }
// Forward workspace of a two-perspective call: the table tiles, then both
// perspectives' rank lists, then (carry: plain outputs and table parts) both
// perspectives' carried sums.
size_t fwd_pair_workspace(const ColMap &m, int64_t B, int K, int64_t N, bool carry) {
  return align256(table_tiles_workspace(m, N)) + 2 * rank_lists_bytes(B, K) +
         (carry && table_parts(N) > 1 ? 2 * carry_bytes(map_tiles(m), B) : 0);
}

// Fold re-layout of the composed table into the workspace's tiles, rank lists
// of both perspectives after them, then one tiled gather of both perspectives
// (plain outputs, or the post-FT epilogue when epi.l0 is set).
static int pair_gather(const int32_t *idx0, const int32_t *idx1, int64_t B, int K, const FoldSrc &src, int64_t N,
                       const ColMap &map, const float *bias, float *out0, float *out1, const FwdEpilogue &epi,
                       void *ws, hipStream_t s, const char *who) {
  const int ntiles = map_tiles(map);
  const int kpad = round_up4(K);
  const size_t lds = rank_lds_bytes(K);
  f32x4 *wt = static_cast<f32x4 *>(ws);
  char *lists = static_cast<char *>(ws) + align256(table_tiles_workspace(map, N));
  const int nparts = table_parts(N);
  const int narrow = lists_narrow(K, N, nparts);
  const RankLists R0 = rank_lists_at(lists, B, K, narrow),
                  R1 = rank_lists_at(lists + rank_lists_bytes(B, K), B, K, narrow);
  f32x4 *carry0 = nullptr, *carry1 = nullptr;
  if (epi.l0 == nullptr && nparts > 1) {
    carry0 = reinterpret_cast<f32x4 *>(lists + 2 * rank_lists_bytes(B, K));
    carry1 = reinterpret_cast<f32x4 *>(lists + 2 * rank_lists_bytes(B, K) + carry_bytes(ntiles, B));
  }
  if (lds > kMaxIndexLds) return fail(SFT_EUNSUPPORTED, std::string(who) + ": max_active too large for the LDS index lists");
  if (tile_rows(N) * (int64_t)kTileRowBytes > (int64_t)UINT32_MAX)
    return fail(SFT_EUNSUPPORTED, std::string(who) + ": more than 2^25 - 1 table rows");
  {
    ProfScope prof(kProfFwdFold, s);
    const int64_t total = N * map.cols4 + 8 * ntiles;
    hipLaunchKernelGGL(fold_relayout_kernel, dim3((unsigned)std::min<int64_t>(ceil_div(total, kBlock), 1 << 16)),
                       dim3(kBlock), 0, s, src, (int)N, map, wt);
  }
  int rc = check_launch(who);
  if (rc != SFT_OK || B == 0) return rc;
  if ((rc = build_rank_lists(idx0, idx1, 2, B, K, (int)N, R0, R1, nparts, s, who)) != SFT_OK) return rc;
  const int nchunks_p = (int)(rank_pad(B) / kRanksPerBlock);
  const int64_t blocks = tile_sched_items_per_xcd(ntiles, 2 * nchunks_p) * kXcds;
  for (int part = 0; part < nparts; ++part) {
    ProfScope prof(kProfFwdTiled, s);
    if (epi.l0 != nullptr)
      hipLaunchKernelGGL((nparts > 1 ? fwd_tiled_kernel<true, true> : fwd_tiled_kernel<true, false>),
                         dim3((unsigned)blocks), dim3(kBlock), lds, s, R0, R1, (int)N, wt,
                         map, reinterpret_cast<const f32x4 *>(bias), (f32x4 *)nullptr, (f32x4 *)nullptr, epi, kpad,
                         ntiles, 2 * nchunks_p, nchunks_p, part, nparts, carry0, carry1, B);
    else
      hipLaunchKernelGGL((nparts > 1 ? fwd_tiled_kernel<false, true> : fwd_tiled_kernel<false, false>),
                         dim3((unsigned)blocks), dim3(kBlock), lds, s, R0, R1, (int)N, wt,
                         map, reinterpret_cast<const f32x4 *>(bias), reinterpret_cast<f32x4 *>(out0),
                         reinterpret_cast<f32x4 *>(out1), epi, kpad, ntiles, 2 * nchunks_p, nchunks_p, part, nparts,
                         carry0, carry1, B);
    if ((rc = check_launch(who)) != SFT_OK) return rc;
  }
  return SFT_OK;
}

int fwd_pair_f32(const int32_t *idx0, const int32_t *idx1, int64_t B, int K, const FoldSrc &src, int64_t N, int L,
                 const float *bias, float *out0, float *out1, void *ws, size_t ws_bytes, hipStream_t s) {
  const ColMap map = plain_map(L / 4);
  if (ws_bytes < fwd_pair_workspace(map, B, K, N, true) || ws == nullptr || (uintptr_t)ws % 256 != 0)
    return fail(SFT_EWORKSPACE, "sft_ft_fwd_pair_f32: workspace smaller than sft_ft_pair_workspace_size() "
                                "or not 256-byte aligned");
  return pair_gather(idx0, idx1, B, K, src, N, map, bias, out0, out1, FwdEpilogue{}, ws, s, "sft_ft_fwd_pair_f32");
}

// Forward of the composed table with the post-FT epilogue.  `saved` holds the
// raw pre-activations of both perspectives in paired tiles (map_tiles x B x
// 128 B each) for the backward; `ws` the table tiles and rank lists.
int fwd_transform_f32(const int32_t *idx0, const int32_t *idx1, int64_t B, int K, const FoldSrc &src, int64_t N,
                      int L, int L1, const float *bias, const float *us, const int64_t *psqt_idx, float *l0,
                      float *psqt, void *saved, size_t saved_bytes, void *ws, size_t ws_bytes, hipStream_t s) {
  const ColMap map = paired_map(L / 4, L1 / 8);
  const size_t raw_bytes = map_tiles_workspace(map, B);
  if (ws_bytes < fwd_pair_workspace(map, B, K, N, false) || ws == nullptr || (uintptr_t)ws % 256 != 0 ||
      saved_bytes < 2 * raw_bytes || saved == nullptr || (uintptr_t)saved % 256 != 0)
    return fail(SFT_EWORKSPACE, "sft_ft_fwd_transform_f32: saved or workspace buffer smaller than "
                                "sft_ft_transform_workspace_size() or not 256-byte aligned");
  FwdEpilogue epi;
  epi.us = us;
  epi.l0 = reinterpret_cast<f32x4 *>(l0);
  epi.raw0 = static_cast<f32x4 *>(saved);
  epi.raw1 = reinterpret_cast<f32x4 *>(static_cast<char *>(saved) + raw_bytes);
  int rc = pair_gather(idx0, idx1, B, K, src, N, map, bias, nullptr, nullptr, epi, ws, s,
                       "sft_ft_fwd_transform_f32");
  if (rc != SFT_OK || B == 0) return rc;
  hipLaunchKernelGGL(psqt_out_kernel, dim3((unsigned)ceil_div(B, kBlock)), dim3(kBlock), 0, s, epi.raw0, epi.raw1,
                     map, B, us, psqt_idx, L - L1, psqt);
  return check_launch("sft_ft_fwd_transform_f32 (psqt)");
}

// PSQT chunks of 4 int32 columns appended to the L / 8 int16 chunks of a row.
static int i16_psqt_chunks(int P) { return P > 0 ? (P + 3) / 4 : 0; }

size_t fwd_i16_tiled_workspace(int64_t N, int L, int P) {
  if (L % 8 != 0) return 0;
  const int64_t ntiles = ceil_div(L / 8 + i16_psqt_chunks(P), kTileCh);
  return (size_t)(ntiles * N * kTileCh) * 16;
}

bool fwd_i16_tiled_supported(int64_t N, int L, int P, const void *W, const void *bias, const void *out) {
  return L % 8 == 0 && ceil_div(L / 8, kTileCh) >= kMinTiles && N * 128 <= (int64_t)(SFT_FWD_TILE_MAX_BYTES) && P <= 8 &&
         (uintptr_t)W % 16 == 0 && (uintptr_t)bias % 16 == 0 && (uintptr_t)out % 16 == 0;
}

int i16_pack(const int16_t *W, int64_t N, int L, const int32_t *psqt, int P, void *packed, size_t bytes,
             hipStream_t s, const char *who) {
  if (bytes < fwd_i16_tiled_workspace(N, L, P) || packed == nullptr || (uintptr_t)packed % 256 != 0)
    return fail(SFT_EWORKSPACE, std::string(who) + ": buffer smaller than the packed table size or not 256-byte aligned");
  const int cols8 = L / 8;
  const int pch = i16_psqt_chunks(P);
  {
    ProfScope prof(kProfFwdRelayout, s);
    const int64_t total = N * (cols8 + pch);
    hipLaunchKernelGGL(i16_relayout_kernel, dim3((unsigned)std::min<int64_t>(ceil_div(total, kBlock), 1 << 16)),
                       dim3(kBlock), 0, s, reinterpret_cast<const i16x8 *>(W), psqt, P, N, cols8, pch,
                       static_cast<i16x8 *>(packed));
  }
  return check_launch((std::string(who) + " (pack)").c_str());
}

int fwd_i16_packed(const int32_t *idx0, const int32_t *idx1, int64_t B, int K, const void *packed, int64_t N, int L,
                   const int16_t *bias, int P, int16_t *out0, int16_t *out1, int32_t *psqt_out0, int32_t *psqt_out1,
                   int lo, int hi, int wrap16, hipStream_t s, const char *who) {
  const int cols8 = L / 8;
  const int pch = i16_psqt_chunks(P);
  const int ntiles = (int)ceil_div(cols8 + pch, kTileCh);
  const int kpad = round_up4(K);
  const size_t lds = index_lds_bytes(kTileCh, K);
  if (lds > kMaxIndexLds) return fail(SFT_EUNSUPPORTED, std::string(who) + ": max_active too large for the LDS index lists");
  if (B == 0) return SFT_OK;
  const int nchunks_p = (int)ceil_div(B, kTiledPosPerBlock);
  const int persp = idx1 != nullptr ? 2 : 1;
  const int64_t blocks = tile_sched_items_per_xcd(ntiles, persp * nchunks_p) * kXcds;
  {
    ProfScope prof(kProfFwdI16Tiled, s);
    hipLaunchKernelGGL(fwd_i16_tiled_kernel, dim3((unsigned)blocks), dim3(kBlock), lds, s, idx0,
                       persp == 2 ? idx1 : idx0, B, K, (int)N, static_cast<const i16x8 *>(packed), (int64_t)cols8,
                       pch, reinterpret_cast<const i16x8 *>(bias), P, reinterpret_cast<i16x8 *>(out0),
                       reinterpret_cast<i16x8 *>(persp == 2 ? out1 : out0), psqt_out0,
                       persp == 2 ? psqt_out1 : psqt_out0, lo, hi, wrap16, kpad, ntiles, persp * nchunks_p,
                       nchunks_p);
  }
  return check_launch((std::string(who) + " (tiled gather)").c_str());
}

// Workspace of the ranked int16 gather: the rank lists of each perspective.
size_t fwd_i16_ranked_workspace(int64_t B, int K, int persp) { return (size_t)persp * rank_lists_bytes(B, K); }

// fwd_i16_packed over rank lists built in the workspace (fwd_i16_ranked_kernel).
int fwd_i16_packed_ranked(const int32_t *idx0, const int32_t *idx1, int64_t B, int K, const void *packed, int64_t N,
                          int L, const int16_t *bias, int P, int16_t *out0, int16_t *out1, int32_t *psqt_out0,
                          int32_t *psqt_out1, int lo, int hi, int wrap16, void *ws, size_t ws_bytes, hipStream_t s,
                          const char *who) {
  const int persp = idx1 != nullptr ? 2 : 1;
  if (ws_bytes < fwd_i16_ranked_workspace(B, K, persp) || ws == nullptr || (uintptr_t)ws % 256 != 0)
    return fail(SFT_EWORKSPACE, std::string(who) + ": workspace smaller than sft_ft_fwd_i16_packed_workspace_size() "
                                                   "or not 256-byte aligned");
  const int cols8 = L / 8;
  const int pch = i16_psqt_chunks(P);
  const int ntiles = (int)ceil_div(cols8 + pch, kTileCh);
  const int kpad = round_up4(K);
  const size_t lds = rank_lds_bytes(K);
  if (lds > kMaxIndexLds) return fail(SFT_EUNSUPPORTED, std::string(who) + ": max_active too large for the LDS index lists");
  if (B == 0) return SFT_OK;
  const int narrow = lists_narrow(K, N, 1);
  char *w = static_cast<char *>(ws);
  const RankLists R0 = rank_lists_at(w, B, K, narrow);
  const RankLists R1 = persp == 2 ? rank_lists_at(w + rank_lists_bytes(B, K), B, K, narrow) : R0;
  int rc = build_rank_lists(idx0, persp == 2 ? idx1 : idx0, persp, B, K, (int)N, R0, R1, 1, s, who);
  if (rc != SFT_OK) return rc;
  const int nchunks_p = (int)(rank_pad(B) / kRanksPerBlock);
  const int64_t blocks = tile_sched_items_per_xcd(ntiles, persp * nchunks_p) * kXcds;
  {
    ProfScope prof(kProfFwdI16Tiled, s);
    hipLaunchKernelGGL(fwd_i16_ranked_kernel, dim3((unsigned)blocks), dim3(kBlock), lds, s, R0, R1, (int)N,
                       static_cast<const i16x8 *>(packed), (int64_t)cols8, pch, reinterpret_cast<const i16x8 *>(bias),
                       P, reinterpret_cast<i16x8 *>(out0), reinterpret_cast<i16x8 *>(persp == 2 ? out1 : out0),
                       psqt_out0, persp == 2 ? psqt_out1 : psqt_out0, lo, hi, wrap16, kpad, ntiles,
                       persp * nchunks_p, nchunks_p);
  }
  return check_launch((std::string(who) + " (ranked gather)").c_str());
}

// Workspace of the per-call tiled int16 forward: the packed table, then the rank lists.
size_t fwd_i16_ex_workspace(int64_t B, int K, int64_t N, int L, int P) {
  return align256(fwd_i16_tiled_workspace(N, L, P)) + fwd_i16_ranked_workspace(B, K, 1);
}

int fwd_i16_tiled(const int32_t *idx, int64_t B, int K, const int16_t *W, int64_t N, int L, const int16_t *bias,
                  const int32_t *psqt, int P, int16_t *out, int32_t *psqt_out, int lo, int hi, int wrap16, void *ws,
                  size_t ws_bytes, hipStream_t s) {
  const char *who = "sft_ft_fwd_i16_ex";
  if (ws_bytes < fwd_i16_ex_workspace(B, K, N, L, P) || ws == nullptr || (uintptr_t)ws % 256 != 0)
    return fail(SFT_EWORKSPACE, "sft_ft_fwd_i16_ex: workspace smaller than sft_ft_fwd_i16_workspace_size() "
                                "or not 256-byte aligned");
  if (rank_lds_bytes(K) > kMaxIndexLds)
    return fail(SFT_EUNSUPPORTED, "sft_ft_fwd_i16_ex: max_active too large for the LDS index lists");
  const size_t packed = align256(fwd_i16_tiled_workspace(N, L, P));
  int rc = i16_pack(W, N, L, psqt, P, ws, packed, s, who);
  if (rc != SFT_OK) return rc;
  return fwd_i16_packed_ranked(idx, nullptr, B, K, ws, N, L, bias, P, out, nullptr, psqt_out, nullptr, lo, hi, wrap16,
                               static_cast<char *>(ws) + packed, ws_bytes - packed, s, who);
}

int fwd_i16(const int32_t *idx, int64_t B, int K, const int16_t *W, int64_t N, int L, const int16_t *bias,
            const int32_t *psqt, int P, int16_t *out, int32_t *psqt_out, int lo, int hi, int wrap16, hipStream_t s) {
  const bool vec = (L % 8 == 0) && ((uintptr_t)W % 16 == 0) && ((uintptr_t)bias % 16 == 0) &&
                   ((uintptr_t)out % 16 == 0);
  const int64_t cols = vec ? L / 8 : L;
  int min_group = 8;
  while (min_group < P) min_group <<= 1;
  const Mapping m = choose_mapping(cols, min_group);
  const int ppb = kWavesPerBlock * (kWave / m.G);
  const dim3 grid((unsigned)ceil_div(B, ppb), (unsigned)m.slabs);
  const size_t lds = index_lds_bytes(m.G, K);
  if (lds > kMaxIndexLds) return fail(SFT_EUNSUPPORTED, "sft_ft_fwd_i16: max_active too large for the LDS index lists");
  const int kpad = round_up4(K);
  ProfScope prof(kProfFwdI16, s);
  if (vec) {
    SFT_G_CASES(launch_fwd_i16, i16x8, grid, lds, s, idx, B, K, (int)N, W, cols, bias, psqt, P, out, psqt_out, lo,
                hi, wrap16, kpad)
  } else {
    SFT_G_CASES(launch_fwd_i16, short, grid, lds, s, idx, B, K, (int)N, W, cols, bias, psqt, P, out, psqt_out, lo,
                hi, wrap16, kpad)
  }
  return check_launch("sft_ft_fwd_i16");
}

int quantize_i16(const float *x, int64_t n, float scale, int16_t *out, hipStream_t s) {
  if (n == 0) return SFT_OK;
  const int64_t blocks = std::min<int64_t>(ceil_div(n, kBlock), 1 << 16);
  ProfScope prof(kProfQuantize, s);
  hipLaunchKernelGGL(quantize_i16_kernel, dim3((unsigned)blocks), dim3(kBlock), 0, s, x, n, scale, out);
  return check_launch("sft_quantize_i16");
}

}  // namespace sft
