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

typedef int i32x4 __attribute__((ext_vector_type(4)));

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
  extern __shared__ int smem[];
  const int wave = uniform(threadIdx.x / kWave);
  const int lane = threadIdx.x % kWave;
  int *list = smem + wave * PPW * kpad;
  int *count = smem + kWavesPerBlock * PPW * kpad + wave * PPW;
  const int64_t pos0 = ((int64_t)blockIdx.x * kWavesPerBlock + wave) * PPW;
  compact_rows(idx, B, K, N, pos0, PPW, list, kpad, count);
  __syncthreads();

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
  extern __shared__ int smem[];
  const int wave = uniform(threadIdx.x / kWave);
  const int lane = threadIdx.x % kWave;
  int *list = smem + wave * PPW * kpad;
  int *count = smem + kWavesPerBlock * PPW * kpad + wave * PPW;
  const int64_t pos0 = ((int64_t)blockIdx.x * kWavesPerBlock + wave) * PPW;
  compact_rows(idx, B, K, N, pos0, PPW, list, kpad, count);
  __syncthreads();

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
constexpr int kTileF = 32;                 // floats per tile row
constexpr int kTileCh = kTileF / 4;        // float4 chunks per tile row (= lane group size)
#ifndef SFT_FWD_TILED_U
#define SFT_FWD_TILED_U 4
#endif
#ifndef SFT_TILED_ROUNDS
#define SFT_TILED_ROUNDS 1
#endif
constexpr int kTiledRounds = SFT_TILED_ROUNDS;                        // position rounds per block
constexpr int kTiledPosPerRound = kWavesPerBlock * (kWave / kTileCh);  // 32
constexpr int kTiledPosPerBlock = kTiledPosPerRound * kTiledRounds;

// Two perspectives share one launch: chunks [0, nchunks_p) read idx0 and write
// out0, chunks [nchunks_p, 2 nchunks_p) idx1 and out1, so an XCD gathers both
// perspectives from a tile while it is in L2.  A single-perspective call passes
// the same arrays twice and nchunks_p = nchunks.
__global__ __launch_bounds__(kBlock) void fwd_tiled_kernel(const int32_t *__restrict__ idx0,
                                                           const int32_t *__restrict__ idx1, int64_t B, int K, int N,
                                                           const f32x4 *__restrict__ Wt, int64_t cols4,
                                                           const f32x4 *__restrict__ bias, f32x4 *__restrict__ out0,
                                                           f32x4 *__restrict__ out1, int kpad, int ntiles, int nchunks,
                                                           int nchunks_p) {
  constexpr int U = SFT_FWD_TILED_U;
  constexpr int PPW = kWave / kTileCh;  // 8 positions per wave per round
  extern __shared__ int smem[];
  TileItem it = tile_sched_item(blockIdx.x, ntiles, nchunks);
  if (it.tile >= ntiles) return;  // whole block: uniform
  const bool second = it.chunk >= nchunks_p;
  if (second) it.chunk -= nchunks_p;
  const int32_t *__restrict__ idx = second ? idx1 : idx0;
  f32x4 *__restrict__ out = second ? out1 : out0;
  const int wave = uniform(threadIdx.x / kWave);
  const int lane = threadIdx.x % kWave;
  int *list = smem + wave * PPW * kpad;
  int *count = smem + kWavesPerBlock * PPW * kpad + wave * PPW;
  const int g = lane / kTileCh, t = lane % kTileCh;
  const int64_t col4 = (int64_t)it.tile * kTileCh + t;
  const bool colok = col4 < cols4;
  const f32x4 b4 = colok ? bias[col4] : f32x4{0.f, 0.f, 0.f, 0.f};
  const f32x4 *wtile = Wt + (int64_t)it.tile * N * kTileCh + t;

  for (int round = 0; round < kTiledRounds; ++round) {
    const int64_t pos0 = (int64_t)it.chunk * kTiledPosPerBlock + round * kTiledPosPerRound + wave * PPW;
    compact_rows(idx, B, K, N, pos0, PPW, list, kpad, count);
    __syncthreads();
    const int64_t pos = pos0 + g;
    const int n = count[g];
    int nmin, nmax;
    group_minmax<kTileCh>(n, nmin, nmax);
    const int *mylist = list + g * kpad;
    f32x4 acc = b4;
    int k = 0;
    for (; k + U <= nmin; k += U) {
      int fi[U];
#pragma unroll
      for (int u = 0; u < U; u += 4) {
        const i32x4 f4 = read4(mylist, k + u);
        fi[u] = f4[0], fi[u + 1] = f4[1], fi[u + 2] = f4[2], fi[u + 3] = f4[3];
      }
      f32x4 w[U];
#pragma unroll
      for (int u = 0; u < U; ++u) w[u] = colok ? wtile[(int64_t)fi[u] * kTileCh] : f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int u = 0; u < U; ++u) acc += w[u];
    }
    for (; k < nmax; k += 4) {
      constexpr int UT = 4;
      const i32x4 f4 = read4(mylist, k);
      f32x4 w[UT];
#pragma unroll
      for (int u = 0; u < UT; ++u) {
        const bool v = k + u < n;
        w[u] = f32x4{0.f, 0.f, 0.f, 0.f};
        if (v && colok) w[u] = wtile[(int64_t)f4[u] * kTileCh];
      }
#pragma unroll
      for (int u = 0; u < UT; ++u)
        if (k + u < n) acc += w[u];
    }
    if (pos < B && colok) __builtin_nontemporal_store(acc, out + pos * cols4 + col4);
    __syncthreads();
  }
}

// ----------------------------------------------------- tiled int16 gather ----
// Same schedule as the fp32 tiled gather over an int16 table re-laid out in
// 64-column tiles (128 B per row; 2.9 MB per tile at N = 22 528).  Lane t of
// an 8-lane group owns 8 int16 columns, widened to int32 before adding (exact);
// PSQT columns (P <= 8 int32 per row) are gathered by the tile-0 workgroups.
__global__ __launch_bounds__(kBlock) void fwd_i16_tiled_kernel(const int32_t *__restrict__ idx, int64_t B, int K,
                                                               int N, const i16x8 *__restrict__ Wt, int64_t cols8,
                                                               const i16x8 *__restrict__ bias,
                                                               const int32_t *__restrict__ psqt, int P,
                                                               i16x8 *__restrict__ out, int32_t *__restrict__ psqt_out,
                                                               int clip_lo, int clip_hi, int wrap16, int kpad,
                                                               int ntiles, int nchunks) {
  constexpr int U = 4;
  constexpr int PPW = kWave / kTileCh;
  extern __shared__ int smem[];
  const TileItem it = tile_sched_item(blockIdx.x, ntiles, nchunks);
  if (it.tile >= ntiles) return;
  const int wave = uniform(threadIdx.x / kWave);
  const int lane = threadIdx.x % kWave;
  int *list = smem + wave * PPW * kpad;
  int *count = smem + kWavesPerBlock * PPW * kpad + wave * PPW;
  const int g = lane / kTileCh, t = lane % kTileCh;
  const int64_t col = (int64_t)it.tile * kTileCh + t;
  const bool colok = col < cols8;
  const bool do_psqt = psqt != nullptr && it.tile == 0 && t < P;
  const i16x8 *wtile = Wt + (int64_t)it.tile * N * kTileCh + t;
  const i32x8 b8 = colok ? Q16<i16x8>::widen(bias[col]) : (i32x8)0;

  for (int round = 0; round < kTiledRounds; ++round) {
    const int64_t pos0 = (int64_t)it.chunk * kTiledPosPerBlock + round * kTiledPosPerRound + wave * PPW;
    compact_rows(idx, B, K, N, pos0, PPW, list, kpad, count);
    __syncthreads();
    const int64_t pos = pos0 + g;
    const int n = count[g];
    int nmin, nmax;
    group_minmax<kTileCh>(n, nmin, nmax);
    (void)nmin;
    const int *mylist = list + g * kpad;
    i32x8 acc = b8;
    int pacc = 0;
    for (int k = 0; k < nmax; k += U) {
      const i32x4 f4 = read4(mylist, k);
      i16x8 w[U];
      int pw[U];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const bool v = k + u < n;
        w[u] = (i16x8)0;
        if (v && colok) w[u] = wtile[(int64_t)f4[u] * kTileCh];
        pw[u] = 0;
        if (v && do_psqt) pw[u] = psqt[(int64_t)f4[u] * P + t];
      }
#pragma unroll
      for (int u = 0; u < U; ++u) {
        acc += Q16<i16x8>::widen(w[u]);
        pacc += pw[u];
      }
    }
    if (pos < B) {
      if (colok) __builtin_nontemporal_store(Q16<i16x8>::finish(acc, clip_lo, clip_hi, wrap16), out + pos * cols8 + col);
      if (do_psqt) psqt_out[pos * P + t] = pacc;
    }
    __syncthreads();
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

// Wt[(t * N + r) * 8 + q] = W[r, 4 * (8 t + q) .. +3]; padding chunks of the last tile are not written.
static __global__ __launch_bounds__(kBlock) void tile_relayout_kernel(const f32x4 *__restrict__ W, int64_t N, int64_t cols4,
                                                               f32x4 *__restrict__ Wt) {
  const int64_t total = N * cols4;
  for (int64_t i = (int64_t)blockIdx.x * kBlock + threadIdx.x; i < total; i += (int64_t)gridDim.x * kBlock) {
    const int64_t r = i / cols4, c = i % cols4;
    const int64_t t = c / 8, q = c % 8;
    Wt[(t * N + r) * 8 + q] = W[i];
  }
}

void launch_tile_relayout(const f32x4 *src, int64_t rows, int64_t cols4, f32x4 *dst, hipStream_t s) {
  const int64_t total = rows * cols4;
  hipLaunchKernelGGL(tile_relayout_kernel, dim3((unsigned)std::min<int64_t>(ceil_div(total, kBlock), 1 << 16)),
                     dim3(kBlock), 0, s, src, rows, cols4, dst);
}

// Composed-table re-layout: merged row r of block s is w_s[r'] (+ v_s[r' %
// period_s] when the block has virtual rows; r' = r - start_s), added in
// binary32 exactly as the table the reference materialises
// (FEAT/halfka_v2_hm.py:69-70, FEAT/composed.py:49-50), and stored straight into
// the 32-column tiles of the tiled gather.  total = N * cols4 < 2^31.
static __global__ __launch_bounds__(kBlock) void fold_relayout_kernel(FoldSrc src, int N, int cols4,
                                                                      f32x4 *__restrict__ Wt) {
  const int total = N * cols4;
  for (int i = blockIdx.x * kBlock + threadIdx.x; i < total; i += gridDim.x * kBlock) {
    const int r = i / cols4, c = i - r * cols4;
    const int s = block_of(r, src.n, src.start);
    const int rl = r - (int)pick(src.start, s);
    f32x4 x = pick(src.w, s)[(int64_t)rl * cols4 + c];
    const f32x4 *v = pick(src.v, s);
    if (v != nullptr) {
      const f32x4 y = v[(int64_t)(rl % (int)pick(src.period, s)) * cols4 + c];
      x += y;
    }
    Wt[((int64_t)(c >> 3) * N + r) * 8 + (c & 7)] = x;
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

size_t fwd_tiled_workspace(int64_t N, int L) {
  if (L % 4 != 0) return 0;
  const int64_t ntiles = ceil_div(L, kTileF);
  return (size_t)(ntiles * N * kTileF) * sizeof(float);
}

#ifndef SFT_FWD_TILE_MAX_BYTES
#define SFT_FWD_TILE_MAX_BYTES (64ll << 20)
#endif
bool fwd_tiled_supported(int64_t N, int L, const void *W, const void *bias, const void *out) {
  return L % 4 == 0 && L >= kTileF * kXcds && N * kTileF * 4 <= (int64_t)(SFT_FWD_TILE_MAX_BYTES) &&
         (uintptr_t)W % 16 == 0 && (uintptr_t)bias % 16 == 0 && (uintptr_t)out % 16 == 0;
}

int fwd_f32_tiled(const int32_t *idx, int64_t B, int K, const float *W, int64_t N, int L, const float *bias, float *out,
                  void *ws, size_t ws_bytes, hipStream_t s) {
  if (ws_bytes < fwd_tiled_workspace(N, L) || ws == nullptr || (uintptr_t)ws % 256 != 0)
    return fail(SFT_EWORKSPACE, "sft_ft_fwd_f32_ex: workspace smaller than sft_ft_fwd_f32_workspace_size() "
                                "or not 256-byte aligned");
  const int64_t cols4 = L / 4;
  const int ntiles = (int)ceil_div(L, kTileF);
  const int kpad = round_up4(K);
  const size_t lds = index_lds_bytes(kTileCh, K);
  if (lds > kMaxIndexLds) return fail(SFT_EUNSUPPORTED, "sft_ft_fwd_f32_ex: max_active too large for the LDS index lists");
  f32x4 *wt = static_cast<f32x4 *>(ws);
  {
    ProfScope prof(kProfFwdRelayout, s);
    launch_tile_relayout(reinterpret_cast<const f32x4 *>(W), N, cols4, wt, s);
  }
  int rc = check_launch("sft_ft_fwd_f32_ex (relayout)");
  if (rc != SFT_OK) return rc;
  const int nchunks = (int)ceil_div(B, kTiledPosPerBlock);
  const int64_t blocks = tile_sched_items_per_xcd(ntiles, nchunks) * kXcds;
  {
    ProfScope prof(kProfFwdTiled, s);
    hipLaunchKernelGGL(fwd_tiled_kernel, dim3((unsigned)blocks), dim3(kBlock), lds, s, idx, idx, B, K, (int)N, wt,
                       cols4, reinterpret_cast<const f32x4 *>(bias), reinterpret_cast<f32x4 *>(out),
                       reinterpret_cast<f32x4 *>(out), kpad, ntiles, nchunks, nchunks);
  }
  return check_launch("sft_ft_fwd_f32_ex (tiled gather)");
}

int fwd_pair_f32(const int32_t *idx0, const int32_t *idx1, int64_t B, int K, const FoldSrc &src, int64_t N, int L,
                 const float *bias, float *out0, float *out1, void *ws, size_t ws_bytes, hipStream_t s) {
  if (ws_bytes < fwd_tiled_workspace(N, L) || ws == nullptr || (uintptr_t)ws % 256 != 0)
    return fail(SFT_EWORKSPACE, "sft_ft_fwd_pair_f32: workspace smaller than sft_ft_pair_workspace_size() "
                                "or not 256-byte aligned");
  const int64_t cols4 = L / 4;
  const int ntiles = (int)ceil_div(L, kTileF);
  const int kpad = round_up4(K);
  const size_t lds = index_lds_bytes(kTileCh, K);
  if (lds > kMaxIndexLds) return fail(SFT_EUNSUPPORTED, "sft_ft_fwd_pair_f32: max_active too large for the LDS index lists");
  f32x4 *wt = static_cast<f32x4 *>(ws);
  {
    const int64_t total = N * cols4;
    ProfScope prof(kProfFwdFold, s);
    hipLaunchKernelGGL(fold_relayout_kernel, dim3((unsigned)std::min<int64_t>(ceil_div(total, kBlock), 1 << 16)),
                       dim3(kBlock), 0, s, src, (int)N, (int)cols4, wt);
  }
  int rc = check_launch("sft_ft_fwd_pair_f32 (fold re-layout)");
  if (rc != SFT_OK || B == 0) return rc;
  const int nchunks_p = (int)ceil_div(B, kTiledPosPerBlock);
  const int64_t blocks = tile_sched_items_per_xcd(ntiles, 2 * nchunks_p) * kXcds;
  {
    ProfScope prof(kProfFwdTiled, s);
    hipLaunchKernelGGL(fwd_tiled_kernel, dim3((unsigned)blocks), dim3(kBlock), lds, s, idx0, idx1, B, K, (int)N, wt,
                       cols4, reinterpret_cast<const f32x4 *>(bias), reinterpret_cast<f32x4 *>(out0),
                       reinterpret_cast<f32x4 *>(out1), kpad, ntiles, 2 * nchunks_p, nchunks_p);
  }
  return check_launch("sft_ft_fwd_pair_f32 (tiled gather)");
}

size_t fwd_i16_tiled_workspace(int64_t N, int L) {
  if (L % 8 != 0) return 0;
  const int64_t ntiles = ceil_div(L / 8, kTileCh);
  return (size_t)(ntiles * N * kTileCh) * 16;
}

bool fwd_i16_tiled_supported(int64_t N, int L, int P, const void *W, const void *bias, const void *out) {
  return L % 8 == 0 && ceil_div(L / 8, kTileCh) >= kXcds && N * 128 <= (int64_t)(SFT_FWD_TILE_MAX_BYTES) && P <= 8 &&
         (uintptr_t)W % 16 == 0 && (uintptr_t)bias % 16 == 0 && (uintptr_t)out % 16 == 0;
}

int fwd_i16_tiled(const int32_t *idx, int64_t B, int K, const int16_t *W, int64_t N, int L, const int16_t *bias,
                  const int32_t *psqt, int P, int16_t *out, int32_t *psqt_out, int lo, int hi, int wrap16, void *ws,
                  size_t ws_bytes, hipStream_t s) {
  if (ws_bytes < fwd_i16_tiled_workspace(N, L) || ws == nullptr || (uintptr_t)ws % 256 != 0)
    return fail(SFT_EWORKSPACE, "sft_ft_fwd_i16_ex: workspace smaller than sft_ft_fwd_i16_workspace_size() "
                                "or not 256-byte aligned");
  const int64_t cols8 = L / 8;
  const int ntiles = (int)ceil_div(cols8, kTileCh);
  const int kpad = round_up4(K);
  const size_t lds = index_lds_bytes(kTileCh, K);
  if (lds > kMaxIndexLds) return fail(SFT_EUNSUPPORTED, "sft_ft_fwd_i16_ex: max_active too large for the LDS index lists");
  i16x8 *wt = static_cast<i16x8 *>(ws);
  {
    ProfScope prof(kProfFwdRelayout, s);
    launch_tile_relayout(reinterpret_cast<const f32x4 *>(W), N, cols8, reinterpret_cast<f32x4 *>(wt), s);
  }
  int rc = check_launch("sft_ft_fwd_i16_ex (relayout)");
  if (rc != SFT_OK) return rc;
  const int nchunks = (int)ceil_div(B, kTiledPosPerBlock);
  const int64_t blocks = tile_sched_items_per_xcd(ntiles, nchunks) * kXcds;
  {
    ProfScope prof(kProfFwdI16Tiled, s);
    hipLaunchKernelGGL(fwd_i16_tiled_kernel, dim3((unsigned)blocks), dim3(kBlock), lds, s, idx, B, K, (int)N, wt,
                       cols8, reinterpret_cast<const i16x8 *>(bias), psqt, P, reinterpret_cast<i16x8 *>(out),
                       psqt_out, lo, hi, wrap16, kpad, ntiles, nchunks);
  }
  return check_launch("sft_ft_fwd_i16_ex (tiled gather)");
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
