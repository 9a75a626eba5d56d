// Sparse FT backward for gfx950.
//
// Default algorithm (SFT_BWD_SORTED), deterministic and in the reference's
// summation order (FT/kernel.py:108-138, 167-186):
//   1. stable radix sort of the flat slots s = b*K + k by feature key
//      (inactive slots get key N and sort to the end); values are positions b.
//   2. seg_start[f] = first sorted slot with key >= f, for f = 0..N.
//   3. one lane group per feature row: acc = 0, acc += grad[b] over the
//      feature's positions in ascending order, then one store of the row
//      (dW[f] + acc, or acc when overwriting).  No atomics touch dW.
// Alternative (SFT_BWD_ATOMIC): position-major scatter, each active slot adds
// the position's grad row into dW[f] with fp32 atomics.
// Bias grad (FT/kernel.py:269): per-block column partial sums, then a fixed-
// order reduction of the partials; deterministic.
#include <rocprim/device/device_radix_sort.hpp>
#include <rocprim/iterator/counting_iterator.hpp>
#include <rocprim/iterator/transform_iterator.hpp>

#include <algorithm>

#include "common.h"

namespace sft {

size_t index_lds_bytes(int G, int K);

namespace {

constexpr int kBiasRowsPerBlock = 128;
constexpr int kBiasMaxParts = 512;

struct SortKey {
  const int32_t *idx;
  unsigned N;
  __host__ __device__ unsigned operator()(int s) const {
    const unsigned v = (unsigned)idx[s];
    return v < N ? v : N;
  }
};
struct SlotPosition {
  int K;
  __host__ __device__ int operator()(int s) const { return s / K; }
};

typedef rocprim::transform_iterator<rocprim::counting_iterator<int>, SortKey, unsigned> KeyIter;
typedef rocprim::transform_iterator<rocprim::counting_iterator<int>, SlotPosition, int> PosIter;

unsigned key_bits(int64_t N) {
  unsigned bits = 1;
  while (((int64_t)1 << bits) <= N) ++bits;  // keys lie in [0, N]
  return bits;
}

hipError_t run_sort(void *temp, size_t &temp_bytes, const int32_t *idx, int64_t M, int K, int64_t N,
                    unsigned *keys_out, int *pos_out, hipStream_t s) {
  KeyIter keys_in(rocprim::counting_iterator<int>(0), SortKey{idx, (unsigned)N});
  PosIter pos_in(rocprim::counting_iterator<int>(0), SlotPosition{K});
  return rocprim::radix_sort_pairs(temp, temp_bytes, keys_in, keys_out, pos_in, pos_out, (unsigned)M, 0u,
                                   key_bits(N), s);
}

// seg_start[f] for f in [0, N]: index of the first sorted key >= f.
__global__ __launch_bounds__(kBlock) void seg_offsets_kernel(const unsigned *__restrict__ keys, int64_t M, int64_t N,
                                                             int32_t *__restrict__ seg_start) {
  const int64_t i = (int64_t)blockIdx.x * kBlock + threadIdx.x;
  if (i > M) return;
  const int64_t cur = i < M ? (int64_t)keys[i] : N + 1;
  const int64_t prev = i > 0 ? (int64_t)keys[i - 1] : -1;
  const int64_t hi = cur < N ? cur : N;
  for (int64_t f = prev + 1; f <= hi; ++f) seg_start[f] = (int32_t)i;
}

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

template <typename T, int G, int CPL, int U>
__global__ __launch_bounds__(kBlock) void gather_rows_kernel(const int32_t *__restrict__ seg_start,
                                                             const int32_t *__restrict__ sorted_pos, int64_t N,
                                                             const T *__restrict__ grad, int64_t cols,
                                                             T *__restrict__ dW, int overwrite) {
  constexpr int PPW = kWave / G;
  const int wave = uniform(threadIdx.x / kWave);
  const int lane = threadIdx.x % kWave;
  const int g = lane / G, t = lane % G;
  const int64_t f = ((int64_t)blockIdx.x * kWavesPerBlock + wave) * PPW + g;
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
  const int n = s1 - s0;
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

  if (live && (n > 0 || overwrite)) {
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
  __syncthreads();
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

// partial[blk, c] = sum of grad[r, c] over the block's rows, 4 interleaved
// accumulators combined as (s0 + s1) + (s2 + s3): a fixed order.
template <typename T>
__global__ __launch_bounds__(kBlock) void bias_partial_kernel(const T *__restrict__ grad, int64_t B, int64_t cols,
                                                              int64_t rows_per_block, T *__restrict__ partial) {
  const int64_t r0 = (int64_t)blockIdx.x * rows_per_block;
  const int64_t r1 = std::min<int64_t>(B, r0 + rows_per_block);
  for (int64_t c = threadIdx.x; c < cols; c += kBlock) {
    T s0 = T(0), s1 = T(0), s2 = T(0), s3 = T(0);
    int64_t r = r0;
    for (; r + 4 <= r1; r += 4) {
      const T *p = grad + r * cols + c;
      s0 += p[0];
      s1 += p[cols];
      s2 += p[2 * cols];
      s3 += p[3 * cols];
    }
    for (; r < r1; ++r) s0 += grad[r * cols + c];
    partial[(int64_t)blockIdx.x * cols + c] = (s0 + s1) + (s2 + s3);
  }
}

// db[c] (+)= sum over parts of partial[p, c]; wave w takes parts w, w+4, ...,
// and the four wave sums are combined in a fixed order.
template <typename T>
__global__ __launch_bounds__(kBlock) void bias_final_kernel(const T *__restrict__ partial, int nparts, int64_t cols,
                                                            T *__restrict__ db, int overwrite) {
  __shared__ T red[kWavesPerBlock][kWave];
  const int wave = threadIdx.x / kWave, lane = threadIdx.x % kWave;
  const int64_t c = (int64_t)blockIdx.x * kWave + lane;
  T s = T(0);
  if (c < cols)
    for (int p = wave; p < nparts; p += kWavesPerBlock) s += partial[(int64_t)p * cols + c];
  red[wave][lane] = s;
  __syncthreads();
  if (wave == 0 && c < cols) {
    const T tot = (red[0][lane] + red[1][lane]) + (red[2][lane] + red[3][lane]);
    db[c] = overwrite ? tot : db[c] + tot;
  }
}

template <typename T, int G, int CPL>
void launch_gather(dim3 grid, hipStream_t s, const int32_t *seg_start, const int32_t *pos, int64_t N, const void *grad,
                   int64_t cols, void *dW, int overwrite) {
  hipLaunchKernelGGL((gather_rows_kernel<T, G, CPL, 4>), grid, dim3(kBlock), 0, s, seg_start, pos, N,
                     static_cast<const T *>(grad), cols, static_cast<T *>(dW), overwrite);
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
  size_t keys, pos, seg, partial, temp, temp_bytes, total;
  int nparts;
};

int bias_parts(int64_t B) {
  return (int)std::max<int64_t>(1, std::min<int64_t>(kBiasMaxParts, ceil_div(B, kBiasRowsPerBlock)));
}

int make_layout(int64_t B, int K, int64_t N, int L, uint32_t flags, BwdLayout &lay) {
  const int64_t M = B * K;
  lay.nparts = bias_parts(B);
  size_t off = 0;
  lay.partial = off;
  off = align256(off + (size_t)lay.nparts * (size_t)L * sizeof(float));
  lay.keys = lay.pos = lay.seg = lay.temp = off;
  lay.temp_bytes = 0;
  if (!(flags & SFT_BWD_ATOMIC) && M > 0) {
    lay.keys = off;
    off = align256(off + (size_t)M * sizeof(unsigned));
    lay.pos = off;
    off = align256(off + (size_t)M * sizeof(int));
    lay.seg = off;
    off = align256(off + (size_t)(N + 1) * sizeof(int32_t));
    size_t tb = 0;
    hipError_t e = run_sort(nullptr, tb, nullptr, M, K, N, nullptr, nullptr, nullptr);
    if (e != hipSuccess) return fail(SFT_EHIP, std::string("sort workspace query: ") + hipGetErrorString(e));
    lay.temp = off;
    lay.temp_bytes = tb;
    off = align256(off + tb);
  }
  lay.total = off;
  return SFT_OK;
}

}  // namespace

int bwd_workspace(int64_t B, int K, int64_t N, int L, uint32_t flags, size_t *bytes) {
  BwdLayout lay;
  int rc = make_layout(B, K, N, L, flags, lay);
  if (rc != SFT_OK) return rc;
  *bytes = lay.total;
  return SFT_OK;
}

int bwd_f32(const int32_t *idx, int64_t B, int K, const float *grad, int64_t N, int L, float *dW, float *db,
            void *ws, size_t ws_bytes, uint32_t flags, hipStream_t s) {
  BwdLayout lay;
  int rc = make_layout(B, K, N, L, flags, lay);
  if (rc != SFT_OK) return rc;
  if (ws_bytes < lay.total || (lay.total > 0 && ws == nullptr))
    return fail(SFT_EWORKSPACE, "workspace smaller than sft_ft_bwd_f32_workspace_size()");
  if ((uintptr_t)ws % 256 != 0) return fail(SFT_EWORKSPACE, "workspace must be 256-byte aligned");
  char *w = static_cast<char *>(ws);
  const int overwrite = (flags & SFT_BWD_OVERWRITE) ? 1 : 0;
  const int64_t M = B * K;

  // ---- bias grad ----
  {
    const bool vec = (L % 4 == 0) && ((uintptr_t)grad % 16 == 0) && ((uintptr_t)db % 16 == 0);
    const int64_t cols = vec ? L / 4 : L;
    const int64_t rows = ceil_div(std::max<int64_t>(B, 1), lay.nparts);
    {
      ProfScope prof(kProfBwdBiasPartial, s);
      if (vec)
        hipLaunchKernelGGL(bias_partial_kernel<f32x4>, dim3(lay.nparts), dim3(kBlock), 0, s,
                           reinterpret_cast<const f32x4 *>(grad), B, cols, rows,
                           reinterpret_cast<f32x4 *>(w + lay.partial));
      else
        hipLaunchKernelGGL(bias_partial_kernel<float>, dim3(lay.nparts), dim3(kBlock), 0, s, grad, B, cols, rows,
                           reinterpret_cast<float *>(w + lay.partial));
    }
    if ((rc = check_launch("bias partial sums")) != SFT_OK) return rc;
    {
      ProfScope prof(kProfBwdBiasFinal, s);
      const dim3 grid((unsigned)ceil_div(cols, kWave));
      if (vec)
        hipLaunchKernelGGL(bias_final_kernel<f32x4>, grid, dim3(kBlock), 0, s,
                           reinterpret_cast<const f32x4 *>(w + lay.partial), lay.nparts, cols,
                           reinterpret_cast<f32x4 *>(db), overwrite);
      else
        hipLaunchKernelGGL(bias_final_kernel<float>, grid, dim3(kBlock), 0, s,
                           reinterpret_cast<const float *>(w + lay.partial), lay.nparts, cols, db, overwrite);
    }
    if ((rc = check_launch("bias reduction")) != SFT_OK) return rc;
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
  unsigned *keys = reinterpret_cast<unsigned *>(w + lay.keys);
  int32_t *pos = reinterpret_cast<int32_t *>(w + lay.pos);
  int32_t *seg = reinterpret_cast<int32_t *>(w + lay.seg);
  if (M > 0) {
    ProfScope prof(kProfBwdSort, s);
    size_t tb = lay.temp_bytes;
    hipError_t e = run_sort(w + lay.temp, tb, idx, M, K, N, keys, pos, s);
    if (e != hipSuccess) return fail(SFT_EHIP, std::string("feature sort: ") + hipGetErrorString(e));
  }
  if (M > 0) {
    ProfScope prof(kProfBwdOffsets, s);
    hipLaunchKernelGGL(seg_offsets_kernel, dim3((unsigned)ceil_div(M + 1, kBlock)), dim3(kBlock), 0, s, keys, M, N,
                       seg);
    if ((rc = check_launch("segment offsets")) != SFT_OK) return rc;
  } else if (!overwrite) {
    return SFT_OK;  // nothing active: dW untouched
  }
  if (M == 0) {
    // overwrite with no slots at all: every row is zero
    const int64_t n = N * (int64_t)L;
    ProfScope prof(kProfBwdZero, s);
    hipLaunchKernelGGL(zero_kernel, dim3((unsigned)std::min<int64_t>(ceil_div(n, kBlock), 1 << 16)), dim3(kBlock), 0,
                       s, dW, n);
    return check_launch("weight grad zero fill");
  }
  {
    const bool vec = (L % 4 == 0) && ((uintptr_t)grad % 16 == 0) && ((uintptr_t)dW % 16 == 0);
    const int64_t cols = vec ? L / 4 : L;
    const Mapping m = choose_mapping(cols);
    const int fpb = kWavesPerBlock * (kWave / m.G);
    const dim3 grid((unsigned)ceil_div(N, fpb), (unsigned)m.slabs);
    ProfScope prof(kProfBwdGather, s);
    if (vec) {
      SFT_G_CASES(launch_gather, f32x4, grid, s, seg, pos, N, grad, cols, dW, overwrite)
    } else {
      SFT_G_CASES(launch_gather, float, grid, s, seg, pos, N, grad, cols, dW, overwrite)
    }
  }
  return check_launch("feature row gather");
}

}  // namespace sft
