// Fused Ranger22 parameter update for the feature-transformer tables: the
// full update the reference compiles with torch.compile
// (src/ranger22/optimizer.py:46-77 for 1-D tensors, :80-111 for 2-D), in one
// pass over p, grad and the optimizer state.
//
// Per element, every operation rounds to binary32 in the order of the
// reference function (no contraction into FMAs):
//   v  = v * beta2 + (g * g) * (1 - beta2)
//   m  = m * beta1^2 + g * (1 - beta1^2)
//   c  = two_nl_factor * (1 - 1 / (||p_row||_2 + eps))     (norm of p before the update)
//   p  = p * (1 - lr * c) - ((m * pnm_a + m_prev * pnm_b) * noise_norm_recip
//                             / (sqrt(v) * inv_sqrt_bc2 + eps)) * step_size
// The twelve scalars are read from device memory (the reference's scalars
// tensor), so the caller needs no host synchronisation.
#include "common.h"

namespace sft {

namespace {

#pragma clang fp contract(off)

// Scalars, in the reference's order (src/ranger22/optimizer.py:239-250).
struct RangerScalars {
  float lr, inv_sqrt_bc2, eps, two_nl_factor, noise_norm_recip, pnm_a, pnm_b, step_size, beta2, one_minus_beta2,
      beta1_sq, one_minus_beta1_sq;
};

__device__ __forceinline__ RangerScalars load_scalars(const float *__restrict__ s) {
  RangerScalars r;
  r.lr = s[0];
  r.inv_sqrt_bc2 = s[1];
  r.eps = s[2];
  r.two_nl_factor = s[3];
  r.noise_norm_recip = s[4];
  r.pnm_a = s[5];
  r.pnm_b = s[6];
  r.step_size = s[7];
  r.beta2 = s[8];
  r.one_minus_beta2 = s[9];
  r.beta1_sq = s[10];
  r.one_minus_beta1_sq = s[11];
  return r;
}

// One element of the update given the row's factor h = 1 - lr * correction.
__device__ __forceinline__ void update_one(float &p, float g, float &v, float &m, float mp, float h,
                                           const RangerScalars &s) {
  const float v1 = v * s.beta2;
  const float gg = g * g;
  const float v2 = v1 + gg * s.one_minus_beta2;
  const float m1 = m * s.beta1_sq;
  const float m2 = m1 + g * s.one_minus_beta1_sq;
  const float denom = sqrtf(v2) * s.inv_sqrt_bc2 + s.eps;
  const float pn = (m2 * s.pnm_a + mp * s.pnm_b) * s.noise_norm_recip;
  const float p1 = p * h;
  p = p1 - (pn / denom) * s.step_size;
  v = v2;
  m = m2;
}

__device__ __forceinline__ float row_factor(float sumsq, const RangerScalars &s) {
  const float unorm = sqrtf(sumsq);
  const float correction = s.two_nl_factor * (1.0f - 1.0f / (unorm + s.eps));
  return 1.0f - s.lr * correction;
}

// Fixed-order wave sum (xor butterfly).
__device__ __forceinline__ float wave_sum(float x) {
#pragma unroll
  for (int m = 1; m < kWave; m <<= 1) x += __shfl_xor(x, m);
  return x;
}

constexpr int kOptRowChunks = 8;  // 16-byte chunks per lane kept in registers (rows up to 2048 floats)

// 2-D tables, cols % 4 == 0 and cols <= 4 * 64 * kOptRowChunks: one wave per row,
// the whole row of all five tensors loaded into registers before the norm's
// reduction, so the loads of a row are all in flight together.
template <int NCH>
__global__ __launch_bounds__(kBlock) void ranger_rows_vec_kernel(f32x4 *__restrict__ p, const f32x4 *__restrict__ g,
                                                                 f32x4 *__restrict__ v, f32x4 *__restrict__ m,
                                                                 const f32x4 *__restrict__ mp, int64_t rows,
                                                                 int cols4, const float *__restrict__ scalars) {
  const int64_t r = (int64_t)blockIdx.x * kWavesPerBlock + uniform(threadIdx.x / kWave);
  if (r >= rows) return;  // wave-uniform
  const int lane = threadIdx.x % kWave;
  const RangerScalars s = load_scalars(scalars);
  const int64_t base = r * cols4;
  const f32x4 z = f32x4{0.f, 0.f, 0.f, 0.f};
  f32x4 pr[NCH], gr[NCH], vr[NCH], mr[NCH], mpr[NCH];
#pragma unroll
  for (int j = 0; j < NCH; ++j) {
    const int c = lane + kWave * j;
    const bool ok = c < cols4;
    pr[j] = ok ? p[base + c] : z;
    gr[j] = ok ? g[base + c] : z;
    vr[j] = ok ? v[base + c] : z;
    mr[j] = ok ? m[base + c] : z;
    mpr[j] = ok ? mp[base + c] : z;
  }
  float sq = 0.f;
#pragma unroll
  for (int j = 0; j < NCH; ++j)
    sq += (pr[j].x * pr[j].x + pr[j].y * pr[j].y) + (pr[j].z * pr[j].z + pr[j].w * pr[j].w);
  const float h = row_factor(wave_sum(sq), s);
#pragma unroll
  for (int j = 0; j < NCH; ++j) {
    const int c = lane + kWave * j;
    if (c >= cols4) continue;
    f32x4 pv, vv, mv;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      float pe = pr[j][e], ve = vr[j][e], me = mr[j][e];
      update_one(pe, gr[j][e], ve, me, mpr[j][e], h, s);
      pv[e] = pe;
      vv[e] = ve;
      mv[e] = me;
    }
    p[base + c] = pv;
    v[base + c] = vv;
    m[base + c] = mv;
  }
}

// Any shape (1-D tensors are one row): one workgroup per row, two passes over
// the row (norm, then update).  Fixed-order block sum.
__global__ __launch_bounds__(kBlock) void ranger_rows_kernel(float *__restrict__ p, const float *__restrict__ g,
                                                             float *__restrict__ v, float *__restrict__ m,
                                                             const float *__restrict__ mp, int64_t cols,
                                                             const float *__restrict__ scalars) {
  __shared__ float red[kWavesPerBlock];
  const int64_t base = (int64_t)blockIdx.x * cols;
  const RangerScalars s = load_scalars(scalars);
  float sq = 0.f;
  for (int64_t c = threadIdx.x; c < cols; c += kBlock) sq += p[base + c] * p[base + c];
  sq = wave_sum(sq);
  if (threadIdx.x % kWave == 0) red[threadIdx.x / kWave] = sq;
  __syncthreads();
  const float h = row_factor((red[0] + red[1]) + (red[2] + red[3]), s);
  for (int64_t c = threadIdx.x; c < cols; c += kBlock) {
    float pv = p[base + c], vv = v[base + c], mv = m[base + c];
    update_one(pv, g[base + c], vv, mv, mp[base + c], h, s);
    p[base + c] = pv;
    v[base + c] = vv;
    m[base + c] = mv;
  }
}

}  // namespace

int ranger_update_f32(float *p, const float *grad, float *variance_ma, float *gma_cur, const float *gma_prev,
                      int64_t rows, int64_t cols, const float *scalars, hipStream_t s) {
  const bool vec = cols % 4 == 0 && cols / 4 <= (int64_t)kWave * kOptRowChunks &&
                   ((uintptr_t)p | (uintptr_t)grad | (uintptr_t)variance_ma | (uintptr_t)gma_cur |
                    (uintptr_t)gma_prev) % 16 == 0;
  ProfScope prof(kProfOptim, s);
  if (vec) {
    const int cols4 = (int)(cols / 4);
    const dim3 grid((unsigned)ceil_div(rows, kWavesPerBlock));
#define SFT_RANGER_VEC(NCH)                                                                                     \
  hipLaunchKernelGGL(ranger_rows_vec_kernel<NCH>, grid, dim3(kBlock), 0, s, reinterpret_cast<f32x4 *>(p),      \
                     reinterpret_cast<const f32x4 *>(grad), reinterpret_cast<f32x4 *>(variance_ma),            \
                     reinterpret_cast<f32x4 *>(gma_cur), reinterpret_cast<const f32x4 *>(gma_prev), rows, cols4, \
                     scalars)
    if (cols4 <= 2 * kWave)
      SFT_RANGER_VEC(2);
    else if (cols4 <= 5 * kWave)
      SFT_RANGER_VEC(5);
    else
      SFT_RANGER_VEC(8);
#undef SFT_RANGER_VEC
  } else
    hipLaunchKernelGGL(ranger_rows_kernel, dim3((unsigned)rows), dim3(kBlock), 0, s, p, grad, variance_ma, gma_cur,
                       gma_prev, cols, scalars);
  return check_launch("sft_ranger22_update_f32");
}

}  // namespace sft
