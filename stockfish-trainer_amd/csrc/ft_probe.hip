// Measurement helper (sft_probe_l2_gather): how fast one dispatch can gather
// 128-byte rows from a table that every XCD's L2 holds -- the access pattern
// of the tiled FT gathers, where an 8-lane group loads one 128-byte tile row as
// eight 16-byte chunks and each XCD gathers from one L2-resident tile.  The
// row numbers come from a per-group linear congruential generator in
// registers, so no index stream competes for the L2; the loads are issued
// eight rows at a time before their adds, as in the FT kernels.  The rate it
// measures (rows x 128 B / duration) is the attainable ceiling for L2-served
// row gathers on the running device, beside the figure derived from the
// hardware's L2 width (16 channels x 128 B per clock per XCD).
#include "common.h"

namespace sft {
namespace {

constexpr int kProbeU = 8;  // row loads in flight per lane group

__global__ __launch_bounds__(kBlock) void l2_gather_probe_kernel(const f32x4 *__restrict__ table, uint32_t row_mask,
                                                                 int rounds, f32x4 *__restrict__ out) {
  const int g = threadIdx.x >> 3, t = threadIdx.x & 7;
  // group-uniform generator state: the 8 lanes of a group read the same rows
  uint32_t x = (uint32_t)(blockIdx.x * (kBlock / 8) + g) * 2654435761u + 12345u;
  f32x4 acc = f32x4{0.f, 0.f, 0.f, 0.f};
  const char *base = reinterpret_cast<const char *>(table);
  const uint32_t lane_off = (uint32_t)t * (uint32_t)sizeof(f32x4);
  for (int r = 0; r < rounds; ++r) {
    f32x4 w[kProbeU];
#pragma unroll
    for (int u = 0; u < kProbeU; ++u) {
      x = x * 1664525u + 1013904223u;
      const uint32_t row = (x >> 8) & row_mask;
      w[u] = *reinterpret_cast<const f32x4 *>(base + (row * 128u + lane_off));
    }
#pragma unroll
    for (int u = 0; u < kProbeU; ++u) acc += w[u];
  }
  out[(int64_t)blockIdx.x * kBlock + threadIdx.x] = acc;  // keeps the loads live
}

}  // namespace

int probe_l2_gather(const float *table, int64_t table_rows, int rounds, int blocks, float *out, hipStream_t s) {
  ProfScope prof(kProfProbeL2Gather, s);
  hipLaunchKernelGGL(l2_gather_probe_kernel, dim3((unsigned)blocks), dim3(kBlock), 0, s,
                     reinterpret_cast<const f32x4 *>(table), (uint32_t)(table_rows - 1), rounds,
                     reinterpret_cast<f32x4 *>(out));
  return check_launch("sft_probe_l2_gather");
}

}  // namespace sft
