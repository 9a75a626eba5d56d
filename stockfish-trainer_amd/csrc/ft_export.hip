// Signed LEB128 encoding of quantized feature-transformer tensors on the GPU,
// the compression of the .nnue writer (src/scripts/serialize.py:61-93,
// _encode_leb_128_array; used by _write_leb_128_array :254-257 for the FT
// bias, weights and PSQT weights).
//
// Per value: 7-bit groups from the least significant, a continuation bit on
// every byte but the last, stopping once the rest of the value is all sign
// bits and the last group's bit 6 equals the sign.  The byte stream is the
// concatenation in element order, so the encoder is a length pass, a scan of
// the lengths and a write pass:
//   leb_len_kernel:   per tile of kLebTile values, the tile's byte count
//   leb_scan_kernel:  one workgroup, exclusive scan of the tile counts (and
//                     the total, into *out_len)
//   leb_write_kernel: per tile, in-tile exclusive scan of the value lengths,
//                     then each value writes its bytes at its offset
#include "common.h"

namespace sft {

namespace {

constexpr int kLebItems = 16;
constexpr int kLebTile = kBlock * kLebItems;  // values per tile

__device__ __forceinline__ int64_t load_value(const void *p, int elem, int64_t i) {
  if (elem == 1) return static_cast<const int8_t *>(p)[i];
  if (elem == 2) return static_cast<const int16_t *>(p)[i];
  return static_cast<const int32_t *>(p)[i];
}

__device__ __forceinline__ int leb_len(int64_t v) {
  int n = 0;
  while (true) {
    const int byte = (int)(v & 0x7f);
    v >>= 7;  // arithmetic shift: keeps the sign
    ++n;
    if ((v == 0 && (byte & 0x40) == 0) || (v == -1 && (byte & 0x40) != 0)) return n;
  }
}

__device__ __forceinline__ void leb_write(int64_t v, uint8_t *out) {
  while (true) {
    const int byte = (int)(v & 0x7f);
    v >>= 7;
    if ((v == 0 && (byte & 0x40) == 0) || (v == -1 && (byte & 0x40) != 0)) {
      *out = (uint8_t)byte;
      return;
    }
    *out++ = (uint8_t)(byte | 0x80);
  }
}

// Exclusive block scan of one value per thread (fixed order); returns the
// block total through *total.
__device__ __forceinline__ int64_t block_exclusive_scan(int64_t x, int64_t *s, int64_t *total) {
  const int tid = threadIdx.x;
  s[tid] = x;
  __syncthreads();
  for (int off = 1; off < kBlock; off <<= 1) {
    const int64_t v = tid >= off ? s[tid - off] : 0;
    __syncthreads();
    s[tid] += v;
    __syncthreads();
  }
  const int64_t incl = s[tid];
  *total = s[kBlock - 1];
  __syncthreads();
  return incl - x;
}

__global__ __launch_bounds__(kBlock) void leb_len_kernel(const void *__restrict__ values, int elem, int64_t n,
                                                         int64_t *__restrict__ tile_bytes) {
  __shared__ int64_t s[kBlock];
  const int64_t base = (int64_t)blockIdx.x * kLebTile + (int64_t)threadIdx.x * kLebItems;
  int64_t mine = 0;
#pragma unroll
  for (int i = 0; i < kLebItems; ++i)
    if (base + i < n) mine += leb_len(load_value(values, elem, base + i));
  int64_t total;
  block_exclusive_scan(mine, s, &total);
  if (threadIdx.x == 0) tile_bytes[blockIdx.x] = total;
}

__global__ __launch_bounds__(kBlock) void leb_scan_kernel(int64_t *__restrict__ tile_bytes, int64_t ntiles,
                                                          int64_t *__restrict__ out_len) {
  __shared__ int64_t s[kBlock];
  const int64_t per = (ntiles + kBlock - 1) / kBlock;
  const int64_t lo = min(ntiles, (int64_t)threadIdx.x * per), hi = min(ntiles, lo + per);
  int64_t mine = 0;
  for (int64_t i = lo; i < hi; ++i) mine += tile_bytes[i];
  int64_t total;
  int64_t run = block_exclusive_scan(mine, s, &total);
  for (int64_t i = lo; i < hi; ++i) {
    const int64_t v = tile_bytes[i];
    tile_bytes[i] = run;
    run += v;
  }
  if (threadIdx.x == 0) *out_len = total;
}

__global__ __launch_bounds__(kBlock) void leb_write_kernel(const void *__restrict__ values, int elem, int64_t n,
                                                           const int64_t *__restrict__ tile_start,
                                                           uint8_t *__restrict__ out) {
  __shared__ int64_t s[kBlock];
  const int64_t base = (int64_t)blockIdx.x * kLebTile + (int64_t)threadIdx.x * kLebItems;
  int64_t v[kLebItems];
  int len[kLebItems];
  int64_t mine = 0;
#pragma unroll
  for (int i = 0; i < kLebItems; ++i) {
    v[i] = base + i < n ? load_value(values, elem, base + i) : 0;
    len[i] = base + i < n ? leb_len(v[i]) : 0;
    mine += len[i];
  }
  int64_t total;
  int64_t off = tile_start[blockIdx.x] + block_exclusive_scan(mine, s, &total);
#pragma unroll
  for (int i = 0; i < kLebItems; ++i) {
    if (base + i < n) leb_write(v[i], out + off);
    off += len[i];
  }
}

}  // namespace

size_t leb128_workspace(int64_t n) { return (size_t)ceil_div(std::max<int64_t>(n, 1), kLebTile) * sizeof(int64_t); }

int leb128_encode(const void *values, int elem, int64_t n, uint8_t *out, int64_t *out_len, void *ws, hipStream_t s) {
  const int64_t ntiles = ceil_div(std::max<int64_t>(n, 1), kLebTile);
  int64_t *tiles = static_cast<int64_t *>(ws);
  ProfScope prof(kProfLeb128, s);
  hipLaunchKernelGGL(leb_len_kernel, dim3((unsigned)ntiles), dim3(kBlock), 0, s, values, elem, n, tiles);
  hipLaunchKernelGGL(leb_scan_kernel, dim3(1), dim3(kBlock), 0, s, tiles, ntiles, out_len);
  hipLaunchKernelGGL(leb_write_kernel, dim3((unsigned)ntiles), dim3(kBlock), 0, s, values, elem, n, tiles, out);
  return check_launch("sft_leb128_encode");
}

}  // namespace sft
