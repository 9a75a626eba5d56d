// Index arithmetic shared by the gfx950 FT kernels and their host launchers:
// magic-number division, the XCD-aware tile schedule, the column maps of the
// 32-column tiles and the long-segment rule of the sorted backward.  Plain
// integer code with no HIP dependency, so that it also builds as host C++ (the
// CPU tests compile it with g++ and the address/undefined-behaviour
// sanitizers).
#pragma once

#include <cstdint>

#if defined(__HIPCC__)
#define SFT_HD __host__ __device__
#else
#define SFT_HD
#endif

namespace sft {

SFT_HD inline int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }
SFT_HD inline int round_up4(int v) { return (v + 3) & ~3; }

// ---- bucket sort over (position chunk, feature) keys: key = chunk * N + f ----
// Buckets hold 2^sb consecutive keys.  The first n buckets hold every key of
// chunk 0 and key N, the first of chunk 1, whose segment start ends chunk 0's
// last segment; n is the fewest that do (0 with one chunk or no features).
SFT_HD inline int buckets_through_chunk0(int64_t N, int nchunks, int sb) {
  if (nchunks < 2 || N <= 0) return 0;
  const int64_t nb = ceil_div((int64_t)nchunks * N, (int64_t)1 << sb);
  const int64_t n = (N >> sb) + 1;
  return (int)(n < nb ? n : nb);
}

// ---- n / d for 32-bit n by a divisor fixed at launch ----
// Multiply-high by a magic number (Granlund & Montgomery 1994, round-up
// variant): with l = ceil(log2 d) and m = floor(2^32 (2^l - d) / d) + 1,
// n / d = (t + ((n - t) >> 1)) >> (l - 1) where t = mulhi(m, n), for d >= 2;
// d = 1 returns n.
SFT_HD inline uint32_t mulhi32(uint32_t a, uint32_t b) { return (uint32_t)(((uint64_t)a * b) >> 32); }
struct FastDiv {
  uint32_t d, mul, shift;
  FastDiv() = default;
  SFT_HD explicit FastDiv(uint32_t div) : d(div), mul(0), shift(0) {
    uint32_t l = 0;
    while (((uint64_t)1 << l) < div) ++l;
    shift = l;
    mul = (uint32_t)((((uint64_t)1 << 32) * (((uint64_t)1 << l) - div)) / div + 1);
  }
  SFT_HD uint32_t operator()(uint32_t n) const {
    if (d == 1) return n;
    const uint32_t t = mulhi32(mul, n);
    return (t + ((n - t) >> 1)) >> (shift - 1);
  }
};

// ---- XCD-aware tile schedule ----
// MI355X runs a dispatch's workgroups round-robin over its 8 XCDs (workgroup i
// on XCD i % 8), and each XCD has its own 4 MB L2.  Tiled kernels give every
// XCD whole column tiles: workgroup i serves the (i / 8)-th item of XCD i % 8,
// where XCD x owns tiles x, x + 8, ... (all chunks of one tile, then the next).
// The rem = ntiles % 8 tiles left after the last full round are cut into 8
// strands each -- strand s of leftover tile t holds its chunks s, s + 8, ...,
// so every strand has the same mix of early (long) and late chunks -- and XCD
// x takes the rem consecutive strands [x rem, (x + 1) rem) of the sequence
// (t, s): every XCD gets the same work (rem strands, +-1 chunk each) from at
// most two leftover tiles, the first one's strands before the second's, in
// chunk order.  (With rem = 5 tiles, whole tiles per XCD group would leave two
// XCDs alone on a tile each while the others share one.)  A workgroup with no
// item gets tile = ntiles.  Any other placement only costs locality, never
// results.
constexpr int kXcds = 8;
struct TileItem {
  int tile, chunk;
};
SFT_HD inline int64_t tile_sched_items_per_xcd(int ntiles, int nchunks) {
  const int full = ntiles / kXcds, rem = ntiles % kXcds;
  return (int64_t)full * nchunks + (int64_t)rem * ((nchunks + kXcds - 1) / kXcds);
}
SFT_HD inline TileItem tile_sched_item(int64_t bid, int ntiles, int nchunks) {
  const int xcd = (int)(bid % kXcds);
  const int64_t j = bid / kXcds;
  const int full = ntiles / kXcds, rem = ntiles % kXcds;
  const int64_t fj = (int64_t)full * nchunks;
  if (j < fj) return TileItem{xcd + kXcds * (int)(j / nchunks), (int)(j % nchunks)};
  if (rem == 0) return TileItem{ntiles, 0};  // no work
  const int64_t rounds = (nchunks + kXcds - 1) / kXcds;  // chunks per strand, the last round partial
  const int s0 = xcd * rem;                              // first strand of this XCD
  const int ta = s0 / kXcds;                             // its first leftover tile
  const int na = ((ta + 1) * kXcds < s0 + rem ? (ta + 1) * kXcds : s0 + rem) - s0;  // strands of tile ta
  int64_t i = j - fj;
  int t = ta, s = s0 % kXcds, n = na;
  if (i >= rounds * na) {  // strands 0 .. rem - na - 1 of the next leftover tile
    i -= rounds * na;
    t = ta + 1;
    s = 0;
    n = rem - na;
    if (n <= 0) return TileItem{ntiles, 0};  // no work
  }
  const int64_t c = (i / n) * kXcds + s + i % n;
  if (c >= nchunks) return TileItem{ntiles, 0};  // no work: past a strand's end
  return TileItem{kXcds * full + t, (int)c};
}

// ---- column maps of the 32-column tiles ----
// Tile t, lane q (one 16-byte chunk of 4 columns) of a tile row holds chunk
// tile_col(m, t, q) of the row-major table (-1: padding).
//   plain  (half4 == 0): chunks tch*t .. tch*t + tch-1.
//   paired (half4 > 0):  for t < t1, chunks 4t .. 4t+3 of the first half
//     (lanes 0-3) and the same chunks of the second half (lanes 4-7), where a
//     half is half4 chunks; tiles t >= t1 hold the chunks after both halves
//     (the PSQT columns), 8 per tile.  Columns j and j + L1/2 of a row, which
//     the post-FT epilogue multiplies together, then sit in lanes q and q ^ 4.
struct ColMap {
  int half4;  // chunks per half (0: plain map)
  int t1;     // paired tiles
  int cols4;  // chunks per row
  int tch;    // plain map: chunks per tile row (8: 32 columns, 4: 16 columns)
};
SFT_HD inline int tile_col(const ColMap &m, int t, int q) {
  if (m.half4 == 0) {
    const int c = m.tch * t + q;
    return (q < m.tch && c < m.cols4) ? c : -1;
  }
  if (t < m.t1) {
    const int j = 4 * t + (q & 3);
    return j < m.half4 ? j + (q >> 2) * m.half4 : -1;
  }
  const int c = 2 * m.half4 + 8 * (t - m.t1) + q;
  return c < m.cols4 ? c : -1;
}
// Inverse: tile and lane of chunk c.
SFT_HD inline void tile_of_col(const ColMap &m, int c, int &t, int &q) {
  if (m.half4 == 0) {
    t = c / m.tch;
    q = c % m.tch;
  } else if (c < 2 * m.half4) {
    const int h = c >= m.half4 ? 1 : 0;
    const int j = c - h * m.half4;
    t = j >> 2;
    q = (j & 3) + 4 * h;
  } else {
    const int k = c - 2 * m.half4;
    t = m.t1 + (k >> 3);
    q = k & 7;
  }
}
SFT_HD inline ColMap plain_map(int cols4, int tch = 8) { return ColMap{0, 0, cols4, tch}; }
SFT_HD inline ColMap paired_map(int cols4, int half4) { return ColMap{half4, (half4 + 3) / 4, cols4, 8}; }
SFT_HD inline int map_tiles(const ColMap &m) {
  return m.half4 == 0 ? (m.cols4 + m.tch - 1) / m.tch : m.t1 + (m.cols4 - 2 * m.half4 + 7) / 8;
}

// ---- long segments of the sorted backward ----
// Whether segment [s0, s1) of the sorted slots is long depends on its bounds
// alone, so the per-feature gathers (which skip long segments) and the segment
// pass (which lists them) agree: it is long when it contains two consecutive
// multiples of `period` ("samples") of the sorted slot index.  Every segment
// of 2 period slots or more is long, none of period slots or fewer.
SFT_HD inline int64_t long_first_sample(int64_t s0, int period) { return (s0 + period - 1) / period * period; }
SFT_HD inline bool long_segment(int64_t s0, int64_t s1, int period) { return long_first_sample(s0, period) + period < s1; }
// The segment pass lists a long segment once, at its first sample i:
// keys[i + period] == keys[i] != keys[i - period] (keys: the M sorted keys).
SFT_HD inline bool long_listed_at(const unsigned *keys, int64_t M, int64_t i, int period) {
  return i % period == 0 && i + period < M && keys[i + period] == keys[i] && (i < period || keys[i - period] != keys[i]);
}

}  // namespace sft
