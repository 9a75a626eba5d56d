// Host checks of the FT kernels' index arithmetic (stockfish-trainer_amd/csrc/
// index_math.h), built with -fsanitize=address,undefined by
// tests/test_index_math_cpu.py.  Every check compares against an independent
// formulation (plain division, brute-force coverage counts, the other map
// direction); the program prints one line per failure and exits non-zero.
#include <cstdio>
#include <cstdlib>
#include <random>
#include <utility>
#include <vector>

#include "index_math.h"

using namespace sft;

static int failures = 0;
#define CHECK(cond, ...)                     \
  do {                                       \
    if (!(cond)) {                           \
      if (++failures <= 20) {                \
        std::printf("FAIL %s: ", #cond);     \
        std::printf(__VA_ARGS__);            \
        std::printf("\n");                   \
      }                                      \
    }                                        \
  } while (0)

// n / d against the hardware divide: every n below 2^14, the neighbours of
// multiples of d up to 2^31 (all of them for d >= 2^15, else 20000 spread over
// the range), and the top of the 31-bit slot range the sort indexes with.
static void check_fastdiv(uint32_t d) {
  const FastDiv f(d);
  for (uint32_t n = 0; n < (1u << 14); ++n) CHECK(f(n) == n / d, "d=%u n=%u", d, n);
  const uint64_t top = 1ull << 31;
  const uint64_t qmax = top / d;
  const uint64_t step = qmax > 65536 ? qmax / 20000 : 1;
  for (uint64_t q = 1; q <= qmax; q += step)
    for (int e = -1; e <= 1; ++e) {
      const uint64_t n = q * d + e;
      if (n < top) CHECK(f((uint32_t)n) == (uint32_t)(n / d), "d=%u n=%llu", d, (unsigned long long)n);
    }
  for (uint64_t n = top - 4096; n < top; ++n) CHECK(f((uint32_t)n) == (uint32_t)(n / d), "d=%u n=%llu", d,
                                                    (unsigned long long)n);
}

// Every (tile, chunk) of ntiles x nchunks is served by exactly one workgroup of
// the launch (tile_sched_items_per_xcd * 8 of them), the others get no work,
// each XCD serves its own tiles only, and the leftover tiles are shared out
// evenly: every XCD gets between rem * floor(nchunks / 8) and
// rem * ceil(nchunks / 8) of their chunks, from at most two consecutive
// leftover tiles (the first one's chunks first), each tile's part a union of
// whole residue classes of the chunk index mod 8.
static void check_schedule(int ntiles, int nchunks) {
  const int64_t blocks = tile_sched_items_per_xcd(ntiles, nchunks) * kXcds;
  std::vector<int> seen((size_t)ntiles * nchunks, 0);
  std::vector<std::vector<int>> xcd_tiles(kXcds);
  for (int64_t b = 0; b < blocks; ++b) {
    const TileItem it = tile_sched_item(b, ntiles, nchunks);
    if (it.tile >= ntiles) {
      CHECK(it.tile == ntiles, "ntiles=%d nchunks=%d b=%lld tile=%d", ntiles, nchunks, (long long)b, it.tile);
      continue;
    }
    CHECK(it.tile >= 0 && it.chunk >= 0 && it.chunk < nchunks, "ntiles=%d nchunks=%d b=%lld (%d,%d)", ntiles,
          nchunks, (long long)b, it.tile, it.chunk);
    if (it.tile < 0 || it.chunk < 0 || it.chunk >= nchunks) continue;
    ++seen[(size_t)it.tile * nchunks + it.chunk];
    xcd_tiles[b % kXcds].push_back(it.tile);
  }
  for (int t = 0; t < ntiles; ++t)
    for (int c = 0; c < nchunks; ++c)
      CHECK(seen[(size_t)t * nchunks + c] == 1, "ntiles=%d nchunks=%d tile %d chunk %d served %d times", ntiles,
            nchunks, t, c, seen[(size_t)t * nchunks + c]);
  // the full rounds: XCD x reads only tiles x, x + 8, ...
  const int full = ntiles / kXcds;
  for (int x = 0; x < kXcds; ++x)
    for (int t : xcd_tiles[x])
      if (t < full * kXcds) CHECK(t % kXcds == x, "ntiles=%d xcd %d got tile %d", ntiles, x, t);
  // the leftover tiles: even shares, at most two tiles per XCD in order,
  // whole residue classes mod 8
  const int rem = ntiles % kXcds;
  if (rem) {
    std::vector<std::vector<std::pair<int, int>>> left(kXcds);  // (tile, chunk) in launch order
    for (int64_t b = 0; b < blocks; ++b) {
      const TileItem it = tile_sched_item(b, ntiles, nchunks);
      if (it.tile >= full * kXcds && it.tile < ntiles) left[b % kXcds].push_back({it.tile, it.chunk});
    }
    const int64_t lo = (int64_t)rem * (nchunks / kXcds), hi = (int64_t)rem * ((nchunks + kXcds - 1) / kXcds);
    for (int x = 0; x < kXcds; ++x) {
      const auto &v = left[x];
      CHECK((int64_t)v.size() >= lo && (int64_t)v.size() <= hi, "ntiles=%d nchunks=%d xcd %d has %zu leftover items",
            ntiles, nchunks, x, v.size());
      for (size_t k = 1; k < v.size(); ++k) {
        CHECK(v[k].first == v[k - 1].first || v[k].first == v[k - 1].first + 1,
              "ntiles=%d nchunks=%d xcd %d: leftover tiles out of order", ntiles, nchunks, x);
        if (v[k].first == v[k - 1].first)
          CHECK(v[k].second > v[k - 1].second, "ntiles=%d nchunks=%d xcd %d: chunks out of order", ntiles, nchunks, x);
      }
      if (!v.empty())
        CHECK(v.back().first - v.front().first <= 1, "ntiles=%d nchunks=%d xcd %d reads more than two leftover tiles",
              ntiles, nchunks, x);
      for (int t = full * kXcds; t < ntiles; ++t) {
        bool cls[kXcds] = {};
        int n = 0;
        for (const auto &e : v)
          if (e.first == t) {
            cls[e.second % kXcds] = true;
            ++n;
          }
        int want = 0;
        for (int c = 0; c < nchunks; ++c) want += cls[c % kXcds] ? 1 : 0;
        CHECK(n == want, "ntiles=%d nchunks=%d xcd %d tile %d: partial residue class", ntiles, nchunks, x, t);
      }
    }
  }
}

// tile_col and tile_of_col are inverse: every chunk of a row lands on exactly
// one (tile, lane), every non-padding (tile, lane) names a chunk, and the
// paired map puts column chunk j and j + half4 in lanes q and q ^ 4 of one tile.
static void check_map(const ColMap &m) {
  const int nt = map_tiles(m);
  std::vector<int> hits(m.cols4, 0);
  const int lanes = m.half4 == 0 ? (m.tch > 8 ? m.tch : 8) : 8;
  for (int t = 0; t < nt; ++t)
    for (int q = 0; q < lanes; ++q) {
      const int c = tile_col(m, t, q);
      if (c < 0) continue;
      CHECK(c < m.cols4, "map(%d,%d,%d,%d) t=%d q=%d -> %d", m.half4, m.t1, m.cols4, m.tch, t, q, c);
      if (c >= m.cols4) continue;
      ++hits[c];
      int t2 = -1, q2 = -1;
      tile_of_col(m, c, t2, q2);
      CHECK(t2 == t && q2 == q, "map(%d,%d,%d,%d) chunk %d: (%d,%d) vs (%d,%d)", m.half4, m.t1, m.cols4, m.tch, c,
            t, q, t2, q2);
      if (m.half4 > 0 && t < m.t1 && c < m.half4) {
        const int partner = tile_col(m, t, q ^ 4);
        CHECK(partner == c + m.half4, "paired map: chunk %d partner %d", c, partner);
      }
    }
  for (int c = 0; c < m.cols4; ++c) CHECK(hits[c] == 1, "map(%d,%d,%d,%d) chunk %d hit %d times", m.half4, m.t1,
                                          m.cols4, m.tch, c, hits[c]);
}

// long_segment(s0, s1) is true exactly for the segments the segment pass lists
// (long_listed_at at one of their samples), and then at exactly one sample.
static void check_long_rule(std::mt19937_64 &rng, int period) {
  for (int trial = 0; trial < 400; ++trial) {
    // sorted keys: runs of random lengths, some around period and 2 period
    std::vector<unsigned> keys;
    unsigned k = 0;
    const int runs = 1 + (int)(rng() % 60);
    for (int r = 0; r < runs; ++r) {
      int len;
      switch (rng() % 4) {
        case 0: len = 1 + (int)(rng() % 8); break;
        case 1: len = period - 3 + (int)(rng() % 8); break;
        case 2: len = 2 * period - 3 + (int)(rng() % 8); break;
        default: len = 1 + (int)(rng() % (5 * period)); break;
      }
      for (int i = 0; i < len; ++i) keys.push_back(k);
      k += 1 + (unsigned)(rng() % 3);
    }
    const int64_t M = (int64_t)keys.size();
    std::vector<int> listed(M + 1, 0);
    for (int64_t i = 0; i < M; ++i)
      if (long_listed_at(keys.data(), M, i, period)) ++listed[i];
    int64_t s0 = 0;
    while (s0 < M) {
      int64_t s1 = s0;
      while (s1 < M && keys[s1] == keys[s0]) ++s1;
      int count = 0;
      for (int64_t i = s0; i < s1; ++i) count += listed[i];
      const bool lng = long_segment(s0, s1, period);
      CHECK(count == (lng ? 1 : 0), "period=%d segment [%lld,%lld) listed %d times, long=%d", period, (long long)s0,
            (long long)s1, count, (int)lng);
      if (s1 - s0 >= 2 * period) CHECK(lng, "segment of %lld slots not long", (long long)(s1 - s0));
      if (s1 - s0 <= period) CHECK(!lng, "segment of %lld slots long", (long long)(s1 - s0));
      s0 = s1;
    }
  }
}

// The buckets that complete position chunk 0 (keys 0 .. N - 1 and key N):
// none of those keys lies in a later bucket, the count is the fewest that
// holds them, and it never exceeds the buckets of the key space.
static void check_chunk0_buckets(int64_t N, int nchunks, int sb) {
  const int n = buckets_through_chunk0(N, nchunks, sb);
  const int64_t nb = ceil_div((int64_t)nchunks * N, (int64_t)1 << sb);
  CHECK(n >= 1 && n <= nb, "N=%lld nchunks=%d sb=%d: %d of %lld buckets", (long long)N, nchunks, sb, n,
        (long long)nb);
  for (int64_t key = 0; key <= N; ++key)
    CHECK((key >> sb) < n, "N=%lld sb=%d: key %lld in bucket %lld of %d", (long long)N, sb, (long long)key,
          (long long)(key >> sb), n);
  CHECK((N >> sb) == n - 1, "N=%lld sb=%d: %d buckets, key N in bucket %lld", (long long)N, sb, n,
        (long long)(N >> sb));
}

int main() {
  // the sort divides slot numbers by max_active (K) and positions by the
  // position-chunk rows (ceil(B / 2) or B); cover every K the ABI allows up to
  // 4096, the workloads' batches and chunk sizes, and powers of two
  for (uint32_t d = 1; d <= 4096; ++d) check_fastdiv(d);
  const uint32_t extra[] = {8192, 16384, 20000, 32767, 32768, 32769, 40000, 65535, 65536, 65537, 100000, 131072,
                            1u << 20, (1u << 20) + 1, 1u << 24, 1u << 30, (1u << 30) + 1, 0x7fffffffu};
  for (uint32_t d : extra) check_fastdiv(d);

  for (int ntiles = 1; ntiles <= 70; ++ntiles)
    for (int nchunks : {1, 2, 3, 5, 7, 8, 9, 64, 255, 256, 257, 982, 1024, 1283})
      check_schedule(ntiles, nchunks);

  for (int cols4 = 1; cols4 <= 600; ++cols4)
    for (int tch : {4, 8, 16}) check_map(plain_map(cols4, tch));
  for (int half4 = 1; half4 <= 300; ++half4)
    for (int psqt4 : {0, 1, 2, 3, 8, 9, 17}) check_map(paired_map(2 * half4 + psqt4, half4));

  for (int sb : {7, 8})
    for (int64_t N = 1; N <= 2100; ++N)
      for (int nchunks : {2, 3}) check_chunk0_buckets(N, nchunks, sb);
  for (int64_t N : {22528, 23232, 24576, 60720, 85296, 85297}) check_chunk0_buckets(N, 2, N >= 65536 ? 8 : 7);
  CHECK(buckets_through_chunk0(1000, 1, 7) == 0, "one chunk has no chunk-0 split");

  std::mt19937_64 rng(12345);
  for (int period : {1, 2, 3, 8, 128, 256}) check_long_rule(rng, period);

  if (failures) {
    std::printf("%d failures\n", failures);
    return 1;
  }
  std::printf("index_math: all checks passed\n");
  return 0;
}
