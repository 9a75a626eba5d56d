// Shared definitions of the gfx950 FT kernels and their host launchers.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <string>

#include "index_math.h"
#include "sft_ft.h"

namespace sft {

// Native clang vectors: elementwise +, 16-byte loads/stores (global_load_dwordx4).
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef short i16x8 __attribute__((ext_vector_type(8)));
typedef int i32x8 __attribute__((ext_vector_type(8)));
typedef int i32x4 __attribute__((ext_vector_type(4)));

constexpr int kWave = 64;          // CDNA wavefront width
constexpr int kWavesPerBlock = 4;  // 256-thread workgroups
constexpr int kBlock = kWave * kWavesPerBlock;
constexpr int kMaxCpl = 8;         // max vector chunks per lane per pass
constexpr size_t kMaxIndexLds = 64 * 1024;  // LDS budget of the per-block index lists

// ---- host-side error plumbing (thread-local, read by sft_last_error) ----
void set_error(const std::string &msg);
void clear_error();
int fail(int code, const std::string &msg);
int check_launch(const char *what);

// ---- fork/join with the calling thread's side stream on the current device ----
// fork_side: work enqueued on *side after the call runs after everything
// already enqueued on s.  mark_side(k) records mark k on the side stream (after
// the work enqueued there so far); wait_side(s, k): work enqueued on s after
// the call runs after that mark.  join_side(s) = mark 0 + wait.  All are stream
// operations (event record / wait), so they capture into a graph like kernels.
constexpr int kSideMarks = 2;
int fork_side(hipStream_t s, hipStream_t *side);
int mark_side(int slot);
int wait_side(hipStream_t s, int slot);
int join_side(hipStream_t s);
// Joins the side stream into s when it goes out of scope unless release()d, so
// an error return after fork_side never leaves side-stream work unordered with
// s (a graph capture stays joined; freed workspace is not reused early).  It
// keeps the error message of the failure that caused the early return.
class SideJoinGuard {
 public:
  explicit SideJoinGuard(hipStream_t s) : s_(s) {}
  ~SideJoinGuard();
  void release() { armed_ = false; }
  SideJoinGuard(const SideJoinGuard &) = delete;
  SideJoinGuard &operator=(const SideJoinGuard &) = delete;

 private:
  hipStream_t s_;
  bool armed_ = true;
};

// ---- kernel timing hooks (active only between sft_prof_enable(1) and (0)) ----
enum ProfKind : int {
  kProfFwdF32 = 0,
  kProfBwdSort,
  kProfBwdOffsets,
  kProfBwdGather,
  kProfBwdBiasPartial,
  kProfBwdBiasFinal,
  kProfBwdAtomic,
  kProfBwdZero,
  kProfFwdI16,
  kProfQuantize,
  kProfFwdRelayout,
  kProfFwdTiled,
  kProfBwdTiled,
  kProfFwdI16Tiled,
  kProfFwdFold,
  kProfBwdVirtual,
  kProfBwdEpilogue,
  kProfOptim,
  kProfEncode,
  kProfLeb128,
  kProfProbeL2Gather,
  kProfFwdRanks,
  kProfNumKinds
};
struct ProfScope {
  ProfScope(int kind, hipStream_t stream);
  ~ProfScope();
  void *slot_;
};

// ---- lane/position mapping shared by the row-gather kernels ----
// A lane group of G lanes (G in {8,16,32,64}) owns one row (a position in the
// forward, a feature in the backward).  Lane t of the group handles vector
// chunks c = slab*G*CPL + t + G*j, j < CPL, so consecutive lanes read
// consecutive 16-byte chunks.  Rows wider than G*CPL chunks use several
// column slabs (grid.y).
struct Mapping {
  int G;
  int cpl;
  int slabs;
};
Mapping choose_mapping(int64_t chunks, int min_group = 8);

// Loads of arrays streamed once per tile pass (index rows, sorted position
// lists).  Marking them non-temporal (SFT_STREAM_NT=1) was measured slower at
// B = 65536 (forward 302 -> 448 us, backward gather 217 -> 244 us per launch),
// so they are plain loads by default.
#ifndef SFT_STREAM_NT
#define SFT_STREAM_NT 0
#endif
#if SFT_STREAM_NT
#define SFT_STREAM_LOAD(p) __builtin_nontemporal_load(p)
#else
#define SFT_STREAM_LOAD(p) (*(p))
#endif

// ---- device helpers ----
__device__ __forceinline__ int lane_id() { return __builtin_amdgcn_mbcnt_hi(~0u, __builtin_amdgcn_mbcnt_lo(~0u, 0)); }

// Number of set bits of `mask` in lanes below the calling lane.
__device__ __forceinline__ int popc_below(uint64_t mask) {
  return __builtin_amdgcn_mbcnt_hi((uint32_t)(mask >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)mask, 0));
}

__device__ __forceinline__ uint64_t ballot(bool p) { return __builtin_amdgcn_ballot_w64(p); }

__device__ __forceinline__ int uniform(int v) { return __builtin_amdgcn_readfirstlane(v); }

// Orders a wave's LDS writes before its later LDS reads by other lanes of the
// same wave (LDS operations of one wave complete in order; this keeps the
// compiler from moving them across).
__device__ __forceinline__ void wave_lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
  __builtin_amdgcn_wave_barrier();
}

constexpr int kCompactRows = 8;  // most rows one compact_rows call takes
// Compacts the active slots of `npos` consecutive index rows (row p at
// idx + (pos0 + p) * K) into list[p * kpad + 0 .. count[p]), keeping slot order.
// Called by one whole wave with npos <= kCompactRows; rows at or past B get count 0.  A slot is active
// when 0 <= v < N.  For K <= 64 one ballot covers 64 / Kp rows (Kp = K rounded
// up to a power of two): lane l reads slot l % Kp of row l / Kp and ranks
// itself among the active lanes of its own Kp-lane segment.  The wave owns
// list/count; before other lanes of the wave read them it calls
// wave_lds_barrier (the rows of one wave need no workgroup barrier).
__device__ __forceinline__ void compact_rows(const int32_t *__restrict__ idx, int64_t B, int K, int N,
                                             int64_t pos0, int npos, int *list, int kpad, int *count) {
  const int lane = lane_id();
  if (K <= kWave) {
    int kp = 1;
    while (kp < K) kp <<= 1;
    const int rows_per_ballot = kWave / kp;
    const int seg = lane / kp, slot = lane % kp;
    const uint64_t segmask = (kp == kWave) ? ~0ull : (((1ull << kp) - 1) << (seg * kp));
    // All loads first (npos <= kCompactRows, so at most kCompactRows ballots),
    // so that their latencies overlap instead of adding up.
    int v[kCompactRows];
#pragma unroll
    for (int i = 0; i < kCompactRows; ++i) {
      const int p = i * rows_per_ballot + seg;
      const int64_t pos = pos0 + p;
      v[i] = -1;
      if (p < npos && pos < B && slot < K) v[i] = SFT_STREAM_LOAD(idx + pos * (int64_t)K + slot);
    }
#pragma unroll
    for (int i = 0; i < kCompactRows; ++i) {
      if (i * rows_per_ballot >= npos) break;  // wave-uniform
      const int p = i * rows_per_ballot + seg;
      const bool ok = (unsigned)v[i] < (unsigned)N;
      const uint64_t m = ballot(ok) & segmask;
      if (ok) list[p * kpad + popc_below(m)] = v[i];
      if (slot == 0 && p < npos) count[p] = __popcll(m);
    }
    return;
  }
  for (int p = 0; p < npos; ++p) {
    const int64_t pos = pos0 + p;
    int base = 0;
    if (pos < B) {
      const int32_t *row = idx + pos * (int64_t)K;
      for (int k0 = 0; k0 < K; k0 += kWave) {
        const int k = k0 + lane;
        int v = -1;
        if (k < K) v = row[k];
        const bool ok = (unsigned)v < (unsigned)N;
        const uint64_t m = ballot(ok);
        if (ok) list[p * kpad + base + popc_below(m)] = v;
        base += __popcll(m);
      }
    }
    if (lane == 0) count[p] = base;
  }
}

#ifndef SFT_MIN_TILES
#define SFT_MIN_TILES 8
#endif
constexpr int kMinTiles = SFT_MIN_TILES;  // fewest column tiles for which the int16 tiled forward is used
// The fp32 backward tiles from 4 column tiles (L > 96): with the leftover
// tiles shared evenly over the XCDs (tile_sched_item), L = 136 (5 tiles) runs
// its gathers in 2 x 37.8 us per perspective against 107.7 us for the row
// gather, and the bias pass, which then also writes the grad tiles, 20.7
// against 10.5 us (step 0.495 -> 0.406 ms).
#ifndef SFT_BWD_MIN_TILES
#define SFT_BWD_MIN_TILES 4
#endif
constexpr int kBwdMinTiles = SFT_BWD_MIN_TILES;

// ---- composed tables ----
// A composed feature transformer's table is the concatenation of up to
// kMaxBlocks row blocks (one per feature set); block s covers merged rows
// [start[s], start[s + 1]).  A block may carry virtual rows: merged row r of
// the block then reads w[r] + v[r % period].
constexpr int kMaxBlocks = 4;
struct FoldSrc {
  int n;
  int64_t start[kMaxBlocks + 1];
  const f32x4 *w[kMaxBlocks];
  const f32x4 *v[kMaxBlocks];  // null: no virtual rows
  int64_t period[kMaxBlocks];
};
// Where the grad of each merged row goes (row-major blocks of cols4 chunks).
struct RowDst {
  int n;
  int64_t start[kMaxBlocks + 1];
  f32x4 *p[kMaxBlocks];
};
// a[s] for a run-time s without indexing the kernel-argument array (selects).
template <typename T, int M>
__device__ __forceinline__ T pick(const T (&a)[M], int s) {
  T x = a[0];
#pragma unroll
  for (int j = 1; j < M; ++j) x = (s == j) ? a[j] : x;
  return x;
}
__device__ __forceinline__ int block_of(int64_t r, int n, const int64_t *start) {
  int s = 0;
#pragma unroll
  for (int j = 1; j < kMaxBlocks; ++j) s += (j < n && r >= start[j]) ? 1 : 0;
  return s;
}

}  // namespace sft
