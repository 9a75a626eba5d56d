// Feature-index encoder: chess positions -> the FT's sparse index rows
// (HalfKAv2_hm, Full_Threats and their composition), on the GPU.
//
// Replaces the reference's per-position index extraction
// (src/rust/feature_extraction.rs: FeatureSet::fill_feature_indices_sparse
// :209-236, fill_row_from_position_without_values :442-477, the HalfKAv2_hm
// indices :389-402, 677-685 and the Full_Threats indices :572-675, 687-833),
// which the reference runs on CPU threads and ships to the GPU as int32 slabs.
// Here the positions travel (65 bytes each) and the slabs are produced in HBM.
//
// Conventions (those of the sfbinpack crate the reference is written
// against): square a1 = 0 .. h8 = 63; piece id = 2 * type + color, types pawn,
// knight, bishop, rook, queen, king = 0..5, white = 0; bitboards are walked
// from the lowest square up.  board[64] holds a piece id or 255 (empty).
//
// One thread per (position, perspective).  Each workgroup first builds, in
// LDS, the empty-board attack masks and the threat offset table
// (threat_feature_calc, :795-833); the threat index's popcount of the attack
// mask below the target (Bitboard::from_before) then reads the mask from LDS.
#include "common.h"

namespace sft {

namespace {

constexpr int kPawn = 0, kKnight = 1, kBishop = 2, kRook = 3, kQueen = 4, kKing = 5;
constexpr int kHalfkaInputs = 24576, kHalfkaMax = 32, kThreatInputs = 60720, kThreatMax = 128;

// src/rust/feature_extraction.rs:27-35
__constant__ int kNumValidTargets[12] = {6, 6, 10, 10, 8, 8, 8, 8, 10, 10, 0, 0};
__constant__ int kThreatMap[6][6] = {
    {0, 1, -1, 2, -1, -1}, {0, 1, 2, 3, 4, -1}, {0, 1, 2, 3, -1, -1},
    {0, 1, 2, 3, -1, -1},  {0, 1, 2, 3, 4, -1}, {-1, -1, -1, -1, -1, -1},
};

__device__ __forceinline__ int popc64(uint64_t x) { return __popcll(x); }
__device__ __forceinline__ int lsb64(uint64_t x) { return __ffsll((unsigned long long)x) - 1; }

// King bucket of an oriented king square (files e-h after orientation):
// (7 - rank) * 4 + (7 - file) (src/rust/feature_extraction.rs:21-25).
__device__ __forceinline__ int king_bucket(int sq) { return (7 - (sq >> 3)) * 4 + (7 - (sq & 7)); }

// Step attacks of knights and kings.
__device__ uint64_t step_attacks(int from, const int (*d)[2], int n) {
  uint64_t a = 0;
  const int f0 = from & 7, r0 = from >> 3;
  for (int i = 0; i < n; ++i) {
    const int f = f0 + d[i][0], r = r0 + d[i][1];
    if (f >= 0 && f < 8 && r >= 0 && r < 8) a |= 1ull << (r * 8 + f);
  }
  return a;
}

// Sliding attacks along 4 directions (rook: orth, bishop: diag), stopping at
// the first occupied square (included).
__device__ uint64_t slide_attacks(int from, uint64_t occ, bool diag) {
  uint64_t a = 0;
  const int f0 = from & 7, r0 = from >> 3;
#pragma unroll
  for (int d = 0; d < 4; ++d) {
    const int df = diag ? ((d & 1) ? 1 : -1) : (d == 0 ? 1 : d == 1 ? -1 : 0);
    const int dr = diag ? ((d & 2) ? 1 : -1) : (d == 2 ? 1 : d == 3 ? -1 : 0);
    int f = f0 + df, r = r0 + dr;
    while (f >= 0 && f < 8 && r >= 0 && r < 8) {
      const int s = r * 8 + f;
      a |= 1ull << s;
      if ((occ >> s) & 1) break;
      f += df;
      r += dr;
    }
  }
  return a;
}

__device__ uint64_t pawn_captures(int color, int from) {
  const int f = from & 7, r = (from >> 3) + (color == 0 ? 1 : -1);
  if (r < 0 || r > 7) return 0;
  uint64_t a = 0;
  if (f > 0) a |= 1ull << (r * 8 + f - 1);
  if (f < 7) a |= 1ull << (r * 8 + f + 1);
  return a;
}

__constant__ int kKnightD[8][2] = {{1, 2}, {2, 1}, {2, -1}, {1, -2}, {-1, -2}, {-2, -1}, {-2, 1}, {-1, 2}};
__constant__ int kKingD[8][2] = {{1, 0}, {1, 1}, {0, 1}, {-1, 1}, {-1, 0}, {-1, -1}, {0, -1}, {1, -1}};

// Attack set on an empty board: index [piece id][square]; pawns: captures and
// push (the mask of the threat index, :723-733); kings are never attackers.
struct EncodeTables {
  uint64_t mask[10][64];
  int table[12][66];  // threat_feature_calc
};

__device__ uint64_t empty_mask(int piece, int from) {
  const int t = piece >> 1, c = piece & 1;
  switch (t) {
    case kPawn: {
      if (from < 8 || from > 55) return 0;
      return pawn_captures(c, from) | 1ull << (c == 0 ? from + 8 : from - 8);
    }
    case kKnight: return step_attacks(from, kKnightD, 8);
    case kBishop: return slide_attacks(from, 0, true);
    case kRook: return slide_attacks(from, 0, false);
    case kQueen: return slide_attacks(from, 0, true) | slide_attacks(from, 0, false);
    default: return step_attacks(from, kKingD, 8);
  }
}

__device__ void build_tables(EncodeTables &T) {
  __shared__ int sizes[12];
  for (int i = threadIdx.x; i < 10 * 64; i += blockDim.x) T.mask[i / 64][i % 64] = empty_mask(i / 64, i % 64);
  __syncthreads();
  if (threadIdx.x < 12) {  // per piece: from-square offsets within its block
    const int p = threadIdx.x;
    int off = 0;
    for (int s = 0; s < 64; ++s) {
      T.table[p][s] = off;
      off += (p >> 1) == kKing ? popc64(step_attacks(s, kKingD, 8)) : popc64(T.mask[p][s]);
    }
    T.table[p][64] = off;
    sizes[p] = off;
  }
  __syncthreads();
  if (threadIdx.x < 12) {
    // base offsets in the reference's piece order: colour outer, type inner
    // (src/rust/feature_extraction.rs:800-828)
    const int p = threadIdx.x;
    int base = 0;
    for (int color = 0; color < 2; ++color)
      for (int t = 0; t < 6; ++t) {
        const int q = 2 * t + color;
        if (q == p) T.table[p][65] = base;
        base += kNumValidTargets[q] * sizes[q];
      }
  }
  __syncthreads();
}

// full_threat_index (src/rust/feature_extraction.rs:687-737); -1: not a feature.
__device__ __forceinline__ int threat_index(const EncodeTables &T, int persp, int attacker, int from, int to,
                                            int attacked, int orient) {
  const bool enemy = (attacker & 1) != (attacked & 1);
  from ^= orient;
  to ^= orient;
  if (persp == 1) {
    attacker ^= 1;
    attacked ^= 1;
  }
  const int at = attacker >> 1, dt = attacked >> 1;
  const int mapped = kThreatMap[at][dt];
  if (mapped < 0 || (at == dt && (enemy || at != kPawn) && from < to)) return -1;
  const uint64_t before = (1ull << to) - 1;  // to >= 0; to == 0 gives 0
  return T.table[attacker][65] + ((attacked & 1) * (kNumValidTargets[attacker] / 2) + mapped) * T.table[attacker][64] +
         T.table[attacker][from] + popc64(before & T.mask[attacker][from]);
}

// Appends features to a row, 4 at a time as 16-byte stores.
struct RowWriter {
  int32_t *row;
  int n, cap_end;  // features written; the component's end slot
  i32x4 buf;
  int nbuf;
  int total;  // uncapped count of the component
  __device__ void push(int v) {
    ++total;
    if (n >= cap_end) return;
    buf[nbuf++] = v;
    ++n;
    if (nbuf == 4) flush();
  }
  __device__ void flush() {
    // n - nbuf is a multiple of 4 except after a component whose count is not;
    // fall back to scalar stores then.
    const int start = n - nbuf;
    if ((start & 3) == 0 && nbuf == 4) {
      *reinterpret_cast<i32x4 *>(row + start) = buf;
    } else {
      for (int i = 0; i < nbuf; ++i) row[start + i] = buf[i];
    }
    nbuf = 0;
  }
};

struct Encoding {
  int ncomp;
  int comp[2];  // 1 = Full_Threats, 2 = HalfKAv2_hm, in feature-set order
  int K;
};

__global__ __launch_bounds__(kBlock) void encode_kernel(const uint8_t *__restrict__ boards,
                                                        const uint8_t *__restrict__ stm, int64_t B, Encoding enc,
                                                        int32_t *__restrict__ white, int32_t *__restrict__ black,
                                                        float *__restrict__ us, int64_t *__restrict__ psqt,
                                                        int64_t *__restrict__ ls, int32_t *__restrict__ count_w,
                                                        int32_t *__restrict__ count_b) {
  __shared__ EncodeTables T;
  if (enc.comp[0] == 1 || (enc.ncomp > 1 && enc.comp[1] == 1)) build_tables(T);  // block-uniform
  const int64_t t = (int64_t)blockIdx.x * kBlock + threadIdx.x;
  const int64_t b = t >> 1;
  const int persp = (int)(t & 1);
  if (b >= B) return;

  // Bitboards of the position.
  uint64_t bb[12];
#pragma unroll
  for (int i = 0; i < 12; ++i) bb[i] = 0;
  const i32x4 *src = reinterpret_cast<const i32x4 *>(boards + 64 * b);
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    const i32x4 w = src[c];
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      const int pc = (w[e >> 2] >> (8 * (e & 3))) & 0xff;
      const uint64_t bit = 1ull << (16 * c + e);
#pragma unroll
      for (int i = 0; i < 12; ++i) bb[i] |= pc == i ? bit : 0ull;
    }
  }
  uint64_t occ = 0;
#pragma unroll
  for (int i = 0; i < 12; ++i) occ |= bb[i];
  const uint64_t pawns = bb[0] | bb[1];
  const int ksq = lsb64(bb[2 * kKing + persp]);
  const uint8_t *board = boards + 64 * b;

  int32_t *row = (persp == 0 ? white : black) + b * enc.K;
  RowWriter w;
  w.row = row;
  w.n = 0;
  w.nbuf = 0;
  int offset = 0, all = 0;
  for (int ci = 0; ci < enc.ncomp; ++ci) {
    const int comp = enc.comp[ci];
    w.cap_end = w.n + (comp == 1 ? kThreatMax : kHalfkaMax);
    w.total = 0;
    if (comp == 2) {
      // fill_halfka_feature_indices_sparse (:389-402)
      const int o = ((ksq & 7) < 4 ? 7 : 0) ^ (persp == 1 ? 56 : 0);
      const int kb = king_bucket(ksq ^ o) * 768;
      for (uint64_t x = occ; x; x &= x - 1) {
        const int s = lsb64(x);
        const int pc = board[s];
        w.push(offset + (s ^ o) + ((pc >> 1) * 2 + ((pc & 1) != persp)) * 64 + kb);
      }
    } else {
      // fill_full_threat_feature_indices_sparse (:572-675)
      const int o = ((ksq & 7) >= 4 ? 7 : 0) ^ (persp == 1 ? 56 : 0);
      const uint64_t A_FILE = 0x0101010101010101ull, H_FILE = 0x8080808080808080ull;
      for (int cr = 0; cr < 2; ++cr) {
        const int color = cr == 0 ? persp : 1 - persp;
        for (int type = 0; type < 6; ++type) {
          const int attacker = 2 * type + color;
          const uint64_t pbb = bb[attacker];
          if (!pbb) continue;
          if (type == kPawn) {
            const uint64_t sets[3] = {
                (color == 0 ? (pbb & ~H_FILE) << 9 : (pbb & ~A_FILE) >> 9) & occ,
                (color == 0 ? (pbb & ~A_FILE) << 7 : (pbb & ~H_FILE) >> 7) & occ,
                (color == 0 ? pbb << 8 : pbb >> 8) & pawns};
            const int delta[3] = {9, 7, 8};
            for (int k = 0; k < 3; ++k)
              for (uint64_t x = sets[k]; x; x &= x - 1) {
                const int to = lsb64(x);
                const int from = color == 0 ? to - delta[k] : to + delta[k];
                const int idx = threat_index(T, persp, attacker, from, to, board[to], o);
                if (idx >= 0) w.push(offset + idx);
              }
          } else {
            for (uint64_t f = pbb; f; f &= f - 1) {
              const int from = lsb64(f);
              uint64_t att;
              if (type == kKnight) att = T.mask[attacker][from];
              else if (type == kKing) att = step_attacks(from, kKingD, 8);
              else if (type == kBishop) att = slide_attacks(from, occ, true);
              else if (type == kRook) att = slide_attacks(from, occ, false);
              else att = slide_attacks(from, occ, true) | slide_attacks(from, occ, false);
              for (uint64_t x = att & occ; x; x &= x - 1) {
                const int to = lsb64(x);
                const int idx = threat_index(T, persp, attacker, from, to, board[to], o);
                if (idx >= 0) w.push(offset + idx);
              }
            }
          }
        }
      }
    }
    if (w.nbuf) w.flush();
    all += w.total;
    offset += comp == 1 ? kThreatInputs : kHalfkaInputs;
  }
  for (int i = w.n; i < enc.K; ++i) row[i] = -1;
  if (persp == 0) {
    if (count_w) count_w[b] = all;
    int pieces = popc64(occ);
    if (us) us[b] = stm[b] == 0 ? 1.0f : 0.0f;
    if (psqt) psqt[b] = (pieces - 1) / 4;
    if (ls) ls[b] = (pieces - 1) / 4;
  } else if (count_b) {
    count_b[b] = all;
  }
}

}  // namespace

int encode_features(const uint8_t *boards, const uint8_t *stm, int64_t B, const int32_t *comps, int ncomp,
                    int32_t *white, int32_t *black, int K, float *us, int64_t *psqt, int64_t *ls, int32_t *count_w,
                    int32_t *count_b, hipStream_t s) {
  Encoding enc{};
  enc.ncomp = ncomp;
  for (int i = 0; i < ncomp; ++i) enc.comp[i] = comps[i];
  enc.K = K;
  ProfScope prof(kProfEncode, s);
  hipLaunchKernelGGL(encode_kernel, dim3((unsigned)ceil_div(2 * B, kBlock)), dim3(kBlock), 0, s, boards, stm, B, enc,
                     white, black, us, psqt, ls, count_w, count_b);
  return check_launch("sft_encode_features");
}

}  // namespace sft
