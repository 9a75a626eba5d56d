/*
 * CPU oracle of the feature-index encoder: chess positions -> the FT's sparse
 * index rows (HalfKAv2_hm, Full_Threats and their composition).
 *
 * TEST INFRASTRUCTURE ONLY.  This file restates, in plain C, the reference's
 * index computation (src/rust/feature_extraction.rs) so that the HIP encoder
 * can be checked against it.  It is never linked into, called by, or used as a
 * fallback for the product library.
 *
 * The reference builds on the sfbinpack crate (0.6.2, Cargo.toml:15; not
 * vendored).  From it this file takes only the published chess conventions the
 * reference's code relies on: squares a1 = 0 .. h8 = 63 (file = sq & 7,
 * rank = sq >> 3); piece id = 2 * type + color with types pawn, knight,
 * bishop, rook, queen, king = 0..5 and white = 0, black = 1; bitboard
 * iteration from the lowest square up; the usual attack sets of each piece;
 * Bitboard::from_before(s) = the squares below s.
 *
 * Position input: board[64] = piece id per square, 255 = empty; stm = 0 white
 * to move, 1 black.
 */
#include <stdint.h>
#include <string.h>

#define EMPTY 255
enum { PAWN = 0, KNIGHT, BISHOP, ROOK, QUEEN, KING };
enum { WHITE = 0, BLACK = 1 };

#define HALFKA_INPUTS 24576
#define HALFKA_MAX 32
#define THREATS_INPUTS 60720
#define THREATS_MAX 128

/* src/rust/feature_extraction.rs:21-25 */
static const int32_t KING_BUCKETS[64] = {
    -1, -1, -1, -1, 31, 30, 29, 28, -1, -1, -1, -1, 27, 26, 25, 24, -1, -1, -1, -1, 23, 22,
    21, 20, -1, -1, -1, -1, 19, 18, 17, 16, -1, -1, -1, -1, 15, 14, 13, 12, -1, -1, -1, -1,
    11, 10, 9,  8,  -1, -1, -1, -1, 7,  6,  5,  4,  -1, -1, -1, -1, 3,  2,  1,  0,
};
/* src/rust/feature_extraction.rs:27-35 */
static const int32_t NUM_VALID_TARGETS[12] = {6, 6, 10, 10, 8, 8, 8, 8, 10, 10, 0, 0};
static const int32_t THREAT_MAP[6][6] = {
    {0, 1, -1, 2, -1, -1}, {0, 1, 2, 3, 4, -1}, {0, 1, 2, 3, -1, -1},
    {0, 1, 2, 3, -1, -1},  {0, 1, 2, 3, 4, -1}, {-1, -1, -1, -1, -1, -1},
};

static int popcount64(uint64_t x) { return __builtin_popcountll(x); }
static int type_of(int piece) { return piece >> 1; }
static int color_of(int piece) { return piece & 1; }

/* Attack set of a piece on `from` by walking rays on an 8 x 8 grid. */
static uint64_t ray_attacks(int from, uint64_t occ, const int (*dirs)[2], int ndirs, int slide) {
    uint64_t a = 0;
    int f0 = from & 7, r0 = from >> 3;
    for (int d = 0; d < ndirs; ++d) {
        int f = f0 + dirs[d][0], r = r0 + dirs[d][1];
        while (f >= 0 && f < 8 && r >= 0 && r < 8) {
            int s = r * 8 + f;
            a |= 1ull << s;
            if (!slide || (occ >> s & 1)) break;
            f += dirs[d][0];
            r += dirs[d][1];
        }
    }
    return a;
}

static const int KNIGHT_D[8][2] = {{1, 2}, {2, 1}, {2, -1}, {1, -2}, {-1, -2}, {-2, -1}, {-2, 1}, {-1, 2}};
static const int KING_D[8][2] = {{1, 0}, {1, 1}, {0, 1}, {-1, 1}, {-1, 0}, {-1, -1}, {0, -1}, {1, -1}};
static const int ROOK_D[4][2] = {{1, 0}, {-1, 0}, {0, 1}, {0, -1}};
static const int BISHOP_D[4][2] = {{1, 1}, {1, -1}, {-1, 1}, {-1, -1}};

static uint64_t piece_attacks(int type, int from, uint64_t occ) {
    switch (type) {
        case KNIGHT: return ray_attacks(from, occ, KNIGHT_D, 8, 0);
        case BISHOP: return ray_attacks(from, occ, BISHOP_D, 4, 1);
        case ROOK: return ray_attacks(from, occ, ROOK_D, 4, 1);
        case QUEEN: return ray_attacks(from, occ, BISHOP_D, 4, 1) | ray_attacks(from, occ, ROOK_D, 4, 1);
        case KING: return ray_attacks(from, occ, KING_D, 8, 0);
        default: return 0;
    }
}

/* Squares a pawn of `color` on `from` attacks (captures). */
static uint64_t pawn_attacks(int color, int from) {
    int f = from & 7, r = from >> 3, dr = color == WHITE ? 1 : -1;
    uint64_t a = 0;
    if (r + dr < 0 || r + dr > 7) return 0;
    if (f > 0) a |= 1ull << ((r + dr) * 8 + f - 1);
    if (f < 7) a |= 1ull << ((r + dr) * 8 + f + 1);
    return a;
}

/* threat_feature_calc, src/rust/feature_extraction.rs:795-833:
 * table[p][s] = offset of from-square s within piece p's block, [64] = the
 * block's per-target size, [65] = the piece's base offset. */
static int32_t g_table[12][66];
static int g_table_total = -1;

static void build_table(void) {
    if (g_table_total >= 0) return;
    int32_t piece_offset = 0;
    for (int color = 0; color < 2; ++color)
        for (int type = 0; type < 6; ++type) {
            int p = 2 * type + color;
            g_table[p][65] = piece_offset;
            int32_t sq_offset = 0;
            for (int from = 0; from < 64; ++from) {
                g_table[p][from] = sq_offset;
                if (type != PAWN) {
                    sq_offset += popcount64(piece_attacks(type, from, 0));
                } else if (from >= 8 && from <= 55) {
                    uint64_t m = pawn_attacks(color, from) | 1ull << (color == WHITE ? from + 8 : from - 8);
                    sq_offset += popcount64(m);
                }
            }
            g_table[p][64] = sq_offset;
            piece_offset += NUM_VALID_TARGETS[p] * sq_offset;
        }
    g_table_total = piece_offset;
}

int feature_oracle_threat_total(void) {
    build_table();
    return g_table_total;
}

int feature_oracle_threat_table(int32_t *out /* [12][66] */) {
    build_table();
    memcpy(out, g_table, sizeof(g_table));
    return 0;
}

/* orient masks, src/rust/feature_extraction.rs:744-762 */
static int halfka_orient(int color, int ksq) { return ((ksq & 7) < 4 ? 7 : 0) ^ (color == BLACK ? 56 : 0); }
static int threat_orient(int color, int ksq) { return ((ksq & 7) >= 4 ? 7 : 0) ^ (color == BLACK ? 56 : 0); }

/* halfka_feature_index, src/rust/feature_extraction.rs:677-685 */
static int32_t halfka_index(int color, int ksq, int sq, int piece) {
    int o = halfka_orient(color, ksq);
    int pidx = type_of(piece) * 2 + (color_of(piece) != color);
    return (sq ^ o) + pidx * 64 + KING_BUCKETS[ksq ^ o] * 768;
}

/* full_threat_index, src/rust/feature_extraction.rs:687-737 */
static int32_t threat_index(int persp, int attacker, int from, int to, int attacked, int ksq) {
    int enemy = color_of(attacker) != color_of(attacked);
    int o = threat_orient(persp, ksq);
    from ^= o;
    to ^= o;
    if (persp == BLACK) {
        attacker ^= 1;
        attacked ^= 1;
    }
    int at = type_of(attacker), dt = type_of(attacked);
    int mapped = THREAT_MAP[at][dt];
    if (mapped < 0 || (at == dt && (enemy || at != PAWN) && from < to)) return -1;
    uint64_t mask;
    if (at == PAWN)
        mask = pawn_attacks(color_of(attacker), from) |
               1ull << (color_of(attacker) == WHITE ? from + 8 : from - 8);
    else
        mask = piece_attacks(at, from, 0);
    int p = attacker; /* piece_index = 2 * type + color = id */
    uint64_t before = to == 0 ? 0 : ((1ull << to) - 1);
    return g_table[p][65] + (color_of(attacked) * (NUM_VALID_TARGETS[p] / 2) + mapped) * g_table[p][64] +
           g_table[p][from] + popcount64(before & mask);
}

static uint64_t pieces_bb(const uint8_t *board, int color, int type) {
    uint64_t b = 0;
    for (int s = 0; s < 64; ++s)
        if (board[s] == 2 * type + color) b |= 1ull << s;
    return b;
}

static int king_sq(const uint8_t *board, int color) {
    for (int s = 0; s < 64; ++s)
        if (board[s] == 2 * KING + color) return s;
    return -1;
}

#define PUSH(v)                                   \
    do {                                          \
        if ((v) >= 0) {                           \
            if (n < cap) out[n] = (v);            \
            ++n;                                  \
        }                                         \
    } while (0)

/* fill_halfka_feature_indices_sparse, src/rust/feature_extraction.rs:389-402 */
static int halfka_features(const uint8_t *board, int color, int32_t *out, int cap) {
    int ksq = king_sq(board, color), n = 0;
    for (int s = 0; s < 64; ++s)
        if (board[s] != EMPTY) PUSH(halfka_index(color, ksq, s, board[s]));
    return n;
}

/* fill_full_threat_feature_indices_sparse, src/rust/feature_extraction.rs:572-675 */
static int threat_features(const uint8_t *board, int persp, int32_t *out, int cap) {
    build_table();
    uint64_t occ = 0;
    for (int s = 0; s < 64; ++s)
        if (board[s] != EMPTY) occ |= 1ull << s;
    const uint64_t A_FILE = 0x0101010101010101ull, H_FILE = 0x8080808080808080ull;
    uint64_t pawns = pieces_bb(board, WHITE, PAWN) | pieces_bb(board, BLACK, PAWN);
    int ksq = king_sq(board, persp), n = 0;
    for (int ci = 0; ci < 2; ++ci) {
        int color = ci == 0 ? persp : 1 - persp;
        for (int type = 0; type < 6; ++type) {
            int attacker = 2 * type + color;
            uint64_t bb = pieces_bb(board, color, type);
            if (type == PAWN) {
                uint64_t left = color == WHITE ? (bb & ~H_FILE) << 9 : (bb & ~A_FILE) >> 9;
                uint64_t right = color == WHITE ? (bb & ~A_FILE) << 7 : (bb & ~H_FILE) >> 7;
                uint64_t fwd = color == WHITE ? bb << 8 : bb >> 8;
                const uint64_t sets[3] = {left & occ, right & occ, fwd & pawns};
                const int delta[3] = {9, 7, 8};
                for (int k = 0; k < 3; ++k)
                    for (int to = 0; to < 64; ++to)
                        if (sets[k] >> to & 1) {
                            int from = color == WHITE ? to - delta[k] : to + delta[k];
                            PUSH(threat_index(persp, attacker, from, to, board[to], ksq));
                        }
            } else {
                for (int from = 0; from < 64; ++from) {
                    if (!(bb >> from & 1)) continue;
                    uint64_t att = piece_attacks(type, from, occ) & occ;
                    for (int to = 0; to < 64; ++to)
                        if (att >> to & 1) PUSH(threat_index(persp, attacker, from, to, board[to], ksq));
                }
            }
        }
    }
    return n;
}

/*
 * Encode B positions for a feature set given as components in order
 * (1 = Full_Threats, 2 = HalfKAv2_hm; e.g. {1, 2} = "Full_Threats+HalfKAv2_hm"),
 * following FeatureSet::fill_feature_indices_sparse and
 * fill_row_from_position_without_values (src/rust/feature_extraction.rs:209-236,
 * 442-477): each component writes after the previous one's features with its
 * indices offset by the previous components' input counts; rows are padded
 * with -1 to K = the sum of the components' maxima.  A component that would
 * exceed its maximum is cut at it and counted in *overflow.
 * Also: us = 1 for white to move, psqt = layer-stack bucket = (pieces - 1) / 4.
 */
int feature_oracle_encode(const uint8_t *boards, const uint8_t *stm, int64_t B, const int32_t *comps, int ncomps,
                          int32_t *white, int32_t *black, float *us, int64_t *psqt, int64_t *count_w,
                          int64_t *count_b, int64_t *overflow) {
    int K = 0;
    for (int c = 0; c < ncomps; ++c) {
        if (comps[c] != 1 && comps[c] != 2) return -1;
        K += comps[c] == 1 ? THREATS_MAX : HALFKA_MAX;
    }
    int64_t over = 0;
    build_table();
#pragma omp parallel for reduction(+ : over) schedule(static)
    for (int64_t b = 0; b < B; ++b) {
        const uint8_t *board = boards + 64 * b;
        for (int persp = 0; persp < 2; ++persp) {
            int32_t *row = (persp == WHITE ? white : black) + b * K;
            int written = 0, offset = 0;
            for (int c = 0; c < ncomps; ++c) {
                int cap = comps[c] == 1 ? THREATS_MAX : HALFKA_MAX;
                int n = comps[c] == 1 ? threat_features(board, persp, row + written, cap)
                                      : halfka_features(board, persp, row + written, cap);
                if (n > cap) {
                    over += 1;
                    n = cap;
                }
                for (int i = 0; i < n; ++i) row[written + i] += offset;
                written += n;
                offset += comps[c] == 1 ? THREATS_INPUTS : HALFKA_INPUTS;
            }
            for (int i = written; i < K; ++i) row[i] = -1;
            (persp == WHITE ? count_w : count_b)[b] = written;
        }
        int pieces = 0;
        for (int s = 0; s < 64; ++s) pieces += board[s] != EMPTY;
        us[b] = stm[b] == WHITE ? 1.0f : 0.0f;
        psqt[b] = (pieces - 1) / 4;
    }
    *overflow = over;
    return 0;
}

/* One threat index (for the tests' enumeration of the index space). */
int feature_oracle_threat_index(int persp, int attacker, int from, int to, int attacked, int ksq) {
    build_table();
    return threat_index(persp, attacker, from, to, attacked, ksq);
}
