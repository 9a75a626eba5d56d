"""Chess positions in the encoder's input format.

A position is a board of 64 piece ids (square a1 = 0 .. h8 = 63; id =
2 * type + color with pawn, knight, bishop, rook, queen, king = 0..5 and
white = 0, black = 1; 255 = empty) plus the side to move (0 = white) — the
conventions of the sfbinpack crate the reference's feature extraction is
written against (src/rust/feature_extraction.rs:4-8).

  board_from_fen(fen) -> (uint8[64], stm)
  random_positions(B, seed) -> (uint8[B, 64], uint8[B])   synthetic positions for tests/benchmarks
  mirror(boards, stm) -> colours swapped and ranks flipped
"""

from __future__ import annotations

import numpy as np

EMPTY = 255
_FEN_TYPES = {"p": 0, "n": 1, "b": 2, "r": 3, "q": 4, "k": 5}
STARTPOS = "rnbqkbnr/pppppppp/8/8/8/8/PPPPPPPP/RNBQKBNR w KQkq - 0 1"


def board_from_fen(fen: str):
    placement, side = fen.split()[:2]
    board = np.full(64, EMPTY, np.uint8)
    for r, rank in enumerate(placement.split("/")):
        f = 0
        for ch in rank:
            if ch.isdigit():
                f += int(ch)
                continue
            board[(7 - r) * 8 + f] = 2 * _FEN_TYPES[ch.lower()] + (0 if ch.isupper() else 1)
            f += 1
    return board, np.uint8(0 if side == "w" else 1)


def random_positions(B: int, seed: int = 0, max_per_side: int = 16):
    """Kings plus a random army per side (up to 8 pawns on ranks 2-7, minor and
    major pieces in at most standard numbers plus promotions), placed on
    distinct random squares; side to move random.  Not necessarily legal."""
    g = np.random.default_rng(seed)
    boards = np.full((B, 64), EMPTY, np.uint8)
    stm = g.integers(0, 2, B).astype(np.uint8)
    for b in range(B):
        free = list(g.permutation(64))
        for color in (0, 1):
            boards[b, free.pop()] = 2 * 5 + color
        for color in (0, 1):
            n = int(g.integers(0, max_per_side))
            pawns = int(g.integers(0, min(8, n) + 1))
            pieces = [0] * pawns + list(g.choice([1, 2, 3, 4], n - pawns, p=[0.3, 0.3, 0.3, 0.1]))
            for t in pieces:
                for k, sq in enumerate(free):
                    if t != 0 or 8 <= sq < 56:
                        boards[b, free.pop(k)] = 2 * t + color
                        break
    return boards, stm


def mirror(boards, stm):
    """The same position seen from the other side: colours swapped, ranks flipped."""
    boards = np.asarray(boards, np.uint8)
    out = np.full_like(boards, EMPTY)
    sq = np.arange(64)
    src = sq ^ 56
    occ = boards[..., src] != EMPTY
    out[..., sq] = np.where(occ, boards[..., src] ^ 1, EMPTY)
    return out, (np.asarray(stm, np.uint8) ^ 1)
