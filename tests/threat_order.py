"""Full_Threats row order restated from the reference's loop structure
(src/rust/feature_extraction.rs:581-675), independently of the oracle's
bitboard walk: every (attacker, from, to) threat of a position is generated
square by square, given the sort key of the loop that emits it, and the
admitted indices are listed in key order.

Loop nesting of fill_full_threat_feature_indices_sparse: colours with the
perspective's own colour first (:592-595); piece types pawn .. king (:598-605);
pawns emit their left captures, then right captures, then pushes onto a pawn
(:611-656), each in ascending target square; other pieces emit, per source
square ascending, their targets ascending (:657-672).  The index of each
threat comes from the oracle's full_threat_index (:687-733), which
test_encode_cpu.py pins separately (a bijection onto [0, 60720)).
"""

from __future__ import annotations

import ctypes

import numpy as np

from oracle import feature_oracle as fo

EMPTY = 255
KNIGHT = [(1, 2), (2, 1), (2, -1), (1, -2), (-1, -2), (-2, -1), (-2, 1), (-1, 2)]
KING = [(1, 0), (1, 1), (0, 1), (-1, 1), (-1, 0), (-1, -1), (0, -1), (1, -1)]
DIAG = [(1, 1), (1, -1), (-1, 1), (-1, -1)]
ORTHO = [(1, 0), (-1, 0), (0, 1), (0, -1)]


def _targets(board, t, frm):
    """Occupied squares a non-pawn piece of type t on frm attacks (sliders stop
    at the first occupied square, which they attack)."""
    f0, r0 = frm % 8, frm // 8
    out = []
    if t in (1, 5):
        for df, dr in (KNIGHT if t == 1 else KING):
            f, r = f0 + df, r0 + dr
            if 0 <= f < 8 and 0 <= r < 8 and board[r * 8 + f] != EMPTY:
                out.append(r * 8 + f)
        return out
    dirs = DIAG if t == 2 else ORTHO if t == 3 else DIAG + ORTHO
    for df, dr in dirs:
        f, r = f0 + df, r0 + dr
        while 0 <= f < 8 and 0 <= r < 8:
            if board[r * 8 + f] != EMPTY:
                out.append(r * 8 + f)
                break
            f, r = f + df, r + dr
    return out


def _index_fn():
    lib = fo._load()
    fn = lib.feature_oracle_threat_index
    fn.restype = ctypes.c_int
    fn.argtypes = [ctypes.c_int] * 6
    return fn


def threat_row(board, persp: int, max_active: int = 128, swap_colors: bool = False,
               push_first: bool = False) -> list[int]:
    """The reference's Full_Threats row of `board` for perspective `persp`
    (0 white); swap_colors / push_first plant two ordering mistakes."""
    index = _index_fn()
    board = np.asarray(board)
    ksq = int(np.nonzero(board == 10 + persp)[0][0])
    keyed = []
    for frm in range(64):
        p = int(board[frm])
        if p == EMPTY:
            continue
        t, c = p // 2, p % 2
        crank = (0 if c == persp else 1) ^ (1 if swap_colors else 0)
        if t == 0:
            f = frm % 8
            fwd = 8 if c == 0 else -8
            moves = []
            if (c == 0 and f < 7) or (c == 1 and f > 0):  # "left": white +9, black -9
                moves.append((0, frm + fwd + (1 if c == 0 else -1)))
            if (c == 0 and f > 0) or (c == 1 and f < 7):  # "right": white +7, black -7
                moves.append((1, frm + fwd - (1 if c == 0 else -1)))
            moves.append((2, frm + fwd))  # push, only onto a pawn of either colour
            for kind, to in moves:
                if not 0 <= to < 64 or board[to] == EMPTY:
                    continue
                if kind == 2 and int(board[to]) // 2 != 0:
                    continue
                k = (0 if kind == 2 else kind + 1) if push_first else kind
                keyed.append(((crank, t, k, to, 0), p, frm, to))
        else:
            for to in _targets(board, t, frm):
                keyed.append(((crank, t, 0, frm, to), p, frm, to))
    keyed.sort(key=lambda e: e[0])
    row = []
    for _, p, frm, to in keyed:
        idx = index(persp, p, frm, to, int(board[to]), ksq)
        if idx >= 0:
            row.append(idx)
    return row[:max_active]
