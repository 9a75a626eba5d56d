"""Feature-encoder oracle (src/rust/feature_extraction.rs): the reference's own
tests and constants, a second restatement of HalfKAv2_hm from the reference's
Python feature module, the threat index space, and colour symmetry."""

import ctypes

import numpy as np
import pytest

from oracle import feature_oracle as fo
from sft_amd import positions
from src.model.modules.features.full_threats import FullThreats
from src.model.modules.features.halfka_v2_hm import HalfKav2Hm, halfka_index

THREAT_MAP = [[0, 1, -1, 2, -1, -1], [0, 1, 2, 3, 4, -1], [0, 1, 2, 3, -1, -1], [0, 1, 2, 3, -1, -1],
              [0, 1, 2, 3, 4, -1], [-1] * 6]


def test_threat_table_total_is_the_input_count():
    # the reference asserts the table sums to FULL_THREATS_INPUTS (feature_extraction.rs:828)
    assert fo.threat_total() == 60720 == FullThreats.NUM_INPUTS


def test_startpos_has_32_halfka_features_per_side():
    # feature_extraction.rs:870-880
    b, s = positions.board_from_fen(positions.STARTPOS)
    out = fo.encode(b[None], np.array([s]), ["HalfKAv2_hm"])
    assert out["count_w"][0] == 32 and out["count_b"][0] == 32
    assert (out["white"][0] >= 0).all() and out["psqt"][0] == (32 - 1) // 4 and out["us"][0] == 1.0


def test_halfka_matches_the_python_feature_module():
    boards, stm = positions.random_positions(200, seed=1)
    out = fo.encode(boards, stm, ["HalfKAv2_hm"])
    for b in range(200):
        for persp, key in ((0, "white"), (1, "black")):
            ksq = int(np.nonzero(boards[b] == 10 + persp)[0][0])
            want = [halfka_index(persp == 0, ksq, s, int(boards[b, s]) // 2 + 1, int(boards[b, s]) % 2 == 0)
                    for s in range(64) if boards[b, s] != positions.EMPTY]
            n = out["count_w" if persp == 0 else "count_b"][b]
            assert list(out[key][b, :n]) == want  # same values, same (square) order
            assert (out[key][b, n:] == -1).all()
    assert (out["white"][out["white"] >= 0] < HalfKav2Hm.NUM_INPUTS).all()


def _empty_board_targets(piece_type, color, frm):
    """Squares a piece attacks on an empty board; a pawn: its two captures and its push."""
    f0, r0 = frm % 8, frm // 8
    out = set()
    if piece_type == 0:
        dr = 1 if color == 0 else -1
        for df in (-1, 1):
            if 0 <= f0 + df < 8:
                out.add((r0 + dr) * 8 + f0 + df)
        out.add((r0 + dr) * 8 + f0)
        return out
    steps = {1: [(1, 2), (2, 1), (2, -1), (1, -2), (-1, -2), (-2, -1), (-2, 1), (-1, 2)],
             2: [(1, 1), (1, -1), (-1, 1), (-1, -1)], 3: [(1, 0), (-1, 0), (0, 1), (0, -1)]}
    dirs = steps[1] if piece_type == 1 else steps[2] if piece_type == 2 else steps[3] if piece_type == 3 \
        else steps[2] + steps[3]
    for df, dr in dirs:
        f, r = f0 + df, r0 + dr
        while 0 <= f < 8 and 0 <= r < 8:
            out.add(r * 8 + f)
            if piece_type == 1:
                break
            f, r = f + df, r + dr
    return out


def test_threat_index_space_is_injective():
    """Every (attacker, from, to in its empty-board attack set, attacked piece)
    the map admits gets a distinct index in [0, 60720), and the blocks of one
    attacker and target class are exactly as large as the attack sets (white
    perspective, king on the a-d files so nothing is flipped)."""
    lib = fo._load()
    lib.feature_oracle_threat_index.restype = ctypes.c_int
    seen = set()
    excluded = 0
    table = fo.threat_table()
    for attacker in range(10):  # kings never attack (map row of -1)
        at, ac = attacker // 2, attacker % 2
        size = sum(len(_empty_board_targets(at, ac, f)) for f in range(64) if at != 0 or 8 <= f < 56)
        assert table[attacker, 64] == size
        for frm in range(64):
            if at == 0 and not 8 <= frm < 56:
                continue
            for to in sorted(_empty_board_targets(at, ac, frm)):
                for dt in range(6):
                    if THREAT_MAP[at][dt] < 0:
                        continue
                    for dc in range(2):
                        idx = lib.feature_oracle_threat_index(0, attacker, frm, to, 2 * dt + dc, 0)
                        if idx < 0:
                            # only same-type pairs counted once (from > to) are dropped
                            assert dt == at and (dc != ac or at != 0) and frm < to
                            excluded += 1
                            continue
                        assert 0 <= idx < 60720
                        assert idx not in seen, (attacker, frm, to, dt, dc)
                        seen.add(idx)
    # a bijection of the admitted combinations and the dropped duplicates onto [0, 60720)
    assert len(seen) + excluded == 60720


def _sorted_rows(out, key, count):
    return [sorted(out[key][b, :out[count][b]].tolist()) for b in range(out[key].shape[0])]


@pytest.mark.parametrize("components", [["HalfKAv2_hm"], ["Full_Threats"], ["Full_Threats", "HalfKAv2_hm"]])
def test_colour_mirror_swaps_perspectives(components):
    boards, stm = positions.random_positions(300, seed=2)
    a = fo.encode(boards, stm, components)
    mb, ms = positions.mirror(boards, stm)
    m = fo.encode(mb, ms, components)
    assert _sorted_rows(a, "white", "count_w") == _sorted_rows(m, "black", "count_b")
    assert _sorted_rows(a, "black", "count_b") == _sorted_rows(m, "white", "count_w")
    assert np.array_equal(a["us"], 1 - m["us"]) and np.array_equal(a["psqt"], m["psqt"])


def test_threat_rows_are_unique_and_in_range():
    boards, stm = positions.random_positions(500, seed=3)
    out = fo.encode(boards, stm, ["Full_Threats", "HalfKAv2_hm"])
    assert out["overflow"] == 0
    for key, cnt in (("white", "count_w"), ("black", "count_b")):
        for b in range(500):
            row = out[key][b, :out[cnt][b]]
            assert len(set(row.tolist())) == len(row)
            assert ((row >= 0) & (row < 85296)).all()
            assert (out[key][b, out[cnt][b]:] == -1).all()


def _rows_and_pushes(boards, stm):
    from threat_order import threat_row

    out = fo.encode(boards, stm, ["Full_Threats"])
    rows = []
    for b in range(boards.shape[0]):
        for persp, key, cnt in ((0, "white", "count_w"), (1, "black", "count_b")):
            n = min(int(out[cnt][b]), 128)
            rows.append((b, persp, out[key][b, :n].tolist(), threat_row(boards[b], persp)))
    return rows


def test_threat_row_order_follows_the_reference_loops():
    """The oracle's (and so the GPU encoder's) Full_Threats rows list the
    threats in the order of the reference's loops, restated independently in
    tests/threat_order.py; two planted ordering mistakes must change rows."""
    from threat_order import threat_row

    boards, stm = positions.random_positions(400, seed=5)
    fens = ["4k3/8/3p4/3P4/8/8/8/4K3 w - - 0 1",          # white pawn pushes onto a black pawn
            "4k3/8/8/2pp4/2PP4/8/8/4K3 b - - 0 1",
            "4k3/3p4/3p4/8/8/3P4/3P4/4K3 w - - 0 1",      # pawns blocked by their own pawns
            positions.STARTPOS]
    fb = [positions.board_from_fen(f) for f in fens]
    boards = np.concatenate([boards, np.stack([b for b, _ in fb])])
    stm = np.concatenate([stm, np.array([s for _, s in fb], np.uint8)])
    rows = _rows_and_pushes(boards, stm)
    for b, persp, got, want in rows:
        assert got == want, (b, persp)
    # the restatement is order-sensitive: both planted mistakes disagree somewhere
    swapped = sum(threat_row(boards[b], p, swap_colors=True) != got for b, p, got, _ in rows)
    pushes_first = sum(threat_row(boards[b], p, push_first=True) != got for b, p, got, _ in rows)
    assert swapped > 100 and pushes_first > 0, (swapped, pushes_first)
