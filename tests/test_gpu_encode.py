"""Feature-index encoder (sft_encode_features) on the GPU against the oracle:
index rows, counts, side to move and buckets identical, for HalfKAv2_hm,
Full_Threats and their composition, on FEN positions and random armies."""

import numpy as np
import pytest
import torch

from gpu_helpers import DEV, announce, host
from oracle import feature_oracle as fo
from sft_amd import positions
from sft_amd.encode import encode_batch

pytestmark = pytest.mark.gpu

FENS = [
    positions.STARTPOS,
    "r1bqkb1r/pppp1ppp/2n2n2/4p3/2B1P3/5N2/PPPP1PPP/RNBQK2R w KQkq - 4 4",
    "8/2p5/3p4/KP5r/1R3p1k/8/4P1P1/8 w - - 0 1",
    "r3k2r/p1ppqpb1/bn2pnp1/3PN3/1p2P3/2N2Q1p/PPPBBPPP/R3K2R b KQkq - 0 1",
    "4k3/8/8/8/8/8/8/4K3 w - - 0 1",
    "rnbq1k1r/pp1Pbppp/2p5/8/2B5/8/PPP1NnPP/RNBQK2R w KQ - 1 8",
]
SETS = {"HalfKAv2_hm": ["HalfKAv2_hm"], "Full_Threats": ["Full_Threats"],
        "Full_Threats+HalfKAv2_hm": ["Full_Threats", "HalfKAv2_hm"]}


def _check(boards, stm, name):
    ref = fo.encode(boards, stm, SETS[name])
    got = encode_batch(torch.from_numpy(boards).to(DEV), torch.from_numpy(stm).to(DEV), name, with_counts=True)
    torch.cuda.synchronize()
    assert np.array_equal(host(got["white"]), ref["white"])
    assert np.array_equal(host(got["black"]), ref["black"])
    assert np.array_equal(host(got["white_count"]), ref["count_w"])
    assert np.array_equal(host(got["black_count"]), ref["count_b"])
    assert np.array_equal(host(got["us"]).reshape(-1), ref["us"])
    assert np.array_equal(host(got["psqt_indices"]), ref["psqt"])
    assert np.array_equal(host(got["layer_stack_indices"]), ref["psqt"])


@pytest.mark.parametrize("name", list(SETS))
def test_encode_fens(name):
    announce(f"encode FENs {name}")
    bs = [positions.board_from_fen(f) for f in FENS]
    _check(np.stack([b for b, _ in bs]), np.array([s for _, s in bs], np.uint8), name)


@pytest.mark.parametrize("name,B,seed", [("HalfKAv2_hm", 3001, 1), ("Full_Threats", 2999, 2),
                                         ("Full_Threats+HalfKAv2_hm", 4096, 3), ("Full_Threats+HalfKAv2_hm", 1, 4)])
def test_encode_random(name, B, seed):
    announce(f"encode random {name} B={B}")
    boards, stm = positions.random_positions(B, seed=seed)
    _check(boards, stm, name)


def test_encode_threat_order_matches_the_reference_loops():
    """The GPU encoder's Full_Threats rows against the loop-order restatement
    (tests/threat_order.py), independently of the oracle's own walk."""
    from threat_order import threat_row

    announce("encode threat order")
    boards, stm = positions.random_positions(300, seed=6)
    got = encode_batch(torch.from_numpy(boards).to(DEV), torch.from_numpy(stm).to(DEV), "Full_Threats",
                       with_counts=True)
    torch.cuda.synchronize()
    for key, cnt, persp in (("white", "white_count", 0), ("black", "black_count", 1)):
        rows, counts = host(got[key]), host(got[cnt])
        for b in range(boards.shape[0]):
            n = min(int(counts[b]), 128)
            assert rows[b, :n].tolist() == threat_row(boards[b], persp), (key, b)
