"""fp32 forward on the GPU vs the ordered oracle: bit-exact, and within 1e-5
row-normwise of binary64."""

import numpy as np
import pytest
import torch

from gpu_helpers import DEV, announce, case, dev, host, rel_err
from oracle import ft_oracle
from sft_amd import _native, workloads

pytestmark = pytest.mark.gpu

SHAPES = [
    # seed, B, N, K, L, lo, hi, sort
    (1, 1, 10, 4, 8, 0, 4, False),
    (2, 37, 517, 32, 136, 0, 32, False),      # narrow rows: 8-lane groups
    (3, 300, 2000, 32, 1048, 16, 32, True),   # 64-lane groups, 5 chunks per lane
    (4, 129, 300, 160, 1048, 32, 160, False),  # K = 160
    (5, 65, 77, 7, 13, 0, 7, False),          # L % 4 != 0: scalar path
    (6, 200, 300, 32, 1040, 16, 32, True),
    (7, 64, 50, 5, 2100, 0, 5, False),        # L > 2048: several column slabs
    (8, 1000, 23232, 32, 136, 16, 32, True),
    (9, 333, 4000, 48, 520, 0, 48, False),    # 32-lane groups
    (10, 5, 3, 70, 12, 0, 3, False),          # K > 64: two compaction rounds
    (11, 1000, 24576, 32, 256, 0, 32, False),  # largest table the tiled gather takes; 8 tiles
    (12, 77, 900, 13, 1040, 0, 13, False),    # K = 13: four rows per ballot
    (13, 700, 40000, 32, 1048, 16, 32, True),  # 32-column tile of 5.1 MB: two table parts
    (14, 300, 85296, 160, 1048, 32, 160, False),  # threat-sized table (4 parts), unsorted rows: all in pass 0
    (15, 500, 3000, 32, 100, 0, 32, False),   # 4 tiles, the last holding one 16-byte chunk
    (16, 400, 2500, 24, 228, 8, 24, True),    # 8 tiles, the last holding one chunk
    (17, 300, 1200, 32, 96, 0, 32, False),    # 3 tiles: row gather
    (18, 900, 3000, 32, 200, 8, 32, True),    # 7 tiles: leftover strands of two tiles per XCD
    # lists of K > 32 built four threads a position (quarters of whole 16-byte pieces)
    (19, 1000, 300, 36, 136, 0, 36, False),   # K = 36: quarters of 12 slots, the last piece of each padding
    (20, 777, 85296, 100, 520, 0, 100, False),  # table parts, quarters of 28 slots, unsorted rows
    (21, 513, 70000, 192, 264, 100, 192, False),  # the widest such lists: quarters of 48 slots
    (22, 300, 85296, 196, 136, 150, 196, True),  # K = 196: one thread a position again
    (23, 400, 60000, 64, 1048, 0, 64, True),  # table parts, sorted rows, many empty quarters
]


@pytest.mark.parametrize("seed,B,N,K,L,lo,hi,sort", SHAPES)
@pytest.mark.parametrize("rows", [False, True])
def test_fwd_matches_oracle(seed, B, N, K, L, lo, hi, sort, rows):
    announce(f"fwd seed={seed} B={B} N={N} K={K} L={L} rows={rows}")
    idx, W, b, _ = case(seed, B, N, K, L, lo, hi, sort)
    out = torch.empty(B, L, device=DEV)
    _native.ft_fwd_f32(dev(idx), dev(W), dev(b), out, rows=rows)
    y = host(out)
    assert np.array_equal(y, ft_oracle.fwd_f32(idx, W, b))
    assert rel_err(y, ft_oracle.fwd_f64(idx, W, b)) <= 1e-5


def test_fwd_repeated_feature_and_last_row():
    announce("fwd repeated features, index N-1")
    N, L = 40, 64
    idx = np.array([[3, 3, 3, -1], [N - 1, 0, N - 1, 5], [-1, -1, -1, -1]], np.int32)
    g = np.random.default_rng(0)
    W = g.standard_normal((N, L)).astype(np.float32)
    b = g.standard_normal(L).astype(np.float32)
    out = torch.empty(3, L, device=DEV)
    _native.ft_fwd_f32(dev(idx), dev(W), dev(b), out)
    assert np.array_equal(host(out), ft_oracle.fwd_f32(idx, W, b))


def test_fwd_out_of_range_indices_are_inactive():
    announce("fwd out-of-range indices")
    N, L = 30, 16
    idx = np.array([[0, 30, 5, -7], [2**31 - 1, 1, -2**31, 29]], np.int32)
    g = np.random.default_rng(1)
    W = g.standard_normal((N, L)).astype(np.float32)
    b = g.standard_normal(L).astype(np.float32)
    out = torch.empty(2, L, device=DEV)
    _native.ft_fwd_f32(dev(idx), dev(W), dev(b), out)
    clean = np.where((idx >= 0) & (idx < N), idx, -1).astype(np.int32)
    assert np.array_equal(host(out), ft_oracle.fwd_f32(clean, W, b))


def test_fwd_unaligned_views_use_the_scalar_path():
    announce("fwd unaligned weight view")
    g = np.random.default_rng(2)
    N, L, B, K = 50, 12, 20, 6
    big = torch.from_numpy(g.standard_normal(N * L + 1).astype(np.float32)).to(DEV)
    W = big[1:].view(N, L)  # 4-byte offset: not 16-byte aligned
    idx = workloads.make_indices(g, B, N, K, 0, K)
    b = g.standard_normal(L).astype(np.float32)
    out = torch.empty(B, L, device=DEV)
    _native.ft_fwd_f32(dev(idx), W, dev(b), out)
    assert np.array_equal(host(out), ft_oracle.fwd_f32(idx, host(W), b))


def test_tiled_workspace_query():
    from test_abi_cpu import _a256, rank_lists_bytes

    # 32-column tiles of N table rows and one pad row, 128 bytes per row, then the rank lists
    n = _native._workspace_bytes("fwd", 65536, 32, 23232, 1048, _native.SFT_FWD_AUTO, DEV)
    assert n == _a256(33 * 23233 * 32 * 4) + rank_lists_bytes(65536, 32)
    assert _native._workspace_bytes("fwd", 65536, 32, 23232, 136, _native.SFT_FWD_AUTO, DEV) == \
        _a256(5 * 23233 * 32 * 4) + rank_lists_bytes(65536, 32)
    assert _native._workspace_bytes("fwd", 65536, 32, 23232, 96, _native.SFT_FWD_AUTO, DEV) == 0  # 3 tiles
    # a table gathered in parts: then the sums carried between the passes, one 128-byte line per position and tile
    assert _native._workspace_bytes("fwd", 65536, 32, 85296, 1048, _native.SFT_FWD_AUTO, DEV) == \
        _a256(33 * 85297 * 32 * 4) + rank_lists_bytes(65536, 32) + _a256(33 * 65536 * 128)
    assert _native._workspace_bytes("fwd", 65536, 32, 600000, 1048, _native.SFT_FWD_AUTO, DEV) == 0  # tile > 64 MiB
    assert _native._workspace_bytes("fwd", 65536, 32, 23232, 1048, _native.SFT_FWD_ROWS, DEV) == 0


@pytest.mark.parametrize("wid", [0, 1, 2, 3])
def test_fwd_full_workload(wid):
    w = workloads.WORKLOADS[wid]
    announce(f"fwd workload {w.name} B={w.B} N={w.N} K={w.K} L={w.L}")
    d = workloads.make_fp32_inputs(w, with_grads=False)
    Wt, bt = dev(d["W"]), dev(d["bias"])
    for key in ("idx_w", "idx_b"):
        ref = ft_oracle.fwd_f32(d[key], d["W"], d["bias"])
        for rows in (False, True):
            out = torch.empty(w.B, w.L, device=DEV)
            _native.ft_fwd_f32(dev(d[key]), Wt, bt, out, rows=rows)
            assert np.array_equal(host(out), ref), (key, rows)


@pytest.mark.parametrize("pair", [False, True])
def test_fwd_table_parts_mixed_rows(pair):
    """A table of several parts (N = 85296 rows: 10.9 MB per 32-column tile) with
    rows whose parts rise (spread over the passes), rows that go back to an
    earlier part (each slot in the pass of the largest part up to it), rows inside one part, rows that
    repeat a feature across a part boundary, empty rows and rows at the table's
    ends -- bit-exact with the ordered oracle in every case."""
    announce(f"fwd table parts, mixed rows, pair={pair}")
    g = np.random.default_rng(21)
    B, N, K, L = 3000, 85296, 160, 1048
    part = -(-N // 4)
    idx = workloads.make_indices(g, B, N, K, 32, 160, sort=True)
    idx[1::7] = workloads.make_indices(g, len(idx[1::7]), N, K, 32, 160, sort=False)  # unsorted rows
    idx[2::7, :] = -1
    for r in range(3, B, 7):  # one part only
        p = (r // 7) % 4
        n = 1 + r % K
        idx[r, :n] = np.sort(g.choice(np.arange(p * part, min(N, (p + 1) * part)), n, replace=False))
    idx[4::7, 10:] = -1
    idx[4::7, 9] = idx[4::7, 0]  # a repeat of the first (part 0) feature after later parts: non-monotone
    idx[5::7, :3] = [0, part - 1, part]  # part boundary, rising
    idx[5::7, 3:] = -1
    idx[6::7, :4] = [N - 1, -1, N - 1, -1]  # last row twice
    idx[6::7, 4:] = -1
    W = (g.standard_normal((N, L)) * 0.01).astype(np.float32)
    b = g.uniform(-0.1, 0.1, L).astype(np.float32)
    ref = ft_oracle.fwd_f32(idx, W, b)
    if not pair:
        out = torch.empty(B, L, device=DEV)
        _native.ft_fwd_f32(dev(idx), dev(W), dev(b), out)
        assert np.array_equal(host(out), ref)
    else:
        o0, o1 = torch.empty(B, L, device=DEV), torch.empty(B, L, device=DEV)
        idx1 = idx[::-1].copy()
        _native.ft_fwd_pair_f32(dev(idx), dev(idx1), [dev(W)], [None], dev(b), o0, o1)
        assert np.array_equal(host(o0), ref)
        assert np.array_equal(host(o1), ft_oracle.fwd_f32(idx1, W, b))


@pytest.mark.parametrize("pair", [False, True])
def test_fwd_table_parts_encoder_rows(pair):
    """Index rows as the feature encoder emits them for Full_Threats+HalfKAv2_hm
    (threats by colour and piece, then HalfKAv2_hm, offset by 60720): about a
    fifth of the rows go back to an earlier table part, most once near a part
    boundary.  Bit-exact with the ordered oracle."""
    from oracle import feature_oracle
    from sft_amd.positions import random_positions

    announce(f"fwd table parts, encoder rows, pair={pair}")
    boards, stm = random_positions(4000, seed=17)
    enc = feature_oracle.encode(boards, stm, ["Full_Threats", "HalfKAv2_hm"])
    idx0, idx1 = enc["white"], enc["black"]
    B, K = idx0.shape
    N, L = 85296, 1048
    part = -(-N // 3)
    back = sum(not np.all(np.diff(r[r >= 0] // part) >= 0) for r in idx0)
    assert back > B // 20  # the case this test is for
    g = np.random.default_rng(23)
    W = (g.standard_normal((N, L)) * 0.01).astype(np.float32)
    b = g.uniform(-0.1, 0.1, L).astype(np.float32)
    ref0, ref1 = ft_oracle.fwd_f32(idx0, W, b), ft_oracle.fwd_f32(idx1, W, b)
    if not pair:
        out = torch.empty(B, L, device=DEV)
        _native.ft_fwd_f32(dev(idx0), dev(W), dev(b), out)
        assert np.array_equal(host(out), ref0)
    else:
        o0, o1 = torch.empty(B, L, device=DEV), torch.empty(B, L, device=DEV)
        _native.ft_fwd_pair_f32(dev(idx0), dev(idx1), [dev(W)], [None], dev(b), o0, o1)
        assert np.array_equal(host(o0), ref0)
        assert np.array_equal(host(o1), ref1)
