"""fp32 backward on the GPU.  Sorted mode: weight grad bit-exact with the
reference-order oracle; bias grad within 1e-5 of binary64.  Atomic mode: both
within 1e-4 row-normwise of binary64 (atomic-order rounding only)."""

import numpy as np
import pytest
import torch

from gpu_helpers import DEV, announce, case, dev, dw_rel_err, host, rel_err
from oracle import ft_oracle
from sft_amd import _native, workloads

pytestmark = pytest.mark.gpu

SHAPES = [
    (1, 1, 10, 4, 8, 0, 4, False),
    (2, 37, 517, 32, 136, 0, 32, False),
    (3, 300, 2000, 32, 1048, 16, 32, True),
    (4, 129, 300, 160, 1048, 32, 160, False),
    (5, 65, 77, 7, 13, 0, 7, False),
    (7, 64, 50, 5, 2100, 0, 5, False),
    (8, 3000, 23232, 32, 136, 16, 32, True),
    (9, 333, 4000, 48, 520, 0, 48, False),
    (10, 40000, 700, 32, 256, 0, 32, True),  # two position chunks (B x 128 B > 4 MB), long segments
    (11, 34000, 5, 3, 1040, 0, 3, False),    # five features: every segment crosses the chunk boundary
    (12, 40000, 3000, 16, 200, 0, 16, True),  # 7 tiles (leftover strands of two tiles per XCD), two chunks
    (13, 5000, 1000, 8, 100, 0, 8, False),    # 4 tiles, the last holding one 16-byte chunk
]


def run_bwd(idx, G, N, flags, dW0=None, db0=None):
    L = G.shape[1]
    dW = torch.zeros(N, L, device=DEV) if dW0 is None else dev(dW0)
    db = torch.zeros(L, device=DEV) if db0 is None else dev(db0)
    if flags & _native.SFT_BWD_OVERWRITE:
        dW.fill_(float("nan"))
        db.fill_(float("nan"))
    _native.ft_bwd_f32(dev(idx), dW, db, dev(G), flags)
    return host(dW), host(db)


@pytest.mark.parametrize("seed,B,N,K,L,lo,hi,sort", SHAPES)
@pytest.mark.parametrize("overwrite", [False, True])
@pytest.mark.parametrize("rows", [False, True])
def test_sorted_bwd_matches_reference_order(seed, B, N, K, L, lo, hi, sort, overwrite, rows):
    announce(f"bwd sorted seed={seed} B={B} N={N} K={K} L={L} overwrite={overwrite} rows={rows}")
    idx, _, _, G = case(seed, B, N, K, L, lo, hi, sort)
    g = np.random.default_rng(seed + 100)
    dW0 = None if overwrite else g.standard_normal((N, L)).astype(np.float32)
    db0 = None if overwrite else g.standard_normal(L).astype(np.float32)
    flags = _native.SFT_BWD_OVERWRITE if overwrite else _native.SFT_BWD_ACCUMULATE
    if rows:
        flags |= _native.SFT_BWD_ROWS
    dW, db = run_bwd(idx, G, N, flags, dW0, db0)
    rW, _ = ft_oracle.bwd_f32(idx, G, N, dW0, db0)
    assert np.array_equal(dW, rW)
    db_ref = (0 if db0 is None else db0.astype(np.float64)) + G.astype(np.float64).sum(0)
    assert rel_err(db, db_ref) <= 1e-5


def skewed_indices(g, B, N, K, hot, p_hot):
    """Rows whose first slots hold 'hot' features with probability p_hot each
    (segment lengths from a few to thousands of slots, as for the most common
    features of real positions), the rest uniform, -1 padded, rows unsorted."""
    idx = np.full((B, K), -1, np.int32)
    hot_ids = g.choice(N, hot, replace=False)
    for b in range(B):
        row = [int(f) for f in hot_ids if g.random() < p_hot]
        rest = g.choice(N, K, replace=False)
        row += [int(f) for f in rest if f not in row][: int(g.integers(0, K - len(row) + 1))]
        g.shuffle(row)
        idx[b, : len(row)] = row
    return idx


@pytest.mark.parametrize("seed,B,N,K,L,hot,p_hot", [
    (21, 40000, 3000, 32, 1048, 12, 0.35),  # tiled: long segments in both position chunks
    (24, 9000, 3000, 32, 1048, 12, 0.35),   # tiled, one position chunk (B x 128 B <= 4 MB)
    (22, 5000, 400, 24, 136, 40, 0.2),      # narrow rows: 5 tiles, or the row gather (rows)
    (25, 40000, 3000, 16, 136, 12, 0.35),   # 5 tiles over 8 XCDs, long segments in both position chunks
    (23, 1200, 50, 16, 520, 6, 0.9),        # segments just above and below the long threshold
])
@pytest.mark.parametrize("overwrite", [False, True])
@pytest.mark.parametrize("rows", [False, True])
def test_sorted_bwd_skewed_segments(seed, B, N, K, L, hot, p_hot, overwrite, rows):
    announce(f"bwd skewed seed={seed} B={B} N={N} K={K} L={L} overwrite={overwrite} rows={rows}")
    g = np.random.default_rng(seed)
    idx = skewed_indices(g, B, N, K, hot, p_hot)
    G = g.standard_normal((B, L)).astype(np.float32)
    dW0 = None if overwrite else g.standard_normal((N, L)).astype(np.float32)
    flags = (_native.SFT_BWD_OVERWRITE if overwrite else _native.SFT_BWD_ACCUMULATE) | (
        _native.SFT_BWD_ROWS if rows else 0)
    dW, _ = run_bwd(idx, G, N, flags, dW0, None if overwrite else np.zeros(L, np.float32))
    rW, _ = ft_oracle.bwd_f32(idx, G, N, dW0)
    assert np.array_equal(dW, rW)


@pytest.mark.parametrize("N", [2500, 1500])
def test_sorted_bwd_every_segment_long(N):
    """Every feature long (~450 and ~750 slots per position chunk): thousands
    of long segments per chunk, many per long-segment slot."""
    announce(f"bwd every segment long N={N}")
    g = np.random.default_rng(41)
    B, K, L = 40000, 64, 256
    idx = workloads.make_indices(g, B, N, K, 48, 64, sort=False)
    G = g.standard_normal((B, L)).astype(np.float32)
    dW, _ = run_bwd(idx, G, N, _native.SFT_BWD_OVERWRITE)
    rW, _ = ft_oracle.bwd_f32(idx, G, N)
    assert np.array_equal(dW, rW)


@pytest.mark.parametrize("L,rows", [(1048, False), (136, True)])
def test_sorted_bwd_long_segments_with_repeated_slots(L, rows):
    """A feature repeated within rows: its long segment holds each such
    position several times, added once per slot (FT/kernel.py:122, 178-181)."""
    announce(f"bwd long segments with repeated slots L={L} rows={rows}")
    g = np.random.default_rng(77)
    B, N, K = 3000, 900, 12
    idx = workloads.make_indices(g, B, N, K, 4, 8, sort=False)
    rep = g.random(B) < 0.6
    idx[rep, 8] = 7
    idx[rep & (g.random(B) < 0.5), 9] = 7  # some rows hold feature 7 three times
    idx[g.random(B) < 0.3, 10] = 11
    G = g.standard_normal((B, L)).astype(np.float32)
    flags = _native.SFT_BWD_OVERWRITE | (_native.SFT_BWD_ROWS if rows else 0)
    dW, _ = run_bwd(idx, G, N, flags)
    rW, _ = ft_oracle.bwd_f32(idx, G, N)
    assert np.array_equal(dW, rW)


@pytest.mark.parametrize("seed,B,N,K,L,lo,hi,sort", SHAPES)
@pytest.mark.parametrize("overwrite", [False, True])
def test_atomic_bwd_within_tolerance(seed, B, N, K, L, lo, hi, sort, overwrite):
    announce(f"bwd atomic seed={seed} B={B} N={N} K={K} L={L} overwrite={overwrite}")
    idx, _, _, G = case(seed, B, N, K, L, lo, hi, sort)
    flags = _native.SFT_BWD_ATOMIC | (_native.SFT_BWD_OVERWRITE if overwrite else 0)
    dW, db = run_bwd(idx, G, N, flags)
    r64, rb64 = ft_oracle.bwd_f64(idx, G, N)
    assert dw_rel_err(dW, r64) <= 1e-4
    assert rel_err(db, rb64) <= 1e-4


def test_bwd_duplicates_and_out_of_range():
    announce("bwd repeated features and out-of-range indices")
    N, L = 12, 20
    idx = np.array([[3, 3, 40, -1], [11, -5, 3, 0], [-1, -1, -1, -1]], np.int32)
    g = np.random.default_rng(5)
    G = g.standard_normal((3, L)).astype(np.float32)
    clean = np.where((idx >= 0) & (idx < N), idx, -1).astype(np.int32)
    for flags in (0, _native.SFT_BWD_OVERWRITE, _native.SFT_BWD_ATOMIC):
        dW, _ = run_bwd(idx, G, N, flags)
        rW, _ = ft_oracle.bwd_f32(clean, G, N)
        if flags & _native.SFT_BWD_ATOMIC:
            assert dw_rel_err(dW, ft_oracle.bwd_f64(clean, G, N)[0]) <= 1e-6
        else:
            assert np.array_equal(dW, rW)


def test_bwd_all_inactive_and_empty_batch():
    announce("bwd all inactive / empty batch")
    N, L = 9, 8
    idx = np.full((4, 3), -1, np.int32)
    G = np.ones((4, L), np.float32)
    dW0 = np.full((N, L), 7.0, np.float32)
    dW, db = run_bwd(idx, G, N, 0, dW0, np.zeros(L, np.float32))
    assert np.array_equal(dW, dW0) and np.array_equal(db, np.full(L, 4.0, np.float32))
    dW, db = run_bwd(idx, G, N, _native.SFT_BWD_OVERWRITE)
    assert not dW.any() and np.array_equal(db, np.full(L, 4.0, np.float32))
    e = np.zeros((0, 3), np.int32)
    dW, db = run_bwd(e, np.zeros((0, L), np.float32), N, _native.SFT_BWD_OVERWRITE)
    assert not dW.any() and not db.any()


@pytest.mark.parametrize("wid", [0, 1, 2, 3])
def test_bwd_full_workload(wid):
    w = workloads.WORKLOADS[wid]
    announce(f"bwd workload {w.name} B={w.B} N={w.N} K={w.K} L={w.L}")
    d = workloads.make_fp32_inputs(w)
    idx, G = d["idx_w"], d["g_w"]
    rW, _ = ft_oracle.bwd_f32(idx, G, w.N)
    for flags in (_native.SFT_BWD_OVERWRITE | _native.SFT_BWD_ROWS, _native.SFT_BWD_OVERWRITE):
        dW = torch.empty(w.N, w.L, device=DEV)
        db = torch.empty(w.L, device=DEV)
        _native.ft_bwd_f32(dev(idx), dW, db, dev(G), flags)
        assert np.array_equal(host(dW), rW), flags
    assert rel_err(host(db), G.astype(np.float64).sum(0)) <= 1e-5
    # adjoint identity at full size: <fwd(W) - b, G> == <W, dW>
    Wt = dev(d["W"])
    out = torch.empty(w.B, w.L, device=DEV)
    _native.ft_fwd_f32(dev(idx), Wt, torch.zeros(w.L, device=DEV), out)
    prod = out.double() * dev(G).double()
    lhs = float(prod.sum())
    rhs = float((Wt.double() * dW.double()).sum())
    assert abs(lhs - rhs) <= 1e-6 * float(prod.abs().sum())


@pytest.mark.parametrize("wid", [1, 3])
def test_atomic_bwd_full_workload(wid):
    w = workloads.WORKLOADS[wid]
    announce(f"bwd atomic workload {w.name}")
    d = workloads.make_fp32_inputs(w)
    idx, G = d["idx_b"], d["g_b"]
    dW = torch.empty(w.N, w.L, device=DEV)
    db = torch.empty(w.L, device=DEV)
    _native.ft_bwd_f32(dev(idx), dW, db, dev(G), _native.SFT_BWD_OVERWRITE | _native.SFT_BWD_ATOMIC)
    r64, _ = ft_oracle.bwd_f64(idx, G, w.N)
    assert dw_rel_err(host(dW), r64) <= 1e-4


def _unaligned(t: torch.Tensor, offset: int) -> torch.Tensor:
    """A copy of t as a view offset by `offset` floats (offset 1: 4-byte aligned only)."""
    if not offset:
        return t
    big = torch.zeros(t.numel() + offset, device=DEV)
    big[offset:] = t.reshape(-1)
    return big[offset:].view(t.shape)


def _prepare(idx, N, L, W=None):
    """The forward with the backward's sort beside it -> (out, idx on the device, prep)."""
    B = idx.shape[0]
    W = np.zeros((N, L), np.float32) if W is None else W
    out = torch.empty(B, L, device=DEV)
    i = dev(idx)
    prep = _native.ft_fwd_f32_prep(i, dev(W), torch.zeros(L, device=DEV), out, _native.SFT_BWD_OVERWRITE)
    return host(out), i, prep


def _prepared_bwd(i, G, N, prep, grad_offset=0, dw_offset=0):
    """The prepared backward; the offsets pass the grad or the weight grad as
    views that are only 4-byte aligned."""
    B, L = G.shape
    g = _unaligned(dev(G), grad_offset)
    dW = _unaligned(torch.full((N, L), float("nan"), device=DEV), dw_offset)
    db = torch.full((L,), float("nan"), device=DEV)
    _native.ft_bwd_f32_prepared(i, dW, db, g, prep, _native.SFT_BWD_OVERWRITE)
    return host(dW), host(db)


def _prepared(idx, G, N, W=None, grad_offset=0):
    out, i, prep = _prepare(idx, N, G.shape[1], W)
    dW, db = _prepared_bwd(i, G, N, prep, grad_offset)
    return out, dW, db


@pytest.mark.parametrize("seed,B,N,K,L,lo,hi,sort", SHAPES)
def test_prepared_bwd_matches_the_backward(seed, B, N, K, L, lo, hi, sort):
    """Sorting under the forward changes nothing: the forward and the prepared
    backward's weight grad are bit-identical to the ordinary calls (tiled and
    row gathers, one and two position chunks, long segments).  The bias grad's
    row blocks differ between the two (the ordinary call's bias pass runs
    beside the whole sort and takes fewer), so both are held to the bias-grad
    bound, 1e-5 of binary64."""
    announce(f"prepared bwd seed={seed} B={B} N={N} K={K} L={L}")
    idx, W, b, G = case(seed, B, N, K, L, lo, hi, sort)
    out, dW, db = _prepared(idx, G, N, W)
    assert np.array_equal(out, ft_oracle.fwd_f32(idx, W, np.zeros(L, np.float32)))
    dW0, db0 = run_bwd(idx, G, N, _native.SFT_BWD_OVERWRITE)
    assert np.array_equal(dW, dW0)
    db64 = G.astype(np.float64).sum(0)
    assert rel_err(db, db64) <= 1e-5 and rel_err(db0, db64) <= 1e-5


@pytest.mark.parametrize("B,L", [(40000, 256), (3000, 256), (40000, 136), (3000, 136)])
def test_prepared_bwd_reads_the_buffer_only(B, L):
    """Two backwards over one prepared buffer (autograd's retain_graph), the
    first with a grad that is only 4-byte aligned (the bias pass reads floats and
    still writes the grad tiles), the second aligned: both match the reference
    order, so the first left the buffer as the forward made it (K = 32 >= L / 20;
    two position chunks at B = 40000, one at 3000).  At L = 136 (K >= L / 5) the
    buffer holds only the sort's radix pass and each backward sorts the buckets
    into its own workspace."""
    announce(f"prepared bwd twice, unaligned then aligned grad B={B} L={L}")
    idx, W, b, G = case(31, B, 900, 32, L, 0, 32, True)
    assert _native.prep_buffer_bytes(B, 32, 900, L, _native.SFT_BWD_OVERWRITE, DEV) > 0
    _, i, prep = _prepare(idx, 900, L)
    ref, _ = ft_oracle.bwd_f32(idx, G, 900)
    db64 = G.astype(np.float64).sum(0)
    for offset in (1, 0):
        dW, db = _prepared_bwd(i, G, 900, prep, grad_offset=offset)
        assert np.array_equal(dW, ref), offset
        assert rel_err(db, db64) <= 1e-5


@pytest.mark.parametrize("N", [1023, 1024, 1025, 1152])
def test_prepared_bwd_chunk0_buckets_edge(N):
    """The split prepared sort's buckets run in two launches, those holding
    every key of position chunk 0 and the first key of chunk 1 (key N, whose
    segment start ends chunk 0's last segment) first.  Feature counts at and
    around a multiple of the 128-key bucket (N = 1024, 1152: key N opens a
    bucket of its own) keep the weight grad bit-exact (B = 40000: two position
    chunks; L = 136: K >= L / 5)."""
    announce(f"prepared bwd, chunk-0 buckets N={N}")
    B, K, L = 40000, 32, 136
    idx, W, b, G = case(40 + N % 7, B, N, K, L, 0, 32, True)
    _, i, prep = _prepare(idx, N, L)
    dW, db = _prepared_bwd(i, G, N, prep)
    assert np.array_equal(dW, ft_oracle.bwd_f32(idx, G, N)[0])
    assert rel_err(db, G.astype(np.float64).sum(0)) <= 1e-5


def test_prepared_bwd_unaligned_weight_grad():
    """A weight grad that is only 4-byte aligned needs the row gather, which
    sorts in one position chunk: refused (before any launch) when the prepared
    sort is in two chunks, and bit-exact when it is in one."""
    announce("prepared bwd, unaligned weight grad")
    for B, chunks in ((40000, 2), (3000, 1)):
        idx, W, b, G = case(32, B, 900, 32, 256, 0, 32, True)
        _, i, prep = _prepare(idx, 900, 256)
        if chunks == 2:
            with pytest.raises(RuntimeError, match="16-byte aligned"):
                _prepared_bwd(i, G, 900, prep, dw_offset=1)
        else:
            dW, _ = _prepared_bwd(i, G, 900, prep, dw_offset=1)
            assert np.array_equal(dW, ft_oracle.bwd_f32(idx, G, 900)[0])
        dW, _ = _prepared_bwd(i, G, 900, prep)  # the buffer is still good
        assert np.array_equal(dW, ft_oracle.bwd_f32(idx, G, 900)[0])


@pytest.mark.parametrize("offset", [1, 2])
def test_bwd_unaligned_grad_keeps_the_tiled_gather(offset):
    """The plain backward with a grad view that is 4- or 8-byte aligned: the bias
    pass reads floats and writes the same grad tiles (two position chunks)."""
    announce(f"bwd unaligned grad offset={offset}")
    idx, W, b, G = case(33, 40000, 700, 32, 1048, 16, 32, True)
    dW = torch.full((700, 1048), float("nan"), device=DEV)
    db = torch.full((1048,), float("nan"), device=DEV)
    _native.ft_bwd_f32(dev(idx), dW, db, _unaligned(dev(G), offset), _native.SFT_BWD_OVERWRITE)
    assert np.array_equal(host(dW), ft_oracle.bwd_f32(idx, G, 700)[0])
    assert rel_err(host(db), G.astype(np.float64).sum(0)) <= 1e-5


def test_prepared_bwd_no_active_slots():
    announce("prepared bwd, every slot inactive")
    idx = np.full((50, 8), -1, np.int32)
    G = np.random.default_rng(4).standard_normal((50, 64)).astype(np.float32)
    _, dW, db = _prepared(idx, G, 30)
    assert not dW.any()
    assert rel_err(db, G.astype(np.float64).sum(0)) <= 1e-5
