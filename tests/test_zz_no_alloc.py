"""sft_ft_fwd_i16_noalloc (static per-GPU scratch, no workspace) against
sft_ft_fwd_i16_ex (caller's workspace), both through the C ABI: bit-identical
outputs on consecutive calls, the later ones smaller, so a packed table left in
the scratch by an earlier call must never leak into a later result."""

import numpy as np
import pytest
import torch

from gpu_helpers import DEV, announce, dev, host
from oracle import ft_oracle
from sft_amd import _native, workloads

pytestmark = pytest.mark.gpu


def _inputs(seed, B, N, K, L, P):
    g = np.random.default_rng(seed)
    idx = workloads.make_indices(g, B, N, K, 0, K, sort=False)
    Wq = g.integers(-32768, 32768, size=(N, L)).astype(np.int16)
    bq = g.integers(-3000, 3000, size=L).astype(np.int16)
    ps = g.integers(-10**6, 10**6, size=(N, P)).astype(np.int32) if P else None
    return idx, Wq, bq, ps


def _run(fn, idx, Wq, bq, ps, lo, hi, wrap16, rows=False):
    B, L = idx.shape[0], Wq.shape[1]
    out = torch.full((B, L), 0x5555, dtype=torch.int16, device=DEV)
    pout = torch.full((B, ps.shape[1]), 0x55555555, dtype=torch.int32, device=DEV) if ps is not None else None
    fn(dev(idx), dev(Wq), dev(bq), out, None if ps is None else dev(ps), pout, lo, hi, wrap16, rows)
    torch.cuda.synchronize()
    return host(out), None if pout is None else host(pout)


# (seed, B, N, K, L, P): consecutive calls, each smaller than the one before;
# the first packs 17 tiles x 22528 rows (47 MiB of the 64 MiB scratch).
CALLS = [
    (1, 8192, 22528, 32, 1040, 8),
    (2, 3000, 5000, 32, 1024, 5),
    (3, 700, 900, 20, 512, 0),
]


@pytest.mark.parametrize("wrap16", [False, True])
def test_noalloc_matches_workspace_entry_on_consecutive_calls(wrap16):
    for seed, B, N, K, L, P in CALLS:
        announce(f"noalloc i16 seed={seed} B={B} N={N} K={K} L={L} P={P} wrap16={wrap16}")
        idx, Wq, bq, ps = _inputs(seed, B, N, K, L, P)
        for lo, hi in ((0, 127), (-32768, 32767)):
            a, pa = _run(_native.ft_fwd_i16_noalloc, idx, Wq, bq, ps, lo, hi, wrap16)
            b, pb = _run(_native.ft_fwd_i16, idx, Wq, bq, ps, lo, hi, wrap16)
            assert np.array_equal(a, b)
            ro, rp = ft_oracle.fwd_i16(idx, Wq, bq, ps, lo, hi, wrap16)
            assert np.array_equal(a, ro)
            if P:
                assert np.array_equal(pa, pb) and np.array_equal(pa, rp)


def test_noalloc_same_shape_new_table():
    """Same shape twice with another table and a smaller batch: the second
    call repacks, so its result follows the new weights."""
    for seed, B in ((11, 4096), (12, 1500)):
        announce(f"noalloc i16 new table seed={seed} B={B}")
        idx, Wq, bq, ps = _inputs(seed, B, 3000, 32, 1040, 8)
        a, pa = _run(_native.ft_fwd_i16_noalloc, idx, Wq, bq, ps, 0, 127, False)
        b, pb = _run(_native.ft_fwd_i16, idx, Wq, bq, ps, 0, 127, False)
        assert np.array_equal(a, b) and np.array_equal(pa, pb)


def test_noalloc_row_gather_shapes():
    """Shapes outside the tiled path (and SFT_Q16_ROWS) run the row gather,
    which uses no scratch."""
    for seed, B, N, K, L, P, rows in ((21, 300, 400, 7, 13, 3, False), (22, 500, 2000, 32, 1040, 8, True)):
        announce(f"noalloc i16 rows seed={seed} B={B} N={N} K={K} L={L} P={P} rows={rows}")
        idx, Wq, bq, ps = _inputs(seed, B, N, K, L, P)
        a, pa = _run(_native.ft_fwd_i16_noalloc, idx, Wq, bq, ps, -100, 255, False, rows)
        b, pb = _run(_native.ft_fwd_i16, idx, Wq, bq, ps, -100, 255, False, rows)
        assert np.array_equal(a, b) and np.array_equal(pa, pb)
