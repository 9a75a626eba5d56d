"""bench.py's contract on the CPU: the one-GPU rule, the roofline pricing
(every fraction a true fraction of the bound it names) and the algorithmic
byte counts the rooflines divide, against a brute-force count over a tiny
index matrix."""

import importlib.util
import os
import subprocess
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


@pytest.fixture(scope="module")
def bench():
    spec = importlib.util.spec_from_file_location("sft_bench", os.path.join(ROOT, "bench.py"))
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def test_more_than_one_gpu_is_refused():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"], capture_output=True,
                       text=True, timeout=120, cwd=ROOT)
    assert r.returncode == 2
    assert "one GPU" in r.stderr and r.stdout == ""


def test_roofline_gather_priced_against_l2(bench):
    # 3.35 GB of requested rows in 0.205 ms, 612 MB of memory-side traffic
    r = bench.roofline("bwd_tiled_gather", 3.35e9, 0.205, traffic=612e6, traffic_source="test", l2_attainable=33281.0)
    assert r["bound"] == "l2" and r["unit"] == "GB/s"
    assert r["achieved"] == pytest.approx(3.35e9 / 0.205e-3 / 1e9)
    assert r["peak"] == pytest.approx(8 * 16 * 128 * 2.4)  # 39 321.6 GB/s
    assert 0 < r["frac"] <= 1 and r["frac"] == pytest.approx(r["achieved"] / r["peak"])
    assert r["frac_of_attainable"] == pytest.approx(r["achieved"] / 33281.0)
    assert r["hbm"]["peak"] == 8000.0
    assert r["hbm"]["frac"] == pytest.approx(612e6 / 0.205e-3 / 1e9 / 8000.0)
    assert 0 < r["hbm"]["frac"] <= 1


def test_roofline_streaming_kernel_priced_against_hbm(bench):
    r = bench.roofline("fwd_tile_relayout", 194.8e6, 0.0346)
    assert r["bound"] == "hbm" and r["peak"] == 8000.0
    assert r["frac"] == pytest.approx(194.8e6 / 0.0346e-3 / 1e9 / 8000.0)
    assert "hbm" not in r and "attainable" not in r


class _W:
    def __init__(self, B, N, L):
        self.B, self.N, self.L = B, N, L


def _brute_counts(idx, N):
    counts = []
    for row in idx.tolist():
        counts.append(sum(1 for v in row if 0 <= v < N))
    return counts


def test_step_bytes_against_a_brute_force_count(bench):
    """Forward: per position K index words, its active rows and one output row;
    backward gather: per active slot a grad row and a position word, the
    segment offsets and every weight-grad row written once."""
    g = np.random.default_rng(3)
    B, K, N, L = 7, 5, 11, 12
    pair = []
    for _ in range(2):
        idx = g.integers(-1, N + 3, (B, K)).astype(np.int32)  # -1 padding and out-of-range slots too
        idx[0, :] = -1  # a position with no active slot
        pair.append(idx)
    w = _W(B, N, L)
    fwd = 0
    bwd = 0
    for idx in pair:
        c = _brute_counts(idx, N)
        for n in c:
            fwd += 4 * K + 4 * L * n + 4 * L
        nnz = sum(c)
        bwd += 4 * L * nnz + 4 * nnz + 4 * (N + 1) + 4 * N * L
    assert bench.kernel_step_bytes("fwd_f32_tiled_gather", w, pair) == fwd
    assert bench.kernel_step_bytes("bwd_tiled_gather", w, pair) == bwd
    assert bench.kernel_step_bytes("fwd_tile_relayout", w, pair) == 2 * 2 * 4 * N * L  # two calls, read + write
    assert bench.kernel_step_bytes("bwd_bias_partial", w, pair) == 2 * 4 * B * L  # the grad read per perspective
    assert bench.kernel_step_bytes("bwd_feature_sort", w, pair) is None  # no byte model: never priced
