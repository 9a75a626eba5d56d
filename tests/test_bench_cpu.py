"""bench.py's contract on the CPU: the one-GPU rule, the roofline pricing
(frac = counter memory-side bytes per launch over HBM's published peak, the
byte model's logical bytes and the L2 view beside it), the repetition
statistics, and the algorithmic byte counts against a brute-force count over a
tiny index matrix."""

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


def test_roofline_gather_priced_against_hbm_from_counter_bytes(bench):
    # 3.35 GB of requested rows in 0.205 ms, 612 MB of memory-side traffic
    r = bench.roofline("bwd_tiled_gather", 3.35e9, 0.205, traffic=612e6, traffic_source="test", l2_attainable=33281.0)
    assert r["bound"] == "hbm" and r["unit"] == "GB/s" and r["peak"] == 8000.0
    assert r["traffic"] == 612e6
    assert r["achieved"] == pytest.approx(612e6 / 0.205e-3 / 1e9)
    assert r["frac"] == pytest.approx(r["achieved"] / 8000.0) and 0 < r["frac"] <= 1
    lg = r["logical"]  # the byte model's rows, L2-served re-reads included: above HBM's peak here
    assert lg["achieved"] == pytest.approx(3.35e9 / 0.205e-3 / 1e9)
    assert lg["frac_of_hbm_peak"] == pytest.approx(lg["achieved"] / 8000.0) and lg["frac_of_hbm_peak"] > 1
    assert r["l2"]["derived_peak"] == pytest.approx(8 * 16 * 128 * 2.4)  # 39 321.6 GB/s
    assert 0 < r["l2"]["frac_of_derived_peak"] <= 1
    assert r["l2"]["frac_of_measured_ceiling"] == pytest.approx(lg["achieved"] / 33281.0)


def test_roofline_without_counter_traffic_says_so(bench):
    r = bench.roofline("fwd_tile_relayout", 194.8e6, 0.0346)
    assert r["bound"] == "hbm" and r["peak"] == 8000.0 and r["traffic"] is None
    assert r["frac"] == pytest.approx(194.8e6 / 0.0346e-3 / 1e9 / 8000.0)
    assert "algorithmic" in r["basis"]
    assert "l2" not in r  # a streaming kernel: no L2 view


def test_repetition_statistics(bench):
    st = bench.rep_stats([1.9, 1.7, 1.72, 1.71, 2.5])
    assert st["ms_per_step"] == 1.72 and st["ms_per_step_min"] == 1.7 and st["ms_per_step_max"] == 2.5
    assert st["reps"] == 5


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


def test_traffic_patterns_cover_the_traced_kernels():
    """Every library kernel in the committed kernel traces of the five workloads
    has a timing kind in sft_amd/traffic.py, so its counter bytes are attributed."""
    import glob
    import re
    import sys

    sys.path.insert(0, os.path.join(ROOT, "stockfish-trainer_amd"))
    from sft_amd import traffic

    names = set()
    for w in ("halfka_b65536", "threats_b65536", "halfka_small_b65536", "halfka_b16384", "halfka_q16_b65536"):
        for path in glob.glob(os.path.join(ROOT, "profiles", f"kernel_trace_{w}.md")):
            for line in open(path):
                m = re.match(r"\| `([^`]+)` \|", line)
                if m:
                    names.add(m.group(1))
    assert names, "no traced kernels found"
    library = [n for n in names if not n.startswith(("at::", "__amd", "l2_gather_probe"))]
    assert library
    missing = [n for n in library if traffic.kind_of(n) is None]
    assert not missing, missing
