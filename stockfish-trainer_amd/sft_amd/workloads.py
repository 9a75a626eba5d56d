"""Synthetic FT workloads and their algorithmic byte counts.

Five workloads (sizes from the reference's feature sets,
src/model/modules/features/halfka_v2_hm.py:41-54, full_threats.py:8-15,
composed.py:24-26, and output width L1 + 8 PSQT columns, src/model/model.py:28):

  0 halfka_b16384       HalfKAv2_hm^ N=23232 K=32 active U[16,32] L=1048, B=16384
  1 halfka_b65536       same at B=65536 (the throughput workload)
  2 threats_b65536      Full_Threats+HalfKAv2_hm^ N=85296 K=160 active U[32,160] L=1048
  3 halfka_small_b65536 HalfKAv2_hm^ N=23232 K=32 active U[16,32] L=136
  4 halfka_q16_b65536   int16 forward, N=22528 (export rows) K=32 active U[16,32] L=1040

Index rows hold `count ~ U{lo..hi}` unique features drawn uniformly from
[0, N), sorted ascending, then -1 padding to K.  Weights are N(0, 0.01),
the bias U(-1/sqrt(N), 1/sqrt(N)) (composed.py:42-47), upstream grads N(0, 1).
Every array comes from numpy.random.default_rng([workload_id, stream]) with
stream 0 = white idx, 1 = black idx, 2 = W, 3 = bias, 4 = grad white,
5 = grad black, so any size can be regenerated bit-for-bit anywhere.
"""

from __future__ import annotations

import hashlib
from dataclasses import dataclass

import numpy as np

S_WHITE, S_BLACK, S_W, S_BIAS, S_GW, S_GB = range(6)


@dataclass(frozen=True)
class Workload:
    wid: int
    name: str
    feature_set: str
    B: int
    N: int
    K: int
    lo: int
    hi: int
    L: int
    quantized: bool = False
    psqt: int = 8

    def scaled(self, B: int) -> "Workload":
        return Workload(self.wid, self.name, self.feature_set, B, self.N, self.K, self.lo, self.hi, self.L,
                        self.quantized, self.psqt)


WORKLOADS = {
    0: Workload(0, "halfka_b16384", "HalfKAv2_hm^", 16384, 23232, 32, 16, 32, 1048),
    1: Workload(1, "halfka_b65536", "HalfKAv2_hm^", 65536, 23232, 32, 16, 32, 1048),
    2: Workload(2, "threats_b65536", "Full_Threats+HalfKAv2_hm^", 65536, 85296, 160, 32, 160, 1048),
    3: Workload(3, "halfka_small_b65536", "HalfKAv2_hm^", 65536, 23232, 32, 16, 32, 136),
    4: Workload(4, "halfka_q16_b65536", "HalfKAv2_hm", 65536, 22528, 32, 16, 32, 1040, quantized=True),
}


def rng(wid: int, stream: int) -> np.random.Generator:
    return np.random.default_rng([wid, stream])


def make_indices(g: np.random.Generator, B: int, N: int, K: int, lo: int, hi: int,
                 sort: bool = True) -> np.ndarray:
    """int32 [B, K]: per row `count ~ U{lo..hi}` distinct values of [0, N), -1 padded.

    Rows are drawn as `hi` i.i.d. uniform values and redrawn whole while they
    hold a repeat, so each row is a uniform random `hi`-subset in random
    order; its first `count` entries are then a uniform random `count`-subset.
    """
    if not (0 <= lo <= hi <= K and hi <= N):
        raise ValueError("need 0 <= lo <= hi <= K and hi <= N")
    if hi * hi <= 2 * N:
        # sparse rows: a whole-row redraw is rarely needed (P(repeat) <~ hi^2 / 2N)
        vals = g.integers(0, N, size=(B, hi), dtype=np.int64)
        while hi > 1:
            s = np.sort(vals, axis=1)
            bad = np.nonzero((s[:, 1:] == s[:, :-1]).any(axis=1))[0]
            if bad.size == 0:
                break
            vals[bad] = g.integers(0, N, size=(bad.size, hi), dtype=np.int64)
    else:
        # dense rows: exact draws without replacement, row by row
        vals = np.stack([g.choice(N, size=hi, replace=False) for _ in range(B)]) if B else \
            np.zeros((0, hi), np.int64)
    counts = g.integers(lo, hi + 1, size=B)
    keep = np.arange(hi)[None, :] < counts[:, None]
    big = np.int64(N) + 1
    vals = np.where(keep, vals, big)
    if sort:
        vals = np.sort(vals, axis=1)
    else:  # keep the random order, but move padding to the end
        order = np.argsort(~keep, axis=1, kind="stable")
        vals = np.take_along_axis(vals, order, axis=1)
    vals = np.where(vals == big, -1, vals)
    out = np.full((B, K), -1, np.int32)
    out[:, :hi] = vals.astype(np.int32)
    return out


def make_zipf_indices(g: np.random.Generator, B: int, N: int, K: int, lo: int, hi: int, alpha: float,
                      offset: float = 10.0, sort: bool = True) -> np.ndarray:
    """Like make_indices, but with skewed feature frequencies, as on real
    positions where a few features are active in a large share of them: the
    features, in a random order, are drawn with probabilities proportional to
    1 / (rank + offset)^alpha; each row keeps the first `count ~ U{lo..hi}`
    distinct values of 2 * hi draws (fewer if the draws hold fewer)."""
    if not (0 <= lo <= hi <= K and hi <= N):
        raise ValueError("need 0 <= lo <= hi <= K and hi <= N")
    perm = g.permutation(N)
    cdf = np.cumsum(1.0 / (np.arange(N) + offset) ** alpha)
    cdf /= cdf[-1]
    D = 2 * hi
    vals = perm[np.minimum(np.searchsorted(cdf, g.random((B, D)), side="right"), N - 1)]
    order = np.argsort(vals, axis=1, kind="stable")  # equal values keep their draw order
    sv = np.take_along_axis(vals, order, axis=1)
    dup_sorted = np.zeros(sv.shape, bool)
    dup_sorted[:, 1:] = sv[:, 1:] == sv[:, :-1]
    dup = np.empty_like(dup_sorted)
    np.put_along_axis(dup, order, dup_sorted, axis=1)
    counts = g.integers(lo, hi + 1, size=B)
    rank = np.cumsum(~dup, axis=1) - 1  # index among the row's distinct draws
    keep = ~dup & (rank < counts[:, None])
    r, c = np.nonzero(keep)
    big = np.int64(N) + 1
    out = np.full((B, hi), big, np.int64)
    out[r, rank[r, c]] = vals[r, c]
    if sort:
        out = np.sort(out, axis=1)
    out = np.where(out == big, -1, out)
    res = np.full((B, K), -1, np.int32)
    res[:, :hi] = out.astype(np.int32)
    return res


def make_fp32_inputs(w: Workload, with_grads: bool = True) -> dict:
    """numpy arrays of an fp32 workload: idx_w, idx_b, W, bias, (g_w, g_b)."""
    d = {
        "idx_w": make_indices(rng(w.wid, S_WHITE), w.B, w.N, w.K, w.lo, w.hi),
        "idx_b": make_indices(rng(w.wid, S_BLACK), w.B, w.N, w.K, w.lo, w.hi),
        "W": rng(w.wid, S_W).standard_normal((w.N, w.L), dtype=np.float32) * np.float32(0.01),
    }
    sigma = float(np.sqrt(1.0 / w.N))
    d["bias"] = rng(w.wid, S_BIAS).uniform(-sigma, sigma, size=w.L).astype(np.float32)
    if with_grads:
        d["g_w"] = rng(w.wid, S_GW).standard_normal((w.B, w.L), dtype=np.float32)
        d["g_b"] = rng(w.wid, S_GB).standard_normal((w.B, w.L), dtype=np.float32)
    return d


def quantize_np(x: np.ndarray, scale: float) -> np.ndarray:
    """round_half_even(float32(x * scale)) saturated to int16 (numpy, host side)."""
    q = np.rint(x.astype(np.float32) * np.float32(scale))
    return np.clip(q, -32768, 32767).astype(np.int16)


def make_q16_inputs(w: Workload, scale: float = 127.0, psqt_scale: float = 600.0 * 16.0) -> dict:
    """int16 workload: W/bias quantized from seeded fp32 N(0, 0.01) / bias draws.

    The PSQT table is int32 [N, psqt] made from N(0, 0.01) draws at the
    export PSQT scale nnue2score * weight_scale_out = 9600
    (src/model/quantize.py:85-89).
    """
    d = {"idx_w": make_indices(rng(w.wid, S_WHITE), w.B, w.N, w.K, w.lo, w.hi)}
    wf = rng(w.wid, S_W).standard_normal((w.N, w.L + w.psqt), dtype=np.float32) * np.float32(0.01)
    sigma = float(np.sqrt(1.0 / w.N))
    bf = rng(w.wid, S_BIAS).uniform(-sigma, sigma, size=w.L).astype(np.float32)
    d["Wq"] = quantize_np(wf[:, :w.L], scale)
    d["bq"] = quantize_np(bf, scale)
    d["psqt"] = np.rint(wf[:, w.L:] * np.float32(psqt_scale)).astype(np.int32)
    return d


def sha256(a: np.ndarray) -> str:
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()[:16]


# ---------------------------------------------------------------- bytes ----
def active_counts(idx: np.ndarray, N: int) -> np.ndarray:
    return ((idx >= 0) & (idx < N)).sum(axis=1)


def step_bytes(idx_w: np.ndarray, idx_b: np.ndarray, N: int, L: int) -> int:
    """Algorithmic bytes of one fwd+bwd step over both perspectives.

    Per perspective and direction: 4*K (index row) + 4*L*(n_active + 1)
    (n_active gathered or scattered rows and one output/grad row), summed
    over positions; plus 4*N*L once for the dense weight-grad write-out.
    """
    K = idx_w.shape[1]
    total = 0
    for idx in (idx_w, idx_b):
        n = active_counts(idx, N).astype(np.int64)
        total += 2 * int((4 * K + 4 * L * (n + 1)).sum())
    return total + 4 * N * L


def step_compulsory_bytes(B: int, K: int, N: int, L: int) -> int:
    """Bytes an fp32 fwd+bwd step of both perspectives through SparseLinearFunction
    cannot avoid moving to or from HBM: both index tensors and the table read
    once, both outputs written, both upstream grads read once, each
    perspective's dense weight grad written and autograd's sum of the two (two
    read, one written).  The bias and its grad are negligible."""
    return 2 * 4 * B * K + 4 * N * L + 2 * 4 * B * L + 2 * 4 * B * L + 2 * 4 * N * L + 3 * 4 * N * L


def q16_compulsory_bytes(B: int, K: int, N: int, L: int, psqt: int = 0) -> int:
    """Bytes the int16 forward of both perspectives cannot avoid: both index
    tensors and the table (with its PSQT columns) read once, both int16 outputs
    and PSQT outputs written."""
    return 2 * 4 * B * K + N * (2 * L + 4 * psqt) + 2 * (2 * B * L + 4 * B * psqt)


def fwd_kernel_bytes(idx: np.ndarray, N: int, L: int) -> int:
    """One fp32 forward launch (one perspective): index rows, gathered rows, output rows."""
    K = idx.shape[1]
    n = active_counts(idx, N).astype(np.int64)
    return int((4 * K + 4 * L * (n + 1)).sum())


def bwd_gather_kernel_bytes(idx: np.ndarray, N: int, L: int) -> int:
    """One per-feature gather launch: a grad row and a sorted position per active
    slot, the N+1 segment offsets, and the N weight-grad rows written."""
    nnz = int(active_counts(idx, N).sum())
    return 4 * L * nnz + 4 * nnz + 4 * (N + 1) + 4 * N * L


def q16_fwd_bytes(idx: np.ndarray, N: int, L: int, psqt: int = 0) -> int:
    """One int16 forward launch: 4*K + 2*L*n_active + 2*L (+ PSQT rows and outputs)."""
    K = idx.shape[1]
    n = active_counts(idx, N).astype(np.int64)
    return int((4 * K + 2 * L * n + 2 * L + 4 * psqt * n + 4 * psqt).sum())
