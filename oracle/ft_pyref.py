"""Pure-Python loop restatement of the FT arithmetic, for small cases.

TEST INFRASTRUCTURE ONLY.  A second, independent restatement of the same
reference semantics as ft_oracle.c, written as explicit scalar loops over
numpy float32 scalars (each `+` is one binary32 add).  Tests use it to check
the C oracle on small random cases, and to show that the golden-fixture
checks catch plausible mistakes: `mutation` plants one such mistake.

Mutations (all planted here, on the CPU, never in product code):
  "bias_last"        add the bias after the rows instead of first
  "reverse_slots"    walk slots k descending
  "no_skip"          treat -1 as row N-1 (negative index wraps) instead of skipping
  "drop_last_slot"   ignore slot K-1
  "bwd_desc"         backward sums a feature's grad rows in descending position order
  "bwd_once_per_row" backward counts a feature once per row even when repeated
  "db_missing_row"   bias grad skips the last position
"""

from __future__ import annotations

import numpy as np

F32 = np.float32


def fwd(idx, W, bias, mutation: str | None = None) -> np.ndarray:
    """Reference order (FT/kernel.py:93-100): acc = bias; acc += W[idx[k]] for k ascending, -1 skipped."""
    idx = np.asarray(idx)
    W = np.asarray(W, F32)
    bias = np.asarray(bias, F32)
    B, K = idx.shape
    L = W.shape[1]
    out = np.empty((B, L), F32)
    slots = list(range(K))
    if mutation == "reverse_slots":
        slots = slots[::-1]
    if mutation == "drop_last_slot":
        slots = slots[:-1]
    for b in range(B):
        for c in range(L):
            acc = F32(0.0) if mutation == "bias_last" else bias[c]
            for k in slots:
                f = int(idx[b, k])
                if f == -1 and mutation != "no_skip":
                    continue
                acc = F32(acc + W[f, c])
            if mutation == "bias_last":
                acc = F32(acc + bias[c])
            out[b, c] = acc
    return out


def bwd(idx, G, N: int, mutation: str | None = None):
    """Reference order (FT/kernel.py:122,171-186,269): per feature, grad rows of its
    slots in ascending flat order summed onto 0; db = column sums (here in
    float64, rounded once, since torch's reduction order is unspecified)."""
    idx = np.asarray(idx)
    G = np.asarray(G, F32)
    B, K = idx.shape
    L = G.shape[1]
    dW = np.zeros((N, L), F32)
    order = list(range(B))
    if mutation == "bwd_desc":
        order = order[::-1]
    acc = {}
    for b in order:
        seen = set()
        for k in range(K):
            f = int(idx[b, k])
            if f == -1:
                continue
            if mutation == "bwd_once_per_row" and f in seen:
                continue
            seen.add(f)
            row = acc.setdefault(f, [F32(0.0)] * L)
            for c in range(L):
                row[c] = F32(row[c] + G[b, c])
    for f, row in acc.items():
        for c in range(L):
            dW[f, c] = F32(dW[f, c] + row[c])
    rows = range(B - 1) if mutation == "db_missing_row" else range(B)
    db = np.array([sum(float(G[b, c]) for b in rows) for c in range(L)], np.float64).astype(F32)
    return dW, db


def fwd_i16(idx, Wq, bq, psqt=None, clip_lo=0, clip_hi=127, wrap16=False):
    """Integer closed form: int16 accumulator semantics emulated with explicit wrapping."""
    idx = np.asarray(idx)
    B, K = idx.shape
    N, L = Wq.shape
    out = np.empty((B, L), np.int16)
    pout = None if psqt is None else np.zeros((B, psqt.shape[1]), np.int64)
    for b in range(B):
        for c in range(L):
            acc = int(bq[c])
            for k in range(K):
                f = int(idx[b, k])
                if f == -1:
                    continue
                acc += int(Wq[f, c])
                if wrap16:
                    acc = (acc + 32768) % 65536 - 32768
            out[b, c] = min(max(acc, clip_lo), clip_hi)
        if psqt is not None:
            for k in range(K):
                f = int(idx[b, k])
                if f != -1:
                    pout[b] += psqt[f].astype(np.int64)
    return out, (None if pout is None else pout.astype(np.int32))
