"""Oracle of the composed feature transformer (both perspectives, virtual rows).

TEST INFRASTRUCTURE ONLY: imported by ``tests/`` and never by the product path.
It composes the pinned per-perspective functions of ``ft_oracle`` the way the
reference composes SparseLinearFunction:

  merged_table(blocks)       torch.cat of each block's merged_weight
                             (src/model/modules/features/composed.py:49-50);
                             HalfKAv2_hm: weight + virtual_weight.repeat(32, 1),
                             one binary32 add per element (halfka_v2_hm.py:69-70);
                             Full_Threats: weight (full_threats.py:27-28)
  composed_fwd(...)          SparseLinearFunction on the merged table, once per
                             perspective (composed.py:52-53)
  composed_bwd(...)          the two reference-order weight grads added in
                             binary32 (autograd's sum of the shared table's
                             grads), split per block (cat's backward); virtual
                             grads are the sum over the 32 repeats (repeat's
                             backward), returned in binary64 with the binary64
                             bias grad, since torch's reduction order is not
                             part of the contract.

A block is (weight [R, L] float32, virtual [V, L] float32 or None).  The
``mutation`` argument plants a mistake (tests check that each one is caught).
"""

from __future__ import annotations

import numpy as np

from . import ft_oracle

MUTATIONS = ("virtual_by_bucket", "blocks_reversed", "bwd_first_only", "virtual_added_twice")


def merged_table(blocks, mutation: str | None = None) -> np.ndarray:
    parts = []
    for w, v in blocks:
        w = np.ascontiguousarray(w, np.float32)
        if v is None:
            parts.append(w)
            continue
        v = np.ascontiguousarray(v, np.float32)
        R, P = w.shape[0], v.shape[0]
        rows = np.arange(R)
        vi = rows // (R // P) if mutation == "virtual_by_bucket" else rows % P
        m = w + v[vi]  # binary32 add, rounded once per element
        if mutation == "virtual_added_twice":
            m = m + v[vi]
        parts.append(m.astype(np.float32))
    if mutation == "blocks_reversed":
        parts = parts[::-1]
    return np.concatenate(parts, axis=0)


def composed_fwd(idx0, idx1, blocks, b, mutation: str | None = None):
    M = merged_table(blocks, mutation)
    return ft_oracle.fwd_f32(idx0, M, b), ft_oracle.fwd_f32(idx1, M, b)


def composed_bwd(idx0, idx1, g0, g1, blocks, mutation: str | None = None):
    """-> ([weight grad per block, float32], [virtual grad per block or None, float64], bias grad float64)."""
    N = sum(np.shape(w)[0] for w, _ in blocks)
    d0, _ = ft_oracle.bwd_f32(idx0, g0, N)
    d1, _ = ft_oracle.bwd_f32(idx1, g1, N)
    d = d0 if mutation == "bwd_first_only" else (d0 + d1).astype(np.float32)
    wgrads, vgrads = [], []
    start = 0
    for w, v in blocks:
        R = np.shape(w)[0]
        dw = d[start:start + R]
        wgrads.append(dw)
        if v is None:
            vgrads.append(None)
        else:
            P = np.shape(v)[0]
            vgrads.append(dw.astype(np.float64).reshape(R // P, P, -1).sum(axis=0))
        start += R
    db = np.asarray(g0, np.float64).sum(axis=0) + np.asarray(g1, np.float64).sum(axis=0)
    return wgrads, vgrads, db
