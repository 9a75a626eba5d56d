"""Oracle of the post-FT epilogue (NNUEModel._transform_inputs,
src/model/model.py:86-115) and of its backward, in numpy binary32.

TEST INFRASTRUCTURE ONLY: imported by ``tests/`` and never by the product path.

  fwd(xw, xb, us, k, l1)                 -> l0 [B, l1], psqt [B, 1]
  bwd(xw, xb, us, k, l1, g_l0, g_psqt)   -> d_xw, d_xb [B, L]

xw / xb are the FT outputs [B, L] of the white / black perspective, us the
side to move [B] or [B, 1] (nonzero: white), k the PSQT bucket [B].  The
backward follows autograd's evaluation of the reference ops step by step
(mul by 127/128, the where() pair summed, the two select() grads summed, the
clamp mask 0 <= x <= 1, gather's scatter-add onto zeros, sub's negation), each
an elementwise binary32 operation, so the results are what torch computes bit
for bit.  ``mutation`` plants a mistake for the tests.
"""

from __future__ import annotations

import numpy as np

MUTATIONS = ("sides_swapped", "no_scale_in_bwd", "strict_clamp_mask", "psqt_sign", "pair_neighbours")
K127 = np.float32(127 / 128)


def _clamp(x):
    return np.where(x < 0, np.float32(0), np.where(x > 1, np.float32(1), x)).astype(np.float32)


def _halves(x, l1, mutation):
    h = l1 // 2
    if mutation == "pair_neighbours":
        return x[:, 0:l1:2], x[:, 1:l1:2]
    return x[:, :h], x[:, h:l1]


def fwd(xw, xb, us, k, l1: int, mutation: str | None = None):
    xw, xb = np.asarray(xw, np.float32), np.asarray(xb, np.float32)
    side = (np.asarray(us, np.float32).reshape(-1, 1) != 0)
    if mutation == "sides_swapped":
        side = ~side
    pw = [np.multiply(*[_clamp(a) for a in _halves(x, l1, mutation)]).astype(np.float32) for x in (xw, xb)]
    first = np.where(side, pw[0], pw[1])
    second = np.where(side, pw[1], pw[0])
    l0 = (np.concatenate([first, second], axis=1) * K127).astype(np.float32)
    kk = np.asarray(k, np.int64).reshape(-1)
    rows = np.arange(xw.shape[0])
    u = np.asarray(us, np.float32).reshape(-1)
    d = (xw[rows, l1 + kk] - xb[rows, l1 + kk]).astype(np.float32)
    psqt = (d * (u - np.float32(0.5))).astype(np.float32).reshape(-1, 1)
    return l0, psqt


def bwd(xw, xb, us, k, l1: int, g_l0, g_psqt, mutation: str | None = None):
    xw, xb = np.asarray(xw, np.float32), np.asarray(xb, np.float32)
    g_l0 = np.asarray(g_l0, np.float32)
    B, L = xw.shape
    h = l1 // 2
    side = (np.asarray(us, np.float32).reshape(-1, 1) != 0)
    if mutation == "sides_swapped":
        side = ~side
    dcat = g_l0 if mutation == "no_scale_in_bwd" else (g_l0 * K127).astype(np.float32)
    d_first, d_second = dcat[:, :h], dcat[:, h:]
    zero = np.float32(0)
    # where(side, w, b) and where(side, b, w): each product gets one selected grad and one +0
    d_pw = [(np.where(side, d_first, zero) + np.where(side, zero, d_second)).astype(np.float32),
            (np.where(side, zero, d_first) + np.where(side, d_second, zero)).astype(np.float32)]
    out = []
    u = np.asarray(us, np.float32).reshape(-1)
    dp = (np.asarray(g_psqt, np.float32).reshape(-1) * (u - np.float32(0.5))).astype(np.float32)
    kk = np.asarray(k, np.int64).reshape(-1)
    for p, x in enumerate((xw, xb)):
        a, b = _halves(x, l1, mutation)
        ca, cb = _clamp(a), _clamp(b)
        da = ((d_pw[p] * cb).astype(np.float32) + zero).astype(np.float32)
        db = ((d_pw[p] * ca).astype(np.float32) + zero).astype(np.float32)
        if mutation == "strict_clamp_mask":
            ma, mb = (a > 0) & (a < 1), (b > 0) & (b < 1)
        else:
            ma, mb = (a >= 0) & (a <= 1), (b >= 0) & (b <= 1)
        dx = np.zeros((B, L), np.float32)
        if mutation == "pair_neighbours":
            dx[:, 0:l1:2] = np.where(ma, da, zero)
            dx[:, 1:l1:2] = np.where(mb, db, zero)
        else:
            dx[:, :h] = np.where(ma, da, zero)
            dx[:, h:l1] = np.where(mb, db, zero)
        sgn = dp if (p == 0 or mutation == "psqt_sign") else -dp
        dx[np.arange(B), l1 + kk] = (zero + sgn).astype(np.float32)
        out.append(dx)
    return out[0], out[1]
