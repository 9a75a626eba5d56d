"""Writes the golden fixtures of tests/golden/*.npz.

The reference ships no test vectors for its FT path, so these fixtures pin the
arithmetic through values fixed by hand or by exact integer arithmetic, never
by the C oracle:

  fwd_tiny    integer-valued rows: every float32 sum is exact, so the expected
              output is the exact integer closed form (computed here with
              Python ints).  Covers interior and suffix -1, a row repeating a
              feature, index N-1, an all -1 row.
  fwd_order   cases whose float32 result depends on the add order; expected
              values derived by hand for the reference order (bias first,
              then slots ascending, FT/kernel.py:93-100).
  bwd_tiny    integer-valued grads: exact dW / db (Python ints).
  bwd_order   a feature hit by three positions whose grads only sum to the
              hand-derived value in ascending position order
              (FT/kernel.py:122 stable sort, :178-181 serial sum).
  q16_tiny    int16 rows that overflow int16 on purpose: expected int32 and
              int16-wrapping results derived by hand.
  quant_tiny  round-half-even and saturation of the export quantizer
              (src/model/quantize.py:83-84) on exactly representable halves.

Run from the repository root:  python tests/golden/make_golden.py
"""

import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))


def exact_fwd(idx, W, b):
    B, K = idx.shape
    L = W.shape[1]
    out = np.zeros((B, L), np.float32)
    for r in range(B):
        for c in range(L):
            s = int(b[c])
            for k in range(K):
                f = int(idx[r, k])
                if f != -1:
                    s += int(W[f, c])
            out[r, c] = s
    return out


def exact_bwd(idx, G, N):
    B, K = idx.shape
    L = G.shape[1]
    dW = [[0] * L for _ in range(N)]
    db = [0] * L
    for r in range(B):
        for c in range(L):
            db[c] += int(G[r, c])
        for k in range(K):
            f = int(idx[r, k])
            if f != -1:
                for c in range(L):
                    dW[f][c] += int(G[r, c])
    return np.array(dW, np.float32), np.array(db, np.float32)


def main():
    g = np.random.default_rng(20261201)

    # ---- fwd_tiny / bwd_tiny ----
    N, L, K = 9, 7, 5
    idx = np.array([
        [0, 3, -1, 8, -1],     # interior -1
        [2, 2, 5, -1, -1],     # repeated feature inside a row (added twice)
        [-1, -1, -1, -1, -1],  # nothing active: out = bias
        [8, 7, 6, 5, 4],       # full row incl. N-1
        [1, -1, -1, -1, -1],
        [4, 0, 8, 2, -1],      # unsorted
    ], np.int32)
    W = g.integers(-8, 9, size=(N, L)).astype(np.float32)
    b = g.integers(-4, 5, size=L).astype(np.float32)
    np.savez(os.path.join(HERE, "fwd_tiny.npz"), idx=idx, W=W, bias=b, out=exact_fwd(idx, W, b))
    Gr = g.integers(-6, 7, size=(idx.shape[0], L)).astype(np.float32)
    dW, db = exact_bwd(idx, Gr, N)
    np.savez(os.path.join(HERE, "bwd_tiny.npz"), idx=idx, G=Gr, N=np.int64(N), dW=dW, db=db)

    # ---- fwd_order ----
    # Column 0 mixes 1e8 (ulp 8 in binary32) with small values, so each row's
    # result depends on the add order; column 1 is an exact control column.
    # A separate case pins "bias first": bias 1 plus 2^-24 twice stays 1
    # ((1 + 2^-24) ties to even), while adding the rows first gives 1 + 2^-23.
    W_o = np.zeros((5, 2), np.float32)
    W_o[0, 0] = np.float32(2.0 ** -24)
    W_o[1, 0] = np.float32(1e8)
    W_o[2, 0] = np.float32(1.0)
    W_o[3, 0] = np.float32(-1e8)
    W_o[4, 0] = np.float32(5.0)
    # column 1: exact small integers, a control column
    W_o[:, 1] = np.array([1, 2, 3, 4, 5], np.float32)
    bias_o = np.array([0.0, 10.0], np.float32)
    idx_o = np.array([
        [0, 0, -1, -1],   # col0: (0 + 2^-24) + 2^-24 = 2^-23 exactly
        [1, 2, 3, -1],    # col0: ((0 + 1e8) + 1) - 1e8 = 0
        [2, 1, 3, -1],    # col0: ((0 + 1) + 1e8) - 1e8 = 0
        [1, 3, 2, -1],    # col0: ((0 + 1e8) - 1e8) + 1 = 1
        [1, -1, 4, 3],    # col0: ((0 + 1e8) + 5) - 1e8 = 8 (1e8 + 5 rounds to 1e8 + 8)
    ], np.int32)
    out_o = np.array([
        [2.0 ** -23, 10 + 1 + 1],
        [0.0, 10 + 2 + 3 + 4],
        [0.0, 10 + 3 + 2 + 4],
        [1.0, 10 + 2 + 4 + 3],
        [8.0, 10 + 2 + 5 + 4],
    ], np.float32)
    # separate bias-first case: bias 1, rows 2^-24 twice -> 1 exactly
    W_b1 = np.array([[2.0 ** -24]], np.float32)
    np.savez(os.path.join(HERE, "fwd_order.npz"), idx=idx_o, W=W_o, bias=bias_o, out=out_o,
             idx_b1=np.array([[0, 0]], np.int32), W_b1=W_b1, bias_b1=np.array([1.0], np.float32),
             out_b1=np.array([[1.0]], np.float32))

    # ---- bwd_order ----
    # feature 2 is active at positions 0, 1, 2 with grads 1e8, -1e8, 1:
    # ascending positions: ((0 + 1e8) - 1e8) + 1 = 1; descending gives
    # ((0 + 1) - 1e8) + 1e8 = 0 (1 - 1e8 rounds to -1e8), and adding the 1
    # second gives 0 as well.  Feature 1 is active at positions 1, 3 with
    # grads -1e8 and 0.5: -1e8 + 0.5 rounds to -1e8.  Feature 0 never occurs.
    idx_bo = np.array([[2, -1], [1, 2], [2, -1], [1, -1]], np.int32)
    G_bo = np.array([[1e8], [-1e8], [1.0], [0.5]], np.float32)
    dW_bo = np.array([[0.0], [-1e8], [1.0]], np.float32)
    np.savez(os.path.join(HERE, "bwd_order.npz"), idx=idx_bo, G=G_bo, N=np.int64(3), dW=dW_bo)

    # ---- q16_tiny ----
    # col 0: bias 30000 + rows 10000 -> int32 40000 -> clamp 127;
    #        int16 wrap: 40000 - 65536 = -25536 -> clamp 0.
    # col 1: bias -30000 + (-10000) -> -40000 -> clamp 0; wrap: 25536 -> 127.
    # col 2: bias 5 + 7 + 9 = 21 in both modes.
    # col 3: bias 0 + 200 - 300 = -100 -> 0.
    Wq = np.array([[10000, -10000, 7, 200], [0, 0, 9, -300]], np.int16)
    bq = np.array([30000, -30000, 5, 0], np.int16)
    idx_q = np.array([[0, 1], [0, -1], [-1, -1]], np.int32)
    out32 = np.array([[127, 0, 21, 0], [127, 0, 12, 127], [127, 0, 5, 0]], np.int16)
    out16 = np.array([[0, 127, 21, 0], [0, 127, 12, 127], [127, 0, 5, 0]], np.int16)
    # raw accumulators (before clamp) for clip range [-32768, 32767] in wrap mode:
    raw16 = np.array([[-25536, 25536, 21, -100], [-25536, 25536, 12, 200], [30000, -30000, 5, 0]], np.int16)
    psqt = np.array([[5, -7], [100000, 3]], np.int32)
    psqt_out = np.array([[100005, -4], [5, -7], [0, 0]], np.int32)
    np.savez(os.path.join(HERE, "q16_tiny.npz"), Wq=Wq, bq=bq, idx=idx_q, out_acc32=out32, out_wrap16=out16,
             raw_wrap16=raw16, psqt=psqt, psqt_out=psqt_out)

    # ---- quant_tiny ----
    x = np.array([0.25, 0.75, 1.25, -0.25, -0.75, 1e9, -1e9, 3.0, -2.5], np.float32)
    q = np.array([0, 2, 2, 0, -2, 32767, -32768, 6, -5], np.int16)  # x * 2, half to even, saturated
    np.savez(os.path.join(HERE, "quant_tiny.npz"), x=x, scale=np.float32(2.0), q=q)
    print("wrote fixtures to", HERE)


if __name__ == "__main__":
    main()
