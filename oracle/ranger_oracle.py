"""Oracle of Ranger22's full parameter update (src/ranger22/optimizer.py:46-111).

TEST INFRASTRUCTURE ONLY: imported by ``tests/`` and never by the product path.

  update(p, g, v, m, m_prev, scalars) -> (p', v', m')

numpy binary32, one rounding per operation in the reference function's order;
the norm of each row of p (the whole tensor for 1-D) is taken in binary64 and
rounded once, so a product that sums it in another order may differ from p'
in the last place.  ``mutation`` plants a mistake for the tests.
"""

from __future__ import annotations

import numpy as np

MUTATIONS = ("pnm_swapped", "norm_over_columns", "norm_after_update", "no_eps_in_denom", "beta1_not_squared")
NAMES = ("lr", "inv_sqrt_bc2", "eps", "two_nl_factor", "noise_norm_recip", "pnm_a", "pnm_b", "step_size", "beta2",
         "one_minus_beta2", "beta1_sq", "one_minus_beta1_sq")


def scalars_array(**kw) -> np.ndarray:
    return np.array([kw[n] for n in NAMES], np.float32)


def update(p, g, v, m, m_prev, scalars, mutation: str | None = None):
    f = np.float32
    s = dict(zip(NAMES, (f(x) for x in np.asarray(scalars, np.float32))))
    p = np.asarray(p, np.float32).copy()
    g, v, m, mp = (np.asarray(a, np.float32) for a in (g, v, m, m_prev))
    one_d = p.ndim == 1
    P, G, V, M, MP = (a.reshape(1, -1) if one_d else a for a in (p, g, v, m, mp))
    V2 = (V * s["beta2"]).astype(f) + ((G * G).astype(f) * s["one_minus_beta2"]).astype(f)
    b1 = s["beta1_sq"] if mutation != "beta1_not_squared" else f(np.sqrt(s["beta1_sq"]))
    M2 = (M * b1).astype(f) + (G * s["one_minus_beta1_sq"]).astype(f)
    V2, M2 = V2.astype(f), M2.astype(f)

    def factor(T):
        axis = 0 if mutation == "norm_over_columns" else 1
        un = f(1) * np.sqrt((T.astype(np.float64) ** 2).sum(axis=axis, keepdims=True)).astype(f)
        corr = (s["two_nl_factor"] * (f(1) - (f(1) / (un + s["eps"]).astype(f)).astype(f)).astype(f)).astype(f)
        return (f(1) - (s["lr"] * corr).astype(f)).astype(f)

    eps_d = f(0) if mutation == "no_eps_in_denom" else s["eps"]
    denom = ((np.sqrt(V2).astype(f) * s["inv_sqrt_bc2"]).astype(f) + eps_d).astype(f)
    a, b = (s["pnm_b"], s["pnm_a"]) if mutation == "pnm_swapped" else (s["pnm_a"], s["pnm_b"])
    pn = (((M2 * a).astype(f) + (MP * b).astype(f)).astype(f) * s["noise_norm_recip"]).astype(f)
    q = ((pn / denom).astype(f) * s["step_size"]).astype(f)
    if mutation == "norm_after_update":
        P2 = (P - q).astype(f)
        P2 = (P2 * factor(P2)).astype(f)
    else:
        P2 = ((P * factor(P)).astype(f) - q).astype(f)
    out = [P2, V2, M2]
    if one_d:
        out = [a.reshape(-1) for a in out]
    return tuple(out)
