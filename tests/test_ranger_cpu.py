"""Ranger22 full-update oracle (src/ranger22/optimizer.py:46-111): a case worked
by hand in exact arithmetic, invariants, and planted mistakes."""

import numpy as np
import pytest

from oracle import ranger_oracle

# lr 0.5, inv_sqrt_bc2 2, eps 0, two_nl_factor 0.25, noise_norm_recip 0.5,
# pnm 2 / -1, step_size 0.5, beta2 0.75, beta1^2 0.5: every value below is exact.
HAND = ranger_oracle.scalars_array(lr=0.5, inv_sqrt_bc2=2.0, eps=0.0, two_nl_factor=0.25, noise_norm_recip=0.5,
                                   pnm_a=2.0, pnm_b=-1.0, step_size=0.5, beta2=0.75, one_minus_beta2=0.25,
                                   beta1_sq=0.5, one_minus_beta1_sq=0.5)


def _hand_case():
    # row 0: p = (3, 4), |p| = 5 -> c = 0.25 (1 - 1/5) = 0.2, 1 - lr c = 0.9 (binary32: 0.9f)
    #   g = 2: v' = 0 * 0.75 + 4 * 0.25 = 1, sqrt 1 * 2 + 0 = 2
    #          m' = 0 * 0.5 + 2 * 0.5 = 1, pn = (1 * 2 + 0.5 * -1) * 0.5 = 0.75, q = 0.75 / 2 * 0.5 = 0.1875
    #   p' = fl(3 * 0.9f) - 0.1875 and fl(4 * 0.9f) - 0.1875, each rounded to binary32
    # row 1: p = (0, 8), |p| = 8 -> c = 0.25 (1 - 1/8) = 0.21875, 1 - lr c = 0.890625
    #   g = (0, 4), v = (4, 0), m = (2, 2), m_prev = (2, 4):
    #   v' = (3, 4), m' = (1, 3); denom = (2 sqrt 3, 4); pn = (0, 1); q = (0, 0.125)
    #   p' = (0, 8 * 0.890625 - 0.125) = (0, 7)
    p = np.array([[3, 4], [0, 8]], np.float32)
    g = np.array([[2, 2], [0, 4]], np.float32)
    v = np.array([[0, 0], [4, 0]], np.float32)
    m = np.array([[0, 0], [2, 2]], np.float32)
    mp = np.array([[0.5, 0.5], [2, 4]], np.float32)
    f = np.float32
    want_p = np.array([[f(f(3) * f(0.9)) - f(0.1875), f(f(4) * f(0.9)) - f(0.1875)], [0, 7]], np.float32)
    want_v = np.array([[1, 1], [3, 4]], np.float32)
    want_m = np.array([[1, 1], [1, 3]], np.float32)
    return (p, g, v, m, mp), (want_p, want_v, want_m)


HAND_EPS = HAND.copy()
HAND_EPS[2] = 1.0  # eps


def _hand_case_eps():
    # eps = 1: p = (0, 3), |p| + eps = 4 -> c = 0.25 * 0.75 = 0.1875, 1 - lr c = 0.90625
    #   g = 0, v = 0: v' = 0, denom = 0 * 2 + 1 = 1;  m = 2, m_prev = 1: m' = 1,
    #   pn = (1 * 2 + 1 * -1) * 0.5 = 0.5, q = 0.5 / 1 * 0.5 = 0.25
    #   p' = (0 - 0.25, 3 * 0.90625 - 0.25) = (-0.25, 2.46875)
    p = np.array([[0, 3]], np.float32)
    z = np.zeros((1, 2), np.float32)
    m = np.full((1, 2), 2, np.float32)
    mp = np.ones((1, 2), np.float32)
    return (p, z, z, m, mp), (np.array([[-0.25, 2.46875]], np.float32), z, np.ones((1, 2), np.float32))


def _hand_ok(mutation=None):
    ok = True
    for case, sc in ((_hand_case, HAND), (_hand_case_eps, HAND_EPS)):
        args, want = case()
        with np.errstate(divide="ignore", invalid="ignore"):
            got = ranger_oracle.update(*args, sc, mutation=mutation)
        ok = ok and all(np.array_equal(a, b) for a, b in zip(got, want))
    return ok


def test_hand_worked_case():
    assert _hand_ok()


@pytest.mark.parametrize("mutation", ranger_oracle.MUTATIONS)
def test_hand_case_catches_mistakes(mutation):
    assert not _hand_ok(mutation)


def _rand(seed, shape):
    g = np.random.default_rng(seed)
    p = g.standard_normal(shape).astype(np.float32)
    grad = (g.standard_normal(shape) * 1e-3).astype(np.float32)
    v = (g.random(shape) * 1e-6).astype(np.float32)
    m = (g.standard_normal(shape) * 1e-3).astype(np.float32)
    mp = (g.standard_normal(shape) * 1e-3).astype(np.float32)
    sc = ranger_oracle.scalars_array(lr=1e-3, inv_sqrt_bc2=1.3, eps=1e-8, two_nl_factor=2e-4, noise_norm_recip=0.5,
                                     pnm_a=2.0, pnm_b=-1.0, step_size=1.7e-3, beta2=0.999, one_minus_beta2=1e-3,
                                     beta1_sq=0.81, one_minus_beta1_sq=0.19)
    return p, grad, v, m, mp, sc


def test_rows_are_independent_and_1d_is_one_row():
    p, g, v, m, mp, sc = _rand(1, (6, 20))
    full = ranger_oracle.update(p, g, v, m, mp, sc)
    perm = np.array([3, 0, 5, 1, 4, 2])
    permuted = ranger_oracle.update(p[perm], g[perm], v[perm], m[perm], mp[perm], sc)
    for a, b in zip(full, permuted):
        assert np.array_equal(a[perm], b)
    one = ranger_oracle.update(p[2], g[2], v[2], m[2], mp[2], sc)
    for a, b in zip(full, one):
        assert np.array_equal(a[2], b)


def test_zero_step_leaves_p_and_updates_state():
    p, g, v, m, mp, sc = _rand(2, (4, 9))
    sc = sc.copy()
    sc[0] = 0.0  # lr
    sc[7] = 0.0  # step_size
    p2, v2, m2 = ranger_oracle.update(p, g, v, m, mp, sc)
    assert np.array_equal(p2, p)
    assert np.array_equal(v2, (v * sc[8]).astype(np.float32) + ((g * g).astype(np.float32) * sc[9]).astype(np.float32))
