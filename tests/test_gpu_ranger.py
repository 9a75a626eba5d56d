"""Fused Ranger22 update (sft_ranger22_update_f32) on the GPU against the
oracle: optimizer states bit-exact, parameters within one unit in the last
place (the row norm is summed in another order than the oracle's binary64)."""

import numpy as np
import pytest
import torch

from gpu_helpers import announce, dev, host
from oracle import ranger_oracle
from src.ranger22.fused_update import get_fused_full_update

pytestmark = pytest.mark.gpu


def _inputs(seed, shape):
    g = np.random.default_rng(seed)
    p = (g.standard_normal(shape) * 0.05).astype(np.float32)
    grad = (g.standard_normal(shape) * 1e-3).astype(np.float32)
    v = (g.random(shape) * 1e-6).astype(np.float32)
    m = (g.standard_normal(shape) * 1e-3).astype(np.float32)
    mp = (g.standard_normal(shape) * 1e-3).astype(np.float32)
    step, beta1, beta2, lr, eps = 7, 0.9, 0.999, 8.75e-4, 1e-7
    sc = ranger_oracle.scalars_array(
        lr=lr, inv_sqrt_bc2=1.0 / np.sqrt(1 - beta2 ** step), eps=eps, two_nl_factor=2 * 1e-4,
        noise_norm_recip=1.0 / np.sqrt((1 + beta2) ** 2 + beta2 ** 2), pnm_a=2.0, pnm_b=-1.0,
        step_size=lr / (1 - beta1 ** step), beta2=beta2, one_minus_beta2=1 - beta2, beta1_sq=beta1 * beta1,
        one_minus_beta1_sq=1 - beta1 * beta1)
    return p, grad, v, m, mp, sc


def _ulps(a, b):
    ai = np.asarray(a, np.float32).view(np.int32).astype(np.int64)
    bi = np.asarray(b, np.float32).view(np.int32).astype(np.int64)
    ai = np.where(ai < 0, np.int64(-2**31) - ai, ai)
    bi = np.where(bi < 0, np.int64(-2**31) - bi, bi)
    return np.abs(ai - bi)


@pytest.mark.parametrize("shape", [(24576, 1048), (768, 1048), (1048,), (37, 13), (5, 2100), (300, 256), (1, 4)])
def test_fused_update_matches_oracle(shape):
    announce(f"ranger22 update shape={shape}")
    p, g, v, m, mp, sc = _inputs(len(shape) * 100 + shape[0], shape)
    tp, tv, tm = dev(p), dev(v), dev(m)
    get_fused_full_update(len(shape))(tp, dev(g), tv, tm, dev(mp), dev(sc))
    torch.cuda.synchronize()
    rp, rv, rm = ranger_oracle.update(p, g, v, m, mp, sc)
    assert np.array_equal(host(tv), rv)
    assert np.array_equal(host(tm), rm)
    assert _ulps(host(tp), rp).max() <= 1


def test_two_steps_alternating_momentum_buffers():
    """Ranger22 swaps grad_ma and neg_grad_ma every step (optimizer.py:357-362)."""
    announce("ranger22 two steps")
    p, g, v, m, mp, sc = _inputs(9, (64, 1048))
    tp, tv, ta, tb = dev(p), dev(v), dev(m), dev(mp)
    upd = get_fused_full_update(2)
    rp, rv, ra, rb = p, v, m, mp
    for step in range(2):
        cur, prev = (ta, tb) if step % 2 == 0 else (tb, ta)
        upd(tp, dev(g), tv, cur, prev, dev(sc))
        if step % 2 == 0:
            rp, rv, ra = ranger_oracle.update(rp, g, rv, ra, rb, sc)
        else:
            rp, rv, rb = ranger_oracle.update(rp, g, rv, rb, ra, sc)
    torch.cuda.synchronize()
    assert np.array_equal(host(tv), rv) and np.array_equal(host(ta), ra) and np.array_equal(host(tb), rb)
    assert _ulps(host(tp), rp).max() <= 1
