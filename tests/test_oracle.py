"""The oracle pinned against hand-derived fixtures, an independent loop
restatement, library routines and the identities of the FT maths (CPU only)."""

import numpy as np
import pytest
import torch

from conftest import golden
from oracle import ft_oracle, ft_pyref
from sft_amd import workloads


def rand_case(seed, B, N, K, L, lo=0, hi=None, sort=False):
    g = np.random.default_rng(seed)
    idx = workloads.make_indices(g, B, N, K, lo, K if hi is None else hi, sort=sort)
    W = g.standard_normal((N, L)).astype(np.float32)
    b = g.standard_normal(L).astype(np.float32)
    G = g.standard_normal((B, L)).astype(np.float32)
    return idx, W, b, G


# ------------------------------------------------------------- fixtures ----
def test_fwd_tiny_fixture():
    d = golden("fwd_tiny")
    assert np.array_equal(ft_oracle.fwd_f32(d["idx"], d["W"], d["bias"]), d["out"])
    assert np.array_equal(ft_oracle.fwd_f64(d["idx"], d["W"], d["bias"]), d["out"].astype(np.float64))


def test_fwd_order_fixture():
    d = golden("fwd_order")
    assert np.array_equal(ft_oracle.fwd_f32(d["idx"], d["W"], d["bias"]), d["out"])
    assert np.array_equal(ft_oracle.fwd_f32(d["idx_b1"], d["W_b1"], d["bias_b1"]), d["out_b1"])


def test_bwd_tiny_fixture():
    d = golden("bwd_tiny")
    dW, db = ft_oracle.bwd_f32(d["idx"], d["G"], int(d["N"]))
    assert np.array_equal(dW, d["dW"]) and np.array_equal(db, d["db"])
    dW64, db64 = ft_oracle.bwd_f64(d["idx"], d["G"], int(d["N"]))
    assert np.array_equal(dW64, d["dW"].astype(np.float64)) and np.array_equal(db64, d["db"].astype(np.float64))


def test_bwd_order_fixture():
    d = golden("bwd_order")
    dW, _ = ft_oracle.bwd_f32(d["idx"], d["G"], int(d["N"]))
    assert np.array_equal(dW, d["dW"])


def test_q16_fixture():
    d = golden("q16_tiny")
    out, pout = ft_oracle.fwd_i16(d["idx"], d["Wq"], d["bq"], d["psqt"], 0, 127, wrap16=False)
    assert np.array_equal(out, d["out_acc32"]) and np.array_equal(pout, d["psqt_out"])
    out, _ = ft_oracle.fwd_i16(d["idx"], d["Wq"], d["bq"], None, 0, 127, wrap16=True)
    assert np.array_equal(out, d["out_wrap16"])
    out, _ = ft_oracle.fwd_i16(d["idx"], d["Wq"], d["bq"], None, -32768, 32767, wrap16=True)
    assert np.array_equal(out, d["raw_wrap16"])


def test_quant_fixture():
    d = golden("quant_tiny")
    assert np.array_equal(ft_oracle.quantize_i16(d["x"], float(d["scale"]), clamp=True), d["q"])
    with pytest.raises(ValueError):
        ft_oracle.quantize_i16(d["x"], float(d["scale"]), clamp=False)  # 1e9 * 2 is out of int16


# ------------------------------------------------ planted mistakes fail ----
FWD_MUTATIONS = ["bias_last", "reverse_slots", "no_skip", "drop_last_slot"]
BWD_MUTATIONS = ["bwd_desc", "bwd_once_per_row", "db_missing_row"]


def _fwd_fixtures_pass(fn) -> bool:
    ok = True
    for name in ("fwd_tiny", "fwd_order"):
        d = golden(name)
        ok &= np.array_equal(fn(d["idx"], d["W"], d["bias"]), d["out"])
    d = golden("fwd_order")
    ok &= np.array_equal(fn(d["idx_b1"], d["W_b1"], d["bias_b1"]), d["out_b1"])
    return bool(ok)


def _bwd_fixtures_pass(fn) -> bool:
    d = golden("bwd_tiny")
    dW, db = fn(d["idx"], d["G"], int(d["N"]))
    ok = np.array_equal(dW, d["dW"]) and np.array_equal(db, d["db"])
    d = golden("bwd_order")
    dW, _ = fn(d["idx"], d["G"], int(d["N"]))
    return bool(ok and np.array_equal(dW, d["dW"]))


def test_loop_restatement_passes_fixtures():
    assert _fwd_fixtures_pass(ft_pyref.fwd)
    assert _bwd_fixtures_pass(ft_pyref.bwd)


@pytest.mark.parametrize("mutation", FWD_MUTATIONS)
def test_fixtures_catch_forward_mistake(mutation):
    assert not _fwd_fixtures_pass(lambda i, w, b: ft_pyref.fwd(i, w, b, mutation=mutation))


@pytest.mark.parametrize("mutation", BWD_MUTATIONS)
def test_fixtures_catch_backward_mistake(mutation):
    assert not _bwd_fixtures_pass(lambda i, g, n: ft_pyref.bwd(i, g, n, mutation=mutation))


# ------------------------------------------ C oracle == loop restatement ----
@pytest.mark.parametrize("seed,B,N,K,L", [(1, 7, 11, 5, 13), (2, 16, 40, 8, 9), (3, 5, 6, 6, 4)])
def test_c_oracle_matches_loops_fwd(seed, B, N, K, L):
    idx, W, b, _ = rand_case(seed, B, N, K, L)
    idx[0, :] = -1
    idx[1, 1] = -1  # interior hole
    assert np.array_equal(ft_oracle.fwd_f32(idx, W, b), ft_pyref.fwd(idx, W, b))


@pytest.mark.parametrize("seed,B,N,K,L", [(4, 9, 12, 5, 6), (5, 20, 7, 4, 3)])
def test_c_oracle_matches_loops_bwd(seed, B, N, K, L):
    idx, _, _, G = rand_case(seed, B, N, K, L)
    idx[2, 0] = idx[2, 1] = 3  # a repeated feature inside one row
    dW, db = ft_oracle.bwd_f32(idx, G, N)
    rW, rb = ft_pyref.bwd(idx, G, N)
    assert np.array_equal(dW, rW) and np.array_equal(db, rb)


def test_c_oracle_matches_loops_i16():
    g = np.random.default_rng(9)
    idx = workloads.make_indices(g, 12, 30, 6, 0, 6, sort=False)
    Wq = g.integers(-20000, 20000, size=(30, 5)).astype(np.int16)
    bq = g.integers(-20000, 20000, size=5).astype(np.int16)
    ps = g.integers(-2**20, 2**20, size=(30, 3)).astype(np.int32)
    for wrap in (False, True):
        for lo, hi in ((0, 127), (-32768, 32767), (-5, 300)):
            o, p = ft_oracle.fwd_i16(idx, Wq, bq, ps, lo, hi, wrap)
            ro, rp = ft_pyref.fwd_i16(idx, Wq, bq, ps, lo, hi, wrap)
            assert np.array_equal(o, ro) and np.array_equal(p, rp)


def test_wrap16_equals_int16_numpy_accumulator():
    """int16 accumulation with numpy's wrapping int16 adds == oracle wrap mode."""
    g = np.random.default_rng(10)
    idx = workloads.make_indices(g, 40, 25, 8, 0, 8)
    Wq = g.integers(-32768, 32768, size=(25, 6)).astype(np.int16)
    bq = g.integers(-32768, 32768, size=6).astype(np.int16)
    acc = np.tile(bq, (40, 1))
    with np.errstate(over="ignore"):
        for k in range(8):
            f = idx[:, k]
            m = f >= 0
            acc[m] = (acc[m] + Wq[f[m]]).astype(np.int16)
    o, _ = ft_oracle.fwd_i16(idx, Wq, bq, None, -32768, 32767, wrap16=True)
    assert np.array_equal(o, acc)


# ---------------------------------------------------- library routines ----
@pytest.mark.parametrize("seed,B,N,K,L", [(11, 64, 300, 32, 136), (12, 33, 50, 7, 13)])
def test_oracle_matches_embedding_bag(seed, B, N, K, L):
    idx, W, b, G = rand_case(seed, B, N, K, L)
    ti = torch.from_numpy(idx.astype(np.int64))
    mask = ti >= 0
    flat = ti[mask]
    offsets = torch.cat([torch.zeros(1, dtype=torch.int64), mask.sum(1).cumsum(0)[:-1]])
    Wt = torch.from_numpy(W.astype(np.float64)).requires_grad_(True)
    out = torch.nn.functional.embedding_bag(flat, Wt, offsets, mode="sum") + torch.from_numpy(b.astype(np.float64))
    out.backward(torch.from_numpy(G.astype(np.float64)))
    y32 = ft_oracle.fwd_f32(idx, W, b)
    assert ft_oracle.rownorm_rel_err(y32, out.detach().numpy()) < 1e-6
    assert np.allclose(ft_oracle.fwd_f64(idx, W, b), out.detach().numpy(), rtol=0, atol=1e-12)
    dW, db = ft_oracle.bwd_f64(idx, G, N)
    assert np.allclose(dW, Wt.grad.numpy(), rtol=0, atol=1e-11)
    assert np.allclose(db, G.astype(np.float64).sum(0), rtol=0, atol=1e-11)


# ---------------------------------------------------------- identities ----
@pytest.mark.parametrize("seed,B,N,K,L", [(21, 200, 97, 16, 24), (22, 64, 1000, 32, 8)])
def test_adjoint_identity(seed, B, N, K, L):
    """<fwd(W) - b, G> == <W, dW(G)>: the backward is the exact transpose of the forward."""
    idx, W, b, G = rand_case(seed, B, N, K, L)
    y = ft_oracle.fwd_f64(idx, W, np.zeros_like(b))
    dW, _ = ft_oracle.bwd_f64(idx, G, N)
    lhs = float((y * G.astype(np.float64)).sum())
    rhs = float((W.astype(np.float64) * dW).sum())
    assert abs(lhs - rhs) <= 1e-9 * max(1.0, abs(lhs))


def test_padding_and_all_inactive_rows():
    idx, W, b, G = rand_case(31, 20, 40, 6, 5)
    padded = np.concatenate([idx, np.full((20, 3), -1, np.int32)], axis=1)
    assert np.array_equal(ft_oracle.fwd_f32(idx, W, b), ft_oracle.fwd_f32(padded, W, b))
    assert np.array_equal(ft_oracle.bwd_f32(idx, G, 40)[0], ft_oracle.bwd_f32(padded, G, 40)[0])
    empty = np.full((3, 6), -1, np.int32)
    assert np.array_equal(ft_oracle.fwd_f32(empty, W, b), np.tile(b, (3, 1)))
    dW, db = ft_oracle.bwd_f32(empty, G[:3], 40)
    assert not dW.any()


def test_permutation_invariance_exact_values():
    g = np.random.default_rng(41)
    idx = workloads.make_indices(g, 30, 50, 8, 0, 8, sort=False)
    W = g.integers(-100, 100, size=(50, 7)).astype(np.float32)
    b = g.integers(-100, 100, size=7).astype(np.float32)
    perm = idx[:, g.permutation(8)]
    assert np.array_equal(ft_oracle.fwd_f32(idx, W, b), ft_oracle.fwd_f32(perm, W, b))


def test_linearity_in_weights():
    idx, W, b, _ = rand_case(51, 25, 30, 5, 6)
    W2 = np.random.default_rng(52).standard_normal(W.shape).astype(np.float32)
    z = np.zeros_like(b)
    lhs = ft_oracle.fwd_f64(idx, W + W2, z)
    rhs = ft_oracle.fwd_f64(idx, W, z) + ft_oracle.fwd_f64(idx, W2, z)
    assert np.allclose(lhs, rhs, rtol=0, atol=1e-5)


def test_bad_index_is_rejected():
    idx = np.array([[0, 5]], np.int32)
    W = np.zeros((5, 2), np.float32)
    with pytest.raises(ValueError):
        ft_oracle.fwd_f32(idx, W, np.zeros(2, np.float32))
    with pytest.raises(ValueError):
        ft_oracle.bwd_f32(idx, np.zeros((1, 2), np.float32), 5)


def test_quantize_matches_numpy_rint_and_torch_round():
    g = np.random.default_rng(61)
    x = (g.standard_normal(10000) * 0.05).astype(np.float32)
    for scale in (127.0, 255.0):
        q = ft_oracle.quantize_i16(x, scale)
        assert np.array_equal(q, workloads.quantize_np(x, scale))
        t = torch.from_numpy(x).mul(scale).round().to(torch.int16).numpy()
        assert np.array_equal(q, t)
