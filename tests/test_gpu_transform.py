"""Composed table + post-FT epilogue (sft_ft_fwd_transform_f32 /
sft_ft_bwd_transform_f32) on the GPU: l0, psqt and the table grads bit-exact
against the composed and epilogue oracles, virtual and bias grads within 1e-5
of binary64, and the fused transform against the reference ops on the GPU."""

import numpy as np
import pytest
import torch

from gpu_helpers import DEV, announce, dev, dw_rel_err, host, rel_err
from oracle import composed_oracle, epilogue_oracle
from sft_amd import _native, workloads
from src.model.modules.features import get_feature_cls
from src.model.transform_inputs import transform_inputs

pytestmark = pytest.mark.gpu


def _bits(a):
    return np.asarray(a, np.float32).view(np.uint32)


SHAPES = [
    # seed, B, K, L1, P, lo, hi, blocks [(rows, virtual rows)]
    (1, 333, 40, 256, 8, 0, 40, [(3072, 96), (700, 0)]),
    (2, 1, 32, 256, 8, 1, 32, [(3072, 768)]),
    (3, 1000, 32, 1040, 8, 16, 32, [(2000, 0)]),                          # half of L1 = 130 chunks
    (4, 257, 24, 248, 12, 0, 24, [(960, 32), (500, 0), (64, 16), (100, 0)]),  # partial paired and PSQT tiles
    (5, 2048, 160, 1040, 8, 32, 160, [(6072, 0), (3072, 768)]),
    (6, 6000, 32, 512, 8, 16, 32, [(40, 8), (24, 0)]),  # 64 rows, one position chunk: every segment long
    (7, 40000, 32, 512, 8, 16, 32, [(40, 8), (24, 0)]),  # two position chunks: long segments in both
    (8, 40000, 32, 512, 8, 16, 32, [(3072, 96), (700, 0)]),  # two chunks, Zipf-skewed: hot and short segments
]
ZIPF = {8: 1.0}  # seeds whose rows draw features with skewed frequencies


def _indices(g, seed, B, N, K, lo, hi, sort):
    if seed in ZIPF:
        return workloads.make_zipf_indices(g, B, N, K, lo, hi, ZIPF[seed], sort=sort)
    return workloads.make_indices(g, B, N, K, lo, hi, sort=sort)


@pytest.mark.parametrize("seed,B,K,L1,P,lo,hi,spec", SHAPES)
def test_transform_matches_oracles(seed, B, K, L1, P, lo, hi, spec):
    announce(f"transform seed={seed} B={B} K={K} L1={L1} P={P} blocks={spec}")
    g = np.random.default_rng(seed)
    L = L1 + P
    N = sum(r for r, _ in spec)
    idx0 = _indices(g, seed, B, N, K, lo, hi, sort=False)
    idx1 = _indices(g, seed, B, N, K, lo, hi, sort=True)
    # weights around the clamp window so that every branch of the epilogue occurs
    blocks = [((g.standard_normal((R, L)) * 0.1).astype(np.float32),
               (g.standard_normal((V, L)) * 0.05).astype(np.float32) if V else None) for R, V in spec]
    bias = g.uniform(0.0, 0.6, L).astype(np.float32)
    us = g.integers(0, 2, B).astype(np.float32)
    k = g.integers(0, P, B).astype(np.int64)
    bad = [r for r in (5, 6) if r < B]
    k_dev = k.copy()
    if bad:
        k_dev[bad[0]] = P          # outside [0, P): psqt 0, no PSQT grad
    if len(bad) > 1:
        k_dev[bad[1]] = -1
    g_l0 = g.standard_normal((B, L1)).astype(np.float32)
    g_psqt = g.standard_normal(B).astype(np.float32)

    tw = [dev(w) for w, _ in blocks]
    tv = [None if v is None else dev(v) for _, v in blocks]
    l0 = torch.full((B, L1), float("nan"), device=DEV)
    psqt = torch.full((B,), float("nan"), device=DEV)
    saved = _native.ft_fwd_transform_f32(dev(idx0), dev(idx1), tw, tv, dev(bias), dev(us), dev(k_dev), L1, l0, psqt)
    dw = [torch.full_like(t, float("nan")) for t in tw]
    dv = [None if t is None else torch.full_like(t, float("nan")) for t in tv]
    db = torch.full((L,), float("nan"), device=DEV)
    _native.ft_bwd_transform_f32(dev(idx0), dev(idx1), dev(g_l0), dev(g_psqt), dev(us), dev(k_dev), saved, L1, dw,
                                 dv, db)
    torch.cuda.synchronize()

    xw, xb = composed_oracle.composed_fwd(idx0, idx1, blocks, bias)
    rl0, rpsqt = epilogue_oracle.fwd(xw, xb, us, k, L1)
    dxw, dxb = epilogue_oracle.bwd(xw, xb, us, k, L1, g_l0, g_psqt)
    rpsqt = rpsqt.reshape(-1)
    for r in bad:
        rpsqt[r] = 0.0
        dxw[r, L1:] = 0.0
        dxb[r, L1:] = 0.0
    assert np.array_equal(_bits(host(l0)), _bits(rl0))
    assert np.array_equal(_bits(host(psqt)), _bits(rpsqt))
    rw, rv, rdb = composed_oracle.composed_bwd(idx0, idx1, dxw, dxb, blocks)
    for s in range(len(spec)):
        assert np.array_equal(host(dw[s]), rw[s]), s
        if rv[s] is not None:
            assert dw_rel_err(host(dv[s]), rv[s]) <= 1e-5, s
    assert rel_err(host(db), rdb) <= 1e-5


def _step(ft, l1, us, iw, ib, k, g_l0, g_psqt, fused):
    for p in ft.parameters():
        p.grad = None
    l0, psqt = transform_inputs(ft, l1, us, iw, ib, k, fused=fused)
    torch.autograd.backward([l0, psqt], [g_l0, g_psqt])
    torch.cuda.synchronize()
    return l0.detach(), psqt.detach(), {n: p.grad.detach().clone() for n, p in ft.named_parameters()}


@pytest.mark.parametrize("name,B", [("HalfKAv2_hm^", 4096), ("Full_Threats+HalfKAv2_hm^", 1500),
                                    ("HalfKAv2_hm^", 65536), ("Full_Threats+HalfKAv2_hm^", 65536)])
def test_fused_transform_equals_reference_ops(name, B):
    announce(f"transform module {name} B={B} fused vs reference ops")
    L1, P = 1040, 8
    torch.manual_seed(4)
    ft = get_feature_cls(name)(L1 + P).to(DEV)
    with torch.no_grad():
        for f in ft.features:
            f.weight.normal_(0, 0.05)
            if hasattr(f, "virtual_weight"):
                f.virtual_weight.normal_(0, 0.02)
        ft.bias.uniform_(0.0, 0.6)
    g = np.random.default_rng(B + 1)
    K = ft.MAX_ACTIVE_FEATURES
    lo = 16 if K == 32 else 32
    iw = dev(workloads.make_indices(g, B, ft.NUM_INPUTS, K, lo, K))
    ib = dev(workloads.make_indices(g, B, ft.NUM_INPUTS, K, lo, K))
    us = dev(g.integers(0, 2, (B, 1)).astype(np.float32))
    k = dev(g.integers(0, P, B).astype(np.int64))
    g_l0 = torch.randn(B, L1, device=DEV)
    g_psqt = torch.randn(B, 1, device=DEV)
    fl0, fps, fg = _step(ft, L1, us, iw, ib, k, g_l0, g_psqt, True)
    rl0, rps, rg = _step(ft, L1, us, iw, ib, k, g_l0, g_psqt, False)
    assert torch.equal(fl0, rl0) and torch.equal(fps, rps)
    for n in fg:
        if n.endswith("virtual_weight") or n == "bias":
            ref = rg[n].double()
            err = ((fg[n].double() - ref).abs().amax(dim=-1) / ref.abs().amax(dim=-1).clamp_min(1e-30)).max().item()
            assert err <= 1e-5, (n, err)
        else:
            assert torch.equal(fg[n], rg[n]), n


@pytest.mark.parametrize("name", ["HalfKAv2_hm^", "Full_Threats+HalfKAv2_hm^"])
def test_transform_encoder_batch_matches_oracles(name):
    """The trainer's data flow end to end: the GPU encoder makes the index rows,
    side to move and PSQT bucket of random positions, and the fused epilogue op
    runs on them over the module's tables (B = 16 384, L1 = 1040, 8 PSQT
    buckets).  l0 and psqt bit-exact, table grads bit-exact, virtual and bias
    grads within 1e-5 of binary64, against the composed and epilogue oracles."""
    from sft_amd import encode, positions

    B, L1, P = 16384, 1040, 8
    L = L1 + P
    announce(f"transform over encoder rows {name} B={B}")
    boards, stm = positions.random_positions(B, seed=9)
    enc = encode.encode_batch(torch.from_numpy(boards).to(DEV), torch.from_numpy(stm).to(DEV), name)
    idx0, idx1 = host(enc["white"]), host(enc["black"])
    us = host(enc["us"]).reshape(-1).astype(np.float32)
    k = host(enc["psqt_indices"]).astype(np.int64)
    assert set(np.unique(us)) <= {0.0, 1.0} and k.min() >= 0 and k.max() < P
    torch.manual_seed(9)
    ft = get_feature_cls(name)(L).to(DEV)
    g = np.random.default_rng(9)
    blocks = []
    for f in ft.features:
        w = (g.standard_normal(tuple(f.weight.shape)) * 0.1).astype(np.float32)
        v = (g.standard_normal(tuple(f.virtual_weight.shape)) * 0.05).astype(np.float32) \
            if hasattr(f, "virtual_weight") else None
        blocks.append((w, v))
    bias = g.uniform(0.0, 0.6, L).astype(np.float32)
    g_l0 = g.standard_normal((B, L1)).astype(np.float32)
    g_psqt = g.standard_normal(B).astype(np.float32)

    tw = [dev(w) for w, _ in blocks]
    tv = [None if v is None else dev(v) for _, v in blocks]
    l0 = torch.full((B, L1), float("nan"), device=DEV)
    psqt = torch.full((B,), float("nan"), device=DEV)
    saved = _native.ft_fwd_transform_f32(enc["white"], enc["black"], tw, tv, dev(bias), dev(us), enc["psqt_indices"],
                                         L1, l0, psqt)
    dw = [torch.full_like(t, float("nan")) for t in tw]
    dv = [None if t is None else torch.full_like(t, float("nan")) for t in tv]
    db = torch.full((L,), float("nan"), device=DEV)
    _native.ft_bwd_transform_f32(enc["white"], enc["black"], dev(g_l0), dev(g_psqt), dev(us), enc["psqt_indices"],
                                 saved, L1, dw, dv, db)
    torch.cuda.synchronize()

    xw, xb = composed_oracle.composed_fwd(idx0, idx1, blocks, bias)
    rl0, rpsqt = epilogue_oracle.fwd(xw, xb, us, k, L1)
    assert np.array_equal(_bits(host(l0)), _bits(rl0))
    assert np.array_equal(_bits(host(psqt)), _bits(rpsqt.reshape(-1)))
    dxw, dxb = epilogue_oracle.bwd(xw, xb, us, k, L1, g_l0, g_psqt)
    rw, rv, rdb = composed_oracle.composed_bwd(idx0, idx1, dxw, dxb, blocks)
    for s in range(len(blocks)):
        assert np.array_equal(host(dw[s]), rw[s]), s
        if rv[s] is not None:
            assert dw_rel_err(host(dv[s]), rv[s]) <= 1e-5, s
    assert rel_err(host(db), rdb) <= 1e-5
