"""Composed table, both perspectives (sft_ft_fwd_pair_f32 / sft_ft_bwd_pair_f32)
on the GPU: against the composed oracle (outputs and block weight grads
bit-exact, virtual and bias grads within 1e-5 of binary64), and the fused
module against the reference composition on the same kernels (bit-identical
outputs and weight grads)."""

import numpy as np
import pytest
import torch

from gpu_helpers import DEV, announce, dev, dw_rel_err, host, rel_err
from oracle import composed_oracle
from sft_amd import _native, workloads
from src.model.modules.features import get_feature_cls

pytestmark = pytest.mark.gpu


def _blocks(g, spec, L):
    out = []
    for R, V in spec:
        w = (g.standard_normal((R, L)) * 0.01).astype(np.float32)
        v = (g.standard_normal((V, L)) * 0.01).astype(np.float32) if V else None
        out.append((w, v))
    return out


def _run_pair(idx0, idx1, blocks, b, g0, g1):
    tw = [dev(w) for w, _ in blocks]
    tv = [None if v is None else dev(v) for _, v in blocks]
    B, L = idx0.shape[0], b.shape[0]
    o0 = torch.full((B, L), float("nan"), device=DEV)
    o1 = torch.full((B, L), float("nan"), device=DEV)
    _native.ft_fwd_pair_f32(dev(idx0), dev(idx1), tw, tv, dev(b), o0, o1)
    dw = [torch.full_like(t, float("nan")) for t in tw]
    dv = [None if t is None else torch.full_like(t, float("nan")) for t in tv]
    db = torch.full((L,), float("nan"), device=DEV)
    _native.ft_bwd_pair_f32(dev(idx0), dev(idx1), dev(g0), dev(g1), dw, dv, db)
    torch.cuda.synchronize()
    return host(o0), host(o1), [host(t) for t in dw], [None if t is None else host(t) for t in dv], host(db)


SHAPES = [
    # seed, B, K, L, lo, hi, blocks [(rows, virtual rows)]
    (1, 333, 40, 264, 0, 40, [(3072, 96), (700, 0)]),
    (2, 1, 32, 256, 1, 32, [(3072, 768)]),              # one position: a single position chunk
    (3, 1000, 32, 1048, 16, 32, [(2000, 0)]),           # no virtual rows
    (4, 257, 24, 260, 0, 24, [(960, 32), (500, 0), (64, 16), (100, 0)]),  # four blocks, partial last tile
    (5, 2048, 160, 1048, 32, 160, [(6072, 0), (3072, 768)]),  # threats-shaped composition
    (6, 6000, 32, 520, 16, 32, [(40, 8), (24, 0)]),  # 64 rows, one position chunk: every segment long
    (7, 40000, 32, 520, 16, 32, [(40, 8), (24, 0)]),  # two position chunks: long segments in both
    (8, 40000, 32, 520, 16, 32, [(3072, 96), (700, 0)]),  # two chunks, Zipf-skewed: hot and short segments
]
ZIPF = {8: 1.0}  # seeds whose rows draw features with skewed frequencies


def _indices(g, seed, B, N, K, lo, hi, sort):
    if seed in ZIPF:
        return workloads.make_zipf_indices(g, B, N, K, lo, hi, ZIPF[seed], sort=sort)
    return workloads.make_indices(g, B, N, K, lo, hi, sort=sort)


@pytest.mark.parametrize("seed,B,K,L,lo,hi,spec", SHAPES)
def test_pair_matches_composed_oracle(seed, B, K, L, lo, hi, spec):
    announce(f"pair seed={seed} B={B} K={K} L={L} blocks={spec}")
    g = np.random.default_rng(seed)
    N = sum(r for r, _ in spec)
    idx0 = _indices(g, seed, B, N, K, lo, hi, sort=False)
    idx1 = _indices(g, seed, B, N, K, lo, hi, sort=True)
    if B > 3:
        idx0[1, 0] = -1
        idx1[2, :] = -1
    blocks = _blocks(g, spec, L)
    b = g.uniform(-0.1, 0.1, L).astype(np.float32)
    g0 = g.standard_normal((B, L)).astype(np.float32)
    g1 = g.standard_normal((B, L)).astype(np.float32)
    o0, o1, dw, dv, db = _run_pair(idx0, idx1, blocks, b, g0, g1)
    r0, r1 = composed_oracle.composed_fwd(idx0, idx1, blocks, b)
    assert np.array_equal(o0, r0) and np.array_equal(o1, r1)
    rw, rv, rdb = composed_oracle.composed_bwd(idx0, idx1, g0, g1, blocks)
    for s in range(len(spec)):
        assert np.array_equal(dw[s], rw[s]), s
        if rv[s] is None:
            assert dv[s] is None
        else:
            assert dw_rel_err(dv[s], rv[s]) <= 1e-5, s
    assert rel_err(db, rdb) <= 1e-5


def test_pair_empty_batch_zeroes_the_grads():
    announce("pair B=0")
    g = np.random.default_rng(7)
    blocks = _blocks(g, [(768 * 2, 768), (100, 0)], 256)
    idx = np.zeros((0, 32), np.int32)
    G = np.zeros((0, 256), np.float32)
    b = g.uniform(-0.1, 0.1, 256).astype(np.float32)
    o0, o1, dw, dv, db = _run_pair(idx, idx, blocks, b, G, G)
    assert o0.shape == (0, 256)
    assert all(not d.any() for d in dw) and not dv[0].any() and dv[1] is None and not db.any()


def test_pair_all_inactive_rows():
    announce("pair all -1")
    g = np.random.default_rng(8)
    blocks = _blocks(g, [(768 * 2, 768)], 264)
    B = 50
    idx = np.full((B, 32), -1, np.int32)
    b = g.uniform(-0.1, 0.1, 264).astype(np.float32)
    g0 = g.standard_normal((B, 264)).astype(np.float32)
    o0, o1, dw, dv, db = _run_pair(idx, idx, blocks, b, g0, g0)
    assert np.array_equal(o0, np.broadcast_to(b, (B, 264))) and np.array_equal(o1, o0)
    assert not dw[0].any() and not dv[0].any()
    assert rel_err(db, 2 * g0.astype(np.float64).sum(0)) <= 1e-5


def _module_step(ft, iw, ib, gw, gb, fused):
    ft.fused = fused
    for p in ft.parameters():
        p.grad = None
    ow, ob = ft(iw, ib)
    torch.autograd.backward([ow, ob], [gw, gb])
    torch.cuda.synchronize()
    return ow.detach(), ob.detach(), {n: p.grad.detach().clone() for n, p in ft.named_parameters()}


@pytest.mark.parametrize("name,B,L", [("HalfKAv2_hm^", 4096, 1048), ("Full_Threats+HalfKAv2_hm^", 1500, 520),
                                      ("HalfKAv2_hm^", 65536, 1048), ("Full_Threats+HalfKAv2_hm^", 65536, 1048)])
def test_fused_module_equals_reference_composition(name, B, L):
    announce(f"module {name} B={B} L={L} fused vs composed")
    torch.manual_seed(3)
    ft = get_feature_cls(name)(L).to(DEV)
    for f in ft.features:
        if hasattr(f, "virtual_weight"):
            with torch.no_grad():
                f.virtual_weight.normal_(0, 0.01)
    g = np.random.default_rng(B)
    K, lo = ft.MAX_ACTIVE_FEATURES, (16 if ft.MAX_ACTIVE_FEATURES == 32 else 32)
    iw = dev(workloads.make_indices(g, B, ft.NUM_INPUTS, K, lo, K))
    ib = dev(workloads.make_indices(g, B, ft.NUM_INPUTS, K, lo, K))
    gw = torch.randn(B, L, device=DEV)
    gb = torch.randn(B, L, device=DEV)
    fw, fb, fg = _module_step(ft, iw, ib, gw, gb, True)
    uw, ub, ug = _module_step(ft, iw, ib, gw, gb, False)
    assert torch.equal(fw, uw) and torch.equal(fb, ub)
    for n in fg:
        if n.endswith("virtual_weight") or n == "bias":
            ref = ug[n].double()
            err = ((fg[n].double() - ref).abs().amax(dim=-1) / ref.abs().amax(dim=-1).clamp_min(1e-30)).max().item()
            assert err <= 1e-5, (n, err)
        else:
            assert torch.equal(fg[n], ug[n]), n
