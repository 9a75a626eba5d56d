"""The exact step bench.py times, at full size, against the oracle.

Both perspectives through SparseLinearFunction (FT/functions.py:12-72): the
custom ops, with the backward's sort made under the forward when the library
prepares it (K >= L / 20: workloads 2 and 3), autograd summing the two weight
grads.  Forward outputs bit-exact with the ordered oracle (FT/kernel.py:93-100),
the summed weight grad bit-exact with the two reference-order weight grads
(FT/kernel.py:122,178-186) added in binary32, the bias grad within 1e-5 of
binary64 (FT/kernel.py:269).  Then the fused ComposedFeatureTransformer
(FEAT/composed.py:49-54) at B = 65 536 for both feature sets against the
composed oracle: outputs and block weight grads bit-exact, virtual and bias
grads within 1e-5 of binary64.  And the headline step over the index rows the
GPU encoder makes from random positions (bench.py's encoder-rows leg)."""

import numpy as np
import pytest
import torch

from gpu_helpers import DEV, announce, dev, dw_rel_err, host, rel_err
from oracle import composed_oracle, ft_oracle
from sft_amd import _native, workloads
from src.model.modules.feature_transformer import SparseLinearFunction
from src.model.modules.features import get_feature_cls

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("wid", [0, 1, 2, 3])
def test_sparse_linear_step_full_workload(wid):
    w = workloads.WORKLOADS[wid]
    prepared = _native.prep_buffer_bytes(w.B, w.K, w.N, w.L, _native.SFT_BWD_OVERWRITE, DEV) > 0
    announce(f"timed step {w.name} B={w.B} N={w.N} K={w.K} L={w.L} sort under the forward={prepared}")
    assert prepared == (wid in (2, 3))  # the path bench.py times for each workload
    d = workloads.make_fp32_inputs(w)
    iw, ib = dev(d["idx_w"]), dev(d["idx_b"])
    W = dev(d["W"]).requires_grad_(True)
    b = dev(d["bias"]).requires_grad_(True)
    ow = SparseLinearFunction.apply(iw, W, b)
    ob = SparseLinearFunction.apply(ib, W, b)
    torch.autograd.backward([ow, ob], [dev(d["g_w"]), dev(d["g_b"])])
    torch.cuda.synchronize()
    assert np.array_equal(host(ow), ft_oracle.fwd_f32(d["idx_w"], d["W"], d["bias"]))
    assert np.array_equal(host(ob), ft_oracle.fwd_f32(d["idx_b"], d["W"], d["bias"]))
    del ow, ob
    rw, _ = ft_oracle.bwd_f32(d["idx_w"], d["g_w"], w.N)
    rb, _ = ft_oracle.bwd_f32(d["idx_b"], d["g_b"], w.N)
    assert np.array_equal(host(W.grad), rw + rb)  # autograd adds the two dense grads in binary32
    db64 = d["g_w"].astype(np.float64).sum(0) + d["g_b"].astype(np.float64).sum(0)
    assert rel_err(host(b.grad), db64) <= 1e-5


@pytest.mark.parametrize("feature_set", ["HalfKAv2_hm", "Full_Threats+HalfKAv2_hm"])
def test_sparse_linear_step_encoder_rows(feature_set):
    """The step over the index rows the GPU encoder makes from random positions
    at B = 65 536, L = 1048: for HalfKAv2_hm bench.py's encoder-rows leg (one
    king bucket's rows per perspective, 2-32 active, -1 after them, over the
    encoder's 24 576-row table); for Full_Threats+HalfKAv2_hm the table-part
    forward and the sort under the forward over rows whose threats come by
    colour and piece, not by index (a fifth of them go back to an earlier
    table part)."""
    import dataclasses

    from sft_amd import encode, positions
    from src.model.modules.features.full_threats import FullThreats
    from src.model.modules.features.halfka_v2_hm import HalfKav2Hm

    threats = feature_set.startswith("Full_Threats")
    N = HalfKav2Hm.NUM_INPUTS + (FullThreats.NUM_INPUTS if threats else 0)
    w = dataclasses.replace(workloads.WORKLOADS[2 if threats else 1], N=N)
    boards, stm = positions.random_positions(w.B, seed=1)
    enc = encode.encode_batch(torch.from_numpy(boards).to(DEV), torch.from_numpy(stm).to(DEV), feature_set)
    iw, ib = enc["white"], enc["black"]
    niw, nib = host(iw), host(ib)
    K = niw.shape[1]
    prepared = _native.prep_buffer_bytes(w.B, K, N, w.L, _native.SFT_BWD_OVERWRITE, DEV) > 0
    announce(f"timed step {feature_set} encoder rows B={w.B} N={N} K={K} L={w.L} sort under the forward={prepared}")
    assert niw.max() < N and (niw >= 0).sum(1).min() >= 2
    assert prepared == threats
    g = np.random.default_rng(7)
    Wn = (g.standard_normal((N, w.L), dtype=np.float32) * 0.01).astype(np.float32)
    bn = g.standard_normal(w.L, dtype=np.float32)
    gw = g.standard_normal((w.B, w.L), dtype=np.float32)
    gb = g.standard_normal((w.B, w.L), dtype=np.float32)
    W = dev(Wn).requires_grad_(True)
    b = dev(bn).requires_grad_(True)
    ow = SparseLinearFunction.apply(iw, W, b)
    ob = SparseLinearFunction.apply(ib, W, b)
    torch.autograd.backward([ow, ob], [dev(gw), dev(gb)])
    torch.cuda.synchronize()
    assert np.array_equal(host(ow), ft_oracle.fwd_f32(niw, Wn, bn))
    assert np.array_equal(host(ob), ft_oracle.fwd_f32(nib, Wn, bn))
    del ow, ob
    rw, _ = ft_oracle.bwd_f32(niw, gw, N)
    rb, _ = ft_oracle.bwd_f32(nib, gb, N)
    assert np.array_equal(host(W.grad), rw + rb)
    db64 = gw.astype(np.float64).sum(0) + gb.astype(np.float64).sum(0)
    assert rel_err(host(b.grad), db64) <= 1e-5


@pytest.mark.parametrize("rows", ["uniform", "encoder"])
@pytest.mark.parametrize("name", ["HalfKAv2_hm^", "Full_Threats+HalfKAv2_hm^"])
def test_fused_module_full_batch_matches_composed_oracle(name, rows):
    """rows="encoder": the index rows the GPU encoder makes from random positions
    (for the composed set: threats by colour and piece, then HalfKAv2_hm offset
    by 60 720), the layout the module sees in training."""
    B, L = 65536, 1048
    announce(f"fused module {name} B={B} L={L} {rows} rows vs composed oracle")
    torch.manual_seed(5)
    ft = get_feature_cls(name)(L).to(DEV)
    assert ft.fused
    for f in ft.features:
        if hasattr(f, "virtual_weight"):
            with torch.no_grad():
                f.virtual_weight.normal_(0, 0.01)
    g = np.random.default_rng(65536 + len(name))
    K = ft.MAX_ACTIVE_FEATURES
    lo = 16 if K == 32 else 32
    if rows == "encoder":
        from sft_amd import encode, positions

        boards, stm = positions.random_positions(B, seed=5)
        enc = encode.encode_batch(torch.from_numpy(boards).to(DEV), torch.from_numpy(stm).to(DEV), name)
        iw, ib = host(enc["white"]), host(enc["black"])
        assert iw.shape == (B, K) and iw.max() < ft.NUM_INPUTS
        del enc
    else:
        iw = workloads.make_indices(g, B, ft.NUM_INPUTS, K, lo, K, sort=False)
        ib = workloads.make_indices(g, B, ft.NUM_INPUTS, K, lo, K, sort=True)
    gw = g.standard_normal((B, L), dtype=np.float32)
    gb = g.standard_normal((B, L), dtype=np.float32)
    ow, ob = ft(dev(iw), dev(ib))
    torch.autograd.backward([ow, ob], [dev(gw), dev(gb)])
    torch.cuda.synchronize()
    blocks = [(host(f.weight), host(f.virtual_weight) if hasattr(f, "virtual_weight") else None)
              for f in ft.features]
    bias = host(ft.bias)
    r0, r1 = composed_oracle.composed_fwd(iw, ib, blocks, bias)
    assert np.array_equal(host(ow), r0) and np.array_equal(host(ob), r1)
    del ow, ob, r0, r1
    rw, rv, rdb = composed_oracle.composed_bwd(iw, ib, gw, gb, blocks)
    for s, f in enumerate(ft.features):
        assert np.array_equal(host(f.weight.grad), rw[s]), s
        if rv[s] is not None:
            assert dw_rel_err(host(f.virtual_weight.grad), rv[s]) <= 1e-5, s
    assert rel_err(host(ft.bias.grad), rdb) <= 1e-5
