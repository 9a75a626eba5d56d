"""The FT step captured in a HIP graph: the library makes no host
synchronisation, allocation or memset inside its calls, so a whole
forward + backward of both perspectives can be captured (torch.cuda.CUDAGraph)
and replayed.  Each replay, with eager work and synchronisation between
replays, must reproduce the eager results bit for bit."""

import numpy as np
import pytest
import torch

from gpu_helpers import DEV, announce, case, dev
from src.model.modules.feature_transformer import SparseLinearFunction
from src.model.modules.features import get_feature_cls
from src.model.transform_inputs import transform_inputs
from sft_amd import workloads

pytestmark = pytest.mark.gpu


def _capture_and_compare(step, outputs, replays=3):
    """step() runs the work and returns the tensors to compare; it is run once
    eagerly (reference), warmed up on a side stream, captured, and replayed."""
    ref = [t.detach().clone() for t in step()]
    torch.cuda.synchronize()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for _ in range(2):
            step()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        static = step()
    noise = torch.randn(1 << 20, device=DEV)
    for r in range(replays):
        noise.mul_(1.0001).add_(1.0)  # eager work between the replays
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        for a, b in zip(static, ref):
            assert torch.equal(a, b), f"replay {r}"


def test_graph_two_perspectives_slf():
    announce("graph: SparseLinearFunction fwd+bwd both perspectives")
    B, N, K, L = 4096, 2000, 32, 1048
    iw, W, b, Gw = case(31, B, N, K, L)
    ib, _, _, Gb = case(32, B, N, K, L)
    iw_t, ib_t, gw, gb = dev(iw), dev(ib), dev(Gw), dev(Gb)
    Wt = dev(W).requires_grad_(True)
    bt = dev(b).requires_grad_(True)

    def step():
        Wt.grad = None
        bt.grad = None
        ow = SparseLinearFunction.apply(iw_t, Wt, bt)
        ob = SparseLinearFunction.apply(ib_t, Wt, bt)
        torch.autograd.backward([ow, ob], [gw, gb])
        return [ow, ob, Wt.grad, bt.grad]

    _capture_and_compare(step, 4)


@pytest.mark.parametrize("L", [1048, 136])
def test_graph_skewed_segments(L):
    """Long segments (listed by the segment pass with atomics, summed by the
    gathers' long-segment workgroups) replay bit-identically."""
    announce(f"graph: SparseLinearFunction fwd+bwd, skewed feature frequencies, L={L}")
    B, N, K = 6000, 3000, 32
    g = np.random.default_rng(41)
    iw_t = dev(workloads.make_zipf_indices(g, B, N, K, 16, 32, alpha=1.0))
    ib_t = dev(workloads.make_zipf_indices(g, B, N, K, 16, 32, alpha=1.0))
    Wt = dev((g.standard_normal((N, L)) * 0.01).astype(np.float32)).requires_grad_(True)
    bt = dev(g.uniform(-0.1, 0.1, L).astype(np.float32)).requires_grad_(True)
    gw = dev(g.standard_normal((B, L)).astype(np.float32))
    gb = dev(g.standard_normal((B, L)).astype(np.float32))

    def step():
        Wt.grad = None
        bt.grad = None
        ow = SparseLinearFunction.apply(iw_t, Wt, bt)
        ob = SparseLinearFunction.apply(ib_t, Wt, bt)
        torch.autograd.backward([ow, ob], [gw, gb])
        return [ow, ob, Wt.grad, bt.grad]

    _capture_and_compare(step, 4)


def test_graph_fused_transform():
    announce("graph: fused composed transform fwd+bwd")
    B, L1 = 2048, 1040
    torch.manual_seed(5)
    ft = get_feature_cls("HalfKAv2_hm^")(L1 + 8).to(DEV)
    with torch.no_grad():
        ft.features[0].weight.normal_(0, 0.05)
        ft.features[0].virtual_weight.normal_(0, 0.02)
        ft.bias.uniform_(0.0, 0.6)
    g = np.random.default_rng(9)
    iw = dev(workloads.make_indices(g, B, 24576, 32, 16, 32))
    ib = dev(workloads.make_indices(g, B, 24576, 32, 16, 32))
    us = dev(g.integers(0, 2, (B, 1)).astype(np.float32))
    k = dev(g.integers(0, 8, B).astype(np.int64))
    gl = torch.randn(B, L1, device=DEV)
    gp = torch.randn(B, 1, device=DEV)

    def step():
        for p in ft.parameters():
            p.grad = None
        l0, psqt = transform_inputs(ft, L1, us, iw, ib, k)
        torch.autograd.backward([l0, psqt], [gl, gp])
        return [l0, psqt] + [p.grad for p in ft.parameters()]

    _capture_and_compare(step, 0)


def test_graph_fused_composed():
    """The fused two-perspective op (ComposedSparseLinearFunction) at a batch
    whose backward runs two position chunks: the side-stream sorts, each
    perspective's bias pass before its gathers and the second perspective's
    sum onto the first all capture and replay bit for bit."""
    announce("graph: fused composed fwd+bwd, two position chunks")
    B = 34000
    torch.manual_seed(6)
    ft = get_feature_cls("HalfKAv2_hm^")(1048).to(DEV)
    with torch.no_grad():
        ft.features[0].weight.normal_(0, 0.05)
        ft.features[0].virtual_weight.normal_(0, 0.02)
    assert ft.fused
    g = np.random.default_rng(10)
    iw = dev(workloads.make_indices(g, B, 24576, 32, 16, 32))
    ib = dev(workloads.make_indices(g, B, 24576, 32, 16, 32, sort=False))
    gw = torch.randn(B, 1048, device=DEV)
    gb = torch.randn(B, 1048, device=DEV)

    def step():
        for p in ft.parameters():
            p.grad = None
        ow, ob = ft(iw, ib)
        torch.autograd.backward([ow, ob], [gw, gb])
        return [ow, ob] + [p.grad for p in ft.parameters()]

    _capture_and_compare(step, 0)
