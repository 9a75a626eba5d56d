"""The composed-table oracle (two perspectives, virtual rows) against torch
autograd of the reference composition on the CPU.  Integer-valued tables make
every sum exact, so the comparison is bit-exact; each planted mistake must be
caught."""

import numpy as np
import pytest
import torch

from oracle import composed_oracle, ft_oracle


def _case(seed, R=12, P=4, R2=7, L=5, B=9, K=6, integer=True):
    g = np.random.default_rng(seed)
    draw = (lambda *s: g.integers(-8, 9, size=s).astype(np.float32)) if integer else \
        (lambda *s: g.standard_normal(s).astype(np.float32))
    w, v, w2, b = draw(R, L), draw(P, L), draw(R2, L), draw(L)
    N = R + R2
    idx = [np.full((B, K), -1, np.int32) for _ in range(2)]
    for t in idx:
        for r in range(B):
            n = g.integers(0, K + 1)
            t[r, :n] = g.choice(N, n, replace=False)
            t[r] = t[r][g.permutation(K)]  # -1 anywhere in the row
    g0, g1 = draw(B, L), draw(B, L)
    return [(w, v), (w2, None)], b, idx[0], idx[1], g0, g1


def _torch_reference(blocks, b, idx0, idx1, g0, g1):
    """The reference composition in torch autograd: cat of merged_weight, a
    masked row sum per perspective, backward of both outputs."""
    (w, v), (w2, _) = blocks
    tw, tv, tw2 = (torch.tensor(a, requires_grad=True) for a in (w, v, w2))
    tb = torch.tensor(b, requires_grad=True)
    merged = torch.cat([tw + tv.repeat(w.shape[0] // v.shape[0], 1), tw2])
    outs = []
    for idx in (idx0, idx1):
        t = torch.tensor(idx, dtype=torch.long)
        rows = merged[t.clamp(min=0)] * (t >= 0).unsqueeze(-1)
        outs.append(tb + rows.sum(1))
    torch.autograd.backward(outs, [torch.tensor(g0), torch.tensor(g1)])
    return [o.detach().numpy() for o in outs], tw.grad.numpy(), tv.grad.numpy(), tw2.grad.numpy(), tb.grad.numpy()


def _matches(seed, mutation=None):
    blocks, b, i0, i1, g0, g1 = _case(seed)
    (o0, o1), dw, dv, dw2, db = _torch_reference(blocks, b, i0, i1, g0, g1)
    r0, r1 = composed_oracle.composed_fwd(i0, i1, blocks, b, mutation)
    wg, vg, rdb = composed_oracle.composed_bwd(i0, i1, g0, g1, blocks, mutation)
    return (np.array_equal(r0, o0) and np.array_equal(r1, o1) and np.array_equal(wg[0], dw)
            and np.array_equal(wg[1], dw2) and np.array_equal(vg[0], dv) and vg[1] is None
            and np.array_equal(rdb, db))


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_composed_oracle_matches_torch_composition(seed):
    assert _matches(seed)


@pytest.mark.parametrize("mutation", composed_oracle.MUTATIONS)
def test_composed_checks_catch_mistakes(mutation):
    assert not any(_matches(s, mutation) for s in (0,)), mutation


def test_merged_table_rounds_once_like_torch():
    blocks, *_ = _case(5, integer=False)
    (w, v), (w2, _) = blocks
    ref = torch.cat([torch.tensor(w) + torch.tensor(v).repeat(3, 1), torch.tensor(w2)]).numpy()
    assert np.array_equal(composed_oracle.merged_table(blocks), ref)


def test_composed_fwd_is_the_plain_forward_on_the_merged_table():
    blocks, b, i0, i1, *_ = _case(6, integer=False)
    M = composed_oracle.merged_table(blocks)
    o0, o1 = composed_oracle.composed_fwd(i0, i1, blocks, b)
    assert np.array_equal(o0, ft_oracle.fwd_f32(i0, M, b)) and np.array_equal(o1, ft_oracle.fwd_f32(i1, M, b))
