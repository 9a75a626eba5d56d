"""The post-FT epilogue oracle against torch autograd of the reference ops
(src/model/model.py:86-115) on the CPU: bit-exact forward and backward,
including pre-activations exactly at the clamp bounds; each planted mistake
must be caught."""

import numpy as np
import pytest
import torch

from oracle import epilogue_oracle


def _case(seed, B=37, l1=16, P=8):
    g = np.random.default_rng(seed)
    L = l1 + P
    xw = g.uniform(-0.5, 1.5, (B, L)).astype(np.float32)
    xb = g.uniform(-0.5, 1.5, (B, L)).astype(np.float32)
    for x in (xw, xb):  # exact bounds and values just outside them
        x[0, :4] = [0.0, 1.0, -1e-8, 1.0000001]
        x[1, l1 // 2:l1 // 2 + 4] = [1.0, 0.0, 0.5, -0.0]
    us = g.integers(0, 2, (B, 1)).astype(np.float32)
    k = g.integers(0, P, B).astype(np.int64)
    g_l0 = g.standard_normal((B, l1)).astype(np.float32)
    g_psqt = g.standard_normal((B, 1)).astype(np.float32)
    return xw, xb, us, k, l1, g_l0, g_psqt


def _torch(xw, xb, us, k, l1, g_l0, g_psqt):
    tw = torch.tensor(xw, requires_grad=True)
    tb = torch.tensor(xb, requires_grad=True)
    tus, tk = torch.tensor(us), torch.tensor(k)
    w, wpsqt = torch.split(tw, l1, dim=1)
    b, bpsqt = torch.split(tb, l1, dim=1)
    half = l1 // 2
    side = tus.bool()
    wc = torch.clamp(w, 0.0, 1.0).reshape(-1, 2, half)
    bc = torch.clamp(b, 0.0, 1.0).reshape(-1, 2, half)
    wpw = wc[:, 0, :] * wc[:, 1, :]
    bpw = bc[:, 0, :] * bc[:, 1, :]
    l0 = torch.cat([torch.where(side, wpw, bpw), torch.where(side, bpw, wpw)], dim=1) * (127 / 128)
    kk = tk.unsqueeze(1)
    psqt = (wpsqt.gather(1, kk) - bpsqt.gather(1, kk)) * (tus - 0.5)
    torch.autograd.backward([l0, psqt], [torch.tensor(g_l0), torch.tensor(g_psqt)])
    return l0.detach().numpy(), psqt.detach().numpy(), tw.grad.numpy(), tb.grad.numpy()


def _bits(a):
    return np.asarray(a, np.float32).view(np.uint32)


def _matches(seed, mutation=None):
    c = _case(seed)
    l0, psqt, dw, db = _torch(*c)
    ol0, opsqt = epilogue_oracle.fwd(*c[:5], mutation=mutation)
    odw, odb = epilogue_oracle.bwd(*c, mutation=mutation)
    # compare bit patterns: also pins the sign of zero grads
    return all(np.array_equal(_bits(a), _bits(b)) for a, b in ((l0, ol0), (psqt, opsqt), (dw, odw), (db, odb)))


@pytest.mark.parametrize("seed", [0, 1, 2, 3])
def test_epilogue_oracle_matches_torch_autograd(seed):
    assert _matches(seed)


@pytest.mark.parametrize("mutation", epilogue_oracle.MUTATIONS)
def test_epilogue_checks_catch_mistakes(mutation):
    assert not _matches(0, mutation)
