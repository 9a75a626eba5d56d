"""Shared helpers of the GPU parity tests (inputs, device transfer, checks)."""

import sys

import numpy as np
import torch

from oracle import ft_oracle
from sft_amd import workloads

DEV = torch.device("cuda:0")


def announce(msg: str) -> None:
    print(f"[case] {msg}", flush=True)
    sys.stdout.flush()


def dev(a: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a)).to(DEV)


def host(t: torch.Tensor) -> np.ndarray:
    return t.detach().cpu().numpy()


def case(seed, B, N, K, L, lo=0, hi=None, sort=False, holes=True):
    g = np.random.default_rng(seed)
    idx = workloads.make_indices(g, B, N, K, lo, K if hi is None else hi, sort=sort)
    if holes and B > 2 and K > 2:
        idx[1, 0] = -1  # interior hole
        idx[2, :] = -1  # all inactive
    W = (g.standard_normal((N, L)) * 0.01).astype(np.float32)
    b = g.uniform(-0.1, 0.1, L).astype(np.float32)
    G = g.standard_normal((B, L)).astype(np.float32)
    return idx, W, b, G


def rel_err(y, y_ref) -> float:
    return ft_oracle.rownorm_rel_err(y, y_ref)


def dw_rel_err(dW, ref64) -> float:
    """max over rows with a nonzero reference of ||dW_f - ref_f||_inf / ||ref_f||_inf;
    rows whose reference is exactly zero must be exactly zero."""
    ref64 = np.asarray(ref64, np.float64)
    dW = np.asarray(dW, np.float64)
    nz = np.abs(ref64).max(axis=1) > 0
    if np.any(dW[~nz] != 0):
        return float("inf")
    return rel_err(dW[nz], ref64[nz]) if nz.any() else 0.0
