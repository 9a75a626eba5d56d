"""PyTorch-CPU restatement of the FT step, used as the benchmark's CPU baseline.

TEST INFRASTRUCTURE ONLY (the benchmark's cpu_baseline leg).  The reference
has no CPU FT (its op asserts CUDA, FT/functions.py:21-23), so this restates
its semantics with library routines: per perspective
`embedding_bag(valid indices, W, offsets, mode="sum") + b` forward, and autograd
of the same for a dense weight grad plus the bias grad (FT/kernel.py:269),
summed over both perspectives like the reference's shared-parameter autograd.
"""

from __future__ import annotations

import numpy as np
import torch


def _bag_inputs(idx: np.ndarray):
    t = torch.from_numpy(idx.astype(np.int64))
    mask = t >= 0
    flat = t[mask]
    counts = mask.sum(1)
    offsets = torch.zeros_like(counts)
    offsets[1:] = counts.cumsum(0)[:-1]
    return flat, offsets


class CpuFtStep:
    """One fwd+bwd step of both perspectives on the CPU (float32)."""

    def __init__(self, idx_w, idx_b, W, bias, g_w, g_b):
        self.bw = _bag_inputs(idx_w)
        self.bb = _bag_inputs(idx_b)
        self.W = torch.from_numpy(np.ascontiguousarray(W)).requires_grad_(True)
        self.b = torch.from_numpy(np.ascontiguousarray(bias)).requires_grad_(True)
        self.gw = torch.from_numpy(np.ascontiguousarray(g_w))
        self.gb = torch.from_numpy(np.ascontiguousarray(g_b))

    def __call__(self):
        self.W.grad = None
        self.b.grad = None
        ow = torch.nn.functional.embedding_bag(self.bw[0], self.W, self.bw[1], mode="sum") + self.b
        ob = torch.nn.functional.embedding_bag(self.bb[0], self.W, self.bb[1], mode="sum") + self.b
        torch.autograd.backward([ow, ob], [self.gw, self.gb])
        return ow, ob
