"""Sparse-input linear forward/backward kernels, backed by libsft_ft.so.

Same factory surface as the reference module
(src/model/modules/feature_transformer/kernel.py:286-319): per (K, L) a cached
callable; batch size and table rows stay dynamic.  The TileLang JIT, its
autotuner and the torch-side sort prep (kernel.py:17-45, 48-63, 108-138,
191-283) are replaced by hand-written gfx950 HIP kernels behind a C ABI
(include/sft_ft.h); launch shapes are chosen per call from L, so there is no
first-call autotune and no main-thread requirement.
"""

from __future__ import annotations

import os
import sys
from collections.abc import Callable

import torch

_PKG_ROOT = os.path.abspath(os.path.join(os.path.dirname(__file__), "..", "..", "..", ".."))
if _PKG_ROOT not in sys.path:
    sys.path.insert(0, _PKG_ROOT)

from sft_amd import _native  # noqa: E402

SparseInputLinearForwardKernel = Callable[
    [torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor], None
]
# (input_indices, weight_grad, bias_grad, output_grad).  The reference alias
# lists six tensors (kernel.py:12-14), but its callable takes these four.
SparseInputLinearBackwardKernel = Callable[
    [torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor], None
]


class _ForwardKernel:
    """fwd(input_indices, weight, bias, output): output[b] = bias + sum_k weight[idx[b, k]].

    Overwrites `output`; -1 slots are skipped wherever they are
    (reference kernel.py:89-103).
    """

    def __init__(self, max_active_indices: int, output_size: int):
        self._max_active_indices = max_active_indices
        self._output_size = output_size

    def __call__(self, input_indices: torch.Tensor, weight: torch.Tensor, bias: torch.Tensor,
                 output: torch.Tensor) -> None:
        if input_indices.shape[1] != self._max_active_indices:
            raise ValueError(f"kernel built for {self._max_active_indices} active slots, "
                             f"got indices of shape {tuple(input_indices.shape)}")
        if weight.shape[1] != self._output_size:
            raise ValueError(f"kernel built for output size {self._output_size}, got weight {tuple(weight.shape)}")
        _native.ft_fwd_f32(input_indices, weight, bias, output)


class _BackwardKernel:
    """bwd(input_indices, weight_grad, bias_grad, output_grad).

    Accumulates like the reference (kernel.py:255-283): weight_grad[f] += sum of
    output_grad rows whose index row holds f (ascending position order),
    bias_grad += output_grad.sum(0).  With accumulate=False both grads are
    overwritten instead (rows of absent features become 0), which lets the
    caller skip the zero-fill.
    """

    def __init__(self, max_active_indices: int, output_size: int):
        self._max_active_indices = max_active_indices
        self._output_size = output_size

    def __call__(self, input_indices: torch.Tensor, weight_grad: torch.Tensor, bias_grad: torch.Tensor,
                 output_grad: torch.Tensor, *, accumulate: bool = True, atomic: bool = False) -> None:
        if input_indices.shape[1] != self._max_active_indices:
            raise ValueError(f"kernel built for {self._max_active_indices} active slots, "
                             f"got indices of shape {tuple(input_indices.shape)}")
        if weight_grad.shape[1] != self._output_size:
            raise ValueError(f"kernel built for output size {self._output_size}, "
                             f"got weight_grad {tuple(weight_grad.shape)}")
        flags = (_native.SFT_BWD_ACCUMULATE if accumulate else _native.SFT_BWD_OVERWRITE)
        if atomic:
            flags |= _native.SFT_BWD_ATOMIC
        _native.ft_bwd_f32(input_indices, weight_grad, bias_grad, output_grad, flags)


_forward_kernel_cache: dict[tuple[int, int], _ForwardKernel] = {}
_backward_kernel_cache: dict[tuple[int, int], _BackwardKernel] = {}


@torch.compiler.disable(recursive=False)
def make_sparse_input_linear_forward_kernel(
    max_active_indices: int, output_size: int
) -> SparseInputLinearForwardKernel:
    key = (max_active_indices, output_size)
    if key not in _forward_kernel_cache:
        _forward_kernel_cache[key] = _ForwardKernel(max_active_indices, output_size)
    return _forward_kernel_cache[key]


@torch.compiler.disable(recursive=False)
def make_sparse_input_linear_backward_kernel(
    max_active_indices: int, output_size: int
) -> SparseInputLinearBackwardKernel:
    key = (max_active_indices, output_size)
    if key not in _backward_kernel_cache:
        _backward_kernel_cache[key] = _BackwardKernel(max_active_indices, output_size)
    return _backward_kernel_cache[key]
