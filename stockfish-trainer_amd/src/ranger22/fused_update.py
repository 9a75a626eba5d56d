"""Ranger22's full parameter update on the GPU (reference
src/ranger22/optimizer.py:46-111, `_compiled_full_update_1d/_2d`, compiled by
`_get_compiled_full_update` at :114-132 and called from Ranger22.step at
:472-480).

`get_fused_full_update(ndim)` returns a callable with the reference's
signature `(p, grad, variance_ma, gma_cur, gma_prev, scalars)` that updates p,
variance_ma and gma_cur in place with one HIP kernel (libsft_ft.so
`sft_ranger22_update_f32`): per-row norm for 2-D tables, whole-tensor norm
for 1-D ones, every elementwise operation rounded to binary32 in the
reference function's order.  A trainer swaps it in for
`_get_compiled_full_update`; no torch.compile, no host synchronisation (the
scalars stay a device tensor).
"""

import torch

from sft_amd import _native


def fused_full_update(p: torch.Tensor, grad: torch.Tensor, variance_ma: torch.Tensor, gma_cur: torch.Tensor,
                      gma_prev: torch.Tensor, scalars: torch.Tensor) -> None:
    assert p.is_cuda and p.dtype == torch.float32 and p.ndim in (1, 2)
    assert p.is_contiguous() and grad.is_contiguous() and variance_ma.is_contiguous()
    assert gma_cur.is_contiguous() and gma_prev.is_contiguous() and scalars.is_contiguous()
    _native.ranger22_update_f32(p, grad, variance_ma, gma_cur, gma_prev, scalars)


def get_fused_full_update(ndim: int):
    if ndim not in (1, 2):
        raise ValueError(f"no fused Ranger22 full-update for ndim={ndim}")
    return fused_full_update
