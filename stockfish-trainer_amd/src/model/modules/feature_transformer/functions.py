"""SparseLinearFunction: the FT's autograd op (reference
src/model/modules/feature_transformer/functions.py:10-72), same inputs, asserts,
outputs and gradients, running the gfx950 kernels of libsft_ft.so.

The kernels are reached through the custom ops sft::sparse_linear_fwd / _bwd
(ops.py); as opaque ops with fake implementations they let torch.compile trace
this function without the graph break the reference's compiler-disabled
factories cause.  The forward op also returns the backward's sort of the
indices (made beside the forward's gather), saved with the inputs."""

import torch
from torch import autograd

from . import ops  # noqa: F401  (registers torch.ops.sft.*)


class SparseLinearFunction(autograd.Function):
    @staticmethod
    def forward(ctx, feature_indices, weight, bias):
        assert len(feature_indices.shape) == 2
        assert feature_indices.dtype == torch.int32
        assert len(weight.shape) == 2
        assert weight.dtype == torch.float32
        assert len(bias.shape) == 1
        assert bias.dtype == torch.float32
        assert feature_indices.is_cuda
        assert weight.is_cuda
        assert bias.is_cuda
        assert weight.device == feature_indices.device
        assert bias.device == feature_indices.device
        assert feature_indices.is_contiguous()
        assert weight.is_contiguous()
        assert bias.is_contiguous()

        # make_sparse_input_linear_forward_kernel(K, L)(idx, W, b, out) on a new
        # [B, L] output, as one opaque op; it also returns the backward's sort of
        # the indices, made beside the forward, which the backward uses
        out, prep = torch.ops.sft.sparse_linear_fwd(feature_indices, weight, bias)
        ctx.save_for_backward(feature_indices, weight, bias, prep)
        return out

    @staticmethod
    def backward(ctx, grad_output):
        assert not ctx.needs_input_grad[0]

        grad_output = grad_output.contiguous()

        feature_indices, weight, _bias, prep = ctx.saved_tensors

        # The backward kernel in overwrite mode writes every row (absent features
        # get 0), so the grads need no zero-fill; the values equal zero-init +
        # accumulate exactly.
        weight_grad, bias_grad = torch.ops.sft.sparse_linear_bwd(feature_indices, grad_output, weight.shape[0], prep)

        return None, weight_grad, bias_grad
