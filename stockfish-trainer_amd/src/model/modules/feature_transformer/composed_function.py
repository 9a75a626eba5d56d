"""Both perspectives of a composed feature transformer in one autograd op.

The reference's ComposedFeatureTransformer.forward
(src/model/modules/features/composed.py:49-54) materialises the merged table
(torch.cat of each block's merged_weight: HalfKAv2_hm's
weight + virtual_weight.repeat(32, 1), src/model/modules/features/halfka_v2_hm.py:69-70;
Full_Threats' weight, src/model/modules/features/full_threats.py:27-28) and runs
SparseLinearFunction once per perspective; autograd then adds the two table
grads, splits the sum over the blocks and reduces the repeated virtual rows.

ComposedSparseLinearFunction computes the same outputs and grads with two
library calls: the forward builds the merged table once, directly in the
gather's tile layout, and gathers both perspectives in one launch; the
backward writes each block's grad (dW_0 + dW_1, one binary32 add, as autograd
sums them) and the virtual-row sums.  Outputs and block grads are bit-identical
to the reference composition run on the same kernels.
"""

import torch
from torch import autograd

from sft_amd import _native

from . import ops  # noqa: F401  (registers torch.ops.sft.*)
from .ops import split_tables  # noqa: F401  (re-exported)


class ComposedSparseLinearFunction(autograd.Function):
    """apply(idx0, idx1, bias, virtual_rows, *tables) -> (out0, out1).

    tables holds, block by block, the block's weight [R_s, L] and, when
    virtual_rows[s] > 0, its virtual table [virtual_rows[s], L]."""

    @staticmethod
    def forward(ctx, feature_indices_0, feature_indices_1, bias, virtual_rows, *tables):
        for idx in (feature_indices_0, feature_indices_1):
            assert len(idx.shape) == 2
            assert idx.dtype == torch.int32
            assert idx.is_cuda
            assert idx.is_contiguous()
        assert feature_indices_0.shape == feature_indices_1.shape
        assert feature_indices_1.device == feature_indices_0.device
        assert len(bias.shape) == 1
        assert bias.dtype == torch.float32
        assert bias.is_cuda and bias.device == feature_indices_0.device
        assert bias.is_contiguous()
        for t in tables:
            assert len(t.shape) == 2
            assert t.dtype == torch.float32
            assert t.is_cuda and t.device == feature_indices_0.device
            assert t.is_contiguous()

        out0, out1 = torch.ops.sft.composed_fwd(feature_indices_0, feature_indices_1, bias, list(virtual_rows),
                                                list(tables))
        ctx.save_for_backward(feature_indices_0, feature_indices_1)
        ctx.virtual_rows = tuple(virtual_rows)
        ctx.table_rows = [t.shape[0] for t in tables]
        return out0, out1

    @staticmethod
    def backward(ctx, grad_0, grad_1):
        assert not ctx.needs_input_grad[0] and not ctx.needs_input_grad[1]
        idx0, idx1 = ctx.saved_tensors
        # Every grad is overwritten by the library: no zero-fill.
        res = torch.ops.sft.composed_bwd(idx0, idx1, grad_0.contiguous(), grad_1.contiguous(),
                                         list(ctx.virtual_rows), list(ctx.table_rows))
        return (None, None, res[-1], None, *res[:-1])


@torch.compiler.assume_constant_result
def _pair_shape_supported(batch_size: int, max_active: int, rows: tuple, vrows: tuple, output_size: int) -> bool:
    # a host-only library query: a constant for torch.compile, not a graph break
    return _native.pair_workspace_bytes(batch_size, max_active, list(rows), list(vrows), output_size) is not None


def composed_pair_supported(batch_size: int, max_active: int, blocks, output_size: int) -> bool:
    """Whether the library runs this composed shape fused (else the caller
    composes the table and runs SparseLinearFunction twice)."""
    rows = tuple(w.shape[0] for w, _ in blocks)
    vrows = tuple(0 if v is None else v.shape[0] for _, v in blocks)
    return _pair_shape_supported(batch_size, max_active, rows, vrows, output_size)
