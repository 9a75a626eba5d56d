"""The feature transformer of both perspectives plus the post-FT epilogue of
NNUEModel._transform_inputs (src/model/model.py:86-115) as one autograd op.

Reference, per position b with x_w / x_b the composed FT outputs
(src/model/modules/features/composed.py:49-54):

    pw_p = clamp(x_p[:, :L1/2], 0, 1) * clamp(x_p[:, L1/2:L1], 0, 1)
    l0   = cat(where(us, pw_w, pw_b), where(us, pw_b, pw_w)) * 127/128
    psqt = (x_w[:, L1 + k] - x_b[:, L1 + k]) * (us - 0.5),  k = psqt_indices

TransformedFeatureFunction computes l0 and psqt with the gather kernel (the FT
outputs never reach memory as [B, L] tensors; the pre-activations are kept in
the gather's tile layout for the backward), and its backward turns the grads
of l0 and psqt straight into the table, virtual and bias grads.  Every output
and table grad is bit-identical to the reference ops on the same kernels.
"""

import torch
from torch import autograd

from sft_amd import _native

from . import ops  # noqa: F401  (registers torch.ops.sft.*)


class TransformedFeatureFunction(autograd.Function):
    """apply(us, idx_w, idx_b, psqt_indices, bias, l1, virtual_rows, *tables) -> (l0, psqt)."""

    @staticmethod
    def forward(ctx, us, feature_indices_0, feature_indices_1, psqt_indices, bias, l1, virtual_rows, *tables):
        for idx in (feature_indices_0, feature_indices_1):
            assert len(idx.shape) == 2
            assert idx.dtype == torch.int32
            assert idx.is_cuda
            assert idx.is_contiguous()
        assert feature_indices_0.shape == feature_indices_1.shape
        assert bias.dtype == torch.float32 and bias.is_contiguous() and bias.is_cuda
        for t in tables:
            assert t.dtype == torch.float32 and t.is_contiguous() and t.is_cuda
        us_flat = us.reshape(-1).to(torch.float32).contiguous()
        psqt_flat = psqt_indices.reshape(-1).to(torch.int64).contiguous()
        l0, psqt, saved = torch.ops.sft.transform_fwd(feature_indices_0, feature_indices_1, bias, us_flat, psqt_flat,
                                                      l1, list(virtual_rows), list(tables))
        # the pre-activations kept for the backward (an opaque uint8 buffer)
        ctx.save_for_backward(feature_indices_0, feature_indices_1, us_flat, psqt_flat, saved)
        ctx.l1 = l1
        ctx.virtual_rows = tuple(virtual_rows)
        ctx.table_rows = [t.shape[0] for t in tables]
        ctx.output_size = bias.shape[0]
        return l0, psqt

    @staticmethod
    def backward(ctx, grad_l0, grad_psqt):
        idx0, idx1, us_flat, psqt_flat, saved = ctx.saved_tensors
        res = torch.ops.sft.transform_bwd(idx0, idx1, grad_l0.contiguous(), grad_psqt.reshape(-1).contiguous(),
                                          us_flat, psqt_flat, saved, ctx.l1, ctx.output_size,
                                          list(ctx.virtual_rows), list(ctx.table_rows))
        return (None, None, None, None, res[-1], None, None, *res[:-1])


@torch.compiler.assume_constant_result
def _transform_shape_supported(batch_size: int, max_active: int, rows: tuple, vrows: tuple, output_size: int,
                               l1: int) -> bool:
    # a host-only library query: a constant for torch.compile, not a graph break
    return _native.transform_workspace_bytes(batch_size, max_active, list(rows), list(vrows), output_size,
                                             l1) is not None


def transform_supported(input_module, batch_size: int, max_active: int, l1: int) -> bool:
    blocks = [f.table_blocks() for f in input_module.features]
    rows = tuple(w.shape[0] for w, _ in blocks)
    vrows = tuple(0 if v is None else v.shape[0] for _, v in blocks)
    return _transform_shape_supported(batch_size, max_active, rows, vrows, input_module.num_outputs, l1)
