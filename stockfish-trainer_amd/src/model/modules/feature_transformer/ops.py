"""The FT's library calls as torch custom operators.

The reference keeps its kernel factories out of compiled graphs with
torch.compiler.disable (src/model/modules/feature_transformer/kernel.py:301,315),
so the model it compiles (src/train/common.py:189) breaks its graph at every
SparseLinearFunction.  Here each call of libsft_ft.so is a torch.library
custom op with a fake (meta) implementation: Dynamo and Inductor see an opaque
op with known output shapes, and the autograd.Functions built on these ops
(SparseLinearFunction, ComposedSparseLinearFunction,
TransformedFeatureFunction) trace without a graph break.  Eager calls run the
same kernels; outputs are bit-identical either way.

Every op allocates and returns its outputs (functional, mutates nothing), and
all of them overwrite: the backward ops return complete grads.
"""

from __future__ import annotations

import torch
from torch import Tensor

from sft_amd import _native



# ---- SparseLinearFunction (FT/functions.py:12-72) ----
# The forward also sorts the indices for the backward (the sort needs nothing
# else), on a side stream beside its gather, into a buffer the autograd
# Function keeps until its backward: the backward then runs the bias pass and
# the gathers only.  The reference sorts inside the backward (FT/kernel.py:108-138).
@torch.library.custom_op("sft::sparse_linear_fwd", mutates_args=(), device_types="cuda")
def sparse_linear_fwd(feature_indices: Tensor, weight: Tensor, bias: Tensor) -> tuple[Tensor, Tensor]:
    out = torch.empty(feature_indices.shape[0], weight.shape[1], dtype=torch.float32, device=feature_indices.device)
    prep = _native.ft_fwd_f32_prep(feature_indices, weight, bias, out, _native.SFT_BWD_OVERWRITE)
    return out, prep


@sparse_linear_fwd.register_fake
def _(feature_indices, weight, bias):
    B, K = feature_indices.shape
    N, L = weight.shape
    if all(type(v) is int for v in (B, K, N, L)):
        nbytes = _native.prep_buffer_bytes(B, K, N, L, _native.SFT_BWD_OVERWRITE, feature_indices.device)
    else:  # symbolic sizes (dynamic shapes): the same layout in SymInt arithmetic
        nbytes = _native.prep_buffer_bytes_formula(B, K, N, L, _native.SFT_BWD_OVERWRITE)
    return (feature_indices.new_empty((B, L), dtype=torch.float32),
            feature_indices.new_empty((nbytes,), dtype=torch.uint8))


@torch.library.custom_op("sft::sparse_linear_bwd", mutates_args=(), device_types="cuda")
def sparse_linear_bwd(feature_indices: Tensor, grad_output: Tensor, num_inputs: int,
                      prep: Tensor) -> tuple[Tensor, Tensor]:
    L = grad_output.shape[1]
    dev = feature_indices.device
    weight_grad = torch.empty(num_inputs, L, dtype=torch.float32, device=dev)
    bias_grad = torch.empty(L, dtype=torch.float32, device=dev)
    _native.ft_bwd_f32_prepared(feature_indices, weight_grad, bias_grad, grad_output, prep,
                                _native.SFT_BWD_OVERWRITE)
    return weight_grad, bias_grad


@sparse_linear_bwd.register_fake
def _(feature_indices, grad_output, num_inputs, prep):
    L = grad_output.shape[1]
    return grad_output.new_empty((num_inputs, L)), grad_output.new_empty((L,))


# ---- ComposedSparseLinearFunction (FEAT/composed.py:49-54) ----
def split_tables(tables, virtual_rows):
    """Flat (w_0, [v_0], w_1, [v_1], ...) -> ([w_s], [v_s or None])."""
    weights, virtuals, i = [], [], 0
    for vr in virtual_rows:
        weights.append(tables[i])
        i += 1
        if vr > 0:
            virtuals.append(tables[i])
            i += 1
        else:
            virtuals.append(None)
    assert i == len(tables)
    return weights, virtuals


@torch.library.custom_op("sft::composed_fwd", mutates_args=(), device_types="cuda")
def composed_fwd(idx0: Tensor, idx1: Tensor, bias: Tensor, virtual_rows: list[int],
                 tables: list[Tensor]) -> tuple[Tensor, Tensor]:
    weights, virtuals = split_tables(tables, virtual_rows)
    B, L = idx0.shape[0], bias.shape[0]
    out0 = torch.empty(B, L, dtype=torch.float32, device=idx0.device)
    out1 = torch.empty(B, L, dtype=torch.float32, device=idx0.device)
    _native.ft_fwd_pair_f32(idx0, idx1, weights, virtuals, bias, out0, out1)
    return out0, out1


@composed_fwd.register_fake
def _(idx0, idx1, bias, virtual_rows, tables):
    shape = (idx0.shape[0], bias.shape[0])
    return bias.new_empty(shape), bias.new_empty(shape)


@torch.library.custom_op("sft::composed_bwd", mutates_args=(), device_types="cuda")
def composed_bwd(idx0: Tensor, idx1: Tensor, grad0: Tensor, grad1: Tensor, virtual_rows: list[int],
                 table_rows: list[int]) -> list[Tensor]:
    """Grads of the tables (in the order of `tables`), then the bias grad."""
    L = grad0.shape[1]
    dev = idx0.device
    grads = [torch.empty(r, L, dtype=torch.float32, device=dev) for r in table_rows]
    bias_grad = torch.empty(L, dtype=torch.float32, device=dev)
    weight_grads, virtual_grads = split_tables(grads, virtual_rows)
    _native.ft_bwd_pair_f32(idx0, idx1, grad0, grad1, weight_grads, virtual_grads, bias_grad)
    return grads + [bias_grad]


@composed_bwd.register_fake
def _(idx0, idx1, grad0, grad1, virtual_rows, table_rows):
    L = grad0.shape[1]
    return [grad0.new_empty((r, L)) for r in table_rows] + [grad0.new_empty((L,))]


# ---- TransformedFeatureFunction (src/model/model.py:86-115) ----
def transform_saved_bytes(batch, output_size: int, l1: int):
    """Bytes of the pre-activations the transform forward keeps for its backward:
    both perspectives in the paired 32-column tiles (L1 / 32 paired tiles and the
    PSQT columns in tiles of 8 chunks), 128 bytes per position and tile."""
    tiles = (l1 // 8 + 3) // 4 + ((output_size - l1) // 4 + 7) // 8
    return 2 * tiles * batch * 128


@torch.library.custom_op("sft::transform_fwd", mutates_args=(), device_types="cuda")
def transform_fwd(idx0: Tensor, idx1: Tensor, bias: Tensor, us: Tensor, psqt_indices: Tensor, l1: int,
                  virtual_rows: list[int], tables: list[Tensor]) -> tuple[Tensor, Tensor, Tensor]:
    """(l0 [B, l1], psqt [B, 1], saved uint8 buffer for transform_bwd)."""
    weights, virtuals = split_tables(tables, virtual_rows)
    B = idx0.shape[0]
    l0 = torch.empty(B, l1, dtype=torch.float32, device=idx0.device)
    psqt = torch.empty(B, 1, dtype=torch.float32, device=idx0.device)
    saved, _ = _native.ft_fwd_transform_f32(idx0, idx1, weights, virtuals, bias, us, psqt_indices, l1, l0, psqt)
    return l0, psqt, saved


@transform_fwd.register_fake
def _(idx0, idx1, bias, us, psqt_indices, l1, virtual_rows, tables):
    B = idx0.shape[0]
    nbytes = transform_saved_bytes(B, bias.shape[0], l1) + 256  # + alignment slack, as the library's buffer
    return (bias.new_empty((B, l1)), bias.new_empty((B, 1)),
            bias.new_empty((nbytes,), dtype=torch.uint8))


@torch.library.custom_op("sft::transform_bwd", mutates_args=(), device_types="cuda")
def transform_bwd(idx0: Tensor, idx1: Tensor, grad_l0: Tensor, grad_psqt: Tensor, us: Tensor, psqt_indices: Tensor,
                  saved: Tensor, l1: int, output_size: int, virtual_rows: list[int],
                  table_rows: list[int]) -> list[Tensor]:
    """Grads of the tables (in the order of `tables`), then the bias grad."""
    dev = idx0.device
    L = output_size
    grads = [torch.empty(r, L, dtype=torch.float32, device=dev) for r in table_rows]
    bias_grad = torch.empty(L, dtype=torch.float32, device=dev)
    weight_grads, virtual_grads = split_tables(grads, virtual_rows)
    sptr = saved.data_ptr() + (-saved.data_ptr()) % 256
    _native.ft_bwd_transform_f32(idx0, idx1, grad_l0, grad_psqt, us, psqt_indices, (saved, sptr), l1,
                                 weight_grads, virtual_grads, bias_grad)
    return grads + [bias_grad]


@transform_bwd.register_fake
def _(idx0, idx1, grad_l0, grad_psqt, us, psqt_indices, saved, l1, output_size, virtual_rows, table_rows):
    return [grad_l0.new_empty((r, output_size)) for r in table_rows] + [grad_l0.new_empty((output_size,))]
