"""The FT custom ops' fake implementations on the CPU (no GPU calls): output
shapes for concrete and symbolic batch sizes, as torch.compile sees them with
dynamic shapes (a varying batch size: the last partial batch, validation), and
the symbolic size of the forward's prepared sort equal to the library's own
size query."""

import itertools

import pytest
import torch

from sft_amd import _native
from src.model.modules.feature_transformer import ops  # noqa: F401  (registers torch.ops.sft.*)

CPU = torch.device("cpu")


def test_prep_size_formula_matches_the_library():
    """prep_buffer_bytes_formula (integer arithmetic, SymInt-safe) against
    sft_ft_bwd_f32_prep_size over batches around the one-chunk limit, K from 1 to
    160, tables of 5 to 85 296 rows, widths on both sides of K >= L / 20 and of
    the tiled domain, and every flag combination the ops pass or reject."""
    flags = [_native.SFT_BWD_ACCUMULATE, _native.SFT_BWD_OVERWRITE, _native.SFT_BWD_OVERWRITE | _native.SFT_BWD_ROWS,
             _native.SFT_BWD_OVERWRITE | _native.SFT_BWD_ATOMIC, _native.SFT_BWD_OVERWRITE | _native.SFT_BWD_PREPARED]
    n = 0
    for B, K, N, L, f in itertools.product([0, 1, 2, 3, 100, 2047, 32768, 32769, 65536, 100001], [1, 7, 32, 160],
                                           [5, 23232, 85296], [8, 100, 124, 128, 136, 1048, 2100], flags):
        assert _native.prep_buffer_bytes_formula(B, K, N, L, f) == _native.prep_buffer_bytes(B, K, N, L, f, CPU), \
            (B, K, N, L, f)
        n += 1
    assert n == 4200


def _meta(*shape, dtype=torch.float32):
    return torch.empty(*shape, dtype=dtype, device="meta")


@pytest.mark.parametrize("N,L", [(4000, 136), (23232, 1048), (85296, 1048)])
def test_sparse_linear_ops_trace_with_dynamic_batch(N, L):
    """torch.compile(dynamic=True, fullgraph=True) over both ops: the fakes run
    with a symbolic batch size, and each batch size gets the prepared buffer the
    library would return (K = 32: prepared from L <= 640; K = 160 always)."""
    def step(idx, W, b, g):
        out, prep = torch.ops.sft.sparse_linear_fwd(idx, W, b)
        dW, db = torch.ops.sft.sparse_linear_bwd(idx, g, W.shape[0], prep)
        return out, prep, dW, db

    torch._dynamo.reset()
    compiled = torch.compile(step, backend="eager", dynamic=True, fullgraph=True)
    K = 160 if N == 85296 else 32
    for B in (300, 301, 40000, 65536):
        out, prep, dW, db = compiled(_meta(B, K, dtype=torch.int32), _meta(N, L), _meta(L), _meta(B, L))
        assert out.shape == (B, L) and dW.shape == (N, L) and db.shape == (L,)
        assert prep.shape == (_native.prep_buffer_bytes(B, K, N, L, _native.SFT_BWD_OVERWRITE, CPU),)
        assert (prep.numel() > 0) == (K * 20 >= L)


def test_composed_and_transform_ops_trace_with_dynamic_batch():
    B0, K, L, L1 = 300, 32, 1048, 1040
    rows, vrows = [24576, 768], [768]

    def step(i0, i1, bias, w, v, g0, g1, us, pk):
        o0, o1 = torch.ops.sft.composed_fwd(i0, i1, bias, vrows, [w, v])
        grads = torch.ops.sft.composed_bwd(i0, i1, g0, g1, vrows, rows)
        l0, psqt, saved = torch.ops.sft.transform_fwd(i0, i1, bias, us, pk, L1, vrows, [w, v])
        tg = torch.ops.sft.transform_bwd(i0, i1, l0, psqt, us, pk, saved, L1, L, vrows, rows)
        return o0, o1, grads, l0, psqt, saved, tg

    torch._dynamo.reset()
    compiled = torch.compile(step, backend="eager", dynamic=True, fullgraph=True)
    for B in (B0, B0 + 7):
        o0, o1, grads, l0, psqt, saved, tg = compiled(
            _meta(B, K, dtype=torch.int32), _meta(B, K, dtype=torch.int32), _meta(L), _meta(24576, L),
            _meta(768, L), _meta(B, L), _meta(B, L), _meta(B, 1), _meta(B, dtype=torch.int64))
        assert o0.shape == o1.shape == (B, L)
        assert [tuple(t.shape) for t in grads] == [(24576, L), (768, L), (L,)]
        assert l0.shape == (B, L1) and psqt.shape == (B, 1)
        assert saved.shape == (ops.transform_saved_bytes(B, L, L1) + 256,)
        assert [tuple(t.shape) for t in tg] == [(24576, L), (768, L), (L,)]
