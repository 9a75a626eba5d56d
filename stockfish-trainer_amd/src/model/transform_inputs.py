"""NNUEModel._transform_inputs (reference src/model/model.py:86-115): the
feature transformer of both perspectives followed by the post-FT epilogue
(clamp to [0, 1], product of the two halves of L1, side-to-move ordering,
x 127/128, and the PSQT difference).

transform_inputs(input_module, l1, us, white, black, psqt_indices) returns
(l0, psqt) like the reference method; with `fused=True` (default) and a shape
the library takes, it runs TransformedFeatureFunction (one forward and one
backward call of libsft_ft.so), otherwise the reference sequence of ops on the
composed FT.  Both give bit-identical l0, psqt and table grads.
"""

import torch

from .modules.feature_transformer.transform_function import TransformedFeatureFunction, transform_supported


def _epilogue(wp, bp, l1, us, psqt_indices):
    """The reference epilogue as torch ops (src/model/model.py:93-115)."""
    w, wpsqt = torch.split(wp, l1, dim=1)
    b, bpsqt = torch.split(bp, l1, dim=1)
    half = l1 // 2
    side = us.bool()
    wc = torch.clamp(w, 0.0, 1.0).reshape(-1, 2, half)
    bc = torch.clamp(b, 0.0, 1.0).reshape(-1, 2, half)
    w_prod = wc[:, 0, :] * wc[:, 1, :]
    b_prod = bc[:, 0, :] * bc[:, 1, :]
    l0 = torch.cat([torch.where(side, w_prod, b_prod), torch.where(side, b_prod, w_prod)], dim=1) * (127 / 128)
    k = psqt_indices.unsqueeze(dim=1)
    psqt = (wpsqt.gather(1, k) - bpsqt.gather(1, k)) * (us - 0.5)
    return l0, psqt


def transform_inputs(input_module, l1: int, us, white_indices, black_indices, psqt_indices, fused: bool = True):
    B, K = white_indices.shape
    if fused and white_indices.is_cuda and transform_supported(input_module, B, K, l1):
        tables, virtual_rows = [], []
        for w, v in (f.table_blocks() for f in input_module.features):
            tables.append(w)
            if v is not None:
                tables.append(v)
            virtual_rows.append(0 if v is None else v.shape[0])
        return TransformedFeatureFunction.apply(us, white_indices, black_indices, psqt_indices, input_module.bias,
                                                l1, tuple(virtual_rows), *tables)
    wp, bp = input_module(white_indices, black_indices)
    return _epilogue(wp, bp, l1, us, psqt_indices)
