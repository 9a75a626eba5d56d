"""int16 quantized FT inference forward (the integer accumulator the export
feeds; the reference holds no such op).

    acc[b]  = bias_q + sum_{k active} W_q[idx[b, k]]        exact int32
    out[b]  = clamp(acc[b], clip_lo, clip_hi)                int16
    psqt[b] = sum_{k active} psqt_q[idx[b, k]]               int32

With wrap16=True the accumulator is int16 with wrapping adds (the engine's
accumulator arithmetic) before the clamp.
"""

from __future__ import annotations

import torch

from . import _native


def quantized_ft_forward(idx: torch.Tensor, weight_q: torch.Tensor, bias_q: torch.Tensor,
                         psqt_q: torch.Tensor | None = None, clip_lo: int = 0, clip_hi: int = 127,
                         wrap16: bool = False, rows: bool = False):
    """One perspective: (out int16 [B, L], psqt_out int32 [B, P] or None)."""
    B = idx.shape[0]
    out = torch.empty(B, weight_q.shape[1], dtype=torch.int16, device=idx.device)
    psqt_out = None
    if psqt_q is not None:
        psqt_out = torch.empty(B, psqt_q.shape[1], dtype=torch.int32, device=idx.device)
    _native.ft_fwd_i16(idx, weight_q, bias_q, out, psqt_q, psqt_out, clip_lo, clip_hi, wrap16, rows)
    return out, psqt_out


def quantize_weight_i16(x: torch.Tensor, scale: float) -> torch.Tensor:
    """round_half_even(x * scale), saturated to int16, on the GPU."""
    return _native.quantize_i16(x.contiguous(), scale)


class QuantizedFeatureTransformer:
    """Both perspectives over one exported int16 table.

    When the shape allows the tiled path, the table and its PSQT columns are
    packed once into 64-column tiles (an inference engine's load-time weight
    permutation) and both perspectives are gathered from them in one launch.
    The pack is rebuilt when torch's version counter of weight_q or psqt_q has
    moved (in-place updates through torch); writes that bypass torch need
    repack().
    """

    def __init__(self, weight_q: torch.Tensor, bias_q: torch.Tensor, psqt_q: torch.Tensor | None = None,
                 clip_lo: int = 0, clip_hi: int = 127, wrap16: bool = False):
        self.weight_q = weight_q.contiguous()
        self.bias_q = bias_q.contiguous()
        self.psqt_q = None if psqt_q is None else psqt_q.contiguous()
        self.clip = (clip_lo, clip_hi)
        self.wrap16 = wrap16
        self.packed = None
        self._packed_key = None
        self.repack()

    def _key(self):
        t = [self.weight_q] + ([] if self.psqt_q is None else [self.psqt_q])
        return tuple((x.data_ptr(), x._version) for x in t)

    def repack(self) -> None:
        """Rebuild the packed tiles from weight_q and psqt_q (no-op outside the tiled path)."""
        ok = self.weight_q.is_cuda and self.bias_q.data_ptr() % 16 == 0
        self.packed = _native.i16_pack(self.weight_q, self.psqt_q) if ok else None
        self._packed_key = self._key()

    def __call__(self, idx_white: torch.Tensor, idx_black: torch.Tensor):
        if self.packed is not None and self._key() != self._packed_key:
            self.repack()
        if self.packed is None or idx_white.shape != idx_black.shape:
            w = quantized_ft_forward(idx_white, self.weight_q, self.bias_q, self.psqt_q, *self.clip, self.wrap16)
            b = quantized_ft_forward(idx_black, self.weight_q, self.bias_q, self.psqt_q, *self.clip, self.wrap16)
            return w, b
        N, L = self.weight_q.shape
        P = 0 if self.psqt_q is None else self.psqt_q.shape[1]
        B = idx_white.shape[0]
        dev = idx_white.device
        ow = torch.empty(B, L, dtype=torch.int16, device=dev)
        ob = torch.empty(B, L, dtype=torch.int16, device=dev)
        pw = torch.empty(B, P, dtype=torch.int32, device=dev) if P else None
        pb = torch.empty(B, P, dtype=torch.int32, device=dev) if P else None
        _native.ft_fwd_i16_packed(self.packed, N, L, P, self.bias_q, idx_white, ow, pw, idx_black, ob, pb,
                                  *self.clip, self.wrap16)
        return (ow, pw), (ob, pb)
