"""The feature-transformer section of the .nnue writer, on the GPU (reference
src/scripts/serialize.py: LEB128_MAGIC :51, _encode_leb_128_array :61-93,
the FT hash word :186, _write_feature_transformer :195-224, _write_tensor /
_write_leb_128_array / int32 :254-275).

FeatureTransformerWriter(input_module, l1, quantization).buf holds the bytes
the reference's NNUEWriter writes from the FT hash word through the PSQT
weights: the quantization runs on the device (sft_quantize_i16 for the
int16 tensors) and the signed LEB128 compression of the bias, weights and PSQT
weights runs as one GPU encoder per tensor (sft_leb128_encode) instead of a
per-value CPU loop.  The header before it and the FC layers after it are not
part of this module.
"""

from __future__ import annotations

import struct

import torch

from sft_amd import _native

LEB128_MAGIC = b"COMPRESSED_LEB128"


def encode_leb_128_array(arr: torch.Tensor) -> bytes:
    """Signed LEB128 of every element, concatenated (serialize.py:61-93)."""
    if not arr.is_cuda:
        raise ValueError("encode_leb_128_array runs on the GPU: pass a device tensor")
    return bytes(_native.leb128_encode(arr.contiguous().view(-1)).cpu().numpy().tobytes())


class FeatureTransformerWriter:
    def __init__(self, input_module, l1: int, quantization, ft_compression: str = "leb128",
                 pad_l1: int | None = None):
        self.buf = bytearray()
        self.effective_l1 = pad_l1 if pad_l1 is not None else l1
        self.pad_amount = self.effective_l1 - l1
        if self.pad_amount < 0:
            raise ValueError(f"pad_l1={pad_l1} is smaller than model L1={l1}")
        self.int32(input_module.HASH ^ (self.effective_l1 * 2))
        self._write_feature_transformer(input_module, l1, quantization, ft_compression)

    def _write_feature_transformer(self, layer, l1: int, quantization, ft_compression: str) -> None:
        with torch.no_grad():
            bias = layer.bias.data[:l1]
            export_weight = layer.get_export_weights()
            weight = export_weight[:, :l1].contiguous()
            psqt_weight = export_weight[:, l1:].contiguous()
            scale = float(quantization.ft_quantized_one)
            bias = _native.quantize_i16(bias.contiguous(), scale)
            weight = _native.quantize_i16(weight, scale)
            psqt_weight = psqt_weight.mul(quantization.psqt_scale).round().to(torch.int32)
            if self.pad_amount > 0:
                bias = torch.nn.functional.pad(bias, (0, self.pad_amount))
                weight = torch.nn.functional.pad(weight, (0, self.pad_amount))
        self._write_tensor(bias.flatten(), ft_compression)
        offset = 0
        for f in layer.features:
            n = int(f.NUM_REAL_FEATURES)
            segment = weight[offset:offset + n]
            if f.EXPORT_WEIGHT_DTYPE == torch.int8:
                self._write_tensor(segment.to(torch.int8).flatten())
            else:
                self._write_tensor(segment.flatten(), ft_compression)
            offset += n
        self._write_tensor(psqt_weight.flatten(), ft_compression)

    def _write_leb_128_array(self, arr: torch.Tensor) -> None:
        payload = encode_leb_128_array(arr)
        self.int32(len(payload))
        self.buf.extend(payload)

    def _write_tensor(self, arr: torch.Tensor, compression: str = "none") -> None:
        if compression == "none":
            self.buf.extend(arr.contiguous().cpu().numpy().tobytes())
        elif compression == "leb128":
            self.buf.extend(LEB128_MAGIC)
            self._write_leb_128_array(arr)
        else:
            raise ValueError(f"Invalid compression mode: {compression}")

    def int32(self, v: int) -> None:
        self.buf.extend(struct.pack("<I", v & 0xFFFFFFFF))
