"""The .nnue writer (reference src/scripts/serialize.py), with the
feature-transformer section on the GPU.

Layout (serialize.py:125-135): header | FT | [router, MoE only] | FC buckets,
all integers little-endian:
  header (:165-180)  VERSION, network hash = FC hash ^ feature hash ^ 2 L1 ^
                     stack-mode salt (^ ROUTER_HASH for MoE), description length
                     and bytes;
  FT (:182-224)      the feature hash ^ 2 L1, then bias, weights per feature
                     block and PSQT weights, int16/int32 (LEB128-compressed by
                     default) or int8 for blocks that export so;
  router (:228-246)  int32 biases[8], int8 weights[8 x 64] (MoE only);
  FC (:188-196, :250-268) per bucket the FC hash, then l1, l2 and output: int32
                     biases and int8 weights, inputs zero-padded to multiples
                     of 32.

FeatureTransformerWriter(input_module, l1, quantization).buf holds the FT
section: the quantization runs on the device (sft_quantize_i16 for the int16
tensors) and the signed LEB128 compression of the bias, weights and PSQT
weights (LEB128_MAGIC :51, _encode_leb_128_array :61-93, _write_tensor /
_write_leb_128_array / int32 :254-275) runs as one GPU encoder per tensor
(sft_leb128_encode) instead of a per-value CPU loop.  NNUEWriter(model) writes
the whole file around it; the model is duck-typed as the reference's NNUEModel:
`input` (the FT module), `L1`, `feature_hash`, `quantization`, `stacks`
("layer" or "none") and `layer_stacks` with `l1`, `l2`, `output` (their
`out_features` per bucket), `get_coalesced_layer_stacks()` yielding each
bucket's (l1, l2, output) nn.Linear, and `router` for MoE stacks.
"""

from __future__ import annotations

import struct

import torch

from sft_amd import _native

LEB128_MAGIC = b"COMPRESSED_LEB128"

# Format version of every stack mode (serialize.py:36).
VERSION = 0x7AF32F20
# Router<64, 8>'s hash word, in the network hash of MoE exports only (:40).
ROUTER_HASH = 0xABCD123C
# Salts per stack mode, the engine's StackModeHashSalt (:43-47).
STACK_MODE_HASH_SALTS = {"layer": 0, "none": 0x61E90A17, "moe": 0}
DEFAULT_DESCRIPTION = (
    "Network trained with the stockfish-trainer "
    "(https://github.com/rgodha24/stockfish-trainer)."
)
ROUTER_EXPERTS, ROUTER_INPUTS = 8, 64


def fc_hash(L1: int, out_features) -> int:
    """The engine's FC-layer hash (serialize.py:95-122): starting from the input
    slice (0xEC42E90D ^ 2 L1), each layer combines 0xCC03DAE4 + its output count
    with the previous hash shifted both ways, and a ClippedReLU (every layer but
    a 1-output one) adds 0x538D24C7."""
    h = (0xEC42E90D ^ (2 * L1)) & 0xFFFFFFFF
    for n in out_features:
        lh = (0xCC03DAE4 + n) & 0xFFFFFFFF
        lh ^= h >> 1
        lh ^= (h << 31) & 0xFFFFFFFF
        if n != 1:
            lh = (lh + 0x538D24C7) & 0xFFFFFFFF
        h = lh
    return h


def stack_mode_of(model, requested: str | None = None) -> str:
    """The model's stack mode (serialize.py:331-347): MoE stacks carry a router."""
    inferred = "moe" if hasattr(model.layer_stacks, "router") else (
        "none" if getattr(model, "stacks", "layer") == "none" else "layer")
    if requested is None:
        return inferred
    if inferred == "moe" and requested != "moe":
        raise ValueError("MoE checkpoints can only be exported with stack_mode='moe'")
    if inferred != "moe" and requested == "moe":
        raise ValueError("Only MoE checkpoints can be exported with stack_mode='moe'")
    return requested


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


class NNUEWriter:
    """The whole .nnue file of a model (serialize.py:125-196), in `buf`."""

    def __init__(self, model, description: str | None = None, ft_compression: str = "leb128",
                 pad_l1: int | None = None, stack_mode: str | None = None):
        self.buf = bytearray()
        self.stack_mode = stack_mode_of(model, stack_mode)
        self.effective_l1 = pad_l1 if pad_l1 is not None else model.L1
        if self.effective_l1 < model.L1:
            raise ValueError(f"pad_l1={pad_l1} is smaller than model L1={model.L1}")
        stacks = model.layer_stacks
        h_fc = fc_hash(model.L1, (stacks.l1.out_features, stacks.l2.out_features, stacks.output.out_features))
        header_hash = h_fc ^ model.feature_hash ^ (self.effective_l1 * 2) ^ STACK_MODE_HASH_SALTS[self.stack_mode]
        if self.stack_mode == "moe":
            header_hash ^= ROUTER_HASH
        desc = (DEFAULT_DESCRIPTION if description is None else description).encode("utf-8")
        self.int32(VERSION)
        self.int32(header_hash)
        self.int32(len(desc))
        self.buf.extend(desc)
        self.buf.extend(FeatureTransformerWriter(model.input, model.L1, model.quantization, ft_compression,
                                                 pad_l1).buf)
        if self.stack_mode == "moe":
            self._write_router(model)
        for index, (l1, l2, output) in enumerate(stacks.get_coalesced_layer_stacks()):
            if self.stack_mode == "none" and index > 0:
                break
            self.int32(h_fc)
            self._write_fc_layer(model, l1, is_output=False)
            self._write_fc_layer(model, l2, is_output=False)
            self._write_fc_layer(model, output, is_output=True)

    def _write_router(self, model) -> None:
        """Router<64, 8>: int32 biases[8], then int8 weights[8 x 64] (serialize.py:228-246)."""
        router = model.layer_stacks.router
        if tuple(router.weight.shape) != (ROUTER_EXPERTS, ROUTER_INPUTS):
            raise ValueError(f"router weight must be [{ROUTER_EXPERTS}, {ROUTER_INPUTS}]")
        b, w = model.quantization.quantize_fc_layer(router.bias.data.cpu(), router.weight.data.cpu(), output_layer=False)
        self.buf.extend(b.flatten().numpy().tobytes())
        self.buf.extend(w.flatten().numpy().tobytes())

    def _write_fc_layer(self, model, layer, *, is_output: bool) -> None:
        """int32 biases, then int8 weights [out, in] with in padded to a multiple of 32
        (serialize.py:250-268)."""
        b, w = model.quantization.quantize_fc_layer(layer.bias.data.cpu(), layer.weight.data.cpu(), is_output)
        n_in = w.shape[1]
        if n_in % 32:
            padded = torch.zeros(w.shape[0], (n_in + 31) // 32 * 32, dtype=torch.int8)
            padded[:, :n_in] = w
            w = padded
        self.buf.extend(b.flatten().numpy().tobytes())
        self.buf.extend(w.flatten().numpy().tobytes())

    def int32(self, v: int) -> None:
        self.buf.extend(struct.pack("<I", v & 0xFFFFFFFF))
