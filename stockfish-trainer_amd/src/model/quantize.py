"""Quantization scales and the export quantizers (reference
src/model/quantize.py:17-23, 26-41, 76-105 for the feature transformer,
107-160 for the FC layers the .nnue writer exports after it).  The training-time
weight-clipping groups of the FC layers live with the layer stacks, which are
not part of this package."""

from dataclasses import dataclass

import torch


@dataclass
class QuantizationConfig:
    nnue2score: float = 600.0
    weight_scale_hidden: float = 64.0
    weight_scale_out: float = 16.0
    ft_quantized_one: float = 255.0
    hidden_quantized_one: float = 127.0


class QuantizationManager:
    def __init__(self, config: QuantizationConfig):
        self.nnue2score = config.nnue2score
        self.weight_scale_hidden = config.weight_scale_hidden
        self.weight_scale_out = config.weight_scale_out
        self.hidden_quantized_one = config.hidden_quantized_one
        self.ft_quantized_one = config.ft_quantized_one

        self.max_hidden_weight = config.hidden_quantized_one / self.weight_scale_hidden
        i8 = torch.iinfo(torch.int8)
        # threat rows export as int8 after the FT scale
        self.min_threat_weight = i8.min / config.ft_quantized_one
        self.max_threat_weight = i8.max / config.ft_quantized_one
        self.max_out_weight = (config.hidden_quantized_one * self.hidden_quantized_one) / (
            self.nnue2score * self.weight_scale_out)

    @property
    def psqt_scale(self) -> float:
        return self.nnue2score * self.weight_scale_out

    def quantize_feature_transformer(self, bias, weight, psqt_weight, callback=lambda *a, **k: None,
                                     clamp: bool = False):
        """bias/weight -> round_half_even(x * ft_quantized_one) as int16; psqt -> round(x * 9600) as int32.

        clamp=True saturates the int16 values first (the reference converts
        without saturation, which is only defined for in-range values).
        """
        b = bias.mul(self.ft_quantized_one).round()
        w = weight.mul(self.ft_quantized_one).round()
        if clamp:
            b = b.clamp(-32768, 32767)
            w = w.clamp(-32768, 32767)
        b = b.to(torch.int16)
        w = w.to(torch.int16)
        p = psqt_weight.mul(self.psqt_scale).round().to(torch.int32)
        callback(b, w, p)
        return b, w, p

    def dequantize_feature_transformer(self, bias, weight, psqt_weight):
        return (bias.divide(self.ft_quantized_one), weight.divide(self.ft_quantized_one),
                psqt_weight.divide(self.psqt_scale))

    def _fc_scales(self, output_layer: bool):
        """(weight scale, bias scale) of an FC layer (src/model/quantize.py:114-121)."""
        if output_layer:
            return self.nnue2score * self.weight_scale_out / self.hidden_quantized_one, \
                self.weight_scale_out * self.nnue2score
        return self.weight_scale_hidden, self.weight_scale_hidden * self.hidden_quantized_one

    def quantize_fc_layer(self, bias, weight, output_layer: bool = False, callback=lambda *a, **k: None):
        """bias -> round(bias * bias scale) as int32; weight -> round(clamp(w, +-127 / weight scale) *
        weight scale) as int8 (src/model/quantize.py:107-140).  The callback gets the quantized
        tensors, the clipped-element count, the element count, the largest clip and the clip bound."""
        w_scale, b_scale = self._fc_scales(output_layer)
        max_w = self.hidden_quantized_one / w_scale
        b = bias.mul(b_scale).round().to(torch.int32)
        clipped_w = weight.clamp(-max_w, max_w)
        diff = clipped_w - weight
        clipped = torch.count_nonzero(diff)
        clipped_max = torch.max(torch.abs(diff)) if diff.numel() else torch.tensor(0.0)
        w = clipped_w.mul(w_scale).round().to(torch.int8)
        callback(b, w, clipped, torch.numel(weight), clipped_max, max_w)
        return b, w

    def dequantize_fc_layer(self, bias, weight, output_layer: bool = False):
        w_scale, b_scale = self._fc_scales(output_layer)
        return bias.divide(b_scale), weight.divide(w_scale)
