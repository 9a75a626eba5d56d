"""FT quantization scales and the FT export quantizer (reference
src/model/quantize.py:17-23, 26-41, 76-105).  Only the feature-transformer part
is here; the dense FC-layer quantizers are outside the FT path."""

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
