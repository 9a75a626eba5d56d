"""A small model with the NNUEModel attributes the .nnue writer reads: an FT
module, L1, the feature hash, the quantization manager and layer stacks of
per-bucket nn.Linear layers (l1: 2 L1 -> L2 + 1, l2: 2 L2 -> L3, output: L3
-> 1, as src/model/modules/layer_stacks.py builds them), plus a router for MoE
stacks.  Shared by the CPU and GPU writer tests."""

from __future__ import annotations

import torch
from torch import nn

from src.model.modules.features import get_feature_cls
from src.model.quantize import QuantizationConfig, QuantizationManager


class _Width:
    def __init__(self, out_features):
        self.out_features = out_features


class Stacks:
    def __init__(self, L1, L2, L3, count, moe, g):
        self.count = count
        self.l1, self.l2, self.output = _Width(L2 + 1), _Width(L3), _Width(1)
        self.buckets = []
        for _ in range(count):
            layers = []
            for n_in, n_out in ((2 * L1, L2 + 1), (2 * L2, L3), (L3, 1)):
                lin = nn.Linear(n_in, n_out)
                with torch.no_grad():
                    lin.weight.copy_(torch.randn(n_out, n_in, generator=g) * 0.8)  # some beyond the clip bound
                    lin.bias.copy_(torch.randn(n_out, generator=g) * 0.3)
                layers.append(lin)
            self.buckets.append(tuple(layers))
        if moe:
            self.router = nn.Linear(64, 8)

    def get_coalesced_layer_stacks(self):
        yield from self.buckets


class Model:
    def __init__(self, features="HalfKAv2_hm^", L1=64, L2=15, L3=32, count=8, stacks="layer", moe=False,
                 device="cpu", seed=3):
        g = torch.Generator().manual_seed(seed)
        self.L1 = L1
        self.stacks = stacks
        self.input = get_feature_cls(features)(L1 + 8)
        with torch.no_grad():
            for f in self.input.features:
                f.weight.copy_(torch.rand(f.weight.shape, generator=g) * 0.8 - 0.4)  # threat rows stay int8
                if hasattr(f, "virtual_weight"):
                    f.virtual_weight.copy_(torch.rand(f.virtual_weight.shape, generator=g) * 0.1 - 0.05)
            self.input.bias.copy_(torch.rand(self.input.bias.shape, generator=g) - 0.5)
        self.input = self.input.to(device)
        self.feature_hash = self.input.HASH
        self.quantization = QuantizationManager(QuantizationConfig())
        self.layer_stacks = Stacks(L1, L2, L3, count, moe, g)
