"""ComposedFeatureTransformer (reference src/model/modules/features/composed.py:8-94):
concatenates the feature blocks' tables and runs the sparse linear op once per
perspective with the shared table and bias."""

import math

import torch
from torch import nn

from ..feature_transformer import ComposedSparseLinearFunction, SparseLinearFunction
from ..feature_transformer.composed_function import composed_pair_supported
from .input_feature import InputFeature


class ComposedFeatureTransformer(nn.Module):
    """Owns the shared bias; each feature block owns its weight rows.

    forward() runs both perspectives through ComposedSparseLinearFunction (one
    fused op, same values) when the library takes the shape; with
    `fused = False`, or for shapes it does not take, it runs the reference
    composition: merged_weight() and SparseLinearFunction per perspective."""

    fused: bool = True

    def __init__(self, features: list):
        super().__init__()
        self.features = nn.ModuleList(features)
        self.num_outputs = features[0].num_outputs
        self.bias = nn.Parameter(torch.empty(self.num_outputs, dtype=torch.float32))

        self.NUM_INPUTS = sum(f.NUM_INPUTS for f in features)
        self.MAX_ACTIVE_FEATURES = sum(f.MAX_ACTIVE_FEATURES for f in features)
        self.NUM_REAL_FEATURES = sum(f.NUM_REAL_FEATURES for f in features)
        self.FEATURE_NAME = "+".join(f.FEATURE_NAME for f in features)
        self.INPUT_FEATURE_NAME = "+".join(f.INPUT_FEATURE_NAME for f in features)
        self.HASH = self._compute_hash()
        self._reset_bias()

    def _compute_hash(self) -> int:
        h = 0
        for f in self.features:
            h = ((h << 1) | (h >> 31)) & 0xFFFFFFFF  # rotate left by one in 32 bits
            h ^= f.HASH
        return h

    def _reset_bias(self):
        bound = math.sqrt(1.0 / self.NUM_INPUTS)
        with torch.no_grad():
            self.bias.uniform_(-bound, bound)

    def merged_weight(self) -> torch.Tensor:
        return torch.cat([f.merged_weight() for f in self.features], dim=0)

    def forward(self, feature_indices_0, feature_indices_1):
        if self.fused and feature_indices_0.is_cuda and feature_indices_0.shape == feature_indices_1.shape:
            blocks = [f.table_blocks() for f in self.features]
            B, K = feature_indices_0.shape
            if composed_pair_supported(B, K, blocks, self.num_outputs):
                tables, virtual_rows = [], []
                for w, v in blocks:
                    tables.append(w)
                    if v is not None:
                        tables.append(v)
                    virtual_rows.append(0 if v is None else v.shape[0])
                return ComposedSparseLinearFunction.apply(
                    feature_indices_0, feature_indices_1, self.bias, tuple(virtual_rows), *tables)
        merged = self.merged_weight()
        return (
            SparseLinearFunction.apply(feature_indices_0, merged, self.bias),
            SparseLinearFunction.apply(feature_indices_1, merged, self.bias),
        )

    @torch.no_grad()
    def coalesce(self) -> None:
        for f in self.features:
            f.coalesce()

    @torch.no_grad()
    def init_weights(self, num_psqt_buckets: int, nnue2score: float) -> None:
        for f in self.features:
            f.init_weights(num_psqt_buckets, nnue2score)
        self.bias[self.num_outputs - num_psqt_buckets:] = 0.0

    @torch.no_grad()
    def get_export_weights(self) -> torch.Tensor:
        return torch.cat([f.get_export_weights() for f in self.features], dim=0)

    @torch.no_grad()
    def load_export_weights(self, export_weight: torch.Tensor) -> None:
        start = 0
        for f in self.features:
            stop = start + f.NUM_REAL_FEATURES
            f.load_export_weights(export_weight[start:stop])
            start = stop

    def clip_weights(self, quantization) -> None:
        for f in self.features:
            f.clip_weights(quantization)


def combine_input_features(*feature_classes: type):
    """Factory num_outputs -> ComposedFeatureTransformer over the given feature classes."""

    def factory(num_outputs: int) -> ComposedFeatureTransformer:
        return ComposedFeatureTransformer([fc(num_outputs) for fc in feature_classes])

    return factory
