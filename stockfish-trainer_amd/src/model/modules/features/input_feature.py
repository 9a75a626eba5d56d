"""Base class of an FT input feature (reference
src/model/modules/features/input_feature.py:8-38): each feature owns its weight
rows and says how many rows, active slots and exported rows it has."""

import math
from abc import ABC, abstractmethod

import torch
from torch import nn


class InputFeature(nn.Module, ABC):
    NAME: str
    HASH: int
    NUM_INPUTS: int
    MAX_ACTIVE_FEATURES: int
    NUM_REAL_FEATURES: int
    EXPORT_WEIGHT_DTYPE: torch.dtype = torch.int16

    @abstractmethod
    def merged_weight(self) -> torch.Tensor:
        """Effective [NUM_INPUTS, num_outputs] table (virtual rows folded in)."""

    def table_blocks(self):
        """(weight, virtual table or None) whose fold is merged_weight(): row r of
        the merged table is weight[r] (+ virtual[r % len(virtual)]).  The default
        hands over merged_weight() itself, without virtual rows."""
        return self.merged_weight(), None

    @abstractmethod
    def coalesce(self) -> None: ...

    @abstractmethod
    def init_weights(self, num_psqt_buckets: int, nnue2score: float) -> None: ...

    @abstractmethod
    def get_export_weights(self) -> torch.Tensor: ...

    @abstractmethod
    def load_export_weights(self, export_weight: torch.Tensor) -> None: ...

    def clip_weights(self, quantization) -> None:
        pass

    def reset_parameters(self):
        bound = math.sqrt(1.0 / self.NUM_INPUTS)
        with torch.no_grad():
            self.weight.uniform_(-bound, bound)
