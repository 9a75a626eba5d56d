"""Full_Threats feature block (reference src/model/modules/features/full_threats.py:7-53):
60 720 rows, up to 128 active, no virtual rows, exported as int8."""

import torch
from torch import nn

from .input_feature import InputFeature


class FullThreats(InputFeature):
    HASH = 0x8F234CB8
    FEATURE_NAME = "Full_Threats"
    INPUT_FEATURE_NAME = "Full_Threats"
    MAX_ACTIVE_FEATURES = 128

    NUM_INPUTS = 60720
    NUM_REAL_FEATURES = 60720
    EXPORT_WEIGHT_DTYPE = torch.int8

    def __init__(self, num_outputs: int):
        super().__init__()
        self.num_outputs = num_outputs
        self.weight = nn.Parameter(torch.empty(self.NUM_INPUTS, num_outputs, dtype=torch.float32))
        self.reset_parameters()

    def merged_weight(self) -> torch.Tensor:
        return self.weight

    def table_blocks(self):
        return self.weight, None

    @torch.no_grad()
    def coalesce(self) -> None:
        return None

    @torch.no_grad()
    def init_weights(self, num_psqt_buckets: int, nnue2score: float) -> None:
        # threats carry no material value: PSQT columns start at zero
        self.weight[:, self.num_outputs - num_psqt_buckets:] = 0.0

    @torch.no_grad()
    def get_export_weights(self) -> torch.Tensor:
        return self.weight.detach().clone()

    @torch.no_grad()
    def load_export_weights(self, export_weight: torch.Tensor) -> None:
        self.weight.copy_(export_weight)

    def clip_weights(self, quantization) -> None:
        self.weight.data.clamp_(quantization.min_threat_weight, quantization.max_threat_weight)
