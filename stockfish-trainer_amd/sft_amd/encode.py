"""Feature-index encoding on the GPU: positions -> the FT's input batch.

The reference's loader (src/rust/pipeline.rs, src/rust/feature_extraction.rs)
decodes binpack entries on CPU threads, computes every position's index rows
there and copies the int32 slabs to the device (src/data/device.py:63-82).
`encode_batch` takes the positions themselves (65 bytes each, already on the
device) and produces the same tensors with one kernel:

    us [B, 1] float32, white / black [B, K] int32, psqt_indices and
    layer_stack_indices [B] int64

for a feature-set name such as "HalfKAv2_hm" or "Full_Threats+HalfKAv2_hm"
(components in that order, src/rust/feature_extraction.rs:239-266).
"""

from __future__ import annotations

import torch

from . import _native

COMPONENTS = {"Full_Threats": _native.SFT_FEATURES_THREATS, "HalfKAv2_hm": _native.SFT_FEATURES_HALFKA}
MAX_ACTIVE = {"Full_Threats": 128, "HalfKAv2_hm": 32}


def parse_feature_set(name: str):
    """"A+B" -> component ids; a trailing '^' (the trainer's factorised variants) is ignored."""
    parts = name.rstrip("^").split("+")
    try:
        return [COMPONENTS[p.rstrip("^")] for p in parts], sum(MAX_ACTIVE[p.rstrip("^")] for p in parts)
    except KeyError as e:
        raise ValueError(f"unknown feature component in {name!r}") from e


def encode_batch(boards: torch.Tensor, side_to_move: torch.Tensor, feature_set: str, with_counts: bool = False):
    comps, K = parse_feature_set(feature_set)
    B = boards.shape[0]
    dev = boards.device
    white = torch.empty(B, K, dtype=torch.int32, device=dev)
    black = torch.empty(B, K, dtype=torch.int32, device=dev)
    us = torch.empty(B, 1, dtype=torch.float32, device=dev)
    psqt = torch.empty(B, dtype=torch.int64, device=dev)
    ls = torch.empty(B, dtype=torch.int64, device=dev)
    counts = (torch.empty(B, dtype=torch.int32, device=dev), torch.empty(B, dtype=torch.int32, device=dev)) \
        if with_counts else (None, None)
    _native.encode_features(boards.contiguous(), side_to_move.contiguous(), comps, white, black, us, psqt, ls,
                            *counts)
    out = {"us": us, "white": white, "black": black, "psqt_indices": psqt, "layer_stack_indices": ls}
    if with_counts:
        out["white_count"], out["black_count"] = counts
    return out
