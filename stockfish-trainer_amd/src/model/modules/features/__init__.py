from collections.abc import Callable

from .composed import ComposedFeatureTransformer, combine_input_features
from .full_threats import FullThreats
from .halfka_v2_hm import HalfKav2Hm
from .input_feature import InputFeature

_FEATURE_COMPONENTS = {
    "HalfKAv2_hm^": HalfKav2Hm,
    "Full_Threats": FullThreats,
}


def get_feature_cls(name: str) -> Callable[[int], ComposedFeatureTransformer]:
    """'A+B' -> factory of a ComposedFeatureTransformer over blocks A then B."""
    return combine_input_features(*(_FEATURE_COMPONENTS[p] for p in name.split("+")))


__all__ = [
    "ComposedFeatureTransformer",
    "combine_input_features",
    "HalfKav2Hm",
    "FullThreats",
    "InputFeature",
    "get_feature_cls",
]
