"""FT-path modules: the sparse linear op and the feature blocks that feed it.
(The reference package also holds the dense layer stacks after the FT; they
run unchanged on PyTorch and are not part of this package.)"""

from .features import get_feature_cls
from .feature_transformer import SparseLinearFunction

__all__ = ["get_feature_cls", "SparseLinearFunction"]
