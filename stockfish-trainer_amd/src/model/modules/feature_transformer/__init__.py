from .functions import SparseLinearFunction

__all__ = [
    "SparseLinearFunction",
]
