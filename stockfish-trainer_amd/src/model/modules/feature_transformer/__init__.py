from .functions import SparseLinearFunction
from .composed_function import ComposedSparseLinearFunction

__all__ = [
    "SparseLinearFunction",
    "ComposedSparseLinearFunction",
]
