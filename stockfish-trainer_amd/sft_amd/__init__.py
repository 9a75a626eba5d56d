"""MI355X-native sparse feature-transformer (FT) library: native binding,
synthetic workloads and the quantized inference op.  The reference-shaped
Python surface lives beside this package under ``src/model``."""

from . import _native  # noqa: F401
