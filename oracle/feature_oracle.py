"""ctypes front-end of the feature-encoder oracle (``oracle/feature_oracle.c``).

TEST INFRASTRUCTURE ONLY: imported by ``tests/`` and the benchmark's
CPU-baseline leg, never by the product path.

  encode(boards, stm, components) -> dict(white, black, us, psqt, count_w, count_b, overflow)
  threat_total(), threat_table()

boards: uint8 [B, 64] piece id per square (2 * type + color; 255 empty),
stm: uint8 [B] (0 white to move); components: a sequence of "Full_Threats" /
"HalfKAv2_hm" in feature-set order (src/rust/feature_extraction.rs:209-236).
"""

from __future__ import annotations

import ctypes
import os

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "_build", "libfeature_oracle.so")
_lib = None
COMPONENT_IDS = {"Full_Threats": 1, "HalfKAv2_hm": 2}
COMPONENT_MAX = {"Full_Threats": 128, "HalfKAv2_hm": 32}


def _load():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            from . import ft_oracle
            ft_oracle.build()
        _lib = ctypes.CDLL(_LIB_PATH)
    return _lib


def _p(a):
    return a.ctypes.data_as(ctypes.c_void_p)


def threat_total() -> int:
    return int(_load().feature_oracle_threat_total())


def threat_table() -> np.ndarray:
    t = np.zeros((12, 66), np.int32)
    _load().feature_oracle_threat_table(_p(t))
    return t


def encode(boards, stm, components) -> dict:
    boards = np.ascontiguousarray(boards, np.uint8)
    stm = np.ascontiguousarray(stm, np.uint8)
    B = boards.shape[0]
    comps = np.array([COMPONENT_IDS[c] for c in components], np.int32)
    K = sum(COMPONENT_MAX[c] for c in components)
    out = {"white": np.empty((B, K), np.int32), "black": np.empty((B, K), np.int32),
           "us": np.empty(B, np.float32), "psqt": np.empty(B, np.int64),
           "count_w": np.empty(B, np.int64), "count_b": np.empty(B, np.int64)}
    over = ctypes.c_int64(0)
    lib = _load()
    lib.feature_oracle_encode.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int64, ctypes.c_void_p,
                                          ctypes.c_int] + [ctypes.c_void_p] * 6 + [ctypes.POINTER(ctypes.c_int64)]
    rc = lib.feature_oracle_encode(_p(boards), _p(stm), B, _p(comps), len(comps), _p(out["white"]),
                                   _p(out["black"]), _p(out["us"]), _p(out["psqt"]), _p(out["count_w"]),
                                   _p(out["count_b"]), ctypes.byref(over))
    if rc != 0:
        raise ValueError("feature_oracle_encode failed")
    out["overflow"] = int(over.value)
    return out
