"""ctypes front-end of the C oracle (``oracle/ft_oracle.c``).

TEST INFRASTRUCTURE ONLY: imported by ``tests/``, the smoke check and the
benchmark's CPU-baseline leg, never by the product path.  Every function takes
and returns numpy arrays and restates one piece of the reference FT arithmetic
(see the C file for the reference file:line each one follows).

Functions:
  fwd_f32(idx, W, b)            ordered binary32 forward  (FT/kernel.py:89-103)
  fwd_f64(idx, W, b)            binary64 forward
  bwd_f32(idx, G, N, dW0, db0)  reference-order binary32 backward (FT/kernel.py:108-138,167-186,269)
  bwd_f64(idx, G, N)            binary64 backward
  fwd_i16(idx, Wq, bq, ...)     integer quantized forward (closed form)
  quantize_i16(x, scale, clamp) export quantization (src/model/quantize.py:83-84)
"""

from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "_build", "libft_oracle.so")
_lib = None

_i32p = ctypes.POINTER(ctypes.c_int32)
_i16p = ctypes.POINTER(ctypes.c_int16)
_f32p = ctypes.POINTER(ctypes.c_float)
_f64p = ctypes.POINTER(ctypes.c_double)
_i64 = ctypes.c_int64
_i32 = ctypes.c_int32


def build() -> str:
    """Compile the oracle with oracle/Makefile (always re-runs make)."""
    subprocess.run(["make", "-s", "-C", _HERE], check=True)
    return _LIB_PATH


def _load():
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(_LIB_PATH):
        build()
    lib = ctypes.CDLL(_LIB_PATH)
    lib.oracle_ft_fwd_f32.argtypes = [_i32p, _i64, _i32, _f32p, _i64, _i32, _f32p, _f32p]
    lib.oracle_ft_fwd_f64.argtypes = [_i32p, _i64, _i32, _f32p, _i64, _i32, _f32p, _f64p]
    lib.oracle_ft_bwd_f32.argtypes = [_i32p, _i64, _i32, _f32p, _i64, _i32, _f32p, _f32p]
    lib.oracle_ft_bwd_f64.argtypes = [_i32p, _i64, _i32, _f32p, _i64, _i32, _f64p, _f64p]
    lib.oracle_ft_fwd_i16.argtypes = [
        _i32p, _i64, _i32, _i16p, _i64, _i32, _i16p, _i32p, _i32, _i16p, _i32p, _i32, _i32, _i32,
    ]
    lib.oracle_quantize_i16.argtypes = [_f32p, _i64, ctypes.c_float, _i32, _i16p]
    for name in ("oracle_ft_fwd_f32", "oracle_ft_fwd_f64", "oracle_ft_bwd_f32",
                 "oracle_ft_bwd_f64", "oracle_ft_fwd_i16", "oracle_quantize_i16"):
        getattr(lib, name).restype = ctypes.c_int
    _lib = lib
    return lib


def _p(a: np.ndarray, t):
    return a.ctypes.data_as(t)


def _c(a, dtype):
    return np.ascontiguousarray(a, dtype=dtype)


def _check(rc: int, what: str) -> None:
    if rc != 0:
        raise ValueError(f"oracle {what} failed with code {rc}")


def fwd_f32(idx, W, b) -> np.ndarray:
    idx, W, b = _c(idx, np.int32), _c(W, np.float32), _c(b, np.float32)
    B, K = idx.shape
    N, L = W.shape
    out = np.empty((B, L), np.float32)
    _check(_load().oracle_ft_fwd_f32(_p(idx, _i32p), B, K, _p(W, _f32p), N, L, _p(b, _f32p),
                                     _p(out, _f32p)), "fwd_f32")
    return out


def fwd_f64(idx, W, b) -> np.ndarray:
    idx, W, b = _c(idx, np.int32), _c(W, np.float32), _c(b, np.float32)
    B, K = idx.shape
    N, L = W.shape
    out = np.empty((B, L), np.float64)
    _check(_load().oracle_ft_fwd_f64(_p(idx, _i32p), B, K, _p(W, _f32p), N, L, _p(b, _f32p),
                                     _p(out, _f64p)), "fwd_f64")
    return out


def bwd_f32(idx, G, N: int, dW0=None, db0=None):
    """Reference-order backward; accumulates onto dW0/db0 (zeros when None)."""
    idx, G = _c(idx, np.int32), _c(G, np.float32)
    B, K = idx.shape
    L = G.shape[1]
    dW = np.zeros((N, L), np.float32) if dW0 is None else _c(dW0, np.float32).copy()
    db = np.zeros((L,), np.float32) if db0 is None else _c(db0, np.float32).copy()
    _check(_load().oracle_ft_bwd_f32(_p(idx, _i32p), B, K, _p(G, _f32p), N, L, _p(dW, _f32p),
                                     _p(db, _f32p)), "bwd_f32")
    return dW, db


def bwd_f64(idx, G, N: int):
    idx, G = _c(idx, np.int32), _c(G, np.float32)
    B, K = idx.shape
    L = G.shape[1]
    dW = np.zeros((N, L), np.float64)
    db = np.zeros((L,), np.float64)
    _check(_load().oracle_ft_bwd_f64(_p(idx, _i32p), B, K, _p(G, _f32p), N, L, _p(dW, _f64p),
                                     _p(db, _f64p)), "bwd_f64")
    return dW, db


def fwd_i16(idx, Wq, bq, psqt=None, clip_lo: int = 0, clip_hi: int = 127, wrap16: bool = False):
    idx, Wq, bq = _c(idx, np.int32), _c(Wq, np.int16), _c(bq, np.int16)
    B, K = idx.shape
    N, L = Wq.shape
    out = np.empty((B, L), np.int16)
    if psqt is not None:
        psqt = _c(psqt, np.int32)
        P = psqt.shape[1]
        pout = np.empty((B, P), np.int32)
        pp, pop = _p(psqt, _i32p), _p(pout, _i32p)
    else:
        P, pout, pp, pop = 0, None, None, None
    _check(_load().oracle_ft_fwd_i16(_p(idx, _i32p), B, K, _p(Wq, _i16p), N, L, _p(bq, _i16p),
                                     pp, P, _p(out, _i16p), pop, clip_lo, clip_hi,
                                     1 if wrap16 else 0), "fwd_i16")
    return out, pout


def quantize_i16(x, scale: float, clamp: bool = True) -> np.ndarray:
    x = _c(x, np.float32)
    out = np.empty(x.shape, np.int16)
    _check(_load().oracle_quantize_i16(_p(x, _f32p), x.size, float(scale), 1 if clamp else 0,
                                       _p(out, _i16p)), "quantize_i16")
    return out


def rownorm_rel_err(y, y_ref) -> float:
    """max over rows of ||y - y_ref||_inf / max(||y_ref||_inf, tiny)."""
    y = np.asarray(y, np.float64)
    y_ref = np.asarray(y_ref, np.float64)
    if y.ndim == 1:
        y, y_ref = y[None, :], y_ref[None, :]
    num = np.abs(y - y_ref).max(axis=1)
    den = np.maximum(np.abs(y_ref).max(axis=1), 1e-30)
    return float((num / den).max()) if num.size else 0.0
