"""Signed LEB128 and the .nnue FT section, restated for the tests.

TEST INFRASTRUCTURE ONLY: imported by ``tests/`` and never by the product path.

  encode(arr) -> bytes               per-value loop of src/scripts/serialize.py:61-73
  decode(buf, n) -> int64 array      vectorised inverse (for round trips)
  ft_section(...) -> bytes           src/scripts/serialize.py:186, 195-224, 254-275 with the
                                     numpy/C quantizers of ft_oracle
"""

from __future__ import annotations

import struct

import numpy as np

from . import ft_oracle

LEB128_MAGIC = b"COMPRESSED_LEB128"


def encode(arr) -> bytes:
    out = bytearray()
    for raw in np.asarray(arr).reshape(-1):
        value = int(raw)
        while True:
            byte = value & 0x7F
            value >>= 7
            if (value == 0 and (byte & 0x40) == 0) or (value == -1 and (byte & 0x40) != 0):
                out.append(byte)
                break
            out.append(byte | 0x80)
    return bytes(out)


def decode(buf: bytes, n: int) -> np.ndarray:
    b = np.frombuffer(buf, np.uint8).astype(np.int64)
    ends = np.nonzero((b & 0x80) == 0)[0]
    if len(ends) != n or (len(b) and ends[-1] != len(b) - 1):
        raise ValueError("malformed LEB128 stream")
    starts = np.concatenate([[0], ends[:-1] + 1])
    pos = np.arange(len(b)) - np.repeat(starts, ends - starts + 1)
    vals = np.zeros(n, np.int64)
    owner = np.repeat(np.arange(n), ends - starts + 1)
    np.add.at(vals, owner, (b & 0x7F) << (7 * pos))
    nbits = 7 * (ends - starts + 1)
    sign = (b[ends] & 0x40) != 0
    vals = np.where(sign, vals - (np.int64(1) << nbits), vals)
    return vals


def _tensor(arr, compression: str) -> bytes:
    if compression == "none":
        return np.ascontiguousarray(arr).tobytes()
    payload = encode(arr)
    return LEB128_MAGIC + struct.pack("<I", len(payload)) + payload


def ft_section(feature_hash: int, l1: int, bias, export_weight, feature_blocks, ft_one: float, psqt_scale: float,
               compression: str = "leb128") -> bytes:
    """feature_blocks: [(num_real_features, export dtype name "int8" or "int16")] in order."""
    out = bytearray(struct.pack("<I", (feature_hash ^ (l1 * 2)) & 0xFFFFFFFF))
    bias_q = ft_oracle.quantize_i16(np.asarray(bias, np.float32)[:l1], ft_one)
    w = np.asarray(export_weight, np.float32)
    weight_q = ft_oracle.quantize_i16(np.ascontiguousarray(w[:, :l1]), ft_one)
    psqt_q = np.rint((w[:, l1:] * np.float32(psqt_scale)).astype(np.float32)).astype(np.int32)
    out += _tensor(bias_q, compression)
    off = 0
    for n, dtype in feature_blocks:
        seg = weight_q[off:off + n]
        out += _tensor(seg.astype(np.int8), "none") if dtype == "int8" else _tensor(seg, compression)
        off += n
    out += _tensor(psqt_q, compression)
    return bytes(out)
