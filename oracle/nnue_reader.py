"""A reader of the .nnue layout, for round trips of the writer.

TEST INFRASTRUCTURE ONLY: imported by ``tests/`` and never by the product path.

Parses what src/scripts/serialize.py writes (layout at :125-196): the header
(:165-180), the FT section (:182-224, LEB128 per :51, :254-275), the MoE router
(:228-246) and the FC buckets (:188-196, :250-268), given the architecture the
file was written for.  It also computes the engine's FC-layer hash as the chain
of layer hashes the engine composes (InputSlice, then per layer AffineTransform
and its ClippedReLU), a different formulation from the writer's single loop.
"""

from __future__ import annotations

import struct

import numpy as np

from . import leb128_oracle as leb


def engine_fc_hash(L1: int, out_features) -> int:
    M = 0xFFFFFFFF

    def input_slice(dims):
        return (0xEC42E90D ^ dims) & M

    def affine(prev, out_dims):
        h = (0xCC03DAE4 + out_dims) & M
        return (h ^ (prev >> 1) ^ ((prev << 31) & M)) & M

    def clipped_relu(prev):
        return (0x538D24C7 + prev) & M

    h = input_slice(2 * L1)
    for n in out_features:
        h = affine(h, n)
        if n != 1:
            h = clipped_relu(h)
    return h


class Reader:
    def __init__(self, buf: bytes):
        self.buf = bytes(buf)
        self.at = 0

    def u32(self) -> int:
        (v,) = struct.unpack_from("<I", self.buf, self.at)
        self.at += 4
        return v

    def raw(self, n: int) -> bytes:
        out = self.buf[self.at:self.at + n]
        if len(out) != n:
            raise ValueError("truncated file")
        self.at += n
        return out

    def array(self, dtype, n: int) -> np.ndarray:
        size = np.dtype(dtype).itemsize * n
        return np.frombuffer(self.raw(size), dtype=dtype).copy()

    def tensor(self, dtype, n: int, compressed: bool) -> np.ndarray:
        if not compressed:
            return self.array(dtype, n)
        if self.raw(len(leb.LEB128_MAGIC)) != leb.LEB128_MAGIC:
            raise ValueError("missing LEB128 magic")
        size = self.u32()
        return leb.decode(self.raw(size), n).astype(dtype)


def read_nnue(buf: bytes, *, L1: int, blocks, psqt: int, fc_shapes, buckets: int, moe: bool = False,
              ft_compressed: bool = True) -> dict:
    """blocks: [(rows, "int8" | "int16")] of the FT; fc_shapes: [(out, in)] of l1, l2, output."""
    r = Reader(buf)
    out = {"version": r.u32(), "hash": r.u32()}
    out["description"] = r.raw(r.u32()).decode("utf-8")
    out["ft_hash"] = r.u32()
    out["ft_bias"] = r.tensor(np.int16, L1, ft_compressed)
    out["ft_blocks"] = []
    for rows, dt in blocks:
        if dt == "int8":
            out["ft_blocks"].append(r.array(np.int8, rows * L1).reshape(rows, L1))
        else:
            out["ft_blocks"].append(r.tensor(np.int16, rows * L1, ft_compressed).reshape(rows, L1))
    out["psqt"] = r.tensor(np.int32, sum(rows for rows, _ in blocks) * psqt, ft_compressed)
    if moe:
        out["router_bias"] = r.array(np.int32, 8)
        out["router_weight"] = r.array(np.int8, 8 * 64).reshape(8, 64)
    out["buckets"] = []
    for _ in range(buckets):
        h = r.u32()
        layers = []
        for n_out, n_in in fc_shapes:
            pad = (n_in + 31) // 32 * 32
            b = r.array(np.int32, n_out)
            w = r.array(np.int8, n_out * pad).reshape(n_out, pad)
            layers.append((b, w))
        out["buckets"].append((h, layers))
    out["trailing"] = len(r.buf) - r.at
    return out
