"""GPU signed LEB128 (sft_leb128_encode) and the .nnue FT section against the
oracle: identical bytes; full-size weights through a decode round trip."""

import numpy as np
import pytest
import torch

from gpu_helpers import DEV, announce, dev, host
from oracle import leb128_oracle as leb
from sft_amd import _native
from src.model.modules.features import get_feature_cls
from src.model.quantize import QuantizationConfig, QuantizationManager
from src.scripts.serialize import FeatureTransformerWriter

pytestmark = pytest.mark.gpu

LIMITS = {np.int8: [0, 1, -1, 63, 64, -64, -65, 127, -128],
          np.int16: [0, 1, -1, 63, 64, -64, -65, 8191, 8192, -8192, -8193, 32767, -32768],
          np.int32: [0, 1, -1, 8191, 8192, -8193, 1048575, -1048576, 2**31 - 1, -2**31]}


@pytest.mark.parametrize("dtype,n", [(np.int8, 1), (np.int8, 5000), (np.int16, 4097), (np.int16, 100003),
                                     (np.int32, 77777)])
def test_leb128_matches_oracle(dtype, n):
    announce(f"leb128 {dtype.__name__} n={n}")
    g = np.random.default_rng(n)
    info = np.iinfo(dtype)
    a = g.integers(info.min, info.max + 1, n, dtype=np.int64).astype(dtype)
    small = g.integers(-300, 300, n).astype(dtype)
    a = np.where(g.random(n) < 0.7, small, a)
    a[:min(n, len(LIMITS[dtype]))] = LIMITS[dtype][:min(n, len(LIMITS[dtype]))]
    got = host(_native.leb128_encode(dev(a))).tobytes()
    assert got == leb.encode(a)


def test_leb128_empty():
    assert _native.leb128_encode(torch.zeros(0, dtype=torch.int16, device=DEV)).numel() == 0


def test_leb128_full_size_round_trip():
    announce("leb128 22528 x 1040 int16 round trip")
    g = np.random.default_rng(5)
    a = np.clip(np.rint(g.standard_normal((22528, 1040)) * 40), -32768, 32767).astype(np.int16)
    a[0, :4] = [32767, -32768, 8192, -8193]
    buf = host(_native.leb128_encode(dev(a))).tobytes()
    assert np.array_equal(leb.decode(buf, a.size), a.reshape(-1).astype(np.int64))


@pytest.mark.parametrize("name,l1", [("HalfKAv2_hm^", 64), ("Full_Threats+HalfKAv2_hm^", 32)])
def test_ft_section_matches_oracle(name, l1):
    announce(f"nnue FT section {name} L1={l1}")
    torch.manual_seed(2)
    ft = get_feature_cls(name)(l1 + 8).to(DEV)
    with torch.no_grad():
        for f in ft.features:
            f.weight.uniform_(-0.4, 0.4)  # within int8 after the 255 scale (threat rows are int8)
            if hasattr(f, "virtual_weight"):
                f.virtual_weight.uniform_(-0.05, 0.05)
        ft.bias.uniform_(-0.5, 0.5)
    q = QuantizationManager(QuantizationConfig())
    got = bytes(FeatureTransformerWriter(ft, l1, q).buf)
    blocks = [(int(f.NUM_REAL_FEATURES), "int8" if f.EXPORT_WEIGHT_DTYPE == torch.int8 else "int16")
              for f in ft.features]
    want = leb.ft_section(ft.HASH, l1, host(ft.bias), host(ft.get_export_weights()), blocks, q.ft_quantized_one,
                          q.psqt_scale)
    assert got == want


@pytest.mark.parametrize("name,l1,mode", [("HalfKAv2_hm^", 64, "layer"), ("Full_Threats+HalfKAv2_hm^", 32, "moe"),
                                          ("HalfKAv2_hm^", 32, "none")])
def test_whole_nnue_file(name, l1, mode):
    """The whole file with the FT section written on the GPU: its FT bytes are
    the oracle's, and the header, router and FC buckets parse back to the
    quantized layers (tests/test_nnue_writer_cpu.py checks the same layout with
    the CPU FT section)."""
    from nnue_model import Model
    from test_nnue_writer_cpu import _check_file
    from src.scripts.serialize import NNUEWriter

    announce(f"whole .nnue {name} L1={l1} {mode}")
    m = Model(name, L1=l1, count=8, stacks="none" if mode == "none" else "layer", moe=mode == "moe", device=DEV)
    buf = bytes(NNUEWriter(m, description="gpu").buf)
    _check_file(m, buf, mode)
    blocks = [(int(f.NUM_REAL_FEATURES), "int8" if f.EXPORT_WEIGHT_DTYPE == torch.int8 else "int16")
              for f in m.input.features]
    q = m.quantization
    want_ft = leb.ft_section(m.input.HASH, l1, host(m.input.bias), host(m.input.get_export_weights()), blocks,
                             q.ft_quantized_one, q.psqt_scale)
    assert buf[12 + 3:12 + 3 + len(want_ft)] == want_ft
