"""The .nnue writer around the FT section (src/scripts/serialize.py): the FC
hash against the engine's chain of layer hashes, the FC quantizer against its
closed form, the stack modes, and whole files parsed back by an independent
reader -- here with the FT section from the oracle's CPU restatement (the GPU
test writes it with the device encoder)."""

import struct

import numpy as np
import pytest
import torch

from nnue_model import Model
from oracle import leb128_oracle as leb
from oracle import nnue_reader
from src.model.quantize import QuantizationConfig, QuantizationManager
from src.scripts import serialize


@pytest.mark.parametrize("L1,outs", [(1024, (16, 32, 1)), (3072, (16, 32, 1)), (128, (8, 1)), (64, (1,)),
                                     (32, (5, 7, 9)), (520, (31, 32, 1))])
def test_fc_hash_is_the_engine_chain(L1, outs):
    assert serialize.fc_hash(L1, outs) == nnue_reader.engine_fc_hash(L1, outs)


def test_fc_hash_sees_every_dimension():
    base = serialize.fc_hash(1024, (16, 32, 1))
    assert base != serialize.fc_hash(1032, (16, 32, 1))
    assert base != serialize.fc_hash(1024, (15, 32, 1))
    assert base != serialize.fc_hash(1024, (16, 31, 1))
    assert base != serialize.fc_hash(1024, (16, 32, 2))


def test_fc_quantizer_closed_form():
    q = QuantizationManager(QuantizationConfig())
    # hidden layers: weight x 64 clamped to +-127/64, bias x 64 * 127; round half to even
    w = torch.tensor([[2.5 / 64, 3.5 / 64, -2.5 / 64, 5.0, -5.0, 0.0]])
    b = torch.tensor([0.5 / (64 * 127), 1.5 / (64 * 127)])
    bq, wq = q.quantize_fc_layer(b, w.repeat(2, 1))
    assert bq.dtype == torch.int32 and wq.dtype == torch.int8
    assert bq.tolist() == [0, 2]
    assert wq[0].tolist() == [2, 4, -2, 127, -127, 0]
    # output layer: weight x 600 * 16 / 127, bias x 16 * 600
    so = 600 * 16 / 127
    bq, wq = q.quantize_fc_layer(torch.tensor([1.0]), torch.tensor([[1.0, 10.0, -10.0]]), output_layer=True)
    assert bq.tolist() == [9600]
    assert wq.tolist() == [[round(so), 127, -127]]
    seen = {}
    q.quantize_fc_layer(b, w, callback=lambda *a: seen.update(n=int(a[2]), total=a[3], bound=a[5]))
    assert seen == {"n": 2, "total": 6, "bound": 127 / 64}
    db, dw = q.dequantize_fc_layer(*q.quantize_fc_layer(b, w))
    assert torch.allclose(dw, torch.clamp(w, -127 / 64, 127 / 64), atol=0.5 / 64)


def test_stack_modes():
    assert serialize.stack_mode_of(Model(count=1)) == "layer"
    assert serialize.stack_mode_of(Model(count=1, stacks="none")) == "none"
    assert serialize.stack_mode_of(Model(count=1, moe=True)) == "moe"
    assert serialize.stack_mode_of(Model(count=1), "none") == "none"
    with pytest.raises(ValueError):
        serialize.stack_mode_of(Model(count=1, moe=True), "layer")
    with pytest.raises(ValueError):
        serialize.stack_mode_of(Model(count=1), "moe")


class _CpuFT:
    """The FT section from the oracle's CPU restatement (the device writer is
    checked against the same bytes in tests/test_gpu_export.py)."""

    def __init__(self, ft, l1, q, ft_compression="leb128", pad_l1=None):
        assert pad_l1 is None
        blocks = [(int(f.NUM_REAL_FEATURES), "int8" if f.EXPORT_WEIGHT_DTYPE == torch.int8 else "int16")
                  for f in ft.features]
        with torch.no_grad():
            self.buf = leb.ft_section(ft.HASH, l1, ft.bias.numpy(), ft.get_export_weights().numpy(), blocks,
                                      q.ft_quantized_one, q.psqt_scale, ft_compression)


def _check_file(m, buf, mode, compressed=True):
    blocks = [(int(f.NUM_REAL_FEATURES), "int8" if f.EXPORT_WEIGHT_DTYPE == torch.int8 else "int16")
              for f in m.input.features]
    st = m.layer_stacks
    shapes = [(b.weight.shape[0], b.weight.shape[1]) for b in st.buckets[0]]
    nb = 1 if mode == "none" else st.count
    got = nnue_reader.read_nnue(buf, L1=m.L1, blocks=blocks, psqt=8, fc_shapes=shapes, buckets=nb,
                                moe=mode == "moe", ft_compressed=compressed)
    assert got["trailing"] == 0
    assert got["version"] == 0x7AF32F20
    h_fc = nnue_reader.engine_fc_hash(m.L1, (st.l1.out_features, st.l2.out_features, 1))
    salt = {"layer": 0, "none": 0x61E90A17, "moe": 0}[mode]
    want_hash = h_fc ^ m.input.HASH ^ (2 * m.L1) ^ salt ^ (0xABCD123C if mode == "moe" else 0)
    assert got["hash"] == want_hash
    assert got["ft_hash"] == m.input.HASH ^ (2 * m.L1)
    q = m.quantization
    for i, (h, layers) in enumerate(got["buckets"]):
        assert h == h_fc
        for j, ((bq, wq), lin) in enumerate(zip(layers, st.buckets[i])):
            wb, ww = q.quantize_fc_layer(lin.bias.data.cpu(), lin.weight.data.cpu(), output_layer=j == 2)
            n_in = ww.shape[1]
            assert np.array_equal(bq, wb.numpy())
            assert np.array_equal(wq[:, :n_in], ww.numpy())
            assert not wq[:, n_in:].any()  # zero padding to 32 inputs
    if mode == "moe":
        rb, rw = q.quantize_fc_layer(st.router.bias.data, st.router.weight.data)
        assert np.array_equal(got["router_bias"], rb.numpy()) and np.array_equal(got["router_weight"], rw.numpy())
    return got


@pytest.mark.parametrize("mode", ["layer", "none", "moe"])
@pytest.mark.parametrize("compression", ["leb128", "none"])
def test_writer_layout_round_trip(monkeypatch, mode, compression):
    monkeypatch.setattr(serialize, "FeatureTransformerWriter", _CpuFT)
    m = Model(L1=64, L2=15, L3=32, count=8, stacks="none" if mode == "none" else "layer", moe=mode == "moe")
    buf = bytes(serialize.NNUEWriter(m, description="test net é", ft_compression=compression).buf)
    got = _check_file(m, buf, mode, compression == "leb128")
    assert got["description"] == "test net é"
    ft = _CpuFT(m.input, m.L1, m.quantization, compression).buf
    assert ft in buf  # the FT section follows the header unchanged
    desc = "test net é".encode()
    assert buf[12 + len(desc):12 + len(desc) + len(ft)] == ft
    assert struct.unpack_from("<I", buf, 8)[0] == len(desc)


def test_writer_default_description_and_pad_check(monkeypatch):
    monkeypatch.setattr(serialize, "FeatureTransformerWriter", _CpuFT)
    m = Model(L1=32, count=2)
    got = _check_file(m, bytes(serialize.NNUEWriter(m).buf), "layer")
    assert got["description"] == serialize.DEFAULT_DESCRIPTION
    with pytest.raises(ValueError):
        serialize.NNUEWriter(m, pad_l1=16)
