"""int16 quantized forward and the device quantizer: bit-exact with the oracle."""

import numpy as np
import pytest
import torch

from conftest import golden
from gpu_helpers import DEV, announce, dev, host
from oracle import ft_oracle
from sft_amd import _native, workloads
from sft_amd.quantized import QuantizedFeatureTransformer, quantize_weight_i16, quantized_ft_forward

pytestmark = pytest.mark.gpu


def test_q16_fixture():
    announce("q16 fixture")
    d = golden("q16_tiny")
    out, pout = quantized_ft_forward(dev(d["idx"]), dev(d["Wq"]), dev(d["bq"]), dev(d["psqt"]), 0, 127, False)
    assert np.array_equal(host(out), d["out_acc32"]) and np.array_equal(host(pout), d["psqt_out"])
    out, _ = quantized_ft_forward(dev(d["idx"]), dev(d["Wq"]), dev(d["bq"]), None, 0, 127, True)
    assert np.array_equal(host(out), d["out_wrap16"])
    out, _ = quantized_ft_forward(dev(d["idx"]), dev(d["Wq"]), dev(d["bq"]), None, -32768, 32767, True)
    assert np.array_equal(host(out), d["raw_wrap16"])


@pytest.mark.parametrize("seed,B,N,K,L,P", [
    (1, 50, 300, 32, 1040, 8), (2, 77, 64, 7, 13, 3), (3, 129, 1000, 160, 256, 0),
    (4, 1000, 22528, 32, 128, 8), (5, 3, 10, 4, 2104, 8), (6, 40, 100, 32, 520, 64),
    (7, 500, 2000, 32, 512, 8), (8, 300, 700, 13, 1040, 3),
    # tiled without PSQT; PSQT columns 0-4 in a tile of their own (L / 8 % 8 == 0)
    (9, 200, 500, 32, 1024, 0), (10, 150, 900, 20, 1024, 5)])
@pytest.mark.parametrize("wrap16", [False, True])
@pytest.mark.parametrize("rows", [False, True])
def test_q16_matches_oracle(seed, B, N, K, L, P, wrap16, rows):
    announce(f"q16 seed={seed} B={B} N={N} K={K} L={L} P={P} wrap16={wrap16} rows={rows}")
    g = np.random.default_rng(seed)
    idx = workloads.make_indices(g, B, N, K, 0, K, sort=False)
    Wq = g.integers(-3000, 3000, size=(N, L)).astype(np.int16)
    bq = g.integers(-3000, 3000, size=L).astype(np.int16)
    ps = g.integers(-10**6, 10**6, size=(N, P)).astype(np.int32) if P else None
    for lo, hi in ((0, 127), (-32768, 32767), (-100, 255)):
        out, pout = quantized_ft_forward(dev(idx), dev(Wq), dev(bq), None if ps is None else dev(ps), lo, hi, wrap16,
                                         rows)
        ro, rp = ft_oracle.fwd_i16(idx, Wq, bq, ps, lo, hi, wrap16)
        assert np.array_equal(host(out), ro)
        if P:
            assert np.array_equal(host(pout), rp)


@pytest.mark.parametrize("wrap16", [False, True])
@pytest.mark.parametrize("rows", [False, True])
def test_q16_extreme_values(wrap16, rows):
    """Weights drawn from the int16 extremes and their neighbours (sign
    extension of 0x8000 / 0x7fff / 0xffff in either half of a packed pair),
    PSQT weights near the int32 limit over K."""
    announce(f"q16 extremes wrap16={wrap16} rows={rows}")
    g = np.random.default_rng(11)
    B, N, K, L, P = 300, 600, 32, 1040, 8
    idx = workloads.make_indices(g, B, N, K, 0, K, sort=False)
    pool = np.array([-32768, -32767, -1, 0, 1, 32766, 32767], dtype=np.int16)
    Wq = pool[g.integers(0, len(pool), size=(N, L))]
    bq = pool[g.integers(0, len(pool), size=L)]
    lim = (2**31 - 1) // (K + 1)
    ps = np.array([-lim, -1, 0, 1, lim], dtype=np.int32)[g.integers(0, 5, size=(N, P))]
    for lo, hi in ((0, 127), (-32768, 32767)):
        out, pout = quantized_ft_forward(dev(idx), dev(Wq), dev(bq), dev(ps), lo, hi, wrap16, rows)
        ro, rp = ft_oracle.fwd_i16(idx, Wq, bq, ps, lo, hi, wrap16)
        assert np.array_equal(host(out), ro) and np.array_equal(host(pout), rp)


@pytest.mark.parametrize("seed,B,N,K,L,P", [
    (21, 300, 1000, 32, 1040, 8), (22, 77, 500, 13, 1024, 0), (23, 129, 800, 20, 2104, 5), (24, 1, 64, 4, 512, 3),
    (25, 1000, 22528, 32, 1040, 8)])
@pytest.mark.parametrize("wrap16", [False, True])
@pytest.mark.parametrize("ranked", [True, False])
def test_packed_table_matches_oracle(seed, B, N, K, L, P, wrap16, ranked):
    """sft_ft_i16_pack + sft_ft_fwd_i16_packed_ex (ranked: rank lists in a
    workspace) or sft_ft_fwd_i16_packed, both perspectives in one launch and one
    perspective alone, against the oracle."""
    announce(f"q16 packed seed={seed} B={B} N={N} K={K} L={L} P={P} wrap16={wrap16} ranked={ranked}")
    g = np.random.default_rng(seed)
    i0 = workloads.make_indices(g, B, N, K, 0, K, sort=False)
    i1 = workloads.make_indices(g, B, N, K, 0, K, sort=False)
    Wq = g.integers(-32768, 32768, size=(N, L)).astype(np.int16)
    bq = g.integers(-3000, 3000, size=L).astype(np.int16)
    ps = g.integers(-10**6, 10**6, size=(N, P)).astype(np.int32) if P else None
    packed = _native.i16_pack(dev(Wq), None if ps is None else dev(ps))
    assert packed is not None
    for lo, hi in ((0, 127), (-32768, 32767)):
        o = [torch.empty(B, L, dtype=torch.int16, device=DEV) for _ in range(3)]
        po = [torch.empty(B, P, dtype=torch.int32, device=DEV) if P else None for _ in range(3)]
        _native.ft_fwd_i16_packed(packed, N, L, P, dev(bq), dev(i0), o[0], po[0], dev(i1), o[1], po[1], lo, hi, wrap16,
                                  ranked=ranked)
        _native.ft_fwd_i16_packed(packed, N, L, P, dev(bq), dev(i1), o[2], po[2], clip_lo=lo, clip_hi=hi,
                                  wrap16=wrap16, ranked=ranked)
        for j, idx in ((0, i0), (1, i1), (2, i1)):
            ro, rp = ft_oracle.fwd_i16(idx, Wq, bq, ps, lo, hi, wrap16)
            assert np.array_equal(host(o[j]), ro), j
            if P:
                assert np.array_equal(host(po[j]), rp), j


def test_quantized_module_repacks_after_in_place_update():
    announce("q16 module repack")
    g = np.random.default_rng(31)
    B, N, K, L, P = 200, 700, 32, 1040, 8
    i0 = workloads.make_indices(g, B, N, K, 0, K, sort=False)
    i1 = workloads.make_indices(g, B, N, K, 0, K, sort=False)
    Wq = g.integers(-3000, 3000, size=(N, L)).astype(np.int16)
    bq = g.integers(-3000, 3000, size=L).astype(np.int16)
    ps = g.integers(-10**5, 10**5, size=(N, P)).astype(np.int32)
    qft = QuantizedFeatureTransformer(dev(Wq), dev(bq), dev(ps), -32768, 32767)
    assert qft.packed is not None
    qft(dev(i0), dev(i1))
    qft.weight_q.add_(7)  # in place through torch: the version counter moves
    qft.psqt_q.mul_(-1)
    (ow, pw), (ob, pb) = qft(dev(i0), dev(i1))
    for idx, o, p in ((i0, ow, pw), (i1, ob, pb)):
        ro, rp = ft_oracle.fwd_i16(idx, Wq + np.int16(7), bq, -ps, -32768, 32767, False)
        assert np.array_equal(host(o), ro) and np.array_equal(host(p), rp)


@pytest.mark.parametrize("scale", [127.0, 255.0])
def test_full_workload_q16(scale):
    w = workloads.WORKLOADS[4]
    announce(f"q16 workload {w.name} scale={scale}")
    d = workloads.make_q16_inputs(w, scale=scale)
    qft = QuantizedFeatureTransformer(dev(d["Wq"]), dev(d["bq"]), dev(d["psqt"]), 0, 127)
    (ow, pw), (ob, pb) = qft(dev(d["idx_w"]), dev(d["idx_w"][::-1].copy()))
    ro, rp = ft_oracle.fwd_i16(d["idx_w"], d["Wq"], d["bq"], d["psqt"], 0, 127, False)
    assert np.array_equal(host(ow), ro) and np.array_equal(host(pw), rp)
    assert np.array_equal(host(ob), ro[::-1]) and np.array_equal(host(pb), rp[::-1])
    o2, p2 = quantized_ft_forward(dev(d["idx_w"]), dev(d["Wq"]), dev(d["bq"]), dev(d["psqt"]), 0, 127, rows=True)
    assert np.array_equal(host(o2), ro) and np.array_equal(host(p2), rp)


def test_device_quantizer_matches_oracle():
    announce("quantize kernel")
    d = golden("quant_tiny")
    assert np.array_equal(host(quantize_weight_i16(dev(d["x"]), float(d["scale"]))), d["q"])
    g = np.random.default_rng(3)
    x = (g.standard_normal((1000, 1040)) * 0.02).astype(np.float32)
    for scale in (127.0, 255.0):
        assert np.array_equal(host(quantize_weight_i16(dev(x), scale)), ft_oracle.quantize_i16(x, scale))


def test_q16_module_encoder_rows():
    """The int16 forward of both perspectives through QuantizedFeatureTransformer
    (the packed table) over the HalfKAv2_hm rows the GPU encoder makes from
    random positions (one king bucket's rows per perspective, 2-32 active, -1
    after them), at B = 65 536 over the encoder's 24 576-row table: bit-exact
    with the oracle."""
    from sft_amd import encode, positions
    from src.model.modules.features.halfka_v2_hm import HalfKav2Hm

    B, N, L, P = 65536, HalfKav2Hm.NUM_INPUTS, 1040, 8
    announce(f"q16 module, encoder rows B={B} N={N} L={L} P={P}")
    boards, stm = positions.random_positions(B, seed=3)
    enc = encode.encode_batch(torch.from_numpy(boards).to(DEV), torch.from_numpy(stm).to(DEV), "HalfKAv2_hm")
    g = np.random.default_rng(13)
    Wq = g.integers(-3000, 3000, size=(N, L)).astype(np.int16)
    bq = g.integers(-3000, 3000, size=L).astype(np.int16)
    ps = g.integers(-10**6, 10**6, size=(N, P)).astype(np.int32)
    qft = QuantizedFeatureTransformer(dev(Wq), dev(bq), dev(ps), 0, 127)
    (ow, pw), (ob, pb) = qft(enc["white"], enc["black"])
    for o, p, i in ((ow, pw, enc["white"]), (ob, pb, enc["black"])):
        ro, rp = ft_oracle.fwd_i16(host(i), Wq, bq, ps, 0, 127, False)
        assert np.array_equal(host(o), ro)
        assert np.array_equal(host(p), rp)
