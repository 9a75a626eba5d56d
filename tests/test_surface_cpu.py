"""Host-side behaviour of the reference-shaped Python surface (no GPU)."""

import numpy as np
import pytest
import torch

from sft_amd import _native, workloads
from src.model.modules.feature_transformer import SparseLinearFunction
from src.model.modules.feature_transformer.kernel import (
    make_sparse_input_linear_backward_kernel,
    make_sparse_input_linear_forward_kernel,
)
from src.model.modules.features import get_feature_cls
from src.model.modules.features.halfka_v2_hm import HalfKav2Hm, KingBuckets, halfka_index
from src.model.quantize import QuantizationConfig, QuantizationManager


def test_sparse_linear_asserts_gpu_tensors_like_the_reference():
    idx = torch.zeros(2, 4, dtype=torch.int32)
    W = torch.zeros(10, 8)
    b = torch.zeros(8)
    with pytest.raises(AssertionError):
        SparseLinearFunction.apply(idx, W, b)
    with pytest.raises(AssertionError):
        SparseLinearFunction.apply(idx.long(), W, b)


def test_native_calls_refuse_cpu_tensors():
    idx = torch.zeros(2, 4, dtype=torch.int32)
    with pytest.raises(ValueError):
        _native.ft_fwd_f32(idx, torch.zeros(10, 8), torch.zeros(8), torch.zeros(2, 8))
    with pytest.raises(ValueError):
        _native.ft_bwd_f32(idx, torch.zeros(10, 8), torch.zeros(8), torch.zeros(2, 8))


def test_factories_cache_per_shape_and_check_shapes():
    f1 = make_sparse_input_linear_forward_kernel(32, 1048)
    assert f1 is make_sparse_input_linear_forward_kernel(32, 1048)
    assert f1 is not make_sparse_input_linear_forward_kernel(32, 136)
    b1 = make_sparse_input_linear_backward_kernel(32, 1048)
    assert b1 is make_sparse_input_linear_backward_kernel(32, 1048)
    with pytest.raises(ValueError):
        f1(torch.zeros(2, 31, dtype=torch.int32), torch.zeros(5, 1048), torch.zeros(1048), torch.zeros(2, 1048))
    with pytest.raises(ValueError):
        b1(torch.zeros(2, 32, dtype=torch.int32), torch.zeros(5, 100), torch.zeros(100), torch.zeros(2, 100))


def test_feature_set_sizes():
    ft = get_feature_cls("HalfKAv2_hm^")(1048)
    assert (ft.NUM_INPUTS, ft.MAX_ACTIVE_FEATURES, ft.NUM_REAL_FEATURES) == (24576, 32, 22528)
    ft2 = get_feature_cls("Full_Threats+HalfKAv2_hm^")(1048)
    assert (ft2.NUM_INPUTS, ft2.MAX_ACTIVE_FEATURES) == (85296, 160)
    assert ft2.FEATURE_NAME == "Full_Threats+HalfKAv2_hm^"
    assert ft.HASH == 0x7F234CB8
    assert ft2.HASH == (((0x8F234CB8 << 1) | (0x8F234CB8 >> 31)) & 0xFFFFFFFF) ^ 0x7F234CB8


def test_merged_weight_tiles_virtual_rows():
    ft = get_feature_cls("HalfKAv2_hm^")(16)
    with torch.no_grad():
        ft.features[0].virtual_weight.normal_()
    m = ft.merged_weight()
    f = ft.features[0]
    r = torch.arange(24576)
    assert torch.equal(m, f.weight + f.virtual_weight[r % 768])


def test_king_buckets_match_reference_table_entries():
    # entries of the reference's KingBuckets table (halfka_v2_hm.py:9-18)
    assert KingBuckets[:8] == [-1, -1, -1, -1, 31, 30, 29, 28]
    assert KingBuckets[56:] == [-1, -1, -1, -1, 3, 2, 1, 0]
    assert KingBuckets[28] == 19 and KingBuckets[39] == 12
    assert sorted(b for b in KingBuckets if b >= 0) == list(range(32))


def test_halfka_index_range_and_psqt_signs():
    assert halfka_index(True, 4, 12, 1, True) == (12 ^ 0) + 0 + 768 * KingBuckets[4]
    vals = HalfKav2Hm.halfka_psqts()
    assert len(vals) == 24576
    assert set(vals) == {0, 126, -126, 781, -781, 825, -825, 1276, -1276, 2538, -2538}


def test_export_roundtrip_of_coalesced_table():
    f = HalfKav2Hm(4)
    with torch.no_grad():
        f.weight.normal_()
        w = f.weight.view(32, 768, 4)
        # make the table exportable: own-king plane only on the bucket square,
        # opponent-king plane zero on that square
        from src.model.modules.features.halfka_v2_hm import InverseKingBuckets
        for b in range(32):
            ksq = InverseKingBuckets[b]
            keep = w[b, 640 + ksq].clone()
            w[b, 640:704] = 0
            w[b, 640 + ksq] = keep
            w[b, 704 + ksq] = 0
    before = f.weight.detach().clone()
    f.load_export_weights(f.get_export_weights())
    assert torch.equal(f.weight, before)


def test_quantize_feature_transformer_mirror():
    qm = QuantizationManager(QuantizationConfig())
    g = torch.Generator().manual_seed(3)
    w = torch.randn(100, 9, generator=g) * 0.01
    b = torch.randn(9, generator=g) * 0.01
    p = torch.randn(100, 8, generator=g) * 0.01
    bq, wq, pq = qm.quantize_feature_transformer(b, w, p)
    assert bq.dtype == torch.int16 and wq.dtype == torch.int16 and pq.dtype == torch.int32
    assert torch.equal(wq, torch.round(w * 255).to(torch.int16))
    assert torch.equal(pq, torch.round(p * 9600).to(torch.int32))
    assert np.array_equal(wq.numpy(), workloads.quantize_np(w.numpy(), 255.0))


def test_workload_indices_contract():
    g = np.random.default_rng(0)
    idx = workloads.make_indices(g, 2000, 500, 32, 16, 32)
    n = workloads.active_counts(idx, 500)
    assert n.min() >= 16 and n.max() <= 32
    for r in idx[:200]:
        a = r[r >= 0]
        assert len(np.unique(a)) == len(a) and np.all(np.diff(a) > 0)
        assert np.all(r[len(a):] == -1)
    again = workloads.make_indices(np.random.default_rng(0), 2000, 500, 32, 16, 32)
    assert np.array_equal(idx, again)


def test_zipf_indices_contract_and_skew():
    g = np.random.default_rng(3)
    B, N = 4000, 2000
    idx = workloads.make_zipf_indices(g, B, N, 32, 16, 32, alpha=1.0)
    n = workloads.active_counts(idx, N)
    assert n.min() >= 14 and n.max() <= 32 and n.mean() > 23
    for r in idx[:300]:
        a = r[r >= 0]
        assert len(np.unique(a)) == len(a) and np.all(np.diff(a) > 0)
        assert np.all(r[len(a):] == -1)
    freq = np.bincount(idx[idx >= 0], minlength=N) / B
    # rank 0 of 1 / (rank + 10): probability 1 / (10 H) per draw, H = sum over ranks
    H = (1.0 / (np.arange(N) + 10.0)).sum()
    assert freq.max() > 0.5 * 24 / (10 * H) and freq.max() > 20 * np.median(freq)
    again = workloads.make_zipf_indices(np.random.default_rng(3), B, N, 32, 16, 32, alpha=1.0)
    assert np.array_equal(idx, again)


def test_step_bytes_formula():
    idx = np.array([[0, 1, -1], [2, -1, -1]], np.int32)
    # per perspective per direction: 4K + 4L(n+1); K=3, L=10: (12+120) + (12+80) = 224
    assert workloads.step_bytes(idx, idx, 5, 10) == 2 * 2 * 224 + 4 * 5 * 10
    w = workloads.WORKLOADS[1]
    assert (w.B, w.N, w.K, w.L) == (65536, 23232, 32, 1048)
    # mean active 24: 2 * 2 * (4*32 + 4*1048*25) = 419 712 bytes per position
    assert 2 * 2 * (4 * 32 + 4 * 1048 * 25) == 419712


def test_workload_indices_dense_rows_terminate():
    """Rows holding most of the table (160 of 300) use exact draws without replacement."""
    idx = workloads.make_indices(np.random.default_rng(4), 129, 300, 160, 32, 160, sort=False)
    for r in idx:
        a = r[r >= 0]
        assert 32 <= len(a) <= 160 and len(np.unique(a)) == len(a) and a.max() < 300
