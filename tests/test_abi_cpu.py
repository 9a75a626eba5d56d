"""The C-ABI library loads, exports what include/sft_ft.h declares, and rejects
bad arguments on the host before any GPU work (no compute calls here)."""

import ctypes
import os
import re

import pytest

from conftest import ROOT
from sft_amd import _native

HEADER = os.path.join(ROOT, "include", "sft_ft.h")
NOALLOC_HEADER = os.path.join(ROOT, "include", "sft_ft_noalloc.h")


def header_functions(path=HEADER):
    text = open(path).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(sft_\w+)\s*\(", text)))


def test_header_declares_the_binding_table():
    assert header_functions() == sorted(_native.SIGNATURES)
    assert header_functions(NOALLOC_HEADER) == sorted(_native.NOALLOC_SIGNATURES)


def test_library_exports_every_declared_symbol():
    lib = _native.lib()
    for name in header_functions():
        assert hasattr(lib, name), name
    noalloc = _native.noalloc_lib()
    for name in header_functions(NOALLOC_HEADER):
        assert hasattr(noalloc, name), name
        assert not hasattr(lib, name), name  # the static scratch lives in the separate library only


def test_abi_version_matches_header():
    m = re.search(r"#define SFT_ABI_VERSION (\d+)", open(HEADER).read())
    assert _native.lib().sft_abi_version() == int(m.group(1))


def test_flag_values_match_header():
    text = open(HEADER).read()
    for name in ("SFT_BWD_OVERWRITE", "SFT_BWD_ATOMIC", "SFT_BWD_ROWS", "SFT_FWD_ROWS", "SFT_Q16_WRAP16", "SFT_Q16_ROWS"):
        m = re.search(rf"#define {name} (0x[0-9a-fA-F]+)u", text)
        assert int(m.group(1), 16) == getattr(_native, name)


P = ctypes.c_void_p(0x1000)  # never dereferenced: every call below must fail validation before any launch


@pytest.mark.parametrize("args,needle", [
    ((None, 4, 2, P, 10, 8, P, P, None), "null pointer"),
    ((P, -1, 2, P, 10, 8, P, P, None), "batch"),
    ((P, 4, 0, P, 10, 8, P, P, None), "max_active"),
    ((P, 4, 2, P, 0, 8, P, P, None), "num_inputs"),
    ((P, 4, 2, P, 10, 0, P, P, None), "output_size"),
    ((P, 4, 2, None, 10, 8, P, P, None), "null pointer"),
    ((P, 2**30, 4, P, 10, 8, P, P, None), "batch * max_active"),
])
def test_fwd_f32_rejects(args, needle):
    lib = _native.lib()
    rc = lib.sft_ft_fwd_f32(*args)
    assert rc == -1
    assert needle in _native.last_error()


def test_fwd_f32_empty_batch_is_a_noop():
    assert _native.lib().sft_ft_fwd_f32(None, 0, 4, P, 10, 8, P, None, None) == 0
    assert _native.last_error() == ""


def test_bwd_rejects_flags_and_pointers():
    lib = _native.lib()
    assert lib.sft_ft_bwd_f32(P, 4, 2, P, 10, 8, P, P, P, 0, 0x100, None) == -1
    assert "flags" in _native.last_error()
    assert lib.sft_ft_bwd_f32(P, 4, 2, P, 10, 8, None, P, P, 0, 0, None) == -1
    assert "null" in _native.last_error()
    n = ctypes.c_size_t(0)
    assert lib.sft_ft_bwd_f32_workspace_size(4, 2, 10, 8, 0x8, ctypes.byref(n)) == -1
    assert lib.sft_ft_bwd_f32_workspace_size(4, 2, 10, 8, 0, None) == -1


def test_i16_rejects():
    lib = _native.lib()
    base = [P, 4, 2, P, 10, 8, P, None, 0, P, None, 0, 127, 0, None]
    a = list(base); a[7] = P  # psqt weight without output
    assert lib.sft_ft_fwd_i16(*a) == -1 and "psqt" in _native.last_error()
    a = list(base); a[7] = P; a[10] = P; a[8] = 65
    assert lib.sft_ft_fwd_i16(*a) == -1 and "psqt_size" in _native.last_error()
    a = list(base); a[11], a[12] = 5, 4
    assert lib.sft_ft_fwd_i16(*a) == -1 and "clip" in _native.last_error()
    a = list(base); a[2] = 70000
    assert lib.sft_ft_fwd_i16(*a) == -1 and "65536" in _native.last_error()
    a = list(base); a[13] = 4  # not a defined flag bit
    assert lib.sft_ft_fwd_i16(*a) == -1 and "flags" in _native.last_error()


def test_i16_noalloc_rejects_before_launch():
    """sft_ft_fwd_i16_noalloc validates like sft_ft_fwd_i16 and refuses a tiled
    shape whose packed table exceeds its static scratch, before any HIP call."""
    lib = _native.noalloc_lib()
    m = re.search(r"#define SFT_NOALLOC_SCRATCH_BYTES \((\d+)u << (\d+)\)", open(NOALLOC_HEADER).read())
    limit = int(m.group(1)) << int(m.group(2))
    base = [P, 4, 32, P, 22528, 1040, P, P, 8, P, P, 0, 127, 0, None]
    a = list(base); a[10] = None  # psqt weight without output
    assert lib.sft_ft_fwd_i16_noalloc(*a) == -1 and "psqt" in _native.last_error()
    a = list(base); a[11], a[12] = 5, 4
    assert lib.sft_ft_fwd_i16_noalloc(*a) == -1 and "clip" in _native.last_error()
    a = list(base); a[13] = 4
    assert lib.sft_ft_fwd_i16_noalloc(*a) == -1 and "flags" in _native.last_error()
    # 500 000 rows x 17 tiles x 128 B = 1.09 GB of packed table (rows x 128 B = 64 MB still tiles)
    a = list(base); a[4] = 500_000
    assert 17 * 500_000 * 128 > limit
    assert lib.sft_ft_fwd_i16_noalloc(*a) == _native.SFT_EWORKSPACE
    err = _native.last_error()
    assert "sft_ft_fwd_i16_noalloc" in err and str(limit) in err and str(17 * 500_000 * 128) in err
    assert 17 * 22528 * 128 <= limit  # the exported HalfKAv2_hm table (1040 + 8 PSQT columns) fits


def test_i16_packed_size_and_pack_checks():
    lib = _native.lib()
    n = ctypes.c_size_t(0)
    # 1040 int16 columns = 130 chunks; 8 PSQT columns = 2 more chunks -> 17 tiles of N * 128 bytes
    assert lib.sft_ft_i16_packed_size(22528, 1040, 8, ctypes.byref(n)) == 0
    assert n.value == 17 * 22528 * 128
    assert lib.sft_ft_i16_packed_size(22528, 1024, 0, ctypes.byref(n)) == 0 and n.value == 16 * 22528 * 128
    assert lib.sft_ft_i16_packed_size(22528, 1024, 5, ctypes.byref(n)) == 0 and n.value == 17 * 22528 * 128
    assert lib.sft_ft_i16_packed_size(22528, 256, 8, ctypes.byref(n)) == _native.SFT_EUNSUPPORTED  # 4 tiles
    assert lib.sft_ft_i16_packed_size(22528, 1040, 9, ctypes.byref(n)) == _native.SFT_EUNSUPPORTED
    assert lib.sft_ft_i16_packed_size(22528, 1040, 8, None) == -1
    assert _native.i16_packed_size(22528, 1044, 8) is None
    # psqt pointer and size must agree; nothing is launched
    assert lib.sft_ft_i16_pack(P, 22528, 1040, None, 8, P, 1 << 30, None) == -1
    assert "psqt_size" in _native.last_error()
    assert lib.sft_ft_i16_pack(P, 22528, 1040, P, 8, P, 1000, None) == _native.SFT_EWORKSPACE


def test_i16_packed_forward_rejects_before_launch():
    lib = _native.lib()
    need = 17 * 22528 * 128
    ok = (P, P, 4, 32, P, need, 22528, 1040, P, 8, P, P, P, P, 0, 127, 0, None)

    def call(**kw):
        names = ["idx0", "idx1", "batch", "max_active", "packed", "packed_bytes", "num_inputs", "output_size",
                 "bias", "psqt_size", "out0", "out1", "psqt_out0", "psqt_out1", "clip_lo", "clip_hi", "flags",
                 "stream"]
        a = dict(zip(names, ok))
        a.update(kw)
        return lib.sft_ft_fwd_i16_packed(*[a[k] for k in names])

    assert call(packed_bytes=need - 1) == -1 and "packed_bytes" in _native.last_error()
    assert call(flags=0x2) == -1 and "flags" in _native.last_error()
    assert call(psqt_out1=None) == -1 and "psqt" in _native.last_error()
    assert call(out1=None) == -1 and "null" in _native.last_error()
    assert call(packed=ctypes.c_void_p(0x1010)) == _native.SFT_EUNSUPPORTED  # not 256-byte aligned
    assert call(psqt_size=9) == _native.SFT_EUNSUPPORTED
    assert call(clip_lo=10, clip_hi=5) == -1
    assert call(batch=0, packed_bytes=need - 1) == -1  # sizes are checked even for an empty batch


def test_i16_packed_ex_workspace_and_rejects_before_launch():
    """The ranked packed forward: its workspace is both perspectives' rank lists;
    it makes the packed forward's checks, then rejects a short or misaligned
    workspace, all before anything runs."""
    lib = _native.lib()
    n = ctypes.c_size_t(0)
    assert lib.sft_ft_fwd_i16_packed_workspace_size(65536, 32, 2, ctypes.byref(n)) == 0
    assert n.value == 2 * rank_lists_bytes(65536, 32)
    assert lib.sft_ft_fwd_i16_packed_workspace_size(65536, 32, 1, ctypes.byref(n)) == 0
    assert n.value == rank_lists_bytes(65536, 32)
    assert lib.sft_ft_fwd_i16_packed_workspace_size(65536, 32, 3, ctypes.byref(n)) == -1
    assert lib.sft_ft_fwd_i16_packed_workspace_size(65536, 65536, 1, ctypes.byref(n)) == -1
    assert lib.sft_ft_fwd_i16_packed_workspace_size(65536, 32, 1, None) == -1
    need = 17 * 22528 * 128
    wsn = 2 * rank_lists_bytes(4, 32)
    ok = (P, P, 4, 32, P, need, 22528, 1040, P, 8, P, P, P, P, 0, 127, P, wsn, 0, None)

    def call(**kw):
        names = ["idx0", "idx1", "batch", "max_active", "packed", "packed_bytes", "num_inputs", "output_size",
                 "bias", "psqt_size", "out0", "out1", "psqt_out0", "psqt_out1", "clip_lo", "clip_hi", "workspace",
                 "workspace_bytes", "flags", "stream"]
        a = dict(zip(names, ok))
        a.update(kw)
        return lib.sft_ft_fwd_i16_packed_ex(*[a[k] for k in names])

    assert call(packed_bytes=need - 1) == -1 and "packed_bytes" in _native.last_error()
    assert call(flags=0x2) == -1 and "flags" in _native.last_error()
    assert call(out1=None) == -1 and "null" in _native.last_error()
    assert call(psqt_size=9) == _native.SFT_EUNSUPPORTED
    assert call(workspace_bytes=wsn - 1) == _native.SFT_EWORKSPACE and "workspace" in _native.last_error()
    assert call(workspace=None) == _native.SFT_EWORKSPACE
    assert call(workspace=ctypes.c_void_p(0x1010)) == _native.SFT_EWORKSPACE  # not 256-byte aligned
    assert call(idx1=None, workspace_bytes=rank_lists_bytes(4, 32) - 1) == _native.SFT_EWORKSPACE


@pytest.mark.parametrize("B", [1, 2, 9000, 16384, 32768, 32769, 65536])
def test_bwd_workspace_holds_the_grad_tiles(B):
    """The tiled backward's bias pass writes ceil(L/32) x B x 128 bytes of grad
    tiles into the workspace whatever the number of position chunks (one for
    batches whose tile fits 4 MB, two above)."""
    n = ctypes.c_size_t(0)
    L, N, K = 1048, 23232, 32
    assert _native.lib().sft_ft_bwd_f32_workspace_size(B, K, N, L, _native.SFT_BWD_OVERWRITE, ctypes.byref(n)) == 0
    assert n.value >= 33 * B * 128 + B * K * 8  # grad tiles + at least the sorted keys and positions


def test_quantize_rejects():
    lib = _native.lib()
    assert lib.sft_quantize_i16(P, -1, 1.0, P, None) == -1
    assert lib.sft_quantize_i16(None, 5, 1.0, P, None) == -1
    assert lib.sft_quantize_i16(None, 0, 1.0, None, None) == 0


def test_error_is_thread_local_and_cleared():
    import threading

    lib = _native.lib()
    assert lib.sft_ft_fwd_f32(None, 4, 2, P, 10, 8, P, P, None) == -1
    seen = []
    t = threading.Thread(target=lambda: seen.append(_native.last_error()))
    t.start()
    t.join()
    assert seen == [""]
    assert "null" in _native.last_error()
    assert lib.sft_abi_version() > 0
    assert lib.sft_ft_fwd_f32(None, 0, 4, P, 10, 8, P, None, None) == 0
    assert _native.last_error() == ""


def test_profiling_kinds_and_empty_collect():
    names = _native.prof_kind_names()
    assert "fwd_f32_gather" in names and "bwd_feature_gather" in names
    _native.prof_enable(True)
    assert _native.prof_collect() == {}
    _native.prof_enable(False)


def _i64s(*v):
    return (ctypes.c_int64 * len(v))(*v)


def _a256(v):
    return (v + 255) // 256 * 256


def rank_lists_bytes(B, K):
    """The forward's rank lists of one perspective: [Bpad][kpad] lists, two
    [Bpad] int32 arrays (position, count) and the [Bpad] 16-byte table-part
    cuts and run offsets, each 256-byte aligned; Bpad = B rounded up to 32,
    kpad = K rounded up to 4."""
    bp, kpad = -(-B // 32) * 32, -(-K // 4) * 4
    return _a256(bp * kpad * 4) + 2 * _a256(bp * 4) + 2 * _a256(bp * 16)


def test_pair_workspace_size_and_shape_checks():
    lib = _native.lib()
    fb, bb = ctypes.c_size_t(0), ctypes.c_size_t(0)
    # HalfKAv2_hm: 24576 rows folded with 768 virtual rows, L = 1048
    rc = lib.sft_ft_pair_workspace_size(65536, 32, 1, _i64s(24576), _i64s(768), 1048, ctypes.byref(fb), ctypes.byref(bb))
    assert rc == 0, _native.last_error()
    # the merged table in 32-column tiles, each with a pad row, then both perspectives' rank lists
    assert fb.value == _a256(33 * 24577 * 32 * 4) + 2 * rank_lists_bytes(65536, 32)
    assert bb.value >= 24576 * 1048 * 4 + 33 * 65536 * 32 * 4  # tmp sums + grad tiles
    # Full_Threats + HalfKAv2_hm
    rc = lib.sft_ft_pair_workspace_size(65536, 160, 2, _i64s(60720, 24576), _i64s(0, 768), 1048, ctypes.byref(fb),
                                        ctypes.byref(bb))
    # three table parts: both perspectives' sums carried between the passes, one 128 B line per position and tile
    assert rc == 0 and fb.value == (_a256(33 * 85297 * 32 * 4) + 2 * rank_lists_bytes(65536, 160) +
                                    2 * _a256(33 * 65536 * 128))
    # shapes the fused path does not take
    rc = lib.sft_ft_pair_workspace_size(65536, 32, 1, _i64s(24576), _i64s(768), 136, ctypes.byref(fb), ctypes.byref(bb))
    assert rc == _native.SFT_EUNSUPPORTED and "output_size" in _native.last_error()
    rc = lib.sft_ft_pair_workspace_size(16, 32, 1, _i64s(600000), _i64s(0), 1048, ctypes.byref(fb), ctypes.byref(bb))
    assert rc == _native.SFT_EUNSUPPORTED
    # invalid descriptions
    for nb, rows, vrows, needle in ((0, (10,), (0,), "num_blocks"), (5, (1,) * 5, (0,) * 5, "num_blocks"),
                                    (1, (1000,), (768,), "divide"), (1, (0,), (0,), "block_rows"),
                                    (1, (100,), (-1,), "divide")):
        rc = lib.sft_ft_pair_workspace_size(16, 32, nb, _i64s(*rows), _i64s(*vrows), 1048, ctypes.byref(fb),
                                            ctypes.byref(bb))
        assert rc == -1 and needle in _native.last_error()


def test_pair_calls_reject_before_launch():
    lib = _native.lib()
    ptrs = (ctypes.c_void_p * 1)(0x1000)
    nulls = (ctypes.c_void_p * 1)(None)
    odd = (ctypes.c_void_p * 1)(0x1008)
    rows, vrows = _i64s(24576), _i64s(768)
    # null virtual table for a block that declares virtual rows
    rc = lib.sft_ft_fwd_pair_f32(P, P, 4, 32, 1, ptrs, nulls, rows, vrows, 1048, P, P, P, P, 1 << 30, None)
    assert rc == -1 and "null" in _native.last_error()
    # misaligned table
    rc = lib.sft_ft_fwd_pair_f32(P, P, 4, 32, 1, odd, ptrs, rows, vrows, 1048, P, P, P, P, 1 << 30, None)
    assert rc == -1 and "aligned" in _native.last_error()
    # unsupported output size
    rc = lib.sft_ft_fwd_pair_f32(P, P, 4, 32, 1, ptrs, ptrs, rows, vrows, 136, P, P, P, P, 1 << 30, None)
    assert rc == _native.SFT_EUNSUPPORTED
    # missing second index tensor
    rc = lib.sft_ft_fwd_pair_f32(P, None, 4, 32, 1, ptrs, ptrs, rows, vrows, 1048, P, P, P, P, 1 << 30, None)
    assert rc == -1 and "null" in _native.last_error()
    rc = lib.sft_ft_bwd_pair_f32(P, P, 4, 32, P, P, 1, rows, vrows, 1048, ptrs, nulls, P, P, 1 << 30, None)
    assert rc == -1 and "null" in _native.last_error()
    rc = lib.sft_ft_bwd_pair_f32(P, P, 4, 32, P, P, 1, rows, vrows, 1048, odd, ptrs, P, P, 1 << 30, None)
    assert rc == -1 and "aligned" in _native.last_error()
    rc = lib.sft_ft_bwd_pair_f32(P, P, 4, 32, P, None, 1, rows, vrows, 1048, ptrs, ptrs, P, P, 1 << 30, None)
    assert rc == -1 and "null" in _native.last_error()


def test_transform_workspace_size_and_checks():
    lib = _native.lib()
    sb, fb, bb = ctypes.c_size_t(0), ctypes.c_size_t(0), ctypes.c_size_t(0)
    args = lambda l1, L=1048: (65536, 32, 1, _i64s(24576), _i64s(768), L, l1, ctypes.byref(sb), ctypes.byref(fb),
                               ctypes.byref(bb))
    assert lib.sft_ft_transform_workspace_size(*args(1040)) == 0, _native.last_error()
    # paired map: 33 tiles for the 2 x 130 chunks of L1 plus one PSQT tile, 128 B per row
    # (the table tiles with one pad row each)
    assert sb.value == 2 * 34 * 65536 * 128 and fb.value == _a256(34 * 24577 * 128) + 2 * rank_lists_bytes(65536, 32)
    assert bb.value >= 2 * 34 * 65536 * 128 + 24576 * 1048 * 4
    for l1 in (1044, 1048, 0, -8):
        assert lib.sft_ft_transform_workspace_size(*args(l1)) == _native.SFT_EUNSUPPORTED
        assert "l1" in _native.last_error()
    assert lib.sft_ft_transform_workspace_size(*args(128, L=136)) == _native.SFT_EUNSUPPORTED


def test_transform_calls_reject_before_launch():
    lib = _native.lib()
    ptrs = (ctypes.c_void_p * 1)(0x1000)
    odd = (ctypes.c_void_p * 1)(0x1008)
    rows, vrows = _i64s(24576), _i64s(768)
    fwd = lambda *a: lib.sft_ft_fwd_transform_f32(*a)
    # null side-to-move, misaligned l0, misaligned table, bad l1
    assert fwd(P, P, 4, 32, 1, ptrs, ptrs, rows, vrows, 1048, 1040, P, None, P, P, P, P, 1 << 30, P, 1 << 30,
               None) == -1 and "null" in _native.last_error()
    assert fwd(P, P, 4, 32, 1, ptrs, ptrs, rows, vrows, 1048, 1040, P, P, P, ctypes.c_void_p(0x1004), P, P, 1 << 30,
               P, 1 << 30, None) == -1 and "aligned" in _native.last_error()
    assert fwd(P, P, 4, 32, 1, odd, ptrs, rows, vrows, 1048, 1040, P, P, P, P, P, P, 1 << 30, P, 1 << 30,
               None) == -1 and "aligned" in _native.last_error()
    assert fwd(P, P, 4, 32, 1, ptrs, ptrs, rows, vrows, 1048, 1036, P, P, P, P, P, P, 1 << 30, P, 1 << 30,
               None) == _native.SFT_EUNSUPPORTED
    bwd = lambda *a: lib.sft_ft_bwd_transform_f32(*a)
    assert bwd(P, P, 4, 32, P, None, P, P, P, 1 << 30, 1, rows, vrows, 1048, 1040, ptrs, ptrs, P, P, 1 << 30,
               None) == -1 and "null" in _native.last_error()
    assert bwd(P, P, 4, 32, P, P, P, P, P, 1 << 30, 1, rows, vrows, 1048, 1040, odd, ptrs, P, P, 1 << 30,
               None) == -1 and "aligned" in _native.last_error()


def test_leb128_rejects_before_launch():
    lib = _native.lib()
    n = ctypes.c_size_t(0)
    assert lib.sft_leb128_workspace_size(100, ctypes.byref(n)) == 0 and n.value >= 8
    ws = ctypes.c_void_p(0x1000)
    # bad element size, too little output capacity, missing workspace, misaligned values
    assert lib.sft_leb128_encode(P, 3, 10, P, 1000, P, ws, 1 << 20, None) == -1 and "elem_bytes" in _native.last_error()
    assert lib.sft_leb128_encode(P, 2, 10, P, 29, P, ws, 1 << 20, None) == -1 and "capacity" in _native.last_error()
    assert lib.sft_leb128_encode(P, 4, 10, P, 50, P, None, 0, None) == _native.SFT_EWORKSPACE
    assert lib.sft_leb128_encode(ctypes.c_void_p(0x1001), 2, 10, P, 30, P, ws, 1 << 20, None) == -1
