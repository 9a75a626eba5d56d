"""ctypes binding of libsft_ft.so, the C-ABI FT library (include/sft_ft.h).

The functions here take torch CUDA tensors, check dtype/shape/device on the
host, and pass raw device pointers plus the caller's current HIP stream to the
library.  There is no CPU or torch fallback: when the library is missing, or a
tensor is not on a GPU, they raise.
"""

from __future__ import annotations

import ctypes
import os
import threading

import torch

PKG_ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
# SFT_LIB selects another build of the library (e.g. one compiled with other tuning constants).
LIB_PATH = os.environ.get("SFT_LIB") or os.path.join(PKG_ROOT, "lib", "libsft_ft.so")
# The allocation-free int16 forward (include/sft_ft_noalloc.h), a library of its own.
NOALLOC_LIB_PATH = os.path.join(PKG_ROOT, "lib", "libsft_ft_noalloc.so")

SFT_OK = 0
SFT_EWORKSPACE = -2
SFT_EUNSUPPORTED = -4
SFT_FWD_AUTO = 0x0
SFT_FWD_ROWS = 0x1
SFT_BWD_ACCUMULATE = 0x0
SFT_BWD_OVERWRITE = 0x1
SFT_BWD_SORTED = 0x00
SFT_BWD_ATOMIC = 0x10
SFT_BWD_ROWS = 0x2
SFT_BWD_PREPARED = 0x20
SFT_Q16_ACC32 = 0x0
SFT_Q16_WRAP16 = 0x1
SFT_Q16_ROWS = 0x2
SFT_FEATURES_THREATS = 1
SFT_FEATURES_HALFKA = 2

_vp = ctypes.c_void_p
_i64 = ctypes.c_int64
_i32 = ctypes.c_int32
_u32 = ctypes.c_uint32

# name -> (restype, argtypes); mirrors include/sft_ft.h
SIGNATURES = {
    "sft_abi_version": (ctypes.c_int, []),
    "sft_last_error": (ctypes.c_char_p, []),
    "sft_ft_fwd_f32": (ctypes.c_int, [_vp, _i64, _i32, _vp, _i64, _i32, _vp, _vp, _vp]),
    "sft_ft_fwd_f32_workspace_size": (
        ctypes.c_int, [_i64, _i32, _i64, _i32, _u32, ctypes.POINTER(ctypes.c_size_t)]),
    "sft_ft_fwd_f32_ex": (
        ctypes.c_int, [_vp, _i64, _i32, _vp, _i64, _i32, _vp, _vp, _vp, ctypes.c_size_t, _u32, _vp]),
    "sft_ft_bwd_f32_workspace_size": (
        ctypes.c_int, [_i64, _i32, _i64, _i32, _u32, ctypes.POINTER(ctypes.c_size_t)]),
    "sft_ft_bwd_f32": (
        ctypes.c_int, [_vp, _i64, _i32, _vp, _i64, _i32, _vp, _vp, _vp, ctypes.c_size_t, _u32, _vp]),
    "sft_ft_bwd_f32_prep_size": (
        ctypes.c_int, [_i64, _i32, _i64, _i32, _u32, ctypes.POINTER(ctypes.c_size_t)]),
    "sft_ft_fwd_f32_prep": (
        ctypes.c_int,
        [_vp, _i64, _i32, _vp, _i64, _i32, _vp, _vp, _vp, ctypes.c_size_t, _u32, _vp, ctypes.c_size_t, _u32, _vp]),
    "sft_ft_bwd_f32_prepared": (
        ctypes.c_int,
        [_vp, _i64, _i32, _vp, _i64, _i32, _vp, _vp, _vp, ctypes.c_size_t, _vp, ctypes.c_size_t, _u32, _vp]),
    "sft_ft_fwd_i16": (
        ctypes.c_int,
        [_vp, _i64, _i32, _vp, _i64, _i32, _vp, _vp, _i32, _vp, _vp, _i32, _i32, _u32, _vp]),
    "sft_ft_fwd_i16_workspace_size": (
        ctypes.c_int, [_i64, _i32, _i64, _i32, _i32, _u32, ctypes.POINTER(ctypes.c_size_t)]),
    "sft_ft_fwd_i16_ex": (
        ctypes.c_int,
        [_vp, _i64, _i32, _vp, _i64, _i32, _vp, _vp, _i32, _vp, _vp, _i32, _i32, _vp, ctypes.c_size_t, _u32, _vp]),
    "sft_ft_i16_packed_size": (ctypes.c_int, [_i64, _i32, _i32, ctypes.POINTER(ctypes.c_size_t)]),
    "sft_ft_i16_pack": (ctypes.c_int, [_vp, _i64, _i32, _vp, _i32, _vp, ctypes.c_size_t, _vp]),
    "sft_ft_fwd_i16_packed": (
        ctypes.c_int,
        [_vp, _vp, _i64, _i32, _vp, ctypes.c_size_t, _i64, _i32, _vp, _i32, _vp, _vp, _vp, _vp, _i32, _i32, _u32,
         _vp]),
    "sft_ft_fwd_i16_packed_workspace_size": (ctypes.c_int, [_i64, _i32, _i32, ctypes.POINTER(ctypes.c_size_t)]),
    "sft_ft_fwd_i16_packed_ex": (
        ctypes.c_int,
        [_vp, _vp, _i64, _i32, _vp, ctypes.c_size_t, _i64, _i32, _vp, _i32, _vp, _vp, _vp, _vp, _i32, _i32, _vp,
         ctypes.c_size_t, _u32, _vp]),
    "sft_ft_pair_workspace_size": (
        ctypes.c_int,
        [_i64, _i32, _i32, ctypes.POINTER(_i64), ctypes.POINTER(_i64), _i32, ctypes.POINTER(ctypes.c_size_t),
         ctypes.POINTER(ctypes.c_size_t)]),
    "sft_ft_fwd_pair_f32": (
        ctypes.c_int,
        [_vp, _vp, _i64, _i32, _i32, ctypes.POINTER(_vp), ctypes.POINTER(_vp), ctypes.POINTER(_i64),
         ctypes.POINTER(_i64), _i32, _vp, _vp, _vp, _vp, ctypes.c_size_t, _vp]),
    "sft_ft_bwd_pair_f32": (
        ctypes.c_int,
        [_vp, _vp, _i64, _i32, _vp, _vp, _i32, ctypes.POINTER(_i64), ctypes.POINTER(_i64), _i32,
         ctypes.POINTER(_vp), ctypes.POINTER(_vp), _vp, _vp, ctypes.c_size_t, _vp]),
    "sft_ft_transform_workspace_size": (
        ctypes.c_int,
        [_i64, _i32, _i32, ctypes.POINTER(_i64), ctypes.POINTER(_i64), _i32, _i32, ctypes.POINTER(ctypes.c_size_t),
         ctypes.POINTER(ctypes.c_size_t), ctypes.POINTER(ctypes.c_size_t)]),
    "sft_ft_fwd_transform_f32": (
        ctypes.c_int,
        [_vp, _vp, _i64, _i32, _i32, ctypes.POINTER(_vp), ctypes.POINTER(_vp), ctypes.POINTER(_i64),
         ctypes.POINTER(_i64), _i32, _i32, _vp, _vp, _vp, _vp, _vp, _vp, ctypes.c_size_t, _vp, ctypes.c_size_t, _vp]),
    "sft_ft_bwd_transform_f32": (
        ctypes.c_int,
        [_vp, _vp, _i64, _i32, _vp, _vp, _vp, _vp, _vp, ctypes.c_size_t, _i32, ctypes.POINTER(_i64),
         ctypes.POINTER(_i64), _i32, _i32, ctypes.POINTER(_vp), ctypes.POINTER(_vp), _vp, _vp, ctypes.c_size_t, _vp]),
    "sft_ranger22_update_f32": (ctypes.c_int, [_vp, _vp, _vp, _vp, _vp, _i64, _i64, _vp, _vp]),
    "sft_encode_features": (
        ctypes.c_int, [_vp, _vp, _i64, ctypes.POINTER(_i32), _i32, _vp, _vp, _i32, _vp, _vp, _vp, _vp, _vp, _vp]),
    "sft_leb128_workspace_size": (ctypes.c_int, [_i64, ctypes.POINTER(ctypes.c_size_t)]),
    "sft_leb128_encode": (ctypes.c_int, [_vp, _i32, _i64, _vp, ctypes.c_size_t, _vp, _vp, ctypes.c_size_t, _vp]),
    "sft_quantize_i16": (ctypes.c_int, [_vp, _i64, ctypes.c_float, _vp, _vp]),
    "sft_probe_l2_gather": (ctypes.c_int, [_vp, _i64, _i32, _i32, _vp, ctypes.c_size_t, _vp]),
    "sft_prof_enable": (ctypes.c_int, [ctypes.c_int]),
    "sft_prof_num_kinds": (ctypes.c_int, []),
    "sft_prof_kind_name": (ctypes.c_char_p, [ctypes.c_int]),
    "sft_prof_collect": (
        ctypes.c_int, [ctypes.POINTER(ctypes.c_double), ctypes.POINTER(ctypes.c_int64), ctypes.c_int]),
}

# name -> (restype, argtypes); mirrors include/sft_ft_noalloc.h
NOALLOC_SIGNATURES = {
    "sft_ft_fwd_i16_noalloc": (
        ctypes.c_int,
        [_vp, _i64, _i32, _vp, _i64, _i32, _vp, _vp, _i32, _vp, _vp, _i32, _i32, _u32, _vp]),
}

_lib = None
_noalloc_lib = None
_lock = threading.Lock()


class NativeLibraryMissing(RuntimeError):
    pass


def lib() -> ctypes.CDLL:
    """Load libsft_ft.so once; raise if it has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not os.path.exists(LIB_PATH):
                raise NativeLibraryMissing(
                    f"{LIB_PATH} not found: build it with `python -c 'import __graft_entry__ as g; g.build()'` "
                    "or `make -C stockfish-trainer_amd/csrc`")
            handle = ctypes.CDLL(LIB_PATH)
            for name, (res, args) in SIGNATURES.items():
                fn = getattr(handle, name)
                fn.restype = res
                fn.argtypes = args
            _lib = handle
    return _lib


def noalloc_lib() -> ctypes.CDLL:
    """Load libsft_ft_noalloc.so once (after libsft_ft.so, which it links); raise
    if it has not been built."""
    global _noalloc_lib
    lib()
    if _noalloc_lib is not None:
        return _noalloc_lib
    with _lock:
        if _noalloc_lib is None:
            if not os.path.exists(NOALLOC_LIB_PATH):
                raise NativeLibraryMissing(f"{NOALLOC_LIB_PATH} not found: build it with "
                                           "`make -C stockfish-trainer_amd/csrc`")
            handle = ctypes.CDLL(NOALLOC_LIB_PATH)
            for name, (res, args) in NOALLOC_SIGNATURES.items():
                fn = getattr(handle, name)
                fn.restype = res
                fn.argtypes = args
            _noalloc_lib = handle
    return _noalloc_lib


def last_error() -> str:
    msg = lib().sft_last_error()
    return msg.decode() if msg else ""


def _check(rc: int, what: str) -> None:
    if rc != SFT_OK:
        raise RuntimeError(f"{what} failed (code {rc}): {last_error()}")


def _ptr(t: torch.Tensor | None):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def _stream(device: torch.device) -> ctypes.c_void_p:
    return ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)


def _require(cond: bool, msg: str) -> None:
    if not cond:
        raise ValueError(msg)


def _on_gpu(device: torch.device, *tensors: torch.Tensor) -> None:
    _require(device.type == "cuda", "sft: tensors must be on a GPU (no CPU path exists)")
    for t in tensors:
        _require(t.device == device, "sft: all tensors must be on the same device")
        _require(t.is_contiguous(), "sft: tensors must be contiguous")


def ft_fwd_f32(idx: torch.Tensor, weight: torch.Tensor, bias: torch.Tensor, out: torch.Tensor,
               rows: bool = False) -> None:
    """out[b] = bias + sum of weight rows selected by idx[b] (reference order, bit-exact).

    By default the library's tiled gather runs when the shape allows it, with a
    workspace taken from torch's allocator; rows=True forces the row gather.
    """
    _require(idx.dim() == 2 and idx.dtype == torch.int32, "idx must be int32 [B, K]")
    _require(weight.dim() == 2 and weight.dtype == torch.float32, "weight must be float32 [N, L]")
    B, K = idx.shape
    N, L = weight.shape
    _require(bias.shape == (L,) and bias.dtype == torch.float32, "bias must be float32 [L]")
    _require(out.shape == (B, L) and out.dtype == torch.float32, "out must be float32 [B, L]")
    _on_gpu(idx.device, idx, weight, bias, out)
    flags = SFT_FWD_ROWS if rows else SFT_FWD_AUTO
    nbytes = _workspace_bytes("fwd", B, K, N, L, flags, idx.device)
    ws, ptr = _workspace(nbytes, idx.device)
    with torch.cuda.device(idx.device):
        _check(lib().sft_ft_fwd_f32_ex(_ptr(idx), B, K, _ptr(weight), N, L, _ptr(bias), _ptr(out), ptr, nbytes,
                                       flags, _stream(idx.device)), "sft_ft_fwd_f32_ex")
    del ws


_ws_cache: dict = {}


_SIZE_FNS = {"fwd": "sft_ft_fwd_f32_workspace_size", "bwd": "sft_ft_bwd_f32_workspace_size",
             "prep": "sft_ft_bwd_f32_prep_size"}


def _workspace_bytes(which: str, B: int, K: int, N: int, L: int, flags: int, device: torch.device) -> int:
    """Bytes of the forward or backward workspace, or of the backward's prepared
    sort ("prep"); a host-only computation, cached per shape."""
    key = (which, device.index, B, K, N, L, flags)
    got = _ws_cache.get(key)
    if got is None:
        n = ctypes.c_size_t(0)
        name = _SIZE_FNS[which]
        _check(getattr(lib(), name)(B, K, N, L, flags, ctypes.byref(n)), name)
        got = _ws_cache[key] = int(n.value)
    return got


def prep_buffer_bytes(B: int, K: int, N: int, L: int, flags: int, device: torch.device) -> int:
    """Size of the uint8 tensor ft_fwd_f32_prep returns: the prepared sort plus
    room to align it to 256 bytes (0 when the backward sorts nothing)."""
    n = _workspace_bytes("prep", B, K, N, L, flags, device)
    return n + 256 if n else 0


# The library's prepared-buffer layout (make_prep_layout in csrc/ft_bwd.hip:
# the radix sort's workspace, then the segment region of nc position chunks)
# restated in integer arithmetic.  Torch's fake tensors call it with symbolic
# sizes (SymInt), which the C size query cannot take; CPU tests check that it
# equals sft_ft_bwd_f32_prep_size over a sweep of shapes.
_SORT_TILE = 2048              # kBlock * kSortItems (csrc/ft_sort.hip)
_SORT_MAX_RADIX = 1024         # kMaxRadix
_BWD_MIN_TILES = 4             # SFT_BWD_MIN_TILES (csrc/common.h)
_BWD_TILE_BYTES = 128          # one 32-column grad tile row
_BWD_ONE_CHUNK_BYTES = 4 << 20  # SFT_BWD_ONE_CHUNK_BYTES
_BWD_CHUNKS = 2                # SFT_BWD_CHUNKS
_BWD_PREP_K_PER_L = 20         # SFT_BWD_PREP_K_PER_L


def _a256(x):
    return (x + 255) // 256 * 256


def prep_buffer_bytes_formula(B, K, N, L, flags: int):
    """prep_buffer_bytes for sizes that may be symbolic (SymInt)."""
    if (flags & SFT_BWD_ATOMIC) or not (B * K > 0) or not (K * _BWD_PREP_K_PER_L >= L):
        return 0
    M = B * K
    tiled = (not (flags & (SFT_BWD_ATOMIC | SFT_BWD_ROWS)) and bool(flags & SFT_BWD_OVERWRITE) and L % 4 == 0
             and (L + 31) // 32 >= _BWD_MIN_TILES and B * _BWD_TILE_BYTES <= 0xFFFFFFFF)
    nc = _BWD_CHUNKS if (tiled and B >= _BWD_CHUNKS and B * _BWD_TILE_BYTES > _BWD_ONE_CHUNK_BYTES) else 1
    sort_ws = 4 * _a256(M * 4) + _a256(_SORT_MAX_RADIX * ((M + _SORT_TILE - 1) // _SORT_TILE) * 4) \
        + _a256(_SORT_MAX_RADIX * 4)
    seg_region = ((2 * nc * N + 1 + nc) * 4 + 15) // 16 * 16 + M * 2 + 16
    return _a256(sort_ws) + _a256(seg_region) + 256


def _aligned(buf: torch.Tensor):
    if buf.numel() == 0:
        return None, 0
    off = (-buf.data_ptr()) % 256
    return ctypes.c_void_p(buf.data_ptr() + off), buf.numel() - off


def bwd_workspace_bytes(B: int, K: int, N: int, L: int, flags: int, device: torch.device) -> int:
    return _workspace_bytes("bwd", B, K, N, L, flags, device)


def _workspace(nbytes: int, device: torch.device):
    """A 256-byte aligned device buffer of nbytes from torch's caching allocator."""
    if nbytes == 0:
        return None, None
    ws = torch.empty(nbytes + 256, dtype=torch.uint8, device=device)
    off = (-ws.data_ptr()) % 256
    return ws, ctypes.c_void_p(ws.data_ptr() + off)


def ft_bwd_f32(idx: torch.Tensor, weight_grad: torch.Tensor, bias_grad: torch.Tensor,
               grad_out: torch.Tensor, flags: int = SFT_BWD_ACCUMULATE) -> None:
    """weight_grad[f] (+)= sum of grad_out rows whose idx row holds f; bias_grad (+)= column sums."""
    _require(idx.dim() == 2 and idx.dtype == torch.int32, "idx must be int32 [B, K]")
    _require(weight_grad.dim() == 2 and weight_grad.dtype == torch.float32, "weight_grad must be float32 [N, L]")
    B, K = idx.shape
    N, L = weight_grad.shape
    _require(bias_grad.shape == (L,) and bias_grad.dtype == torch.float32, "bias_grad must be float32 [L]")
    _require(grad_out.shape == (B, L) and grad_out.dtype == torch.float32, "grad_out must be float32 [B, L]")
    _on_gpu(idx.device, idx, weight_grad, bias_grad, grad_out)
    nbytes = bwd_workspace_bytes(B, K, N, L, flags, idx.device)
    ws, ptr = _workspace(nbytes, idx.device)
    with torch.cuda.device(idx.device):
        _check(lib().sft_ft_bwd_f32(_ptr(idx), B, K, _ptr(grad_out), N, L, _ptr(weight_grad), _ptr(bias_grad),
                                    ptr, nbytes, flags, _stream(idx.device)), "sft_ft_bwd_f32")
    del ws


def ft_fwd_f32_prep(idx: torch.Tensor, weight: torch.Tensor, bias: torch.Tensor, out: torch.Tensor,
                    bwd_flags: int = SFT_BWD_OVERWRITE) -> torch.Tensor:
    """ft_fwd_f32, and the backward's sort of idx run beside it: returns the
    prepared buffer for ft_bwd_f32_prepared with the same idx, sizes and flags."""
    _require(idx.dim() == 2 and idx.dtype == torch.int32, "idx must be int32 [B, K]")
    _require(weight.dim() == 2 and weight.dtype == torch.float32, "weight must be float32 [N, L]")
    B, K = idx.shape
    N, L = weight.shape
    _require(bias.shape == (L,) and bias.dtype == torch.float32, "bias must be float32 [L]")
    _require(out.shape == (B, L) and out.dtype == torch.float32, "out must be float32 [B, L]")
    _on_gpu(idx.device, idx, weight, bias, out)
    prep = torch.empty(prep_buffer_bytes(B, K, N, L, bwd_flags, idx.device), dtype=torch.uint8, device=idx.device)
    pptr, pbytes = _aligned(prep)
    nbytes = _workspace_bytes("fwd", B, K, N, L, SFT_FWD_AUTO, idx.device)
    ws, ptr = _workspace(nbytes, idx.device)
    with torch.cuda.device(idx.device):
        _check(lib().sft_ft_fwd_f32_prep(_ptr(idx), B, K, _ptr(weight), N, L, _ptr(bias), _ptr(out), ptr, nbytes,
                                         SFT_FWD_AUTO, pptr, pbytes, bwd_flags, _stream(idx.device)),
               "sft_ft_fwd_f32_prep")
    del ws
    return prep


def ft_bwd_f32_prepared(idx: torch.Tensor, weight_grad: torch.Tensor, bias_grad: torch.Tensor,
                        grad_out: torch.Tensor, prep: torch.Tensor, flags: int = SFT_BWD_OVERWRITE) -> None:
    """ft_bwd_f32 from the buffer ft_fwd_f32_prep returned for the same idx and flags."""
    _require(idx.dim() == 2 and idx.dtype == torch.int32, "idx must be int32 [B, K]")
    _require(weight_grad.dim() == 2 and weight_grad.dtype == torch.float32, "weight_grad must be float32 [N, L]")
    B, K = idx.shape
    N, L = weight_grad.shape
    _require(bias_grad.shape == (L,) and bias_grad.dtype == torch.float32, "bias_grad must be float32 [L]")
    _require(grad_out.shape == (B, L) and grad_out.dtype == torch.float32, "grad_out must be float32 [B, L]")
    _require(prep.dtype == torch.uint8 and prep.numel() == prep_buffer_bytes(B, K, N, L, flags, idx.device),
             "prep must be the buffer ft_fwd_f32_prep returned for these sizes and flags")
    _on_gpu(idx.device, idx, weight_grad, bias_grad, grad_out, prep)
    pptr, pbytes = _aligned(prep)
    nbytes = bwd_workspace_bytes(B, K, N, L, flags | SFT_BWD_PREPARED, idx.device)
    ws, ptr = _workspace(nbytes, idx.device)
    with torch.cuda.device(idx.device):
        _check(lib().sft_ft_bwd_f32_prepared(_ptr(idx), B, K, _ptr(grad_out), N, L, _ptr(weight_grad),
                                             _ptr(bias_grad), pptr, pbytes, ptr, nbytes, flags, _stream(idx.device)),
               "sft_ft_bwd_f32_prepared")
    del ws


def ft_fwd_i16(idx: torch.Tensor, weight: torch.Tensor, bias: torch.Tensor, out: torch.Tensor,
               psqt_weight: torch.Tensor | None = None, psqt_out: torch.Tensor | None = None,
               clip_lo: int = 0, clip_hi: int = 127, wrap16: bool = False, rows: bool = False) -> None:
    """int16 forward (exact): out = clamp(bias + sum of rows), psqt_out = sum of PSQT rows.

    The tiled gather runs when the shape allows it (workspace from torch);
    rows=True forces the row gather.
    """
    _require(idx.dim() == 2 and idx.dtype == torch.int32, "idx must be int32 [B, K]")
    _require(weight.dim() == 2 and weight.dtype == torch.int16, "weight must be int16 [N, L]")
    B, K = idx.shape
    N, L = weight.shape
    _require(bias.shape == (L,) and bias.dtype == torch.int16, "bias must be int16 [L]")
    _require(out.shape == (B, L) and out.dtype == torch.int16, "out must be int16 [B, L]")
    tensors = [idx, weight, bias, out]
    P = 0
    if psqt_weight is not None or psqt_out is not None:
        _require(psqt_weight is not None and psqt_out is not None, "psqt_weight and psqt_out go together")
        _require(psqt_weight.dim() == 2 and psqt_weight.shape[0] == N and psqt_weight.dtype == torch.int32,
                 "psqt_weight must be int32 [N, P]")
        P = psqt_weight.shape[1]
        _require(psqt_out.shape == (B, P) and psqt_out.dtype == torch.int32, "psqt_out must be int32 [B, P]")
        tensors += [psqt_weight, psqt_out]
    _on_gpu(idx.device, *tensors)
    flags = (SFT_Q16_WRAP16 if wrap16 else SFT_Q16_ACC32) | (SFT_Q16_ROWS if rows else 0)
    key = ("i16", idx.device.index, B, K, N, L, P, flags)
    nbytes = _ws_cache.get(key)
    if nbytes is None:
        n = ctypes.c_size_t(0)
        _check(lib().sft_ft_fwd_i16_workspace_size(B, K, N, L, P, flags, ctypes.byref(n)),
               "sft_ft_fwd_i16_workspace_size")
        nbytes = _ws_cache[key] = int(n.value)
    ws, ptr = _workspace(nbytes, idx.device)
    with torch.cuda.device(idx.device):
        _check(lib().sft_ft_fwd_i16_ex(_ptr(idx), B, K, _ptr(weight), N, L, _ptr(bias), _ptr(psqt_weight), P,
                                       _ptr(out), _ptr(psqt_out), clip_lo, clip_hi, ptr, nbytes, flags,
                                       _stream(idx.device)), "sft_ft_fwd_i16_ex")
    del ws


def ft_fwd_i16_noalloc(idx: torch.Tensor, weight: torch.Tensor, bias: torch.Tensor, out: torch.Tensor,
                       psqt_weight: torch.Tensor | None = None, psqt_out: torch.Tensor | None = None,
                       clip_lo: int = 0, clip_hi: int = 127, wrap16: bool = False, rows: bool = False) -> None:
    """ft_fwd_i16 through sft_ft_fwd_i16_noalloc (libsft_ft_noalloc.so): no
    workspace, nothing allocated by the library; the packed tiles go to its
    static per-GPU scratch array."""
    _require(idx.dim() == 2 and idx.dtype == torch.int32, "idx must be int32 [B, K]")
    _require(weight.dim() == 2 and weight.dtype == torch.int16, "weight must be int16 [N, L]")
    B, K = idx.shape
    N, L = weight.shape
    _require(bias.shape == (L,) and bias.dtype == torch.int16, "bias must be int16 [L]")
    _require(out.shape == (B, L) and out.dtype == torch.int16, "out must be int16 [B, L]")
    tensors = [idx, weight, bias, out]
    P = 0
    if psqt_weight is not None or psqt_out is not None:
        _require(psqt_weight is not None and psqt_out is not None, "psqt_weight and psqt_out go together")
        _require(psqt_weight.dim() == 2 and psqt_weight.shape[0] == N and psqt_weight.dtype == torch.int32,
                 "psqt_weight must be int32 [N, P]")
        P = psqt_weight.shape[1]
        _require(psqt_out.shape == (B, P) and psqt_out.dtype == torch.int32, "psqt_out must be int32 [B, P]")
        tensors += [psqt_weight, psqt_out]
    _on_gpu(idx.device, *tensors)
    flags = (SFT_Q16_WRAP16 if wrap16 else SFT_Q16_ACC32) | (SFT_Q16_ROWS if rows else 0)
    with torch.cuda.device(idx.device):
        _check(noalloc_lib().sft_ft_fwd_i16_noalloc(_ptr(idx), B, K, _ptr(weight), N, L, _ptr(bias), _ptr(psqt_weight), P,
                                            _ptr(out), _ptr(psqt_out), clip_lo, clip_hi, flags,
                                            _stream(idx.device)), "sft_ft_fwd_i16_noalloc")


def i16_packed_size(N: int, L: int, P: int) -> int | None:
    """Bytes of the packed int16 table, or None when the shape is outside the tiled path."""
    n = ctypes.c_size_t(0)
    rc = lib().sft_ft_i16_packed_size(N, L, P, ctypes.byref(n))
    if rc == SFT_EUNSUPPORTED:
        return None
    _check(rc, "sft_ft_i16_packed_size")
    return int(n.value)


def i16_pack(weight: torch.Tensor, psqt_weight: torch.Tensor | None = None) -> torch.Tensor | None:
    """The int16 table (and PSQT columns) in the packed 64-column tiles, as a uint8
    device tensor; None when the shape is outside the tiled path."""
    _require(weight.dim() == 2 and weight.dtype == torch.int16, "weight must be int16 [N, L]")
    N, L = weight.shape
    P = 0
    tensors = [weight]
    if psqt_weight is not None:
        _require(psqt_weight.dim() == 2 and psqt_weight.shape[0] == N and psqt_weight.dtype == torch.int32,
                 "psqt_weight must be int32 [N, P]")
        P = psqt_weight.shape[1]
        tensors.append(psqt_weight)
    _on_gpu(weight.device, *tensors)
    nbytes = i16_packed_size(N, L, P)
    if nbytes is None or weight.data_ptr() % 16 != 0:
        return None
    packed = torch.empty(nbytes, dtype=torch.uint8, device=weight.device)
    with torch.cuda.device(weight.device):
        _check(lib().sft_ft_i16_pack(_ptr(weight), N, L, _ptr(psqt_weight), P, _ptr(packed), nbytes,
                                     _stream(weight.device)), "sft_ft_i16_pack")
    return packed


def ft_fwd_i16_packed(packed: torch.Tensor, N: int, L: int, P: int, bias: torch.Tensor, idx0: torch.Tensor,
                      out0: torch.Tensor, psqt_out0: torch.Tensor | None, idx1: torch.Tensor | None = None,
                      out1: torch.Tensor | None = None, psqt_out1: torch.Tensor | None = None,
                      clip_lo: int = 0, clip_hi: int = 127, wrap16: bool = False, ranked: bool = True) -> None:
    """int16 forward of one (idx1 None) or both perspectives from a table packed by i16_pack.
    ranked: through sft_ft_fwd_i16_packed_ex (rank lists in a workspace), else
    sft_ft_fwd_i16_packed (index rows compacted per tile, no workspace)."""
    _require(packed.dtype == torch.uint8 and packed.dim() == 1, "packed must come from i16_pack")
    _require(idx0.dim() == 2 and idx0.dtype == torch.int32, "idx0 must be int32 [B, K]")
    B, K = idx0.shape
    _require(bias.shape == (L,) and bias.dtype == torch.int16, "bias must be int16 [L]")
    tensors = [packed, bias, idx0, out0]
    for i, o, po in ((idx0, out0, psqt_out0), (idx1, out1, psqt_out1)):
        if i is None:
            continue
        _require(i.shape == (B, K) and i.dtype == torch.int32, "idx must be int32 [B, K], same shape for both")
        _require(o is not None and o.shape == (B, L) and o.dtype == torch.int16, "out must be int16 [B, L]")
        tensors += [i, o]
        if P:
            _require(po is not None and po.shape == (B, P) and po.dtype == torch.int32,
                     "psqt_out must be int32 [B, P]")
            tensors.append(po)
    _on_gpu(idx0.device, *tensors)
    flags = SFT_Q16_WRAP16 if wrap16 else SFT_Q16_ACC32
    with torch.cuda.device(idx0.device):
        if not ranked:
            _check(lib().sft_ft_fwd_i16_packed(_ptr(idx0), _ptr(idx1), B, K, _ptr(packed), packed.numel(), N, L,
                                               _ptr(bias), P, _ptr(out0), _ptr(out1), _ptr(psqt_out0),
                                               _ptr(psqt_out1), clip_lo, clip_hi, flags, _stream(idx0.device)),
                   "sft_ft_fwd_i16_packed")
            return
        n = ctypes.c_size_t(0)
        _check(lib().sft_ft_fwd_i16_packed_workspace_size(B, K, 1 if idx1 is None else 2, ctypes.byref(n)),
               "sft_ft_fwd_i16_packed_workspace_size")
        ws = torch.empty(n.value + 256, dtype=torch.uint8, device=idx0.device)
        wp, wn = _aligned(ws)
        _check(lib().sft_ft_fwd_i16_packed_ex(_ptr(idx0), _ptr(idx1), B, K, _ptr(packed), packed.numel(), N, L,
                                              _ptr(bias), P, _ptr(out0), _ptr(out1), _ptr(psqt_out0), _ptr(psqt_out1),
                                              clip_lo, clip_hi, wp, wn, flags, _stream(idx0.device)),
               "sft_ft_fwd_i16_packed_ex")


# ---- composed table, both perspectives ----
def _i64_array(vals):
    return (_i64 * len(vals))(*[int(v) for v in vals])


def _ptr_array(tensors):
    return (_vp * len(tensors))(*[None if t is None else t.data_ptr() for t in tensors])


def pair_workspace_bytes(B: int, K: int, rows, virtual_rows, L: int):
    """(forward bytes, backward bytes) of the composed-table pair calls, or None
    when the library does not run this shape fused (then the caller composes the
    table itself)."""
    key = ("pair", B, K, tuple(rows), tuple(virtual_rows), L)
    if key in _ws_cache:
        return _ws_cache[key]
    fb, bb = ctypes.c_size_t(0), ctypes.c_size_t(0)
    rc = lib().sft_ft_pair_workspace_size(B, K, len(rows), _i64_array(rows), _i64_array(virtual_rows), L,
                                          ctypes.byref(fb), ctypes.byref(bb))
    if rc == SFT_EUNSUPPORTED:
        got = None
    else:
        _check(rc, "sft_ft_pair_workspace_size")
        got = (int(fb.value), int(bb.value))
    _ws_cache[key] = got
    return got


def _pair_shapes(idx0, idx1, tables, virtuals):
    _require(idx0.dim() == 2 and idx0.dtype == torch.int32, "idx0 must be int32 [B, K]")
    _require(idx1.shape == idx0.shape and idx1.dtype == torch.int32, "idx1 must be int32 [B, K] like idx0")
    _require(1 <= len(tables) <= 4 and len(virtuals) == len(tables), "1 to 4 table blocks, one virtual entry each")
    L = tables[0].shape[1]
    rows, vrows = [], []
    for w, v in zip(tables, virtuals):
        _require(w.dim() == 2 and w.shape[1] == L and w.dtype == torch.float32, "block tables must be float32 [R, L]")
        rows.append(w.shape[0])
        if v is None:
            vrows.append(0)
        else:
            _require(v.dim() == 2 and v.shape[1] == L and v.dtype == torch.float32, "virtual tables must be float32 [V, L]")
            _require(w.shape[0] % v.shape[0] == 0, "block rows must be a multiple of its virtual rows")
            vrows.append(v.shape[0])
    return idx0.shape[0], idx0.shape[1], L, rows, vrows


def ft_fwd_pair_f32(idx0, idx1, tables, virtuals, bias, out0, out1) -> None:
    """out_p = bias + sum of merged-table rows selected by idx_p, p = 0, 1; merged
    row r of a block with virtual rows V is table[r] + V[r % len(V)]."""
    B, K, L, rows, vrows = _pair_shapes(idx0, idx1, tables, virtuals)
    _require(bias.shape == (L,) and bias.dtype == torch.float32, "bias must be float32 [L]")
    for o in (out0, out1):
        _require(o.shape == (B, L) and o.dtype == torch.float32, "outputs must be float32 [B, L]")
    dev = idx0.device
    _on_gpu(dev, idx0, idx1, bias, out0, out1, *tables, *[v for v in virtuals if v is not None])
    sizes = pair_workspace_bytes(B, K, rows, vrows, L)
    _require(sizes is not None, f"sft: shape not supported by the composed pair path: {last_error()}")
    ws, ptr = _workspace(sizes[0], dev)
    with torch.cuda.device(dev):
        _check(lib().sft_ft_fwd_pair_f32(_ptr(idx0), _ptr(idx1), B, K, len(rows), _ptr_array(tables),
                                         _ptr_array(virtuals), _i64_array(rows), _i64_array(vrows), L, _ptr(bias),
                                         _ptr(out0), _ptr(out1), ptr, sizes[0], _stream(dev)), "sft_ft_fwd_pair_f32")
    del ws


def ft_bwd_pair_f32(idx0, idx1, grad0, grad1, table_grads, virtual_grads, bias_grad) -> None:
    """Overwrites table_grads (dW_0 + dW_1 per block), virtual_grads (sum over
    repeats) and bias_grad (sum of both grads' rows)."""
    B, K, L, rows, vrows = _pair_shapes(idx0, idx1, table_grads, virtual_grads)
    _require(bias_grad.shape == (L,) and bias_grad.dtype == torch.float32, "bias_grad must be float32 [L]")
    for g in (grad0, grad1):
        _require(g.shape == (B, L) and g.dtype == torch.float32, "grads must be float32 [B, L]")
    dev = idx0.device
    _on_gpu(dev, idx0, idx1, grad0, grad1, bias_grad, *table_grads, *[v for v in virtual_grads if v is not None])
    sizes = pair_workspace_bytes(B, K, rows, vrows, L)
    _require(sizes is not None, f"sft: shape not supported by the composed pair path: {last_error()}")
    ws, ptr = _workspace(sizes[1], dev)
    with torch.cuda.device(dev):
        _check(lib().sft_ft_bwd_pair_f32(_ptr(idx0), _ptr(idx1), B, K, _ptr(grad0), _ptr(grad1), len(rows),
                                         _i64_array(rows), _i64_array(vrows), L, _ptr_array(table_grads),
                                         _ptr_array(virtual_grads), _ptr(bias_grad), ptr, sizes[1], _stream(dev)),
               "sft_ft_bwd_pair_f32")
    del ws


# ---- composed table + post-FT epilogue ----
def transform_workspace_bytes(B: int, K: int, rows, virtual_rows, L: int, L1: int):
    """(saved, forward workspace, backward workspace) bytes of the transform
    calls, or None when the library does not run this shape fused."""
    key = ("transform", B, K, tuple(rows), tuple(virtual_rows), L, L1)
    if key in _ws_cache:
        return _ws_cache[key]
    sb, fb, bb = ctypes.c_size_t(0), ctypes.c_size_t(0), ctypes.c_size_t(0)
    rc = lib().sft_ft_transform_workspace_size(B, K, len(rows), _i64_array(rows), _i64_array(virtual_rows), L, L1,
                                               ctypes.byref(sb), ctypes.byref(fb), ctypes.byref(bb))
    if rc == SFT_EUNSUPPORTED:
        got = None
    else:
        _check(rc, "sft_ft_transform_workspace_size")
        got = (int(sb.value), int(fb.value), int(bb.value))
    _ws_cache[key] = got
    return got


def _transform_checks(idx0, idx1, tables, virtuals, us, psqt_idx, L1):
    B, K, L, rows, vrows = _pair_shapes(idx0, idx1, tables, virtuals)
    _require(us.dtype == torch.float32 and us.numel() == B, "us must be float32 with one value per position")
    _require(psqt_idx.dtype == torch.int64 and psqt_idx.numel() == B, "psqt_indices must be int64 [B]")
    sizes = transform_workspace_bytes(B, K, rows, vrows, L, L1)
    _require(sizes is not None, f"sft: shape not supported by the fused transform: {last_error()}")
    return B, K, L, rows, vrows, sizes


def ft_fwd_transform_f32(idx0, idx1, tables, virtuals, bias, us, psqt_idx, L1: int, l0, psqt):
    """l0 [B, L1] and psqt [B] of the post-FT epilogue over the composed forward.
    Returns the saved pre-activations (a uint8 tensor and the aligned pointer
    into it) that ft_bwd_transform_f32 needs."""
    B, K, L, rows, vrows, (sbytes, fbytes, _) = _transform_checks(idx0, idx1, tables, virtuals, us, psqt_idx, L1)
    _require(l0.shape == (B, L1) and l0.dtype == torch.float32, "l0 must be float32 [B, L1]")
    _require(psqt.numel() == B and psqt.dtype == torch.float32, "psqt must be float32 [B]")
    dev = idx0.device
    _on_gpu(dev, idx0, idx1, bias, us, psqt_idx, l0, psqt, *tables, *[v for v in virtuals if v is not None])
    saved, sptr = _workspace(sbytes, dev)
    ws, ptr = _workspace(fbytes, dev)
    with torch.cuda.device(dev):
        _check(lib().sft_ft_fwd_transform_f32(_ptr(idx0), _ptr(idx1), B, K, len(rows), _ptr_array(tables),
                                              _ptr_array(virtuals), _i64_array(rows), _i64_array(vrows), L, L1,
                                              _ptr(bias), _ptr(us), _ptr(psqt_idx), _ptr(l0), _ptr(psqt), sptr,
                                              sbytes, ptr, fbytes, _stream(dev)), "sft_ft_fwd_transform_f32")
    del ws
    return saved, sptr


def ft_bwd_transform_f32(idx0, idx1, g_l0, g_psqt, us, psqt_idx, saved, L1: int, table_grads, virtual_grads,
                         bias_grad) -> None:
    """Overwrites table_grads, virtual_grads and bias_grad with the grads of the
    transform given the grads of l0 and psqt and the forward's saved buffer."""
    B, K, L, rows, vrows, (sbytes, _, bbytes) = _transform_checks(idx0, idx1, table_grads, virtual_grads, us,
                                                                   psqt_idx, L1)
    _require(g_l0.shape == (B, L1) and g_l0.dtype == torch.float32, "grad of l0 must be float32 [B, L1]")
    _require(g_psqt.numel() == B and g_psqt.dtype == torch.float32, "grad of psqt must be float32 [B]")
    _require(bias_grad.shape == (L,) and bias_grad.dtype == torch.float32, "bias_grad must be float32 [L]")
    dev = idx0.device
    _on_gpu(dev, idx0, idx1, g_l0, g_psqt, us, psqt_idx, bias_grad, *table_grads,
            *[v for v in virtual_grads if v is not None])
    saved_tensor, sptr = saved
    _require(saved_tensor is None or saved_tensor.device == dev, "saved buffer on another device")
    ws, ptr = _workspace(bbytes, dev)
    with torch.cuda.device(dev):
        _check(lib().sft_ft_bwd_transform_f32(_ptr(idx0), _ptr(idx1), B, K, _ptr(g_l0), _ptr(g_psqt), _ptr(us),
                                              _ptr(psqt_idx), sptr, sbytes, len(rows), _i64_array(rows),
                                              _i64_array(vrows), L, L1, _ptr_array(table_grads),
                                              _ptr_array(virtual_grads), _ptr(bias_grad), ptr, bbytes,
                                              _stream(dev)), "sft_ft_bwd_transform_f32")
    del ws


def ranger22_update_f32(p, grad, variance_ma, gma_cur, gma_prev, scalars) -> None:
    """In-place Ranger22 full update of one fp32 tensor (row norms for 2-D,
    whole-tensor norm for 1-D); scalars is the reference's 12-float device tensor."""
    _require(p.dim() in (1, 2) and p.dtype == torch.float32, "p must be a 1-D or 2-D float32 tensor")
    for t in (grad, variance_ma, gma_cur, gma_prev):
        _require(t.shape == p.shape and t.dtype == torch.float32, "grad and states must match p")
    _require(scalars.numel() == 12 and scalars.dtype == torch.float32, "scalars must be 12 float32 values")
    _on_gpu(p.device, p, grad, variance_ma, gma_cur, gma_prev, scalars)
    rows, cols = (1, p.shape[0]) if p.dim() == 1 else p.shape
    with torch.cuda.device(p.device):
        _check(lib().sft_ranger22_update_f32(_ptr(p), _ptr(grad), _ptr(variance_ma), _ptr(gma_cur), _ptr(gma_prev),
                                             rows, cols, _ptr(scalars), _stream(p.device)), "sft_ranger22_update_f32")


def encode_features(boards, side_to_move, components, white, black, us=None, psqt=None, layer_stack=None,
                    white_count=None, black_count=None) -> None:
    """Index rows of both perspectives from positions (uint8 boards [B, 64],
    side to move [B]); components: SFT_FEATURES_* in feature-set order."""
    _require(boards.dim() == 2 and boards.shape[1] == 64 and boards.dtype == torch.uint8, "boards must be uint8 [B, 64]")
    B = boards.shape[0]
    _require(side_to_move.dtype == torch.uint8 and side_to_move.numel() == B, "side_to_move must be uint8 [B]")
    K = white.shape[1] if white.dim() == 2 else -1
    for t in (white, black):
        _require(t.dtype == torch.int32 and t.shape == (B, K), "index rows must be int32 [B, K]")
    opt = [t for t in (us, psqt, layer_stack, white_count, black_count) if t is not None]
    _on_gpu(boards.device, boards, side_to_move, white, black, *opt)
    comps = (_i32 * len(components))(*components)
    with torch.cuda.device(boards.device):
        _check(lib().sft_encode_features(_ptr(boards), _ptr(side_to_move), B, comps, len(components), _ptr(white),
                                         _ptr(black), K, _ptr(us), _ptr(psqt), _ptr(layer_stack), _ptr(white_count),
                                         _ptr(black_count), _stream(boards.device)), "sft_encode_features")


def leb128_encode(values: torch.Tensor) -> torch.Tensor:
    """Signed LEB128 codes of an int8 / int16 / int32 device tensor, concatenated
    in element order: a uint8 device tensor of exactly the encoded length."""
    elem = {torch.int8: 1, torch.int16: 2, torch.int32: 4}.get(values.dtype)
    _require(elem is not None, "values must be int8, int16 or int32")
    _on_gpu(values.device, values)
    n = values.numel()
    cap = n * {1: 2, 2: 3, 4: 5}[elem]
    dev = values.device
    out = torch.empty(max(cap, 1), dtype=torch.uint8, device=dev)
    out_len = torch.zeros(1, dtype=torch.int64, device=dev)
    nb = ctypes.c_size_t(0)
    _check(lib().sft_leb128_workspace_size(n, ctypes.byref(nb)), "sft_leb128_workspace_size")
    ws, ptr = _workspace(int(nb.value), dev)
    with torch.cuda.device(dev):
        _check(lib().sft_leb128_encode(_ptr(values), elem, n, _ptr(out), cap, _ptr(out_len), ptr, int(nb.value),
                                       _stream(dev)), "sft_leb128_encode")
    length = int(out_len.item())  # synchronises the stream
    del ws
    return out[:length]


def quantize_i16(x: torch.Tensor, scale: float) -> torch.Tensor:
    """round_half_even(x * scale) saturated to int16, computed by the library on the GPU."""
    _require(x.dtype == torch.float32, "x must be float32")
    _on_gpu(x.device, x)
    out = torch.empty(x.shape, dtype=torch.int16, device=x.device)
    with torch.cuda.device(x.device):
        _check(lib().sft_quantize_i16(_ptr(x), x.numel(), float(scale), _ptr(out), _stream(x.device)),
               "sft_quantize_i16")
    return out


# ---- per-launch kernel timing ----
def probe_l2_gather(table: torch.Tensor, rounds: int, blocks: int, out: torch.Tensor) -> int:
    """One dispatch of the L2 row-gather probe over `table` (float32 [rows, 32],
    rows a power of two); returns the bytes it gathers."""
    _require(table.dim() == 2 and table.shape[1] == 32 and table.dtype == torch.float32,
             "table must be float32 [rows, 32]")
    _require(out.dtype == torch.float32 and out.numel() >= blocks * 256 * 4, "out must hold blocks * 1024 floats")
    _on_gpu(table.device, table, out)
    with torch.cuda.device(table.device):
        _check(lib().sft_probe_l2_gather(_ptr(table), table.shape[0], rounds, blocks, _ptr(out), out.numel() * 4,
                                         _stream(table.device)), "sft_probe_l2_gather")
    return blocks * 32 * 8 * rounds * 128


def prof_enable(on: bool) -> None:
    _check(lib().sft_prof_enable(1 if on else 0), "sft_prof_enable")


def prof_kind_names() -> list[str]:
    n = lib().sft_prof_num_kinds()
    return [lib().sft_prof_kind_name(i).decode() for i in range(n)]


def prof_collect() -> dict:
    """{kind_name: (total_ms, launches)} for launches since the last collect."""
    names = prof_kind_names()
    n = len(names)
    ms = (ctypes.c_double * n)()
    cnt = (ctypes.c_int64 * n)()
    _check(lib().sft_prof_collect(ms, cnt, n), "sft_prof_collect")
    return {names[i]: (ms[i], cnt[i]) for i in range(n) if cnt[i] > 0}
