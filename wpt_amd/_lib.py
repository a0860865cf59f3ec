"""Loads libwptv.so (the HIP kernels of the verify step) through ctypes and
declares its C ABI (include/wptv.h).

The library is loaded after torch, so that its HIP runtime is the one torch
already holds.  A missing or stale library is KernelUnavailable: nothing in
this package computes the verify step any other way.
"""

import ctypes
from pathlib import Path

import torch

LIBRARY = Path(__file__).resolve().parent / "lib" / "libwptv.so"
ABI_VERSION = 10

WPTV_F32, WPTV_BF16 = 0, 1
DTYPES = {torch.float32: WPTV_F32, torch.bfloat16: WPTV_BF16}
WPTV_I64, WPTV_I32 = 8, 9
INDEX_DTYPES = {torch.int64: WPTV_I64, torch.int32: WPTV_I32}
FORCE_GENERIC = 1
RANGE_FROM_POSITIONS = 2
KEY_SPLIT = 4
OUT_FM = 8
ROWS32 = 16


class KernelUnavailable(RuntimeError):
    """The HIP kernels cannot work here: the reason says why.  Nothing has
    been computed (the reference's kernels.KernelUnavailable,
    packages/wpt-model/src/wpt_model/kernels.py:57-59)."""


_P, _I, _I64, _F, _SZ = ctypes.c_void_p, ctypes.c_int, ctypes.c_int64, ctypes.c_float, ctypes.c_size_t

# name -> argument types, in the order of include/wptv.h
SIGNATURES = {
    "wptv_abi_version": [],
    "wptv_last_error": [],
    "wptv_attention_workspace": [_I, _I, _I, _I, _I, _I, _I, _I, ctypes.POINTER(_I), ctypes.POINTER(_SZ)],
    "wptv_verify_attention": [_P, _P, _I64, _I64, _P, _I64, _I64, _I, _P, _I, _P, _P, _P, _I, _I, _I, _I, _I, _F, _I,
                              _I, _P, _P, _P, _SZ, _P],
    "wptv_verify_attention_static": [_P, _P, _I64, _I64, _P, _I64, _I64, _I, _P, _I, _P, _P, _P, _I, _I, _I, _I, _I,
                                     _F, _I, _I, _P, _P, _P],
    "wptv_sparse_attention_workspace": [_I, _I, _I, _I, _I, _I, _I, _I, ctypes.POINTER(_I), ctypes.POINTER(_SZ)],
    "wptv_sparse_attention": [_P, _P, _I64, _I64, _P, _I64, _I64, _I, _P, _I, _P, _I, _P, _P, _I64, _I, _I, _I, _I, _I,
                              _F, _I, _P, _P, _P, _SZ, _P],
    "wptv_window_attention_workspace": [_I, _I, _I, _I, _I, _I, ctypes.POINTER(_I), ctypes.POINTER(_SZ)],
    "wptv_window_attention": [_P, _P, _I64, _I64, _P, _I64, _I64, _I, _P, _P, _I, _I, _P, _P, _I64, _I, _I, _I, _I,
                              _F, _I, _P, _P, _SZ, _P],
    "wptv_choice_workspace": [_I, _I, _I, ctypes.POINTER(_SZ)],
    "wptv_exact_choice": [_P, _P, _I64, _I64, _I, _P, _P, _I, _I, _I, _I, _I, _F, _I, _I, _P, _P, _SZ, _P],
    "wptv_kv_append": [_P, _I64, _I64, _I64, _P, _I64, _I64, _P, _P, _I, _I, _I, _I, _P],
    "wptv_add_rms_norm": [_P, _P, _P, _P, _I, _I, _I, _F, _P],
    "wptv_qkv_post": [_P, _I64, _P, _P, _P, _P, _I64, _I64, _I64, _P, _P, _I, _I, _I, _I, _I, _F, _P],
    "wptv_window_qkv_post": [_P, _I64, _P, _P, _P, _P, _I64, _I64, _I, _P, _P, _I, _I, _I, _I, _I, _P, _I, _F, _P],
    "wptv_heads_rms_norm": [_P, _I64, _P, _P, _I, _I, _I, _I, _F, _P],
    "wptv_heads_rms_norm_rope": [_P, _I64, _P, _P, _I, _I, _I, _I, _F, _P, _I, _P, _P],
    "wptv_embed_rms_norm": [_P, _P, _I64, _P, _P, _P, _I, _I, _I, _I, _F, _P, _P, _I, _P],
    "wptv_cache_lengths": [_P, _P, _P, _I, _I, _I, _P],
    "wptv_next_feeds": [_P, _I64, _P, _P, _I64, _I, _I, _P, _P, _P],
    "wptv_swiglu": [_P, _P, _I, _I, _I, _P],
    "wptv_gemm_workspace": [_I, _I, _I, _P, _P],
    "wptv_gemm": [_P, _I64, _P, _I64, _I, _I, _I, _P, _I64, _I, _I, _P, _SZ, _P],
    "wptv_gemm_swiglu": [_P, _I64, _P, _I64, _I, _I, _I, _P, _I64, _P],
    "wptv_gemm_parts": [_P, _I64, _P, _I64, _I, _I, _I, _I, _P, _SZ, _P],
    "wptv_fm_pack": [_P, _I64, _I, _I, _I, _P, _P],
    "wptv_fm_row_blocks": [_I],
    "wptv_gemm_fm_plan": [_I, _I, _I, _I, ctypes.POINTER(_I), ctypes.POINTER(_SZ)],
    "wptv_gemm_fm_parts": [_P, _P, _I, _I, _I, _I, _P, _SZ, _P],
    "wptv_gemm_fm_swiglu": [_P, _P, _I, _I, _I, _P, _P],
    "wptv_gemm_fm_wide": [_P, _I, _P, _I, _I, _I, _P, _I64, _I, _P],
    "wptv_gemm_fm_wide_argmax_workspace": [_I, _I, _P],
    "wptv_gemm_fm_wide_argmax": [_P, _I, _P, _I, _I, _I, _P, _P, _SZ, _P],
    "wptv_add_rms_norm_parts": [_P, _P, _I, _P, _P, _I, _I, _I, _I, _F, _P],
    "wptv_qkv_post_parts": [_P, _I, _P, _P, _P, _P, _I64, _I64, _I64, _P, _P, _I, _I, _I, _I, _I, _F, _P],
    "wptv_accept_workspace": [_I, _I, ctypes.POINTER(_SZ)],
    "wptv_accept": [_P, _I64, _I64, _I, _P, _P, _I64, _I64, _P, _I64, _P, _P, _P, _F, _I, _I, _I, _I, _I, _P, _P,
                    _P, _SZ, _P],
    "wptv_accept_commit": [_P, _I64, _I64, _I, _P, _P, _I64, _I64, _P, _I64, _P, _P, _P, _F, _I, _I, _I, _I, _I, _P,
                           _P, _P, _SZ, _P, _P, _P, _I64, _P, _P, _P],
    "wptv_accept_in_order": [_P, _I64, _I64, _I, _P, _P, _I64, _I64, _P, _I64, _P, _P, _P, _I, _F, _I, _I, _I, _I,
                             _P, _P, _P, _SZ, _P, _P, _P, _I64, _P, _P, _P],
    "wptv_greedy_tree": [_P, _I64, _I64, _I, _P, _P, _I, _I, _I, _P, _P, _P, _P, _SZ, _P],
    "wptv_greedy_tree_best": [_P, _P, _P, _I, _I, _P, _P, _P, _P],
}

_handle = None


def lib():
    """The loaded library, its functions declared."""
    global _handle
    if _handle is None:
        if not LIBRARY.exists():
            raise KernelUnavailable(f"the HIP library {LIBRARY} is not built: run `python -m wpt_amd.build` "
                                    "(or __graft_entry__.build()) first")
        try:
            handle = ctypes.CDLL(str(LIBRARY))
        except OSError as error:
            raise KernelUnavailable(f"the HIP library does not load: {error}") from error
        for name, argtypes in SIGNATURES.items():
            try:
                function = getattr(handle, name)
            except AttributeError as error:
                raise KernelUnavailable(f"the HIP library lacks {name}: it is stale, build it again") from error
            function.argtypes = argtypes
            function.restype = ctypes.c_char_p if name == "wptv_last_error" else ctypes.c_int
        if handle.wptv_abi_version() != ABI_VERSION:
            raise KernelUnavailable(f"the HIP library has ABI {handle.wptv_abi_version()}, this package "
                                    f"{ABI_VERSION}: build it again")
        _handle = handle
    return _handle


def check(status, what):
    """Raises the error a non-zero status of `what` stands for."""
    if status == 0:
        return
    message = f"{what}: {lib().wptv_last_error().decode(errors='replace')}"
    if status == -1:
        raise ValueError(message)
    if status == -3:
        raise NotImplementedError(message)
    raise RuntimeError(message)


def ptr(tensor):
    """The device address of a tensor, or None."""
    return None if tensor is None else ctypes.c_void_p(tensor.data_ptr())


def stream(device):
    """The current HIP stream of device, as the library takes it."""
    return ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)


def fm_row_blocks(rows):
    """The 16-row blocks a fragment-major operand of `rows` rows is stored
    with (include/wptv.h: 2 ceil(rows / 32))."""
    return 2 * ((int(rows) + 31) // 32)


def dtype_code(dtype):
    try:
        return DTYPES[dtype]
    except KeyError:
        raise NotImplementedError(f"the HIP kernels take fp32 or bf16, not {dtype}") from None
