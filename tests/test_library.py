"""The C-ABI library (CPU side): it loads, exports every entry point
include/wptv.h declares, and answers its host-only queries (no kernel runs
here)."""

import ctypes
import re
from pathlib import Path

import pytest

from wpt_amd import _lib

HEADER = Path(__file__).resolve().parents[1] / "include" / "wptv.h"


def declared():
    text = HEADER.read_text()
    return sorted(set(re.findall(r"^(?:int|const char\*)\s+(wptv_\w+)\(", text, flags=re.M)))


def test_the_header_declares_the_entry_points_the_loader_binds():
    assert declared() == sorted(_lib.SIGNATURES)


def test_the_library_loads_and_exports_every_declared_entry_point():
    library = _lib.lib()
    for name in declared():
        assert hasattr(library, name), name
    assert library.wptv_abi_version() == _lib.ABI_VERSION


def test_the_workspace_query_plans_the_verify_attention_workload():
    library = _lib.lib()
    splits, size = ctypes.c_int(8), ctypes.c_size_t(0)
    status = library.wptv_attention_workspace(32, 5, 16, 128, 4096, 0, _lib.WPTV_BF16, 0, ctypes.byref(splits),
                                              ctypes.byref(size))
    assert status == 0 and splits.value == 8
    # eight parts of 80 query rows x 128 bf16 values plus an FP32
    # log-sum-exp each
    assert size.value >= 32 * 8 * 80 * (128 * 2 + 4)
    status = library.wptv_attention_workspace(32, 5, 16, 128, 4096, 0, _lib.WPTV_BF16, _lib.KEY_SPLIT,
                                              ctypes.byref(splits), ctypes.byref(size))
    assert status == 0 and size.value >= 32 * 8 * 80 * (128 * 2 + 4)


def test_bad_arguments_are_reported_with_a_message():
    library = _lib.lib()
    splits, size = ctypes.c_int(0), ctypes.c_size_t(0)
    status = library.wptv_attention_workspace(0, 5, 16, 128, 4096, 0, _lib.WPTV_BF16, 0, ctypes.byref(splits),
                                              ctypes.byref(size))
    assert status == -1
    assert b"positive" in library.wptv_last_error()
    with pytest.raises(ValueError, match="positive"):
        _lib.check(status, "attention_workspace")
    status = library.wptv_attention_workspace(1, 1, 1, 128, 8, 0, 7, 0, ctypes.byref(splits), ctypes.byref(size))
    with pytest.raises(NotImplementedError):
        _lib.check(status, "attention_workspace")
