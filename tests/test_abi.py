"""CPU checks of the C ABI: the library loads, exports every function that
include/zealot_hip.h declares, the ctypes binding covers them with matching
struct sizes, and calls that must fail do so with a status, not a crash."""

import ctypes as C
import os
import re

import pytest

from zealot_amd import _ffi

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "zealot_hip.h")


def header_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(zl_[a-z0-9_]+)\s*\(", text)))


def test_header_parses():
    fns = header_functions()
    assert "zl_init" in fns and "zl_ppo_update" in fns and len(fns) >= 40


def test_library_exports_every_declared_symbol():
    lib = _ffi.load_library()
    missing = [f for f in header_functions() if not hasattr(lib, f)]
    assert not missing, missing


def test_binding_covers_header():
    assert sorted(_ffi.SIGNATURES) == header_functions()


def test_struct_sizes_match_binding():
    lib = _ffi.load_library()
    out = (C.c_size_t * 3)()
    lib.zl_abi_struct_sizes(out)
    assert list(out) == [C.sizeof(_ffi.zl_ppo_config), C.sizeof(_ffi.zl_batch), C.sizeof(_ffi.zl_ppo_stats)]


def test_null_context_is_rejected():
    lib = _ffi.load_library()
    assert lib.zl_gemm(None, None, None, 0, None, 0, 1, 1, 1) == _ffi.ZL_ERR_INVALID
    assert lib.zl_ppo_update(None, None, None, None) == _ffi.ZL_ERR_INVALID
    assert lib.zl_version().startswith(b"zealot_hip")


def test_init_without_gpu_reports_error():
    """With no usable GPU, zl_init returns a status and an error string
    (the caller's fallback signal) instead of crashing."""
    lib = _ffi.load_library()
    h = C.c_void_p()
    st = lib.zl_init(0, C.byref(h))
    if st == _ffi.ZL_OK:
        lib.zl_destroy(h)
        pytest.skip("a GPU is present")
    assert st in (_ffi.ZL_ERR_HIP, _ffi.ZL_ERR_CODE_OBJECT, _ffi.ZL_ERR_INVALID)
    assert h.value is None
    assert len(lib.zl_global_error()) > 0


def test_init_rejects_bad_device_index():
    lib = _ffi.load_library()
    h = C.c_void_p()
    assert lib.zl_init(-1, C.byref(h)) != _ffi.ZL_OK
