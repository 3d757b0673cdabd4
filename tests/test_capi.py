"""CPU-side checks of the C ABI library: it loads, exports exactly what
include/rembed_hip.h declares, and reports a missing device as a distinct
status (the host's cue to fall back to its CPU path). No compute calls.
"""
import ctypes
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "rembed_hip.h")


def header_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(rh_[a-z0-9_]+)\s*\(", text)))


def test_header_and_binding_agree():
    from rembed_amd import _lib
    assert header_functions() == sorted(_lib.EXPORTS)


def test_library_exports_every_declared_symbol():
    from rembed_amd import _lib
    lib = ctypes.CDLL(_lib.LIB_PATH)
    missing = [f for f in header_functions() if not hasattr(lib, f)]
    assert not missing, missing
    assert _lib.lib.rh_version() >= 100


def test_library_is_built_for_gfx950():
    from rembed_amd import _lib
    blob = open(_lib.LIB_PATH, "rb").read()
    assert b"gfx950" in blob


def test_no_device_is_a_distinct_status():
    import torch
    if torch.cuda.is_available():
        pytest.skip("a GPU is present")
    from rembed_amd import _lib
    n = ctypes.c_int(-1)
    assert _lib.lib.rh_device_count(ctypes.byref(n)) == _lib.RH_ERR_NO_DEVICE
    assert n.value == 0
    h = ctypes.c_void_p()
    assert _lib.lib.rh_context_create(0, ctypes.byref(h)) == _lib.RH_ERR_NO_DEVICE
    assert b"no HIP device" in _lib.lib.rh_last_error()


def test_null_arguments_are_rejected_without_a_device():
    from rembed_amd import _lib
    L = _lib.lib
    assert L.rh_context_create(0, None) == _lib.RH_ERR_INVALID
    assert L.rh_context_sync(None) == _lib.RH_ERR_INVALID
    assert L.rh_pack_weight(None, 0, None, None, 4, 16, None) == _lib.RH_ERR_INVALID
    assert L.rh_weight_info(None, None, None, None) == _lib.RH_ERR_INVALID
    assert L.rh_model_create(None, None, 0, None) == _lib.RH_ERR_INVALID
    assert L.rh_model_embed(None, None, None, 0, 1, None) == _lib.RH_ERR_INVALID
    assert L.rh_model_share(None, None, None) == _lib.RH_ERR_INVALID
