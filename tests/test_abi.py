"""CPU checks of the C ABI: the library loads, exports every function that
include/lanternl_hip.h declares, the ctypes binding declares the same set, and
entry points refuse to run before lhip_init (no GPU work is attempted here)."""
import ctypes
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "lanternl_hip.h")


def header_functions():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"LHIP_API\s+[\w\s\*]+?\b(lhip_\w+)\s*\(", text)))


def test_header_parses():
    fns = header_functions()
    assert "lhip_init" in fns and "lhip_sgemm" in fns and len(fns) >= 20


def test_library_exports_every_declared_symbol():
    from lanternl_amd.build import LIB_PATH
    assert os.path.exists(LIB_PATH), "build the library first (__graft_entry__.build())"
    L = ctypes.CDLL(LIB_PATH)
    missing = [f for f in header_functions() if not hasattr(L, f)]
    assert not missing, missing


def test_ctypes_binding_matches_header():
    from lanternl_amd._lib import SIGNATURES
    assert sorted(SIGNATURES) == header_functions()


def test_calls_before_init_fail_cleanly():
    from lanternl_amd import _lib
    L = _lib.lib()
    if L.lhip_is_ready():
        pytest.skip("library already initialised in this process")
    rc = L.lhip_sgemm(0, 0, 4, 4, 4, 1.0, None, 4, None, 4, 0.0, None, 4)
    assert rc == -4
    assert "not initialised" in _lib.last_error()
    L.lhip_clear_error()
    assert _lib.last_error() == ""
    with pytest.raises(_lib.LanternlHipError, match="DEVICE"):
        _lib.call("lhip_sync")
