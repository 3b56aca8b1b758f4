"""CPU checks of the C ABI library: it loads and exports every function the header declares.
No compute call is made here (there is no GPU in this environment)."""
import ctypes
import os

import pytest

from momij_amd import _lib


def test_library_exports_every_header_symbol():
    if not os.path.exists(_lib.LIB_PATH):
        pytest.fail("libmomij_hip.so is not built (run __graft_entry__.build())")
    lib = ctypes.CDLL(_lib.LIB_PATH)
    names = _lib.header_symbols()
    assert len(names) >= 30
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing
    # every header function has a ctypes signature in the binding
    assert set(names) == set(_lib._SIGS), set(names) ^ set(_lib._SIGS)


def test_pure_helpers():
    lib = _lib.load()
    assert lib.mj_abi_version() == 1
    assert lib.mj_status_str(3) == b"unsupported shape"
    assert lib.mj_status_str(5) == b"aborted"
