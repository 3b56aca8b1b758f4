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


def test_build_refuses_scratch_in_counted_wait_kernels():
    """The build's guard reads the compiler's resource remarks: VGPR spills and scratch memory
    in a kernel whose waits count its own outstanding requests fail the build; SGPR spills into
    VGPR lanes (no memory requests) and other kernels pass."""
    from momij_amd import build

    def remarks(name, vspill, sspill, scratch):
        return (f"x.hip:1:1: remark: Function Name: {name} [-Rpass-analysis=kernel-resource-usage]\n"
                f"x.hip:1:1: remark:     SGPRs Spill: {sspill} [-Rpass-analysis=kernel-resource-usage]\n"
                f"x.hip:1:1: remark:     VGPRs Spill: {vspill} [-Rpass-analysis=kernel-resource-usage]\n"
                f"x.hip:1:1: remark:     ScratchSize [bytes/lane]: {scratch} [-Rpass-analysis=kernel-resource-usage]\n")

    g5 = "_Z9k_gather5ILi8ELi64ELi2ELi8ELi2ELb1ELb0ELb1EEv10GatherArgsii"
    assert build._spills(remarks(g5, 0, 6, 0)) == []
    assert build._spills(remarks("_Z7k_otherv", 9, 0, 64)) == []
    assert [w for _, w in build._spills(remarks(g5, 14, 0, 56))] == ["14 VGPR spills",
                                                                     "56 scratch bytes a lane"]
    assert [k for k, _ in build._spills(remarks("k_lm_head", 0, 0, 16))] == ["k_lm_head"]
