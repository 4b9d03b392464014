"""The C-ABI library: it loads and exports every function the header declares
(no compute calls: this runs without a GPU)."""
import os
import subprocess

import pytest

from ds4f_hip import lib as L


def _has_gpu():
    return os.path.exists("/dev/kfd")


def test_library_built_and_loads():
    assert os.path.exists(L.LIB_PATH), "run __graft_entry__.build() first"
    L.load()


def test_exports_every_header_function():
    names = L.header_functions()
    assert "ds4f_gpu_gqa_decode" in names and "ds4f_gpu_lin_decode" in names
    lib = L.load()
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing
    # and the binding covers exactly the header's functions
    assert sorted(L._SIGS) == names


def test_exported_dynamic_symbols():
    out = subprocess.run(["nm", "-D", "--defined-only", L.LIB_PATH], capture_output=True,
                         text=True, check=True).stdout
    syms = {line.split()[-1] for line in out.splitlines() if line.strip()}
    for n in L.header_functions():
        assert n in syms, n


def test_kernels_are_gfx950_code_objects():
    # the fat binary of this build carries a gfx950 code object
    blob = open(L.LIB_PATH, "rb").read()
    assert b"amdgcn-amd-amdhsa--gfx950" in blob


@pytest.mark.skipif(_has_gpu(), reason="checks the no-device behaviour")
def test_no_device_means_fallback():
    lib = L.load()
    assert lib.ds4f_gpu_init() == -1
    assert lib.ds4f_gpu_attn_sync(-1, 0, 0) == -1
    assert lib.ds4f_gpu_gqa_decode(3, 0, None, None, None, None, None, None) == -1
    assert lib.ds4f_gpu_lin_decode(0, 0, None, None, None, None, None, None, None, None,
                                   None) == -1
    assert L.last_error()
