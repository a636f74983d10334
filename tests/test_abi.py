"""CPU-side checks of the C-ABI library: it loads, exports every entry point
that include/*.h declares, and reports errors through lrs_last_error()
without a GPU (no compute call is made here)."""
import ctypes as C
import glob
import os
import re

import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB = os.path.join(REPO, "llama.rs_amd", "liblrs.so")


def declared_symbols():
    names = set()
    for h in glob.glob(os.path.join(REPO, "include", "*.h")):
        src = open(h).read()
        src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
        for m in re.finditer(r"\b(lrs_[a-z0-9_]+)\s*\(", src):
            names.add(m.group(1))
    return sorted(names)


def test_headers_declare_entry_points():
    names = declared_symbols()
    assert "lrs_matvec_f32" in names and "lrs_dequant_f32" in names
    assert len(names) >= 20


def test_library_exports_every_declared_symbol():
    assert os.path.exists(LIB), "liblrs.so not built (run __graft_entry__.build())"
    lib = C.CDLL(LIB)
    missing = [n for n in declared_symbols() if not hasattr(lib, n)]
    assert not missing, missing


def test_measurement_probe_is_a_library_of_its_own():
    """the load-only read kernel bench.py measures with lives in
    liblrs_probe.so, not in the product library or its header"""
    probe = C.CDLL(os.path.join(REPO, "llama.rs_amd", "liblrs_probe.so"))
    assert hasattr(probe, "lrsp_read_time")
    lib = C.CDLL(LIB)
    assert not hasattr(lib, "lrs_read_dev") and not hasattr(lib, "lrsp_read_time")
    assert "lrs_read_dev" not in declared_symbols()


def test_library_is_built_for_gfx950_only():
    data = open(LIB, "rb").read()
    assert b"gfx950" in data
    for other in (b"gfx942", b"gfx90a", b"sm_"):
        assert b"amdgcn-amd-amdhsa--" + other not in data


def test_error_path_without_device(lrs):
    import ctypes

    if lrs.lib.lrs_ctx_create(-1, ctypes.byref(ctypes.c_void_p())) == 0:
        pytest.skip("a GPU is visible here")
    msg = lrs.lib.lrs_last_error().decode()
    assert "HIP" in msg or "device" in msg
    with pytest.raises(lrs.ModelError):
        lrs.Context()


def test_null_arguments_are_rejected(lrs):
    assert lrs.lib.lrs_ctx_sync(None) == -1
    assert "null" in lrs.lib.lrs_last_error().decode()
    assert lrs.lib.lrs_matvec_f32(None, None, None, None, 1) == -1
    assert lrs.lib.lrs_matvec_set_geom(48, 2, 4) == -1
    assert lrs.lib.lrs_matvec_set_geom(0, 0, 0) == 0


def test_no_oracle_in_product():
    """The product package never imports or links the CPU oracle."""
    for f in glob.glob(os.path.join(REPO, "llama.rs_amd", "**", "*"), recursive=True):
        if f.endswith((".py", ".hip", ".h", ".cpp")):
            src = open(f).read()
            assert "lrs_oracle" not in src and "import oracle" not in src, f
