"""CPU-side checks of the C ABI: the library loads and exports every entry
point include/cpv.h declares (no compute calls without a GPU)."""
import ctypes
import os
import re

import pytest

from codpiece_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared_symbols():
    src = open(os.path.join(ROOT, "include", "cpv.h")).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    return sorted(set(re.findall(r"\b(cpv_[a-z0-9_]+)\s*\(", src)))


def test_header_declares_the_entry_points():
    names = declared_symbols()
    for n in ["cpv_init", "cpv_free", "cpv_qgemm", "cpv_attn", "cpv_spec_accept", "cpv_weight_upload"]:
        assert n in names


def test_library_exports_every_declared_symbol():
    lib = ctypes.CDLL(_lib.LIB_PATH)
    missing = [n for n in declared_symbols() if not hasattr(lib, n)]
    assert not missing, missing


def test_python_binding_covers_the_header():
    assert set(declared_symbols()) == set(_lib.SIGNATURES)


def test_load_binds_all_signatures():
    lib = _lib.load()
    assert lib.cpv_init.restype is ctypes.c_int


def test_init_without_a_device_fails_cleanly():
    import torch
    if torch.cuda.is_available():
        pytest.skip("a GPU is present")
    lib = _lib.load()
    h = ctypes.c_void_p()
    assert lib.cpv_init(0, ctypes.byref(h)) == _lib.CPV_EDEVICE
    assert lib.cpv_last_error(None) == b"null context"
