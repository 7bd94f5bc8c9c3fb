"""CPU-only checks of the product library: it loads without a GPU, exports
every entry point include/zkml_gpu.h declares, and reports errors instead of
exiting; the Python front end raises when the library is missing."""
import ctypes
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "zkml_gpu.h")
LIB = os.path.join(ROOT, "cuda-zkml_amd", "libzkml_gpu.so")


def declared_symbols():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"\b(zk_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_the_boundary():
    names = declared_symbols()
    for must in ("zk_ntt", "zk_coset_ntt", "zk_msm_g1", "zk_msm_g2", "zk_quotient_h", "zk_pk_load",
                 "zk_setup", "zk_prove", "zk_r1cs_create"):
        assert must in names


def test_library_exports_every_declared_symbol():
    assert os.path.exists(LIB), "run __graft_entry__.build() first"
    lib = ctypes.CDLL(LIB)
    missing = [s for s in declared_symbols() if not hasattr(lib, s)]
    assert not missing, missing


def test_status_strings_and_null_context():
    lib = ctypes.CDLL(LIB)
    lib.zk_status_string.restype = ctypes.c_char_p
    assert lib.zk_status_string(0) == b"ok"
    assert b"witness" in lib.zk_status_string(6)
    # null context is rejected, never dereferenced
    assert lib.zk_ntt(None, None, None, 10, 0, 1, None) == 1
    assert lib.zk_msm_g1(None, None, None, 0, None, None) == 1


def test_front_end_fails_loudly_without_library(monkeypatch, tmp_path):
    import zkml_amd
    monkeypatch.setattr(zkml_amd, "LIB_PATH", str(tmp_path / "missing.so"))
    monkeypatch.setattr(zkml_amd, "_lib", None)
    with pytest.raises(zkml_amd.ZkError):
        zkml_amd.lib()
