"""ctypes bindings used by the tests: the CPU oracle (oracle/liboracle.so), the
reference-code checker (oracle/_ref/libzkref.so) and the product C ABI
(cuda-zkml_amd/libzkml_gpu.so, through cuda-zkml_amd/zkml_amd.py)."""
import ctypes
import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
ORACLE_SO = os.path.join(ROOT, "oracle", "liboracle.so")
REF_SO = os.path.join(ROOT, "oracle", "_ref", "libzkref.so")
PKG_DIR = os.path.join(ROOT, "cuda-zkml_amd")

if PKG_DIR not in sys.path:
    sys.path.insert(0, PKG_DIR)

u64p = ctypes.POINTER(ctypes.c_uint64)
vp = ctypes.c_void_p


def ptr(a):
    """Pointer to a contiguous numpy array's data."""
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data_as(ctypes.c_void_p)


def words(n, width=4):
    return np.zeros((n, width), dtype=np.uint64)


_oracle = None
_ref = None


def oracle():
    global _oracle
    if _oracle is None:
        lib = ctypes.CDLL(ORACLE_SO)
        lib.orc_r1cs_new.restype = vp
        lib.orc_r1cs_new.argtypes = [ctypes.c_int] * 4
        lib.orc_r1cs_free.argtypes = [vp]
        lib.orc_r1cs_add.argtypes = [vp, ctypes.c_int, vp, vp, vp, ctypes.c_size_t]
        lib.orc_r1cs_verify.argtypes = [vp, vp, ctypes.c_size_t]
        lib.orc_compute_h.argtypes = [vp, vp, ctypes.c_size_t, vp, ctypes.c_int]
        lib.orc_setup.argtypes = [vp, ctypes.c_uint64, ctypes.c_char_p, ctypes.c_char_p, ctypes.c_int]
        lib.orc_prove.argtypes = [ctypes.c_char_p, vp, vp, ctypes.c_size_t, ctypes.c_uint64, ctypes.c_int, vp, vp]
        lib.orc_prove_g2mode.argtypes = [ctypes.c_char_p, vp, vp, ctypes.c_size_t, ctypes.c_uint64, ctypes.c_int,
                                         vp, vp, ctypes.c_int]
        lib.orc_msm_g1.argtypes = [vp, vp, ctypes.c_size_t, ctypes.c_int, ctypes.c_int, vp]
        lib.orc_msm_g2.argtypes = [vp, vp, ctypes.c_size_t, ctypes.c_int, ctypes.c_int, vp]
        lib.orc_g1_gen_batch.argtypes = [vp, ctypes.c_size_t, vp, ctypes.c_int]
        lib.orc_g2_gen_batch.argtypes = [vp, ctypes.c_size_t, vp, ctypes.c_int]
        lib.orc_ntt.argtypes = [vp, ctypes.c_int, ctypes.c_int, ctypes.c_int]
        lib.orc_coset_scale.argtypes = [vp, ctypes.c_int, ctypes.c_uint64, ctypes.c_int]
        lib.orc_fr_dot_std.argtypes = [vp, vp, ctypes.c_size_t, vp]
        lib.orc_dft_naive.argtypes = [vp, vp, ctypes.c_int, ctypes.c_int]
        lib.orc_fr_from_u64_array.argtypes = [vp, ctypes.c_size_t, vp]
        lib.orc_fr_batch_from_std.argtypes = [vp, ctypes.c_size_t, vp]
        lib.orc_pk_read.argtypes = [ctypes.c_char_p, vp, vp, vp, vp, vp, vp, vp, vp]
        for name in ("orc_fr_mul", "orc_fq_mul", "orc_fr_add", "orc_fr_sub", "orc_fq_add", "orc_fq_sub",
                     "orc_g1_mul", "orc_g2_mul", "orc_g1_add", "orc_g2_add"):
            getattr(lib, name).argtypes = [vp, vp, vp]
        for name in ("orc_fr_inv", "orc_fq_inv", "orc_fr_from_std", "orc_fr_to_std", "orc_fq_from_std",
                     "orc_fq_to_std"):
            getattr(lib, name).argtypes = [vp, vp]
        lib.orc_omega.argtypes = [ctypes.c_int, ctypes.c_int, vp]
        lib.orc_g1_generator.argtypes = [vp]
        lib.orc_g2_generator.argtypes = [vp]
        lib.orc_g1_on_curve.argtypes = [vp]
        _oracle = lib
    return _oracle


def ref_available():
    return os.path.exists(REF_SO)


def ref():
    global _ref
    if _ref is None:
        lib = ctypes.CDLL(REF_SO)
        for name in ("ref_fr_mul", "ref_fq_mul", "ref_g1_mul", "ref_g2_mul", "ref_g1_add", "ref_g2_add"):
            getattr(lib, name).argtypes = [vp, vp, vp]
        lib.ref_fr_inv.argtypes = [vp, vp]
        lib.ref_fq_from_std.argtypes = [vp, vp]
        lib.ref_g1_generator.argtypes = [vp]
        lib.ref_g2_generator.argtypes = [vp]
        lib.ref_msm_g1_small.argtypes = [vp, vp, ctypes.c_size_t, vp]
        lib.ref_msm_g2_small.argtypes = [vp, vp, ctypes.c_size_t, vp]
        lib.ref_verify_files.argtypes = [ctypes.c_char_p] * 3
        lib.ref_verify_witness.argtypes = [ctypes.c_int, ctypes.c_int, vp, vp, vp, vp, vp]
        lib.ref_export_r1cs.argtypes = [ctypes.c_int] * 4 + [vp, vp, vp, vp, ctypes.c_char_p]
        lib.ref_export_wtns.argtypes = [vp, ctypes.c_int, ctypes.c_char_p]
        lib.ref_pairing.argtypes = [vp, vp, vp]
        lib.ref_statement_tiny_cnn_b.argtypes = [ctypes.c_char_p, ctypes.c_char_p, vp]
        lib.ref_statement_mlp.argtypes = [ctypes.c_uint64] + [ctypes.c_int] * 6 + [ctypes.c_char_p, ctypes.c_char_p, vp]
        lib.ref_poseidon_constants.argtypes = [vp, vp]
        lib.ref_poseidon_constants.restype = None
        lib.ref_statement_generic.argtypes = [ctypes.c_int, vp, vp, vp, vp, vp, ctypes.c_int, ctypes.c_int, vp, vp,
                                              ctypes.c_int64, vp, ctypes.c_uint64, ctypes.c_char_p, ctypes.c_char_p,
                                              vp, ctypes.c_char_p, ctypes.c_size_t]
        _ref = lib
    return _ref


# ------------------------------------------------------------------ helpers
class OracleR1CS:
    """An R1CS held by the oracle, built from COO arrays."""

    def __init__(self, nc, nv, npub, npriv, mats):
        self.lib = oracle()
        self.h = self.lib.orc_r1cs_new(nc, nv, npub, npriv)
        self.nc, self.nv, self.npub = nc, nv, npub
        for which, (rows, cols, vals) in enumerate(mats):
            rows = np.ascontiguousarray(rows, dtype=np.int32)
            cols = np.ascontiguousarray(cols, dtype=np.int32)
            vals = np.ascontiguousarray(vals, dtype=np.uint64)
            self.lib.orc_r1cs_add(self.h, which, ptr(rows), ptr(cols), ptr(vals), len(rows))

    def verify(self, w):
        w = np.ascontiguousarray(w, dtype=np.uint64)
        return bool(self.lib.orc_r1cs_verify(self.h, ptr(w), w.shape[0]))

    def compute_h(self, w, threads=4):
        w = np.ascontiguousarray(w, dtype=np.uint64)
        n = 1 << self.lib.orc_qap_log_n(self.nc)
        out = words(n)
        got = self.lib.orc_compute_h(self.h, ptr(w), w.shape[0], ptr(out), threads)
        assert got == n
        return out

    def setup(self, seed, pk_path, vk_path, threads=4):
        rc = self.lib.orc_setup(self.h, seed, pk_path.encode(), vk_path.encode(), threads)
        assert rc == 0, rc

    def prove(self, pk_path, w, seed, threads=4, g2_affine_ref=False):
        """g2_affine_ref: the B term on the reference's affine-inversion G2
        arithmetic (src/curve/g2.cuh:103-146) instead of Jacobian G2."""
        w = np.ascontiguousarray(w, dtype=np.uint64)
        out = np.zeros(256, dtype=np.uint8)
        ms = np.zeros(4, dtype=np.float64)
        rc = self.lib.orc_prove_g2mode(pk_path.encode(), self.h, ptr(w), w.shape[0], seed, threads, ptr(out),
                                       ptr(ms), int(g2_affine_ref))
        return rc, out.tobytes(), ms

    def __del__(self):
        try:
            self.lib.orc_r1cs_free(self.h)
        except Exception:
            pass
