"""Python (ctypes) front end of libzkml_gpu.so, the MI355X Groth16 prover core.

Used by the tests, bench.py and __graft_entry__.py.  It calls the C ABI of
include/zkml_gpu.h directly; there is no CPU fallback: if the library is not
built, or a call fails, a ZkError is raised.
"""
import ctypes
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libzkml_gpu.so")

vp = ctypes.c_void_p
_lib = None


class ZkError(RuntimeError):
    pass


class ZkLayer(ctypes.Structure):
    """zk_layer of include/zkml_gpu.h (reference NNModel::Layer)."""
    _fields_ = [("type", ctypes.c_int32), ("in_size", ctypes.c_int32), ("out_size", ctypes.c_int32),
                ("conv_in_c", ctypes.c_int32), ("conv_in_h", ctypes.c_int32), ("conv_in_w", ctypes.c_int32),
                ("conv_out_c", ctypes.c_int32), ("conv_kh", ctypes.c_int32), ("conv_kw", ctypes.c_int32),
                ("conv_stride", ctypes.c_int32), ("conv_pad", ctypes.c_int32),
                ("relu_bits", ctypes.c_int32), ("relu_shift", ctypes.c_int32),
                ("relu_c", ctypes.c_int64 * 4), ("relu_scale", ctypes.c_int64),
                ("weights", ctypes.c_void_p), ("bias", ctypes.c_void_p)]


class ZkStatementOptions(ctypes.Structure):
    """zk_statement_options of include/zkml_gpu.h (reference StatementV2Options)."""
    _fields_ = [("model_tag", ctypes.c_uint64 * 4), ("has_context", ctypes.c_int32),
                ("context", ctypes.c_uint64 * 4), ("private_input", ctypes.c_int32),
                ("input_blinding", ctypes.c_void_p), ("private_model", ctypes.c_int32),
                ("private_outputs", ctypes.c_int32), ("route", ctypes.c_int32),
                ("route_threshold", ctypes.c_int64), ("compare_bits", ctypes.c_int32)]


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise ZkError(f"{LIB_PATH} is not built (run __graft_entry__.build())")
        L = ctypes.CDLL(LIB_PATH)
        L.zk_create.argtypes = [ctypes.c_int, ctypes.POINTER(vp)]
        L.zk_destroy.argtypes = [vp]
        L.zk_status_string.restype = ctypes.c_char_p
        L.zk_status_string.argtypes = [ctypes.c_int]
        L.zk_last_error.restype = ctypes.c_char_p
        L.zk_last_error.argtypes = [vp]
        L.zk_synchronize.argtypes = [vp]
        L.zk_get_stream.restype = vp
        L.zk_get_stream.argtypes = [vp]
        L.zk_dev_alloc.argtypes = [vp, ctypes.c_size_t, ctypes.POINTER(vp)]
        L.zk_dev_free.argtypes = [vp, vp]
        for f in ("zk_memcpy_h2d", "zk_memcpy_d2h", "zk_memcpy_d2d"):
            getattr(L, f).argtypes = [vp, vp, vp, ctypes.c_size_t]
        L.zk_set_profiling.argtypes = [vp, ctypes.c_int]
        L.zk_set_profiling_only.argtypes = [vp, ctypes.c_char_p]
        L.zk_kernel_stats.argtypes = [vp, ctypes.c_char_p, ctypes.POINTER(ctypes.c_uint64),
                                      ctypes.POINTER(ctypes.c_double)]
        L.zk_reset_kernel_stats.argtypes = [vp]
        L.zk_kernel_stats_names.restype = ctypes.c_char_p
        L.zk_kernel_stats_names.argtypes = [vp]
        L.zk_ntt.argtypes = [vp, vp, vp, ctypes.c_int, ctypes.c_int, ctypes.c_int, vp]
        L.zk_ntt_noalloc.argtypes = [vp, vp, vp, ctypes.c_int, ctypes.c_int, ctypes.c_int, vp]
        L.zk_coset_ntt.argtypes = [vp, vp, vp, ctypes.c_int, ctypes.c_uint64, ctypes.c_int, ctypes.c_int, vp]
        L.zk_msm_g1.argtypes = [vp, vp, vp, ctypes.c_size_t, vp, vp]
        L.zk_msm_g2.argtypes = [vp, vp, vp, ctypes.c_size_t, vp, vp]
        L.zk_msm_record_bytes.argtypes = [ctypes.c_int]
        L.zk_msm_record_bytes.restype = ctypes.c_size_t
        L.zk_msm_prepare_points.argtypes = [vp, vp, ctypes.c_size_t, ctypes.c_int, vp, vp]
        L.zk_msm_g1_prepared.argtypes = [vp, vp, vp, ctypes.c_size_t, vp, vp]
        L.zk_msm_g2_prepared.argtypes = [vp, vp, vp, ctypes.c_size_t, vp, vp]
        L.zk_msm_config.argtypes = [ctypes.c_size_t, ctypes.c_int, ctypes.POINTER(ctypes.c_int),
                                    ctypes.POINTER(ctypes.c_int)]
        L.zk_msm_g1_host.argtypes = [vp, vp, vp, ctypes.c_int, vp]
        L.zk_msm_g2_host.argtypes = [vp, vp, vp, ctypes.c_int, vp]
        L.zk_g1_generator_mul.argtypes = [vp, vp, ctypes.c_size_t, vp, vp]
        L.zk_g2_generator_mul.argtypes = [vp, vp, ctypes.c_size_t, vp, vp]
        L.zk_r1cs_create.argtypes = [vp, ctypes.c_int, ctypes.c_int, ctypes.c_int, vp, ctypes.c_size_t, vp,
                                     ctypes.c_size_t, vp, ctypes.c_size_t, ctypes.POINTER(vp)]
        L.zk_r1cs_destroy.argtypes = [vp]
        L.zk_r1cs_domain.argtypes = [vp, ctypes.POINTER(ctypes.c_int)]
        L.zk_quotient_h.argtypes = [vp, vp, vp, ctypes.c_size_t, vp, vp]
        L.zk_pk_load.argtypes = [vp, ctypes.c_char_p, ctypes.POINTER(vp)]
        L.zk_pk_destroy.argtypes = [vp]
        L.zk_pk_info.argtypes = [vp] + [ctypes.POINTER(ctypes.c_int)] * 3
        L.zk_setup.argtypes = [vp, vp, ctypes.c_uint64, ctypes.c_char_p, ctypes.c_char_p]
        L.zk_prove.argtypes = [vp, vp, vp, vp, ctypes.c_size_t, ctypes.c_int, ctypes.c_uint64, ctypes.c_int, vp, vp]
        ip = ctypes.POINTER(ctypes.c_int)
        sp = ctypes.POINTER(ctypes.c_size_t)
        L.zk_iden3_r1cs_info.argtypes = [ctypes.c_char_p, ip, ip, ip, ip, sp, sp, sp]
        L.zk_iden3_r1cs_read.argtypes = [ctypes.c_char_p, vp, vp, vp]
        L.zk_iden3_r1cs_write.argtypes = [ctypes.c_char_p, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                          vp, ctypes.c_size_t, vp, ctypes.c_size_t, vp, ctypes.c_size_t]
        L.zk_wtns_info.argtypes = [ctypes.c_char_p, sp]
        L.zk_wtns_read.argtypes = [ctypes.c_char_p, vp, ctypes.c_size_t]
        L.zk_wtns_write.argtypes = [ctypes.c_char_p, vp, ctypes.c_size_t]
        L.zk_synthetic_r1cs.argtypes = [ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_uint64, vp, sp, vp, sp,
                                        vp, sp, vp]
        L.zk_pairing.argtypes = [vp, vp, vp]
        L.zk_verify.argtypes = [vp, ctypes.c_size_t, vp, vp, ctypes.c_int, ctypes.POINTER(ctypes.c_int)]
        L.zk_verify_files.argtypes = [ctypes.c_char_p, ctypes.c_char_p, ctypes.c_char_p,
                                      ctypes.POINTER(ctypes.c_int)]
        L.zk_kzg_commit.argtypes = [vp, vp, vp, ctypes.c_size_t, vp, vp]
        L.zk_kzg_open.argtypes = [vp, vp, vp, ctypes.c_size_t, vp, vp, vp, vp]
        L.zk_poseidon_permute.argtypes = [vp]
        L.zk_poseidon_hash2.argtypes = [vp, vp, vp]
        L.zk_poseidon_commit.argtypes = [vp, ctypes.c_size_t, ctypes.c_uint64, vp]
        L.zk_poseidon_constants.argtypes = [vp, vp]
        L.zk_statement_v2_build.argtypes = [ctypes.POINTER(ZkLayer), ctypes.c_int, vp, ctypes.c_int, ctypes.c_int,
                                            ctypes.POINTER(ZkStatementOptions), ctypes.POINTER(vp),
                                            ctypes.c_char_p, ctypes.c_size_t]
        L.zk_statement_destroy.argtypes = [vp]
        L.zk_statement_destroy.restype = None
        L.zk_statement_info.argtypes = [vp, ip, ip, ip, ip, sp, sp, sp]
        L.zk_statement_layout.argtypes = [vp, vp]
        L.zk_statement_r1cs.argtypes = [vp, vp, vp, vp]
        L.zk_statement_witness.argtypes = [vp, vp]
        L.zk_statement_scores.argtypes = [vp, vp]
        L.zk_statement_check.argtypes = [vp]
        L.zk_statement_write.argtypes = [vp, ctypes.c_char_p, ctypes.c_char_p]
        L.zk_statement_meta_json.argtypes = [vp, ctypes.c_uint64, ctypes.c_char_p, ctypes.c_size_t, sp]
        _lib = L
    return _lib


def _np_ptr(a):
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data_as(vp)


R_WORDS = np.array([0x43E1F593F0000001, 0x2833E84879B97091, 0xB85045B68181585D, 0x30644E72E131A029],
                   dtype=np.uint64)


def random_fr(n, rng):
    """n uniform elements of [0, r) as (n, 4) uint64 words (rejection sampling).
    Any value below r is a valid Montgomery-form element."""
    out = np.empty((n, 4), dtype=np.uint64)
    filled = 0
    while filled < n:
        k = (n - filled) * 5 // 4 + 16
        w = rng.integers(0, 2**64, size=(k, 4), dtype=np.uint64)
        w[:, 3] &= np.uint64((1 << 62) - 1)
        # lexicographic compare from the top limb
        lt = np.zeros(k, dtype=bool)
        eq = np.ones(k, dtype=bool)
        for i in (3, 2, 1, 0):
            lt |= eq & (w[:, i] < R_WORDS[i])
            eq &= w[:, i] == R_WORDS[i]
        w = w[lt]
        take = min(len(w), n - filled)
        out[filled:filled + take] = w[:take]
        filled += take
    return out


SPARSE_DTYPE = np.dtype([("row", "<i4"), ("col", "<i4"), ("value", "<u8", (4,))])  # 40 bytes


def sparse_entries(rows, cols, vals):
    """reference SparseEntry array (src/prover/circuit.cuh:32-36)."""
    e = np.zeros(len(rows), dtype=SPARSE_DTYPE)
    e["row"] = rows
    e["col"] = cols
    e["value"] = np.asarray(vals, dtype=np.uint64).reshape(-1, 4)
    return e


class DeviceBuffer:
    def __init__(self, ctx, nbytes):
        self.ctx = ctx
        self.nbytes = nbytes
        p = vp()
        ctx._check(lib().zk_dev_alloc(ctx.h, nbytes, ctypes.byref(p)))
        self.ptr = p.value

    def free(self):
        if self.ptr:
            lib().zk_dev_free(self.ctx.h, vp(self.ptr))
            self.ptr = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class Context:
    def __init__(self, device=0):
        self.h = vp()
        st = lib().zk_create(device, ctypes.byref(self.h))
        if st != 0:
            raise ZkError(f"zk_create failed: {lib().zk_status_string(st).decode()}")

    def _check(self, st, what=""):
        if st != 0:
            msg = lib().zk_last_error(self.h).decode(errors="replace")
            raise ZkError(f"{what} failed ({lib().zk_status_string(st).decode()}): {msg}")

    def close(self):
        if self.h:
            lib().zk_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    # ---- memory
    def alloc(self, nbytes):
        return DeviceBuffer(self, int(nbytes))

    def upload(self, arr):
        arr = np.ascontiguousarray(arr)
        buf = self.alloc(max(arr.nbytes, 1))
        self._check(lib().zk_memcpy_h2d(self.h, vp(buf.ptr), _np_ptr(arr), arr.nbytes), "h2d")
        return buf

    def h2d(self, buf, arr):
        arr = np.ascontiguousarray(arr)
        assert arr.nbytes <= buf.nbytes
        self._check(lib().zk_memcpy_h2d(self.h, vp(buf.ptr), _np_ptr(arr), arr.nbytes), "h2d")

    def d2h(self, buf, shape, dtype=np.uint64):
        out = np.empty(shape, dtype=dtype)
        self._check(lib().zk_memcpy_d2h(self.h, _np_ptr(out), vp(buf.ptr), out.nbytes), "d2h")
        return out

    def sync(self):
        self._check(lib().zk_synchronize(self.h), "synchronize")

    # ---- profiling
    def set_profiling(self, on, only=None):
        """Per-kernel HIP-event timing; `only` restricts it to one kernel name."""
        self._check(lib().zk_set_profiling_only(self.h, only.encode() if only else None))
        self._check(lib().zk_set_profiling(self.h, 1 if on else 0))

    def kernel_stats(self, name):
        n = ctypes.c_uint64()
        ms = ctypes.c_double()
        self._check(lib().zk_kernel_stats(self.h, name.encode(), ctypes.byref(n), ctypes.byref(ms)))
        return n.value, ms.value

    def reset_kernel_stats(self):
        self._check(lib().zk_reset_kernel_stats(self.h))

    def kernel_names(self):
        s = lib().zk_kernel_stats_names(self.h).decode()
        return [x for x in s.split(",") if x]

    # ---- NTT
    def ntt(self, d_out, d_in, log_n, inverse=False, batch=1):
        self._check(lib().zk_ntt(self.h, vp(d_out.ptr), vp(d_in.ptr), log_n, int(inverse), batch, None), "zk_ntt")

    def ntt_noalloc(self, d_out, d_in, log_n, inverse=False, batch=1):
        """zk_ntt_noalloc: the same transform with no device allocation."""
        self._check(lib().zk_ntt_noalloc(self.h, vp(d_out.ptr), vp(d_in.ptr), log_n, int(inverse), batch, None),
                    "zk_ntt_noalloc")

    def coset_ntt(self, d_out, d_in, log_n, g, inverse=False, batch=1):
        self._check(lib().zk_coset_ntt(self.h, vp(d_out.ptr), vp(d_in.ptr), log_n, g, int(inverse), batch, None),
                    "zk_coset_ntt")

    # ---- MSM
    def msm_g1(self, d_points, d_scalars, n):
        out = np.zeros(8, dtype=np.uint64)
        self._check(lib().zk_msm_g1(self.h, vp(d_points.ptr), vp(d_scalars.ptr), n, _np_ptr(out), None), "zk_msm_g1")
        return out

    def msm_g2(self, d_points, d_scalars, n):
        out = np.zeros(16, dtype=np.uint64)
        self._check(lib().zk_msm_g2(self.h, vp(d_points.ptr), vp(d_scalars.ptr), n, _np_ptr(out), None), "zk_msm_g2")
        return out

    def msm_prepare(self, d_points, n, g2=False):
        """Point records of n points for repeated MSMs (zk_msm_prepare_points)."""
        d_recs = self.alloc(max(1, n) * lib().zk_msm_record_bytes(int(g2)))
        self._check(lib().zk_msm_prepare_points(self.h, vp(d_points.ptr), n, int(g2), vp(d_recs.ptr), None),
                    "zk_msm_prepare_points")
        return d_recs

    def msm_g1_prepared(self, d_recs, d_scalars, n):
        out = np.zeros(8, dtype=np.uint64)
        self._check(lib().zk_msm_g1_prepared(self.h, vp(d_recs.ptr), vp(d_scalars.ptr), n, _np_ptr(out), None),
                    "zk_msm_g1_prepared")
        return out

    def msm_g2_prepared(self, d_recs, d_scalars, n):
        out = np.zeros(16, dtype=np.uint64)
        self._check(lib().zk_msm_g2_prepared(self.h, vp(d_recs.ptr), vp(d_scalars.ptr), n, _np_ptr(out), None),
                    "zk_msm_g2_prepared")
        return out

    def kzg_commit(self, d_srs, d_coeffs, degree):
        """sum f_i [tau^i]_1 as (8,) u64 affine (Montgomery words)."""
        out = np.zeros(8, dtype=np.uint64)
        self._check(lib().zk_kzg_commit(self.h, vp(d_srs.ptr), vp(d_coeffs.ptr), degree, _np_ptr(out), None),
                    "zk_kzg_commit")
        return out

    def kzg_open(self, d_srs, d_coeffs, degree, z_mont):
        """(opening proof (8,) u64 affine, f(z) (4,) u64 Montgomery)."""
        out = np.zeros(8, dtype=np.uint64)
        fz = np.zeros(4, dtype=np.uint64)
        z = np.ascontiguousarray(z_mont, dtype=np.uint64).reshape(4)
        self._check(lib().zk_kzg_open(self.h, vp(d_srs.ptr), vp(d_coeffs.ptr), degree, _np_ptr(z), _np_ptr(out),
                                      _np_ptr(fz), None), "zk_kzg_open")
        return out, fz

    @staticmethod
    def msm_config(n, g2=False):
        """(window bits, windows) the MSM uses for n points."""
        c, w = ctypes.c_int(), ctypes.c_int()
        st = lib().zk_msm_config(n, int(g2), ctypes.byref(c), ctypes.byref(w))
        if st:
            raise ZkError(f"zk_msm_config failed ({lib().zk_status_string(st).decode()})")
        return c.value, w.value

    def g1_generator_mul(self, d_scalars, n, d_out):
        self._check(lib().zk_g1_generator_mul(self.h, vp(d_scalars.ptr), n, vp(d_out.ptr), None), "g1_generator_mul")

    def g2_generator_mul(self, d_scalars, n, d_out):
        self._check(lib().zk_g2_generator_mul(self.h, vp(d_scalars.ptr), n, vp(d_out.ptr), None), "g2_generator_mul")

    # ---- Groth16
    def r1cs(self, num_constraints, num_variables, num_public, A, B, C):
        """A, B, C: SPARSE_DTYPE arrays (or (rows, cols, vals) triples)."""
        mats = []
        for M in (A, B, C):
            if not isinstance(M, np.ndarray):
                M = sparse_entries(*M)
            mats.append(np.ascontiguousarray(M))
        h = vp()
        self._check(lib().zk_r1cs_create(self.h, num_constraints, num_variables, num_public,
                                         _np_ptr(mats[0]), len(mats[0]), _np_ptr(mats[1]), len(mats[1]),
                                         _np_ptr(mats[2]), len(mats[2]), ctypes.byref(h)), "zk_r1cs_create")
        return R1CS(self, h, num_constraints, num_variables, num_public)

    def load_pk(self, path):
        h = vp()
        self._check(lib().zk_pk_load(self.h, str(path).encode(), ctypes.byref(h)), "zk_pk_load")
        return ProvingKey(self, h)

    def setup(self, r1cs, seed, pk_path, vk_path):
        self._check(lib().zk_setup(self.h, r1cs.h, seed, str(pk_path).encode(), str(vk_path).encode()), "zk_setup")

    def prove(self, pk, r1cs, witness, num_public, seed, check_witness=True):
        """witness: (m, 4) uint64 Montgomery words.  Returns (256 bytes, timings)."""
        w = np.ascontiguousarray(witness, dtype=np.uint64)
        out = np.zeros(256, dtype=np.uint8)
        t = np.zeros(8, dtype=np.float64)
        self._check(lib().zk_prove(self.h, pk.h, r1cs.h, _np_ptr(w), w.shape[0], num_public, seed,
                                   int(check_witness), _np_ptr(out), _np_ptr(t)), "zk_prove")
        names = ("total", "quotient", "A", "B_g2", "L", "H", "B_g1", "host")
        return out.tobytes(), dict(zip(names, t.tolist()))

    def quotient_h(self, r1cs, d_witness, m, d_h):
        self._check(lib().zk_quotient_h(self.h, r1cs.h, vp(d_witness.ptr), m, vp(d_h.ptr), None), "zk_quotient_h")


def _status(st, what):
    if st:
        raise ZkError(f"{what} failed ({lib().zk_status_string(st).decode()})")


def _opt_ptr(a):
    return _np_ptr(a) if len(a) else None


def iden3_r1cs_read(path):
    """(num_constraints, num_variables, num_public, num_private, A, B, C) from an
    iden3 .r1cs file; A, B, C as SPARSE_DTYPE arrays (Montgomery values)."""
    nc, nv, npub, npriv = (ctypes.c_int() for _ in range(4))
    na, nb, ncc = (ctypes.c_size_t() for _ in range(3))
    _status(lib().zk_iden3_r1cs_info(path.encode(), ctypes.byref(nc), ctypes.byref(nv), ctypes.byref(npub),
                                     ctypes.byref(npriv), ctypes.byref(na), ctypes.byref(nb), ctypes.byref(ncc)),
            "zk_iden3_r1cs_info")
    mats = [np.zeros(k.value, dtype=SPARSE_DTYPE) for k in (na, nb, ncc)]
    _status(lib().zk_iden3_r1cs_read(path.encode(), *[_opt_ptr(m) for m in mats]), "zk_iden3_r1cs_read")
    return (nc.value, nv.value, npub.value, npriv.value, *mats)


def iden3_r1cs_write(path, num_constraints, num_variables, num_public, num_private, A, B, C):
    mats = [np.ascontiguousarray(M if isinstance(M, np.ndarray) else sparse_entries(*M)) for M in (A, B, C)]
    _status(lib().zk_iden3_r1cs_write(path.encode(), num_constraints, num_variables, num_public, num_private,
                                      _opt_ptr(mats[0]), len(mats[0]), _opt_ptr(mats[1]), len(mats[1]),
                                      _opt_ptr(mats[2]), len(mats[2])), "zk_iden3_r1cs_write")


def wtns_read(path):
    m = ctypes.c_size_t()
    _status(lib().zk_wtns_info(path.encode(), ctypes.byref(m)), "zk_wtns_info")
    w = np.zeros((m.value, 4), dtype=np.uint64)
    _status(lib().zk_wtns_read(path.encode(), _np_ptr(w), m.value), "zk_wtns_read")
    return w


def wtns_write(path, w_mont):
    w = np.ascontiguousarray(w_mont, dtype=np.uint64).reshape(-1, 4)
    _status(lib().zk_wtns_write(path.encode(), _np_ptr(w), w.shape[0]), "zk_wtns_write")


def synthetic_r1cs(num_constraints, num_public, num_inputs, seed):
    """Config-5 style random R1CS: (A, B, C, witness) with the witness in
    Montgomery words; num_variables = witness rows."""
    A = np.zeros(3 * num_constraints, dtype=SPARSE_DTYPE)
    B = np.zeros(3 * num_constraints, dtype=SPARSE_DTYPE)
    C = np.zeros(num_constraints, dtype=SPARSE_DTYPE)
    w = np.zeros((1 + num_public + num_inputs + num_constraints, 4), dtype=np.uint64)
    na, nb, ncc = (ctypes.c_size_t() for _ in range(3))
    _status(lib().zk_synthetic_r1cs(num_constraints, num_public, num_inputs, seed, _opt_ptr(A), ctypes.byref(na),
                                    _opt_ptr(B), ctypes.byref(nb), _opt_ptr(C), ctypes.byref(ncc), _np_ptr(w)),
            "zk_synthetic_r1cs")
    return A[:na.value].copy(), B[:nb.value].copy(), C[:ncc.value].copy(), w


def pairing(p_std, q_std):
    """e(P, Q): P (8,) u64 standard form x, y; Q (16,) u64.  Returns (48,) u64,
    the Fp12 value in standard form (12 Fq elements, reference order)."""
    p = np.ascontiguousarray(p_std, dtype=np.uint64)
    q = np.ascontiguousarray(q_std, dtype=np.uint64)
    out = np.zeros(48, dtype=np.uint64)
    st = lib().zk_pairing(_np_ptr(p), _np_ptr(q), _np_ptr(out))
    if st:
        raise ZkError(f"zk_pairing failed ({lib().zk_status_string(st).decode()})")
    return out


def verify(vk_bytes, proof_bytes, publics_std):
    """Groth16 verification (host).  publics_std: (npub, 4) u64 standard form."""
    pub = np.ascontiguousarray(publics_std, dtype=np.uint64).reshape(-1, 4)
    vk = np.frombuffer(bytes(vk_bytes), dtype=np.uint8).copy()
    pr = np.frombuffer(bytes(proof_bytes), dtype=np.uint8).copy()
    ok = ctypes.c_int(0)
    st = lib().zk_verify(_np_ptr(vk), vk.size, _np_ptr(pr), _np_ptr(pub) if pub.size else None, pub.shape[0],
                         ctypes.byref(ok))
    if st:
        raise ZkError(f"zk_verify failed ({lib().zk_status_string(st).decode()})")
    return bool(ok.value)


def verify_files(vk_path, proof_path, publics_path):
    ok = ctypes.c_int(0)
    st = lib().zk_verify_files(vk_path.encode(), proof_path.encode(), publics_path.encode(), ctypes.byref(ok))
    if st:
        raise ZkError(f"zk_verify_files failed ({lib().zk_status_string(st).decode()})")
    return bool(ok.value)


R_INT = 21888242871839275222246405745257275088548364400416034343698204186575808495617


def std_words(x):
    """Python int -> 4 little-endian u64 words of x mod r (standard form)."""
    x %= R_INT
    return np.array([(x >> (64 * k)) & ((1 << 64) - 1) for k in range(4)], dtype=np.uint64)


def words_int(w):
    w = np.asarray(w, dtype=np.uint64).reshape(-1)
    return sum(int(w[k]) << (64 * k) for k in range(4))


# ---- Poseidon (host) -----------------------------------------------------------
DOMAIN_MODEL = 0x4D4F44454C
DOMAIN_INPUT = 0x494E505554


def poseidon_permute(state):
    """Poseidon t = 3 permutation of three field elements (Python ints)."""
    s = np.concatenate([std_words(x) for x in state])
    _status(lib().zk_poseidon_permute(_np_ptr(s)), "zk_poseidon_permute")
    return [words_int(s[4 * i:4 * i + 4]) for i in range(3)]


def poseidon_hash2(a, b):
    """circomlib Poseidon([a, b])."""
    out = np.zeros(4, dtype=np.uint64)
    _status(lib().zk_poseidon_hash2(_np_ptr(std_words(a)), _np_ptr(std_words(b)), _np_ptr(out)),
            "zk_poseidon_hash2")
    return words_int(out)


def poseidon_commit(values, domain):
    """Rate-2 sponge commitment of the statement (capacity (len << 64) | domain)."""
    v = np.concatenate([std_words(x) for x in values]) if len(values) else np.zeros(0, dtype=np.uint64)
    out = np.zeros(4, dtype=np.uint64)
    _status(lib().zk_poseidon_commit(_opt_ptr(v), len(values), domain, _np_ptr(out)), "zk_poseidon_commit")
    return words_int(out)


def poseidon_constants():
    """(round constants: 195 ints, MDS: 3 x 3 ints)."""
    rc = np.zeros(195 * 4, dtype=np.uint64)
    mds = np.zeros(9 * 4, dtype=np.uint64)
    _status(lib().zk_poseidon_constants(_np_ptr(rc), _np_ptr(mds)), "zk_poseidon_constants")
    rci = [words_int(rc[4 * i:4 * i + 4]) for i in range(195)]
    m = [words_int(mds[4 * i:4 * i + 4]) for i in range(9)]
    return rci, [m[0:3], m[3:6], m[6:9]]


# ---- statement producer (host) ---------------------------------------------------
LINEAR, RELU_APPROX, SOFTMAX_APPROX, SELF_ATTENTION, RELU_EXACT, CONV2D = range(6)
LAYOUT_KEYS = ("batch", "n_in", "n_out", "outputs_start", "model_tag_index", "context_index",
               "model_commitment_index", "inputs_start", "input_slot_size", "route_start", "num_public")


def layer_linear(in_size, out_size, weights, bias):
    return {"type": LINEAR, "in_size": in_size, "out_size": out_size,
            "weights": np.asarray(weights, dtype=np.int64).reshape(-1),
            "bias": np.asarray(bias, dtype=np.int64).reshape(-1)}


def layer_conv2d(in_c, in_h, in_w, out_c, kh, kw, stride, pad, weights, bias):
    return {"type": CONV2D, "conv": (in_c, in_h, in_w, out_c, kh, kw, stride, pad),
            "weights": np.asarray(weights, dtype=np.int64).reshape(-1),
            "bias": np.asarray(bias, dtype=np.int64).reshape(-1)}


def layer_relu_exact(size, bits, shift):
    return {"type": RELU_EXACT, "in_size": size, "out_size": size, "bits": bits, "shift": shift}


def layer_relu_approx(size, c=(64, 64, 1, 0), scale=1):
    """Defaults are NNModel::make_relu_layer's coefficients."""
    return {"type": RELU_APPROX, "in_size": size, "out_size": size, "c": tuple(c), "scale": scale}


def layer_softmax(size):
    return {"type": SOFTMAX_APPROX, "in_size": size, "out_size": size}


class Statement:
    """R1CS + witness of zk_statement_v2_build (reference build_statement_v2)."""

    def __init__(self, h):
        self.h = h
        nc, nv, npub, npriv = (ctypes.c_int() for _ in range(4))
        na, nb, ncc = (ctypes.c_size_t() for _ in range(3))
        _status(lib().zk_statement_info(h, ctypes.byref(nc), ctypes.byref(nv), ctypes.byref(npub),
                                        ctypes.byref(npriv), ctypes.byref(na), ctypes.byref(nb), ctypes.byref(ncc)),
                "zk_statement_info")
        self.nc, self.nv, self.npub, self.npriv = nc.value, nv.value, npub.value, npriv.value
        self.A, self.B, self.C = (np.zeros(k.value, dtype=SPARSE_DTYPE) for k in (na, nb, ncc))
        _status(lib().zk_statement_r1cs(h, _opt_ptr(self.A), _opt_ptr(self.B), _opt_ptr(self.C)),
                "zk_statement_r1cs")
        self.w = np.zeros((self.nv, 4), dtype=np.uint64)
        _status(lib().zk_statement_witness(h, _np_ptr(self.w)), "zk_statement_witness")
        lay = np.zeros(len(LAYOUT_KEYS), dtype=np.int32)
        _status(lib().zk_statement_layout(h, _np_ptr(lay)), "zk_statement_layout")
        self.layout = dict(zip(LAYOUT_KEYS, (int(x) for x in lay)))
        sc = np.zeros(self.layout["batch"] * self.layout["n_out"], dtype=np.int64)
        _status(lib().zk_statement_scores(h, _np_ptr(sc)), "zk_statement_scores")
        self.scores = sc.reshape(self.layout["batch"], self.layout["n_out"])

    def check(self):
        """True when the witness satisfies every row (host check)."""
        st = lib().zk_statement_check(self.h)
        if st not in (0, 6):
            _status(st, "zk_statement_check")
        return st == 0

    def write(self, r1cs_path=None, wtns_path=None):
        _status(lib().zk_statement_write(self.h, r1cs_path.encode() if r1cs_path else None,
                                         wtns_path.encode() if wtns_path else None), "zk_statement_write")

    def meta_json(self, model_tag64=0):
        n = ctypes.c_size_t()
        _status(lib().zk_statement_meta_json(self.h, model_tag64, None, 0, ctypes.byref(n)),
                "zk_statement_meta_json")
        buf = ctypes.create_string_buffer(n.value + 1)
        _status(lib().zk_statement_meta_json(self.h, model_tag64, buf, n.value + 1, ctypes.byref(n)),
                "zk_statement_meta_json")
        return buf.value.decode()

    def publics_std(self):
        """Public inputs w[1..npub] as (npub, 4) standard-form words."""
        out = np.zeros((self.npub, 4), dtype=np.uint64)
        for i in range(self.npub):
            out[i] = std_words(words_int(self.w[1 + i]) * pow(1 << 256, -1, R_INT))
        return out

    def close(self):
        if self.h:
            lib().zk_statement_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def statement_v2(layers, inputs, model_tag=0, context=None, private_input=False, input_blinding=None,
                 private_model=False, private_outputs=False, route_threshold=None, compare_bits=48):
    """Build the statement for `inputs` (batch x n_in signed ints) through the
    product's builder.  route_threshold not None enables in-circuit routing."""
    x = np.asarray(inputs, dtype=np.int64)
    x = np.ascontiguousarray(x.reshape(len(inputs), -1) if x.size else x.reshape(len(inputs), 0))
    keep = [x]
    arr = (ZkLayer * max(1, len(layers)))()
    for i, d in enumerate(layers):
        L = arr[i]
        L.type = d["type"]
        L.in_size = d.get("in_size", 0)
        L.out_size = d.get("out_size", 0)
        if "conv" in d:
            (L.conv_in_c, L.conv_in_h, L.conv_in_w, L.conv_out_c, L.conv_kh, L.conv_kw, L.conv_stride,
             L.conv_pad) = d["conv"]
        L.relu_bits, L.relu_shift = d.get("bits", 0), d.get("shift", 0)
        for k, c in enumerate(d.get("c", (0, 0, 0, 0))):
            L.relu_c[k] = c
        L.relu_scale = d.get("scale", 0)
        for f in ("weights", "bias"):
            if f in d:
                a = np.ascontiguousarray(d[f], dtype=np.int64)
                keep.append(a)
                setattr(L, f, a.ctypes.data if a.size else None)
    o = ZkStatementOptions()
    for k, wd in enumerate(std_words(model_tag)):
        o.model_tag[k] = int(wd)
    if context is not None:
        o.has_context = 1
        for k, wd in enumerate(std_words(context)):
            o.context[k] = int(wd)
    if private_input:
        o.private_input = 1
        if input_blinding is not None:
            bl = np.concatenate([std_words(v) for v in input_blinding])
            keep.append(bl)
            o.input_blinding = bl.ctypes.data
    o.private_model = int(bool(private_model))
    o.private_outputs = int(bool(private_outputs))
    if route_threshold is not None:
        o.route = 1
        o.route_threshold = int(route_threshold)
    o.compare_bits = compare_bits
    h = vp()
    err = ctypes.create_string_buffer(256)
    st = lib().zk_statement_v2_build(arr, len(layers), _np_ptr(x) if x.size else None, x.shape[0],
                                     x.shape[1] if x.ndim == 2 else 0, ctypes.byref(o), ctypes.byref(h), err, 256)
    if st:
        raise ZkError(f"zk_statement_v2_build failed: {err.value.decode()}")
    del keep
    return Statement(h)


class R1CS:
    def __init__(self, ctx, h, nc, nv, npub):
        self.ctx, self.h, self.nc, self.nv, self.npub = ctx, h, nc, nv, npub
        ln = ctypes.c_int()
        lib().zk_r1cs_domain(h, ctypes.byref(ln))
        self.log_n = ln.value

    def close(self):
        if self.h:
            lib().zk_r1cs_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class ProvingKey:
    def __init__(self, ctx, h):
        self.ctx, self.h = ctx, h
        n, m, p = ctypes.c_int(), ctypes.c_int(), ctypes.c_int()
        lib().zk_pk_info(h, ctypes.byref(n), ctypes.byref(m), ctypes.byref(p))
        self.n, self.m, self.npub = n.value, m.value, p.value

    def close(self):
        if self.h:
            lib().zk_pk_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
