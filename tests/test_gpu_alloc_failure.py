"""Error paths of the NTT's cached tables: a device allocation that fails
while a transform builds its plan or its coset tables returns ZK_ERR_OOM,
caches nothing half-built, and the same context's next transforms (same size,
same coset) are bit-exact against the CPU oracle.  The failures are injected
with the library's zk_debug_fail_device_alloc hook; no device memory is
exhausted.  (The reference has no such path: it exits on any CUDA error,
src/common.cuh:11-19.)"""
import numpy as np
import pytest

from test_gpu_ntt import oracle_coset, oracle_ntt, rand_words

pytestmark = pytest.mark.gpu


def _fail_at(nth):
    import zkml_amd
    assert zkml_amd.lib().zk_debug_fail_device_alloc(nth) == 0


@pytest.mark.parametrize("log_n", [11, 17])
def test_table_allocation_failure_then_recovery(log_n):
    import zkml_amd
    ctx = zkml_amd.Context(0)  # fresh: no plan, coset table or pass buffer yet
    try:
        a = rand_words(1 << log_n, 100 + log_n)
        d_in = ctx.upload(a)
        d_out = ctx.alloc(a.nbytes)
        # A first coset transform allocates the plan's tables, then the coset
        # tables, then the pass-to-pass buffer.  Fail each in turn: the plan
        # (1st), the coset tables (2nd, after the plan is cached), the pass
        # buffer (2nd again, after the coset tables are cached).
        for nth in (1, 2, 2):
            _fail_at(nth)
            with pytest.raises(zkml_amd.ZkError, match="ZK_ERR_OOM|out of memory|allocation"):
                ctx.coset_ntt(d_out, d_in, log_n, 7, False)
            _fail_at(0)
        ctx.coset_ntt(d_out, d_in, log_n, 7, False)
        assert np.array_equal(ctx.d2h(d_out, a.shape), oracle_coset(a, log_n, 7, False))
        # plan cached, a new coset generator needs new tables: fail them once
        _fail_at(1)
        with pytest.raises(zkml_amd.ZkError):
            ctx.coset_ntt(d_out, d_in, log_n, 5, True)
        _fail_at(0)
        ctx.coset_ntt(d_out, d_in, log_n, 5, True)
        assert np.array_equal(ctx.d2h(d_out, a.shape), oracle_coset(a, log_n, 5, True))
        ctx.ntt(d_out, d_in, log_n, False)
        assert np.array_equal(ctx.d2h(d_out, a.shape), oracle_ntt(a, log_n, False))
    finally:
        _fail_at(0)
        ctx.close()


def _free_bytes():
    import ctypes
    hip = ctypes.CDLL("libamdhip64.so")
    free, total = ctypes.c_size_t(), ctypes.c_size_t()
    assert hip.hipMemGetInfo(ctypes.byref(free), ctypes.byref(total)) == 0
    return free.value


def test_pk_window_table_allocation_failure_falls_back(tmp_path):
    """zk_pk_load of a key with 2^15 variables builds window tables for its
    queries (each table, then its temporary, in the order A, B1, L, B2, H).
    A failed allocation of a table or of its temporary drops every table: the
    load still succeeds, leaves no error behind and holds a fraction of the
    tables' memory, and the next proof is byte-identical to a table-backed
    proof and to the oracle's prove on the same key and seed."""
    import zkml_amd
    from test_gpu_groth16 import PROVE_SEED, SETUP_SEED, _oracle_of
    ctx = zkml_amd.Context(0)
    try:
        nc, npub = (1 << 15) - 64, 4
        A, B, C, w = zkml_amd.synthetic_r1cs(nc, npub, 16, 15)
        r = ctx.r1cs(nc, w.shape[0], npub, A, B, C)
        pk_path, vk_path = str(tmp_path / "pk.bin"), str(tmp_path / "vk.bin")
        ctx.setup(r, SETUP_SEED, pk_path, vk_path)
        ctx.sync()
        before = _free_bytes()
        pk = ctx.load_pk(pk_path)
        with_tables = before - _free_bytes()
        proof, _ = ctx.prove(pk, r, w, npub, PROVE_SEED)
        pk.close()
        # 1: A's table, 2: A's temporary, 7: B2's table, 10: H's temporary
        for nth in (1, 2, 7, 10):
            print(f"[pk tables] allocation {nth} fails", flush=True)
            ctx.sync()
            before = _free_bytes()
            _fail_at(nth)
            try:
                pk = ctx.load_pk(pk_path)
            finally:
                _fail_at(0)
            used = before - _free_bytes()
            assert used < with_tables // 2, (nth, used, with_tables)
            assert zkml_amd.lib().zk_last_error(ctx.h) in (None, b"")
            again, _ = ctx.prove(pk, r, w, npub, PROVE_SEED)
            assert again == proof, nth
            pk.close()
        oc = _oracle_of(A, B, C, nc, w.shape[0], npub)
        rc, proof_o, _ = oc.prove(pk_path, w, PROVE_SEED, threads=16)
        assert rc == 0 and proof_o == proof
        r.close()
    finally:
        _fail_at(0)
        ctx.close()
