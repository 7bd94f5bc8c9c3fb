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
