"""zk_ntt_noalloc (the NTT entry point that allocates no device memory)
against zk_ntt through the C ABI: bit-identical outputs on two calls in a
row, the second smaller (so it reuses the fixed scratch with other tables),
forward and inverse, batched; sizes beyond the fixed scratch are refused;
device free memory is unchanged across the calls."""
import ctypes

import numpy as np
import pytest

import zkml_amd

pytestmark = pytest.mark.gpu


def _free_bytes():
    hip = ctypes.CDLL("libamdhip64.so")
    free, total = ctypes.c_size_t(), ctypes.c_size_t()
    assert hip.hipMemGetInfo(ctypes.byref(free), ctypes.byref(total)) == 0
    return free.value


@pytest.fixture(scope="module")
def ctx():
    c = zkml_amd.Context(0)
    yield c
    c.close()


def _run_pair(ctx, log_n, batch, inverse, rng):
    a = zkml_amd.random_fr(batch << log_n, rng)
    d_in = ctx.upload(a)
    d_ref = ctx.alloc(a.nbytes)
    d_out = ctx.alloc(a.nbytes)
    ctx.ntt(d_ref, d_in, log_n, inverse=inverse, batch=batch)
    ctx.sync()
    want = ctx.d2h(d_ref, a.shape)
    before = _free_bytes()
    ctx.ntt_noalloc(d_out, d_in, log_n, inverse=inverse, batch=batch)
    ctx.sync()
    assert _free_bytes() == before
    got = ctx.d2h(d_out, a.shape)
    assert np.array_equal(got, want), (log_n, batch, inverse)
    # in place as well
    ctx.ntt_noalloc(d_in, d_in, log_n, inverse=inverse, batch=batch)
    ctx.sync()
    assert np.array_equal(ctx.d2h(d_in, a.shape), want)


@pytest.mark.parametrize("inverse", [False, True])
def test_noalloc_equals_ntt_two_calls_second_smaller(ctx, inverse):
    rng = np.random.default_rng(11 + inverse)
    _run_pair(ctx, 16, 4, inverse, rng)   # 2^18 elements: the whole buffer
    _run_pair(ctx, 12, 3, inverse, rng)   # smaller, other tables
    _run_pair(ctx, 5, 2, inverse, rng)    # one pass
    _run_pair(ctx, 12, 1, inverse, rng)   # back to the size before


def test_noalloc_rejects_sizes_beyond_the_scratch(ctx):
    rng = np.random.default_rng(3)
    a = zkml_amd.random_fr(1 << 17, rng)
    d = ctx.upload(a)
    o = ctx.alloc(a.nbytes)
    with pytest.raises(zkml_amd.ZkError, match="log_n outside"):
        ctx.ntt_noalloc(o, d, 17)
    b = zkml_amd.random_fr(5 << 16, rng)
    db = ctx.upload(b)
    ob = ctx.alloc(b.nbytes)
    with pytest.raises(zkml_amd.ZkError, match="above 2\\^18"):
        ctx.ntt_noalloc(ob, db, 16, batch=5)
    # the entry point still works after a refusal
    ctx.ntt_noalloc(o, d, 16, batch=2)
    ref = ctx.alloc(a.nbytes)
    ctx.ntt(ref, d, 16, batch=2)
    ctx.sync()
    assert np.array_equal(ctx.d2h(o, a.shape), ctx.d2h(ref, a.shape))
