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


def test_noalloc_graph_replays_after_other_sizes(ctx):
    """zk_ntt_noalloc captured into HIP graphs (one size whose tables were
    already filled by an eager call, one whose first call is the captured
    one), replayed three times each with eager calls of other sizes in
    between: every replay equals zk_ntt, and so does an eager call of the
    size first seen under capture."""
    hip = ctypes.CDLL("libamdhip64.so")
    vp = ctypes.c_void_p
    rng = np.random.default_rng(29)
    st = vp()
    assert hip.hipStreamCreate(ctypes.byref(st)) == 0

    def sync():
        assert hip.hipStreamSynchronize(st) == 0

    def call(d_out, d_in, log_n, inverse=0):
        rc = zkml_amd.lib().zk_ntt_noalloc(ctx.h, vp(d_out.ptr), vp(d_in.ptr), log_n, inverse, 1, st)
        assert rc == 0, zkml_amd.lib().zk_last_error(ctx.h)

    def reference(d_in, log_n, inverse=0):
        d = ctx.alloc(32 << log_n)
        ctx.ntt(d, d_in, log_n, inverse=bool(inverse))
        ctx.sync()
        return ctx.d2h(d, (1 << log_n, 4))

    def capture(d_out, d_in, log_n, inverse):
        graph, exe = vp(), vp()
        assert hip.hipStreamBeginCapture(st, 0) == 0  # global capture mode
        call(d_out, d_in, log_n, inverse)
        assert hip.hipStreamEndCapture(st, ctypes.byref(graph)) == 0
        assert hip.hipGraphInstantiate(ctypes.byref(exe), graph, None, None, ctypes.c_size_t(0)) == 0
        return graph, exe

    cases = []
    for log_n, inverse, eager_first in ((12, 0, True), (10, 1, False)):
        a = zkml_amd.random_fr(1 << log_n, rng)
        d_in, d_out = ctx.upload(a), ctx.alloc(a.nbytes)
        if eager_first:
            call(d_out, d_in, log_n, inverse)
            sync()
        print(f"[noalloc graph] capture log_n={log_n} inverse={inverse} eager_first={eager_first}", flush=True)
        graph, exe = capture(d_out, d_in, log_n, inverse)
        cases.append((log_n, inverse, d_in, d_out, graph, exe, reference(d_in, log_n, inverse)))
    others = [13, 9, 16, 3]
    try:
        for rep in range(3):
            for (log_n, inverse, d_in, d_out, graph, exe, want) in cases:
                # an eager call of another size between the replays
                o = others[(rep + log_n) % len(others)]
                b = zkml_amd.random_fr(1 << o, rng)
                db, ob = ctx.upload(b), ctx.alloc(b.nbytes)
                call(ob, db, o)
                sync()
                assert np.array_equal(ctx.d2h(ob, b.shape), reference(db, o))
                assert hip.hipMemsetAsync(vp(d_out.ptr), 0, ctypes.c_size_t(32 << log_n), st) == 0
                assert hip.hipGraphLaunch(exe, st) == 0
                sync()
                assert np.array_equal(ctx.d2h(d_out, want.shape), want), (rep, log_n, inverse)
        # the size first seen under capture, eagerly
        log_n, inverse, d_in, d_out, _, _, want = cases[1]
        call(d_out, d_in, log_n, inverse)
        sync()
        assert np.array_equal(ctx.d2h(d_out, want.shape), want)
    finally:
        for c in cases:
            hip.hipGraphExecDestroy(c[5])
            hip.hipGraphDestroy(c[4])
        hip.hipStreamDestroy(st)
