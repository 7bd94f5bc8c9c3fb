"""GPU MSM (G1, G2) and fixed-base generation through the C ABI.

Pins: bit-exact canonical affine output against
  * the CPU oracle's restatement of the reference Pippenger (msm.cu:320-598)
    and its per-point double-and-add path, for n up to a few thousand;
  * the closed form sum_i s_i * (k_i G) = (sum_i k_i s_i mod r) G for the
    BASELINE config-3 inputs P_i = k_i G at 2^16 ... 2^20, for uniform and
    witness-like scalars;
  * edge cases the reference handles: n = 0, infinity points, zero scalars,
    hot buckets (many equal scalars), duplicate points, P and -P cancelling.
"""
import ctypes

import numpy as np
import pytest

import zkpy as Z
from bindings import oracle, ptr

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ctx():
    import zkml_amd
    c = zkml_amd.Context(0)
    yield c
    c.close()


def std_words(vals):
    return np.array([Z.limbs(v % Z.R) for v in vals], dtype=np.uint64).reshape(-1, 4)


def to_mont(std):
    std = np.ascontiguousarray(std, dtype=np.uint64)
    out = np.zeros_like(std)
    oracle().orc_fr_batch_from_std(ptr(std), std.shape[0], ptr(out))
    return out


def from_std_arr(arr):
    a = arr.astype(object)
    return [int(a[i, 0]) | (int(a[i, 1]) << 64) | (int(a[i, 2]) << 128) | (int(a[i, 3]) << 192)
            for i in range(arr.shape[0])]


def rand_std(n, rng):
    import zkml_amd
    return zkml_amd.random_fr(n, rng)  # uniform in [0, r) as words


def witness_like(n, rng):
    """70% in [0, 2^16), 10% r - small, 20% uniform."""
    s = rand_std(n, rng)
    u = rng.random(n)
    small = u < 0.7
    s[small] = 0
    s[small, 0] = rng.integers(0, 1 << 16, size=int(small.sum()), dtype=np.uint64)
    neg = (u >= 0.7) & (u < 0.8)
    vals = from_std_arr(s[neg])
    small_neg = rng.integers(1, 1 << 16, size=len(vals))
    s[neg] = std_words([Z.R - int(x) for x in small_neg])
    return s


def gpu_points(ctx, k_mont, g2=False):
    n = k_mont.shape[0]
    dk = ctx.upload(k_mont)
    dp = ctx.alloc(n * (128 if g2 else 64))
    (ctx.g2_generator_mul if g2 else ctx.g1_generator_mul)(dk, n, dp)
    return dp


def oracle_points(k_mont, g2=False):
    n = k_mont.shape[0]
    out = np.zeros((n, 16 if g2 else 8), dtype=np.uint64)
    (oracle().orc_g2_gen_batch if g2 else oracle().orc_g1_gen_batch)(ptr(np.ascontiguousarray(k_mont)), n,
                                                                    ptr(out), 8)
    return out


def closed_form_g1(ks, ss):
    return Z.g1.pmul(Z.G1, sum(k * s for k, s in zip(ks, ss)) % Z.R)


def closed_form_scalar(kstd, sstd):
    """sum k_i s_i mod r for (n, 4) standard-form words (oracle Fr arithmetic,
    itself pinned against Python big integers)."""
    out = np.zeros(4, dtype=np.uint64)
    oracle().orc_fr_dot_std(ptr(np.ascontiguousarray(kstd)), ptr(np.ascontiguousarray(sstd)), kstd.shape[0],
                            ptr(out))
    return Z.from_limbs(out)


# ------------------------------------------------------------------ fixed base
@pytest.mark.parametrize("n", [1, 5, 1000])
def test_g1_generator_mul_matches_oracle(ctx, n):
    rng = np.random.default_rng(n)
    ks = rand_std(n, rng)
    ks[0] = 0
    if n > 2:
        ks[1] = std_words([1])[0]
        ks[2] = std_words([Z.R - 1])[0]
    km = to_mont(ks)
    dp = gpu_points(ctx, km)
    got = ctx.d2h(dp, (n, 8))
    assert np.array_equal(got, oracle_points(km))


@pytest.mark.parametrize("n", [1, 7, 200])
def test_g2_generator_mul_matches_oracle(ctx, n):
    rng = np.random.default_rng(50 + n)
    km = to_mont(rand_std(n, rng))
    dp = gpu_points(ctx, km, g2=True)
    got = ctx.d2h(dp, (n, 16))
    assert np.array_equal(got, oracle_points(km, g2=True))


# ------------------------------------------------------------------ G1 MSM vs oracle
def run_msm(ctx, pts, sc_mont, g2=False):
    dp = ctx.upload(pts)
    ds = ctx.upload(sc_mont)
    return (ctx.msm_g2 if g2 else ctx.msm_g1)(dp, ds, pts.shape[0])


def oracle_msm(pts, sc_mont, g2=False, mode=0):
    out = np.zeros(16 if g2 else 8, dtype=np.uint64)
    f = oracle().orc_msm_g2 if g2 else oracle().orc_msm_g1
    f(ptr(np.ascontiguousarray(pts)), ptr(np.ascontiguousarray(sc_mont)), pts.shape[0], mode, 8, ptr(out))
    return out


@pytest.mark.parametrize("n", [1, 2, 3, 64, 257, 1000, 4096])
def test_msm_g1_small_vs_oracle(ctx, n):
    rng = np.random.default_rng(1000 + n)
    km = to_mont(rand_std(n, rng))
    pts = oracle_points(km)
    sc = to_mont(rand_std(n, rng))
    got = run_msm(ctx, pts, sc)
    assert np.array_equal(got, oracle_msm(pts, sc))


def test_msm_g1_n0_is_infinity(ctx):
    d = ctx.alloc(64)
    out = ctx.msm_g1(d, d, 0)
    assert not out.any()


def test_msm_g1_edge_cases(ctx):
    """Zero scalars, scalar 1 and r-1, infinity points, duplicate points,
    P and -P with the same scalar, many equal scalars (hot bucket)."""
    rng = np.random.default_rng(7)
    n = 3000
    ks = from_std_arr(rand_std(n, rng))
    ss = from_std_arr(rand_std(n, rng))
    ks[10] = ks[11] = ks[12]          # duplicate points
    ss[10] = ss[11] = ss[12]
    ks[20], ss[20] = ks[21], ss[21]   # same point, same scalar
    ks[30] = (-ks[31]) % Z.R          # P and -P ...
    ss[30] = ss[31]                   # ... cancel
    for i in range(100, 1600):        # hot bucket: 1500 scalars equal to 1
        ss[i] = 1
    for i in range(1600, 1700):
        ss[i] = 0
    ss[1700] = Z.R - 1
    ks[5] = 0                         # infinity point
    km = to_mont(std_words(ks))
    pts = oracle_points(km)
    assert not pts[5].any()
    sc = to_mont(std_words(ss))
    got = run_msm(ctx, pts, sc)
    assert Z.g1_from_words(got) == closed_form_g1(ks, ss)
    assert np.array_equal(got, oracle_msm(pts, sc))


@pytest.mark.parametrize("g2", [False, True])
def test_msm_equal_partials(ctx, g2):
    """One point repeated with one scalar: every chunk partial and every
    bucket's running sum meets an equal point, so the chunk combine and the
    bucket reduction take their doubling branch (P == 0 in the addition),
    in the plain and the split lane layouts.  Closed form: (n s mod r) k G."""
    n = 4096 if not g2 else 1024
    rng = np.random.default_rng(90 + g2)
    k = from_std_arr(rand_std(1, rng))[0]
    s = from_std_arr(rand_std(1, rng))[0]
    km = to_mont(std_words([k] * n))
    pts = oracle_points(km[:1], g2=g2)
    pts = np.repeat(pts, n, axis=0)
    sc = to_mont(std_words([s] * n))
    got = run_msm(ctx, pts, sc, g2=g2)
    assert np.array_equal(got, oracle_msm(pts, sc, g2=g2))
    if not g2:
        assert Z.g1_from_words(got) == Z.g1.pmul(Z.G1, k * s * n % Z.R)


@pytest.mark.parametrize("log_n", [14, 20])
def test_msm_g1_all_equal_scalars(ctx, log_n):
    """Every scalar equal: one bucket per window holds all n points (at 2^20
    every placement wave holds a single bucket, and the chunk-combine tree
    spans 2^14 chunks)."""
    rng = np.random.default_rng(8)
    n = 1 << log_n
    ks = from_std_arr(rand_std(n, rng))
    s = 0x1234567890ABCDEF1234567890ABCDEF
    km = to_mont(std_words(ks))
    dp = gpu_points(ctx, km)
    ds = ctx.upload(to_mont(std_words([s] * n)))
    got = ctx.msm_g1(dp, ds, n)
    assert Z.g1_from_words(got) == Z.g1.pmul(Z.G1, sum(ks) * s % Z.R)


@pytest.mark.parametrize("log_n,dist", [(16, "uniform"), (16, "witness"), (18, "uniform"), (18, "witness"),
                                        (20, "uniform"), (20, "witness"), (22, "uniform"), (22, "witness")])
def test_msm_g1_closed_form_large(ctx, log_n, dist):
    """BASELINE config 3 at every size it names: P_i = k_i G1 generated on
    the GPU (spot-checked against the oracle), MSM checked against
    (sum k_i s_i) G1, for uniform and witness-like scalars."""
    n = 1 << log_n
    rng = np.random.default_rng(log_n * 10 + (dist == "witness"))
    kstd = rand_std(n, rng)
    km = to_mont(kstd)
    dp = gpu_points(ctx, km)
    idx = np.array([0, 1, n // 2, n - 1])
    spot = ctx.d2h(dp, (n, 8))[idx]
    assert np.array_equal(spot, oracle_points(np.ascontiguousarray(km[idx])))
    sstd = witness_like(n, rng) if dist == "witness" else rand_std(n, rng)
    ds = ctx.upload(to_mont(sstd))
    print(f"[msm g1 2^{log_n} {dist}]", flush=True)
    got = ctx.msm_g1(dp, ds, n)
    assert Z.g1_from_words(got) == Z.g1.pmul(Z.G1, closed_form_scalar(kstd, sstd))
    # repeat on the same context: workspace reuse gives the same bytes
    again = ctx.msm_g1(dp, ds, n)
    assert np.array_equal(again, got)


def add_mod_r(a, b):
    """(a + b) mod r on (n, 4) uint64 words below r, vectorized.  Montgomery
    forms add like the values they stand for."""
    import zkml_amd
    s = np.empty_like(a)
    carry = np.zeros(a.shape[0], dtype=np.uint64)
    for k in range(4):
        t = a[:, k] + b[:, k]
        c1 = t < a[:, k]
        t2 = t + carry
        s[:, k] = t2
        carry = (c1 | (t2 < t)).astype(np.uint64)
    assert not carry.any()  # a + b < 2r < 2^256
    r = zkml_amd.R_WORDS
    ge = np.ones(a.shape[0], dtype=bool)  # s >= r, decided from the top word down
    decided = np.zeros(a.shape[0], dtype=bool)
    for k in range(3, -1, -1):
        gt, lt = s[:, k] > r[k], s[:, k] < r[k]
        ge = np.where(~decided & gt, True, np.where(~decided & lt, False, ge))
        decided |= gt | lt
    borrow = np.zeros(a.shape[0], dtype=np.uint64)
    out = s.copy()
    for k in range(4):
        t = s[:, k] - r[k]
        b1 = s[:, k] < r[k]
        t2 = t - borrow
        out[:, k] = t2
        borrow = (b1 | (t < borrow)).astype(np.uint64)
    return np.where(ge[:, None], out, s)


def test_add_mod_r_helper():
    rng = np.random.default_rng(4)
    a, b = rand_std(500, rng), rand_std(500, rng)
    a[0] = std_words([Z.R - 1])[0]
    b[0] = std_words([1])[0]
    got = from_std_arr(add_mod_r(a, b))
    assert got == [(x + y) % Z.R for x, y in zip(from_std_arr(a), from_std_arr(b))]


@pytest.mark.parametrize("g2", [False, True])
def test_msm_2_22_linearity(ctx, g2):
    """BASELINE config 3 / config 5 at 2^22 points, where a Python closed form
    is too slow: MSM(P, s) + MSM(P, t) = MSM(P, s + t) and
    MSM(P, s) + MSM(P, s) = MSM(P, 2s), uniform scalars."""
    n = 1 << 22
    rng = np.random.default_rng(22 + g2)
    dp = gpu_points(ctx, rand_std(n, rng), g2=g2)  # any words below r are valid Montgomery scalars
    s, t = rand_std(n, rng), rand_std(n, rng)
    run = ctx.msm_g2 if g2 else ctx.msm_g1
    G, from_words = (Z.g2, Z.g2_from_words) if g2 else (Z.g1, Z.g1_from_words)
    res = {}
    for name, sc in (("s", s), ("t", t), ("s+t", add_mod_r(s, t)), ("2s", add_mod_r(s, s))):
        ds = ctx.upload(sc)
        print(f"[msm 2^22 {'g2' if g2 else 'g1'}] scalars {name}", flush=True)
        res[name] = from_words(run(dp, ds, n))
        del ds
    assert res["s"] is not None and res["t"] is not None
    assert G.padd(res["s"], res["t"]) == res["s+t"]
    assert G.padd(res["s"], res["s"]) == res["2s"]


# ------------------------------------------------------------------ G2
@pytest.mark.parametrize("n", [1, 16, 129, 700])
def test_msm_g2_vs_oracle(ctx, n):
    rng = np.random.default_rng(3000 + n)
    km = to_mont(rand_std(n, rng))
    pts = oracle_points(km, g2=True)
    sc = to_mont(rand_std(n, rng))
    got = run_msm(ctx, pts, sc, g2=True)
    assert np.array_equal(got, oracle_msm(pts, sc, g2=True))


def test_msm_g2_all_equal_scalars(ctx):
    """G2, every scalar equal at 2^16: each window's one bucket spans more
    than 512 chunks, so a standalone G2 MSM takes the tree combine on lane
    pairs (the proofs take it on split lanes).  Closed form (s sum k_i) G2."""
    n = 1 << 16
    rng = np.random.default_rng(17)
    ks = from_std_arr(rand_std(n, rng))
    s = 0xFEDCBA9876543210FEDCBA9876543210
    dp = gpu_points(ctx, to_mont(std_words(ks)), g2=True)
    ds = ctx.upload(to_mont(std_words([s] * n)))
    got = ctx.msm_g2(dp, ds, n)
    assert Z.g2_from_words(got) == Z.g2.pmul(Z.G2, sum(ks) * s % Z.R)


@pytest.mark.parametrize("log_n,dist", [(14, "witness"), (16, "uniform"), (16, "witness"), (22, "uniform")])
def test_msm_g2_closed_form(ctx, log_n, dist):
    """G2 MSM over Q_i = k_i G2 against (sum k_i s_i) G2: the proof sizes of
    configs 4 (2^16) and 5 (2^22)."""
    n = 1 << log_n
    rng = np.random.default_rng(99 + log_n)
    kstd = rand_std(n, rng)
    dp = gpu_points(ctx, to_mont(kstd), g2=True)
    sstd = witness_like(n, rng) if dist == "witness" else rand_std(n, rng)
    ds = ctx.upload(to_mont(sstd))
    print(f"[msm g2 2^{log_n} {dist}]", flush=True)
    got = ctx.msm_g2(dp, ds, n)
    assert Z.g2_from_words(got) == Z.g2.pmul(Z.G2, closed_form_scalar(kstd, sstd))


# ------------------------------------------------------------------ converted once
@pytest.mark.parametrize("g2,log_n", [(False, 0), (False, 10), (False, 16), (False, 20), (True, 10), (True, 16)])
def test_msm_prepared_records(ctx, g2, log_n):
    """zk_msm_prepare_points + zk_msm_g*_prepared: over points P_i = k_i G
    the result equals zk_msm_g* over the same points and the closed form
    (sum k_i s_i) G, for two scalar vectors in a row over the same records,
    the second over a shorter prefix."""
    n = 1 << log_n
    rng = np.random.default_rng(700 + log_n + 50 * g2)
    kstd = rand_std(n, rng)
    dp = gpu_points(ctx, to_mont(kstd), g2=g2)
    drecs = ctx.msm_prepare(dp, n, g2=g2)
    G, from_words = (Z.g2, Z.g2_from_words) if g2 else (Z.g1, Z.g1_from_words)
    base = Z.G2 if g2 else Z.G1
    run, run_prep = (ctx.msm_g2, ctx.msm_g2_prepared) if g2 else (ctx.msm_g1, ctx.msm_g1_prepared)
    for m in (n, max(1, n // 3)):
        sstd = rand_std(m, rng)
        ds = ctx.upload(to_mont(sstd))
        print(f"[msm prepared {'g2' if g2 else 'g1'} 2^{log_n} m={m}]", flush=True)
        got = run_prep(drecs, ds, m)
        assert np.array_equal(got, run(dp, ds, m))
        assert from_words(got) == G.pmul(base, closed_form_scalar(kstd[:m], sstd))


def test_msm_prepare_rejects_overlap(ctx):
    """Records written over their own points are refused before any launch."""
    import zkml_amd
    n = 64
    dp = gpu_points(ctx, to_mont(rand_std(n, np.random.default_rng(1))))
    st = zkml_amd.lib().zk_msm_prepare_points(ctx.h, zkml_amd.vp(dp.ptr), n, 0, zkml_amd.vp(dp.ptr + 64), None)
    with pytest.raises(zkml_amd.ZkError, match="overlap"):
        ctx._check(st, "zk_msm_prepare_points")


# ------------------------------------------------------------------ host-pointer drop-in
def test_msm_g1_host_reference_layout(ctx):
    """zk_msm_g1_host takes the reference's 72-byte G1Affine structs and
    returns a 96-byte G1Jacobian (msm.cuh:67)."""
    import zkml_amd
    n = 300
    rng = np.random.default_rng(5)
    km = to_mont(rand_std(n, rng))
    pts = oracle_points(km)
    pts[3] = 0
    recs = np.zeros((n, 9), dtype=np.uint64)  # 72 bytes each
    recs[:, :8] = pts
    recs[3, 8] = 1  # bool infinity at byte 64
    sc = to_mont(rand_std(n, rng))
    out = np.zeros(12, dtype=np.uint64)
    L = zkml_amd.lib()
    st = L.zk_msm_g1_host(ctx.h, ptr(recs), ptr(sc), n, ptr(out))
    assert st == 0
    expect = oracle_msm(pts, sc)
    assert np.array_equal(out[:8], expect)
    assert Z.from_mont(Z.from_limbs(out[8:12]), Z.P) == 1


def test_msm_g2_host_reference_layout(ctx):
    """zk_msm_g2_host takes the reference's 136-byte G2Affine structs (x, y in
    Fp2, bool infinity at byte 128) and returns a 192-byte G2Jacobian
    (msm.cuh:68); a point flagged infinity is skipped whatever its words."""
    import zkml_amd
    n = 200
    rng = np.random.default_rng(6)
    km = to_mont(rand_std(n, rng))
    pts = oracle_points(km, g2=True)
    recs = np.zeros((n, 17), dtype=np.uint64)  # 136 bytes each
    recs[:, :16] = pts
    recs[7, 16] = 1  # bool infinity at byte 128; its coordinates stay a valid point
    sc = to_mont(rand_std(n, rng))
    out = np.zeros(24, dtype=np.uint64)
    L = zkml_amd.lib()
    assert L.zk_msm_g2_host(ctx.h, ptr(recs), ptr(sc), n, ptr(out)) == 0
    pts_inf = pts.copy()
    pts_inf[7] = 0
    expect = oracle_msm(pts_inf, sc, g2=True)
    assert np.array_equal(out[:16], expect)
    # z = 1 in Fq2 (Montgomery): c0 = 1, c1 = 0
    assert Z.from_mont(Z.from_limbs(out[16:20]), Z.P) == 1 and not out[20:24].any()
