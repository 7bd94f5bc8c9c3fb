"""CPU unit tests of the kernels' own field and curve arithmetic.

cuda-zkml_amd/csrc/field.hpp and curve.hpp are header-only and compile for the
host as well; tests/native/field_host_check.cpp exposes them through a small C
shim.  Expectations come from Python big integers (tests/zkpy.py), so a wrong
limb, carry or range assumption fails here before any kernel runs:

  fmul / fsqr / fmul_sum  a*b*2^-261 (sums of 2 and 4 products) mod q, result < 2q, limbs < 2^29,
                          at the edges of the documented input ranges
  fsub_lazy / fneg_lazy   exact a - b + 2q and 2q - a (and the 4q forms)
  fsub3, fis_zero(4)      a - b - 2c into [0, 2q); zero tests over [0, 2q) / [0, 4q)
  fadd / fsub / fmul_sub  congruence and the [0, 2q) output range
  fadd_wide / fcsub       exact a + b below 4q; a - 2q when a >= 2q
  NTT lazy butterfly      over Fr: X, Y in [0, 4r) give X' +- Y*w in [0, 4r)
  XYZZ madd/add/dbl/mdbl  G1 and G2 against affine formulas, with coordinates
                          given in non-canonical [q, 2q) representatives and
                          random Z, plus the doubling / inverse / infinity cases
"""
import ctypes
import os
import random
import subprocess

import pytest

from zkpy import G1, G2, P as Q, R as ORDER, g1, g2, f2_inv, f2_mul

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CSRC = os.path.join(ROOT, "cuda-zkml_amd", "csrc")
SRC = os.path.join(ROOT, "tests", "native", "field_host_check.cpp")
RP = 1 << 261          # internal Montgomery radix
RP_INV = pow(RP, -1, Q)
U32x9 = ctypes.c_uint32 * 9


@pytest.fixture(scope="module")
def fh(tmp_path_factory):
    so = tmp_path_factory.mktemp("fh") / "field_host_check.so"
    subprocess.run(["g++", "-O2", "-std=c++17", "-shared", "-fPIC", "-I", CSRC, SRC, "-o", str(so)], check=True)
    lib = ctypes.CDLL(str(so))
    lib.fh_op.restype = ctypes.c_int
    lib.fh_xyzz.restype = ctypes.c_int
    lib.fh_fr_op.restype = ctypes.c_int
    return lib


def to_l(x):
    assert 0 <= x < 1 << 261
    return [(x >> (29 * i)) & ((1 << 29) - 1) for i in range(9)]


def from_l(ws):
    return sum(int(w) << (29 * i) for i, w in enumerate(ws))


def op(fh, code, a, b=0, c=0, d=0):
    out = U32x9()
    assert fh.fh_op(code, U32x9(*to_l(a)), U32x9(*to_l(b)), U32x9(*to_l(c)), U32x9(*to_l(d)), out) == 0
    ws = list(out)
    assert all(w < 1 << 29 for w in ws), "limb not normalized"
    return from_l(ws)


def samples(rng, hi, k=40):
    """Values in [0, hi): the edges plus random ones."""
    return [0, 1, hi - 1, hi - 2, Q - 1, Q, Q + 1][: 7 if hi > Q + 1 else 4] + [rng.randrange(hi) for _ in range(k)]


def test_fmul_fsqr_ranges(fh):
    rng = random.Random(1)
    for a in samples(rng, 8 * Q):
        for b in samples(rng, 8 * Q, 6):
            r = op(fh, 0, a, b)
            assert r < 2 * Q and r % Q == a * b * RP_INV % Q
    for a in samples(rng, 8 * Q):
        r = op(fh, 1, a)
        assert r < 2 * Q and r % Q == a * a * RP_INV % Q


def test_fmul2_ranges(fh):
    rng = random.Random(2)
    vals = samples(rng, 4 * Q, 12)
    for a in vals:
        for b in vals[:6]:
            c, e = rng.choice(vals), rng.choice(vals)
            r = op(fh, 2, a, b, c, e)
            assert r < 2 * Q and r % Q == (a * b + c * e) * RP_INV % Q
    m = 4 * Q - 1  # every operand at its maximum
    r = op(fh, 2, m, m, m, m)
    assert r < 2 * Q and r % Q == 2 * m * m * RP_INV % Q
    # four products (a, c < 2q; b, d < 4q), including all at their maxima
    for _ in range(200):
        a, c = rng.randrange(2 * Q), rng.randrange(2 * Q)
        b, d = rng.randrange(4 * Q), rng.randrange(4 * Q)
        r = op(fh, 8, a, b, c, d)
        assert r < 2 * Q and r % Q == (a * b + c * d + a * d + c * b) * RP_INV % Q
    a, b = 2 * Q - 1, 4 * Q - 1
    r = op(fh, 8, a, b, a, b)
    assert r < 2 * Q and r % Q == 4 * a * b * RP_INV % Q


def test_lazy_sub_neg_exact(fh):
    rng = random.Random(3)
    for a in samples(rng, 2 * Q):
        for b in samples(rng, 2 * Q, 4):
            assert op(fh, 3, a, b) == a + 2 * Q - b
    for a in samples(rng, 2 * Q) + [2 * Q]:
        assert op(fh, 4, a) == 2 * Q - a


def test_fused_sub_lazy4_zero_tests(fh):
    rng = random.Random(7)
    for a in samples(rng, 2 * Q, 20):
        for b in samples(rng, 2 * Q, 3):
            c = rng.randrange(2 * Q)
            r = op(fh, 9, a, b, c)  # a - b - 2c into [0, 2q)
            assert r < 2 * Q and r % Q == (a - b - 2 * c) % Q
    for a, b, c in ((0, 2 * Q - 1, 2 * Q - 1), (2 * Q - 1, 0, 0), (Q, Q, Q)):
        r = op(fh, 9, a, b, c)
        assert r < 2 * Q and r % Q == (a - b - 2 * c) % Q
    for a in samples(rng, 4 * Q, 10):
        for b in samples(rng, 4 * Q, 3) + [4 * Q]:
            assert op(fh, 10, a, b) == a + 4 * Q - b
    for a in samples(rng, 4 * Q, 10) + [4 * Q]:
        assert op(fh, 11, a) == 4 * Q - a
    # zero tests: exactly the multiples of q inside the documented ranges
    for a in [0, Q, 1, Q - 1, Q + 1, 2 * Q - 1] + [rng.randrange(2 * Q) for _ in range(50)]:
        assert op(fh, 12, a) == (1 if a % Q == 0 else 0)
    for a in [0, Q, 2 * Q, 3 * Q, 1, 2 * Q + 1, 3 * Q - 1, 4 * Q - 1] + [rng.randrange(4 * Q) for _ in range(50)]:
        assert op(fh, 13, a) == (1 if a % Q == 0 else 0)


def test_wide_add_and_conditional_subtract(fh):
    rng = random.Random(11)
    for a in samples(rng, 2 * Q):
        for b in samples(rng, 2 * Q, 4):
            assert op(fh, 14, a, b) == a + b  # exact, below 4q
    for a in samples(rng, 4 * Q, 60) + [2 * Q, 2 * Q - 1, 2 * Q + 1, 4 * Q - 1]:
        assert op(fh, 15, a) == (a - 2 * Q if a >= 2 * Q else a)


def fr_op(fh, code, a, b=0):
    out = U32x9()
    assert fh.fh_fr_op(code, U32x9(*to_l(a)), U32x9(*to_l(b)), out) == 0
    ws = list(out)
    assert all(w < 1 << 29 for w in ws), "limb not normalized"
    return from_l(ws)


def test_ntt_lazy_butterfly_bounds(fh):
    """The NTT's lazy radix-2 step: inputs X, Y in [0, 4r), a canonical
    twiddle w; T = Y*w (Montgomery), X' = X mod 2r, outputs X' + T and
    X' - T + 2r must stay in [0, 4r) and be congruent to X +- Y*w/R'."""
    rng = random.Random(12)
    r = ORDER
    rinv = pow(RP, -1, r)
    edge = [0, 1, r - 1, r, 2 * r - 1, 2 * r, 3 * r, 4 * r - 1]
    xs = edge + [rng.randrange(4 * r) for _ in range(40)]
    ws = [0, 1, r - 1] + [rng.randrange(r) for _ in range(8)]
    for x in xs:
        for y in xs[:12]:
            w = rng.choice(ws)
            t = fr_op(fh, 0, y, w)
            assert t < 2 * r and t % r == y * w * rinv % r
            xc = fr_op(fh, 2, x)
            assert xc == (x - 2 * r if x >= 2 * r else x)
            s, d = fr_op(fh, 1, xc, t), fr_op(fh, 3, xc, t)
            assert s == xc + t and s < 4 * r
            assert d == xc + 2 * r - t and 0 < d < 4 * r
            assert (s - x - y * w * rinv) % r == 0 and (d - x + y * w * rinv) % r == 0


def test_ntt_offset_subtract_and_reduce(fh):
    """The NTT pass's lazy helpers: fsub_off<K>(a, b) = a - b + K r exactly for
    b < K r (K = 2, 4, 8; a up to 26r), and freduce gives the canonical value
    of any normalized input below 2^261 (its top-limb quotient estimate may
    fall 2 short: the two conditional subtractions must absorb that)."""
    rng = random.Random(21)
    r = ORDER
    for code, K in ((7, 2), (4, 4), (5, 8)):
        for _ in range(60):
            a = rng.randrange(26 * r)
            b = rng.choice([0, K * r - 1, rng.randrange(K * r)])
            assert fr_op(fh, code, a, b) == a - b + K * r
    edge = [0, 1, r - 1, r, r + 1, 2 * r - 1, 2 * r, 3 * r - 1, 26 * r, (1 << 261) - 1, (1 << 260) + 12345]
    # values just below and above multiples of r, where the estimate is tight
    edge += [k * r + d for k in (1, 5, 17, 100, 168) for d in (-1, 0, 1) if 0 <= k * r + d < 1 << 261]
    for x in edge + [rng.randrange(1 << 261) for _ in range(200)]:
        assert fr_op(fh, 6, x) == x % r, hex(x)


def test_ntt_grow_butterfly_chain(fh):
    """The pass kernel's arithmetic on one element path: a first radix-8 step
    with twiddle-free butterflies (offsets 2r, 4r, 8r) and five twiddled
    stages (u + w v, u - w v + 2r, no reduction) keep normalized limbs and
    values below 26r, congruent to the exact result; freduce finishes."""
    rng = random.Random(22)
    r = ORDER
    rinv = pow(RP, -1, r)
    for _ in range(30):
        u, v = rng.randrange(2 * r), rng.randrange(2 * r)
        exact_u = u
        for code, K in ((7, 2), (4, 4), (5, 8)):   # sub-stages 0..2, twiddle 1 (worst-case growth path)
            u, v = fr_op(fh, 1, u, v), fr_op(fh, code, u, v)
            assert u < 2 * K * r and v < 2 * K * r
        exact_u, exact_v = u % r, v % r
        for _ in range(5):
            w = rng.randrange(r)
            t = fr_op(fh, 0, v, w)
            assert t < 2 * r
            u, v = fr_op(fh, 1, u, t), fr_op(fh, 7, u, t)
            tv = exact_v * w * rinv % r
            exact_u, exact_v = (exact_u + tv) % r, (exact_u - tv) % r
        assert u < 26 * r and v < 26 * r
        assert fr_op(fh, 6, u) == exact_u and fr_op(fh, 6, v) == exact_v


def test_add_sub_mulsub(fh):
    rng = random.Random(4)
    for a in samples(rng, 2 * Q):
        for b in samples(rng, 2 * Q, 4):
            s = op(fh, 5, a, b)
            d = op(fh, 6, a, b)
            assert s < 2 * Q and s % Q == (a + b) % Q
            assert d < 2 * Q and d % Q == (a - b) % Q
    for _ in range(200):
        c, d = (rng.randrange(2 * Q) for _ in range(2))
        a, b = rng.randrange(4 * Q), rng.randrange(4 * Q)  # the lazy factors
        r = op(fh, 7, a, b, c, d)
        assert r < 2 * Q and r % Q == (a * b - c * d) * RP_INV % Q


# ----------------------------------------------------------------- XYZZ
def rep(rng, v):
    """Internal representative of v (standard form): v*2^261 mod q, with q
    added at random so that [q, 2q) inputs are exercised."""
    x = v * RP % Q
    return x + Q if rng.random() < 0.5 else x


def enc1(rng, pt, z):
    if pt is None:
        return [0] * 36
    x, y = pt
    zz, zzz = z * z % Q, z * z * z % Q
    out = []
    for v in (x * zz % Q, y * zzz % Q, zz, zzz):
        out += to_l(rep(rng, v))
    return out


def dec1(ws):
    X, Y, ZZ, ZZZ = (from_l(ws[9 * i: 9 * i + 9]) for i in range(4))
    for v in (X, Y, ZZ, ZZZ):
        assert v < 2 * Q
    if ZZ % Q == 0:
        return None
    return (X * pow(ZZ, Q - 2, Q) % Q, Y * pow(ZZZ, Q - 2, Q) % Q)


def enc2(rng, pt, z):
    if pt is None:
        return [0] * 72
    x, y = pt
    zz = f2_mul(z, z)
    zzz = f2_mul(zz, z)
    out = []
    for v in (f2_mul(x, zz), f2_mul(y, zzz), zz, zzz):
        out += to_l(rep(rng, v[0])) + to_l(rep(rng, v[1]))
    return out


def dec2(ws):
    parts = [(from_l(ws[18 * i: 18 * i + 9]), from_l(ws[18 * i + 9: 18 * i + 18])) for i in range(4)]
    for v in parts:
        assert v[0] < 2 * Q and v[1] < 2 * Q
    X, Y, ZZ, ZZZ = ((a % Q, b % Q) for a, b in parts)
    if ZZ == (0, 0):
        return None
    return (f2_mul(X, f2_inv(ZZ)), f2_mul(Y, f2_inv(ZZZ)))


def xyzz_call(fh, g2flag, code, p, q):
    nw = 72 if g2flag else 36
    arr = ctypes.c_uint32 * nw
    out = arr()
    assert fh.fh_xyzz(g2flag, code, arr(*p), arr(*(q + [0] * (nw - len(q)))), out) == 0
    return list(out)


@pytest.mark.parametrize("g2flag", [0, 1])
def test_xyzz_formulas(fh, g2flag):
    rng = random.Random(5 + g2flag)
    grp, gen = (g2, G2) if g2flag else (g1, G1)
    enc, dec = (enc2, dec2) if g2flag else (enc1, dec1)

    def rz():
        return (rng.randrange(1, Q), rng.randrange(Q)) if g2flag else rng.randrange(1, Q)

    def affine_words(pt):  # Z = 1, the record form madd/mdbl read
        return enc(rng, pt, (1, 0) if g2flag else 1)[: 36 if g2flag else 18]

    pts = [grp.pmul(gen, rng.randrange(1, ORDER)) for _ in range(6)]
    for i in range(len(pts) - 1):
        a, b = pts[i], pts[i + 1]
        # madd, add, dbl, mdbl on generic inputs
        assert dec(xyzz_call(fh, g2flag, 0, enc(rng, a, rz()), affine_words(b))) == grp.padd(a, b)
        assert dec(xyzz_call(fh, g2flag, 1, enc(rng, a, rz()), enc(rng, b, rz()))) == grp.padd(a, b)
        assert dec(xyzz_call(fh, g2flag, 2, enc(rng, a, rz()), [])) == grp.padd(a, a)
        assert dec(xyzz_call(fh, g2flag, 3, [0] * (72 if g2flag else 36), affine_words(a))) == grp.padd(a, a)
    a = pts[0]
    # special cases: P + P (doubling branch), P + (-P), infinity operands
    assert dec(xyzz_call(fh, g2flag, 0, enc(rng, a, rz()), affine_words(a))) == grp.padd(a, a)
    assert dec(xyzz_call(fh, g2flag, 1, enc(rng, a, rz()), enc(rng, a, rz()))) == grp.padd(a, a)
    assert dec(xyzz_call(fh, g2flag, 0, enc(rng, a, rz()), affine_words(grp.pneg(a)))) is None
    assert dec(xyzz_call(fh, g2flag, 1, enc(rng, a, rz()), enc(rng, grp.pneg(a), rz()))) is None
    assert dec(xyzz_call(fh, g2flag, 0, enc(rng, None, rz()), affine_words(a))) == a
    assert dec(xyzz_call(fh, g2flag, 1, enc(rng, None, rz()), enc(rng, a, rz()))) == a
    assert dec(xyzz_call(fh, g2flag, 1, enc(rng, a, rz()), enc(rng, None, rz()))) == a
