"""CPU unit tests of the host group arithmetic (cuda-zkml_amd/csrc/host_bn254.hpp).

The proof assembly (A = alpha1 + A_msm + r delta1, C = s A_msm + r B1_msm + L
+ H + ..., reference src/prover/groth16.cu:769-840), the MSM window
combination and the verifier run on these Jacobian formulas.  Expectations
come from affine Python big-integer arithmetic (tests/zkpy.py), so a wrong
branch of an addition fails here before any proof is compared:

  add (G1, G2)   affine + affine and Jacobian + affine (the z = 1 path),
                 affine + Jacobian, Jacobian + Jacobian (the general path);
                 P + P (doubling inside both paths), P + (-P) and infinity
  limbs29_scaled the device's nine 29-bit limbs as an integer below 2^261,
                 reduced mod q (the host's MSM window combination takes the
                 ratios X / ZZ, Y / ZZZ of such values, the radix cancelling)
  mul2 (G1)      a P + b Q with one doubling chain (Shamir's trick) for
                 64-bit blinding-size and full-size scalars, 0, 1, r - 1,
                 P = Q and Q = -P; against mul and the Python reference
"""
import ctypes
import os
import random
import subprocess

import pytest

from zkpy import G1, G2, P as Q, R, g1, g2, g1_to_words, g1_from_words, g2_to_words, g2_from_words, to_mont, limbs

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CSRC = os.path.join(ROOT, "cuda-zkml_amd", "csrc")
SRC = os.path.join(ROOT, "tests", "native", "host_bn254_check.cpp")
W8 = ctypes.c_uint64 * 8
W16 = ctypes.c_uint64 * 16
W4 = ctypes.c_uint64 * 4


@pytest.fixture(scope="module")
def hb(tmp_path_factory):
    so = tmp_path_factory.mktemp("hb") / "host_bn254_check.so"
    subprocess.run(["g++", "-O2", "-std=c++17", "-mbmi2", "-madx", "-shared", "-fPIC", "-I", CSRC, SRC, "-o", str(so)],
                   check=True)
    return ctypes.CDLL(str(so))


def zw(z, fq2=False):
    """Montgomery words of a Jacobian z (Fq or Fq2); None stays affine."""
    if z is None:
        return None
    if fq2:
        return W8(*(limbs(to_mont(z[0], Q)) + limbs(to_mont(z[1], Q))))
    return W4(*limbs(to_mont(z, Q)))


def fr_w(k):
    return W4(*limbs(to_mont(k % R, R)))


def g1_add(hb, p, zp, q, zq):
    out = W8()
    assert hb.hb_g1_add(W8(*g1_to_words(p)), zw(zp), W8(*g1_to_words(q)), zw(zq), out) == 0
    return g1_from_words(out)


def g2_add(hb, p, zp, q, zq):
    out = W16()
    assert hb.hb_g2_add(W16(*g2_to_words(p)), zw(zp, True), W16(*g2_to_words(q)), zw(zq, True), out) == 0
    return g2_from_words(out)


def test_g1_add_paths(hb):
    rng = random.Random(11)
    pts = [g1.pmul(G1, rng.randrange(1, R)) for _ in range(6)]
    zs = [None, rng.randrange(2, Q)]
    for p in pts:
        for q in pts[:3] + [p, g1.pneg(p), None]:
            want = g1.padd(p, q)
            for zp in zs:
                for zq in zs:
                    assert g1_add(hb, p, zp, q, zq) == want, (zp is None, zq is None)
    # infinity on the left, through both representations of the right
    for zq in zs:
        assert g1_add(hb, None, None, pts[0], zq) == pts[0]


def test_g2_add_paths(hb):
    rng = random.Random(12)
    pts = [g2.pmul(G2, rng.randrange(1, R)) for _ in range(3)]
    zs = [None, (rng.randrange(Q), rng.randrange(1, Q))]
    for p in pts:
        for q in pts[:2] + [p, g2.pneg(p), None]:
            want = g2.padd(p, q)
            for zp in zs:
                for zq in zs:
                    assert g2_add(hb, p, zp, q, zq) == want, (zp is None, zq is None)


def test_g1_mul_and_mul2(hb):
    rng = random.Random(13)
    p = g1.pmul(G1, rng.randrange(1, R))
    q = g1.pmul(G1, rng.randrange(1, R))
    scalars = [0, 1, 2, R - 1, (1 << 64) - 1] + [rng.randrange(1 << 64) for _ in range(3)] + \
              [rng.randrange(R) for _ in range(3)]
    for a in scalars:
        out = W8()
        assert hb.hb_g1_mul(W8(*g1_to_words(p)), fr_w(a), out) == 0
        assert g1_from_words(out) == g1.pmul(p, a)
    pairs = [(rng.choice(scalars), rng.choice(scalars)) for _ in range(12)] + [(0, 0), (1, R - 1), (R - 1, 1)]
    for a, b in pairs:
        for qq in (q, p, g1.pneg(p), None):
            out = W8()
            assert hb.hb_g1_mul2(W8(*g1_to_words(p)), fr_w(a), W8(*g1_to_words(qq)), fr_w(b), out) == 0
            assert g1_from_words(out) == g1.padd(g1.pmul(p, a), g1.pmul(qq, b) if qq else None), (a, b)


def test_g2_mul(hb):
    rng = random.Random(14)
    p = g2.pmul(G2, rng.randrange(1, R))
    for a in (0, 1, R - 1, rng.randrange(1 << 64), rng.randrange(R)):
        out = W16()
        assert hb.hb_g2_mul(W16(*g2_to_words(p)), fr_w(a), out) == 0
        assert g2_from_words(out) == g2.pmul(p, a)


def test_fq_from_limbs29_scaled(hb):
    rng = random.Random(15)
    U9 = ctypes.c_uint32 * 9
    vals = [0, 1, Q - 1, Q, Q + 1, 2 * Q - 1, 2 * Q, (1 << 256) - 1, 1 << 256, (1 << 261) - 1, 127 * Q, 128 * Q - 1]
    vals += [rng.randrange(2 * Q) for _ in range(200)] + [rng.randrange(1 << 261) for _ in range(200)]
    for v in vals:
        out = W4()
        assert hb.hb_fq_from_limbs29_scaled(U9(*[(v >> (29 * i)) & ((1 << 29) - 1) for i in range(9)]), out) == 0
        assert sum(int(w) << (64 * i) for i, w in enumerate(out)) == v % Q, hex(v)


def test_ratio_of_scaled_values_is_exact(hb):
    """x = X / ZZ from device-form limbs equals the affine x (the 2^5 of the
    radix cancels): checked through the G1 adder, whose affine output divides
    by z^2 = ZZ."""
    rng = random.Random(16)
    RP = 1 << 261
    U9 = ctypes.c_uint32 * 9
    for _ in range(20):
        p = g1.pmul(G1, rng.randrange(1, R))
        z = rng.randrange(1, Q)
        X, Y, ZZ = p[0] * z * z % Q, p[1] * z * z * z % Q, z * z % Q
        dev = [v * RP % Q for v in (X, Y, ZZ)]  # the device's internal form
        words = []
        for v in dev:
            out = W4()
            hb.hb_fq_from_limbs29_scaled(U9(*[(v >> (29 * i)) & ((1 << 29) - 1) for i in range(9)]), out)
            words.append(sum(int(w) << (64 * i) for i, w in enumerate(out)))
        inv_mont = pow(1 << 256, -1, Q)
        xs, ys, zzs = (w * inv_mont % Q for w in words)  # the values the host arithmetic sees
        assert xs * pow(zzs, -1, Q) % Q == p[0]
