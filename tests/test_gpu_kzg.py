"""GPU tests of the KZG commitment and opening (cuda-zkml_amd/csrc/kzg.hip;
zk_kzg_commit / zk_kzg_open, reference KZGCommitment, src/prover/groth16.cu:
393-438).

Pins (closed forms over an SRS built from a known tau, [tau^i]_1 = tau^i G1):
  commit  = f(tau) G1;
  open    = q(tau) G1 with q(tau) = (f(tau) - f(z)) / (tau - z), and the
            returned f(z) equals Horner's f(z) in Python;
  the pairing equation e(C - f(z) G1, G2) = e(proof, [tau]_2 - z G2) holds
  (host pairing), and fails for a wrong f(z);
  degrees 0 and 1 give the identity proof (the reference's rule); the sizes
  cross the blocked scan's chunk (32) and recursion (32^2, 32^3) edges.
The expected points come from the oracle's CPU fixed-base multiply.
"""
import random

import numpy as np
import pytest

import zkml_amd
from bindings import oracle, ptr
from zkpy import G1, G2, MONT, P as Q, R, g1, g2

pytestmark = pytest.mark.gpu


def mont_words(vals):
    return np.array([[(v * MONT % R) >> (64 * k) & ((1 << 64) - 1) for k in range(4)] for v in vals],
                    dtype=np.uint64).reshape(-1, 4)


def gen_points(scalars):
    """k G1 for each k (oracle, CPU), (n, 8) Montgomery affine words."""
    k = mont_words(scalars)
    out = np.zeros((len(scalars), 8), dtype=np.uint64)
    oracle().orc_g1_gen_batch(ptr(k), len(scalars), ptr(out), 8)
    return out


def horner(coeffs, x):
    acc = 0
    for c in reversed(coeffs):
        acc = (acc * x + c) % R
    return acc


@pytest.fixture(scope="module")
def ctx():
    return zkml_amd.Context(0)


SIZES = [0, 1, 2, 3, 31, 32, 33, 1024, 1025, 1057, 40000]


@pytest.fixture(scope="module")
def srs():
    rng = random.Random(77)
    tau = rng.randrange(2, R)
    n = max(SIZES)
    return tau, gen_points([pow(tau, i, R) for i in range(n)])


@pytest.mark.parametrize("degree", SIZES)
def test_commit_and_open_closed_forms(ctx, srs, degree):
    tau, pts = srs
    rng = random.Random(degree)
    f = [rng.randrange(R) for _ in range(degree)]
    z = rng.randrange(R)
    print(f"[kzg] degree {degree}", flush=True)
    d_srs = ctx.upload(pts[:max(degree, 1)])
    d_f = ctx.upload(mont_words(f) if degree else np.zeros((1, 4), dtype=np.uint64))
    com = ctx.kzg_commit(d_srs, d_f, degree)
    proof, fz = ctx.kzg_open(d_srs, d_f, degree, mont_words([z])[0])
    ft, fzv = horner(f, tau), horner(f, z)
    assert zkml_amd.words_int(fz) * pow(MONT, -1, R) % R == fzv
    expect_c = gen_points([ft])[0] if ft else np.zeros(8, dtype=np.uint64)
    assert np.array_equal(com, expect_c)
    if degree <= 1:
        assert not proof.any()
        return
    qt = (ft - fzv) * pow((tau - z) % R, -1, R) % R
    expect_p = gen_points([qt])[0] if qt else np.zeros(8, dtype=np.uint64)
    assert np.array_equal(proof, expect_p)


def _std_point_g1(pt):
    return np.array([v for c in pt for v in zkml_amd.std_words(c)], dtype=np.uint64)


def _std_point_g2(pt):
    return np.array([v for c2 in pt for c in c2 for v in zkml_amd.std_words(c)], dtype=np.uint64)


def test_pairing_equation(ctx, srs):
    tau, pts = srs
    rng = random.Random(5)
    degree = 200
    f = [rng.randrange(R) for _ in range(degree)]
    z = rng.randrange(R)
    d_srs = ctx.upload(pts[:degree])
    d_f = ctx.upload(mont_words(f))
    com = ctx.kzg_commit(d_srs, d_f, degree)
    proof, fz = ctx.kzg_open(d_srs, d_f, degree, mont_words([z])[0])
    fzv = zkml_amd.words_int(fz) * pow(MONT, -1, R) % R

    def affine(w):  # Montgomery Fq words -> Python ints
        x = zkml_amd.words_int(w[:4]) * pow(MONT, -1, Q) % Q
        y = zkml_amd.words_int(w[4:]) * pow(MONT, -1, Q) % Q
        return (x, y)

    C, Pi = affine(com), affine(proof)
    lhs_pt = g1.padd(C, g1.pneg(g1.pmul(G1, fzv)))
    rhs_q = g2.padd(g2.pmul(G2, tau), g2.pneg(g2.pmul(G2, z)))
    lhs = zkml_amd.pairing(_std_point_g1(lhs_pt), _std_point_g2(G2))
    rhs = zkml_amd.pairing(_std_point_g1(Pi), _std_point_g2(rhs_q))
    assert np.array_equal(lhs, rhs)
    wrong = g1.padd(C, g1.pneg(g1.pmul(G1, (fzv + 1) % R)))
    assert not np.array_equal(zkml_amd.pairing(_std_point_g1(wrong), _std_point_g2(G2)), rhs)
