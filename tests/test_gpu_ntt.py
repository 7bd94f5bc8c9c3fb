"""GPU NTT / iNTT / coset NTT through the C ABI, bit-exact against the CPU
oracle's radix-2 restatement of ntt_gpu (src/ntt/ntt.cu:354-465) and the
coset steps of compute_h (src/prover/groth16.cu:350-383)."""
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


def oracle_ntt(a, log_n, inverse, threads=8):
    b = np.ascontiguousarray(a.copy())
    oracle().orc_ntt(ptr(b), log_n, int(inverse), threads)
    return b


def oracle_coset(a, log_n, g, inverse, threads=16):
    """forward: NTT(a_i g^i); inverse: iNTT(a)_i g^-i, on Montgomery words (the
    oracle's restatement of compute_h's coset loops, groth16.cu:352-383)."""
    lib = oracle()
    b = np.ascontiguousarray(a.copy())
    if inverse:
        lib.orc_ntt(ptr(b), log_n, 1, threads)
        lib.orc_coset_scale(ptr(b), log_n, g, 1)
    else:
        lib.orc_coset_scale(ptr(b), log_n, g, 0)
        lib.orc_ntt(ptr(b), log_n, 0, threads)
    return b


def rand_words(n, seed):
    import zkml_amd
    w = zkml_amd.random_fr(n, np.random.default_rng(seed))
    if n >= 4:
        w[0] = 0
        w[1] = np.array(Z.limbs(Z.R - 1), dtype=np.uint64)
        w[2] = np.array(Z.fr_words(1), dtype=np.uint64)
    return w


def run_gpu(ctx, a, log_n, inverse, batch=1, coset=0, inplace=False):
    d_in = ctx.upload(a)
    d_out = d_in if inplace else ctx.alloc(a.nbytes)
    if coset:
        ctx.coset_ntt(d_out, d_in, log_n, coset, inverse, batch)
    else:
        ctx.ntt(d_out, d_in, log_n, inverse, batch)
    return ctx.d2h(d_out, a.shape)


def test_ntt_kat_1234(ctx):
    """tests/test_ntt.cu:65-93: NTT([1,2,3,4])[0] = 10."""
    a = np.array([Z.fr_words(v) for v in (1, 2, 3, 4)], dtype=np.uint64)
    out = run_gpu(ctx, a, 2, False)
    vals = [Z.fr_from_words(r) for r in out]
    assert vals[0] == 10
    assert vals == Z.dft([1, 2, 3, 4], Z.omega(2))
    back = run_gpu(ctx, out, 2, True)
    assert np.array_equal(back, a)


@pytest.mark.parametrize("log_n", list(range(1, 19)) + [20])
def test_ntt_forward_inverse_vs_oracle(ctx, log_n):
    n = 1 << log_n
    a = rand_words(n, log_n)
    for inverse in (False, True):
        got = run_gpu(ctx, a, log_n, inverse)
        assert np.array_equal(got, oracle_ntt(a, log_n, inverse)), (log_n, inverse)


def test_ntt_2_22_vs_oracle_and_round_trip(ctx):
    log_n = 22
    a = rand_words(1 << log_n, 22)
    fwd = run_gpu(ctx, a, log_n, False)
    assert np.array_equal(fwd, oracle_ntt(a, log_n, False))
    back = run_gpu(ctx, fwd, log_n, True)
    assert np.array_equal(back, a)


@pytest.mark.parametrize("log_n,g", [(3, 5), (10, 7), (13, 5), (16, 7), (20, 7), (22, 7)])
def test_coset_ntt_vs_oracle(ctx, log_n, g):
    a = rand_words(1 << log_n, 100 + log_n)
    for inverse in (False, True):
        got = run_gpu(ctx, a, log_n, inverse, coset=g)
        assert np.array_equal(got, oracle_coset(a, log_n, g, inverse)), (log_n, g, inverse)


def test_coset_ntt_horner_spot_check(ctx):
    """Coset NTT output j equals the polynomial evaluated at g w^j (Horner)."""
    log_n, g = 8, 7
    a = rand_words(1 << log_n, 5)
    out = run_gpu(ctx, a, log_n, False, coset=g)
    coeffs = [Z.fr_from_words(r) for r in a]
    w = Z.omega(log_n)
    for j in (0, 1, 77, 255):
        assert Z.fr_from_words(out[j]) == Z.poly_eval(coeffs, g * pow(w, j, Z.R) % Z.R)


@pytest.mark.parametrize("log_n", [4, 11, 17])
def test_ntt_batch_and_inplace(ctx, log_n):
    n = 1 << log_n
    a = rand_words(3 * n, 7 + log_n)
    got = run_gpu(ctx, a, log_n, False, batch=3)
    for b in range(3):
        assert np.array_equal(got[b * n:(b + 1) * n], oracle_ntt(a[b * n:(b + 1) * n], log_n, False))
    inpl = run_gpu(ctx, a[:n].copy(), log_n, True, inplace=True)
    assert np.array_equal(inpl, oracle_ntt(a[:n], log_n, True))


def test_ntt_rejects_bad_sizes(ctx):
    import zkml_amd
    a = rand_words(8, 1)
    d = ctx.upload(a)
    with pytest.raises(zkml_amd.ZkError):
        ctx.ntt(d, d, 25, False)
    with pytest.raises(zkml_amd.ZkError):
        ctx.ntt(d, d, 0, False)
