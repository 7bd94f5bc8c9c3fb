"""The CPU oracle pinned against closed forms, the reference's own KATs and
golden artefacts, and the reference's own code compiled in oracle/_ref/.

Pins per oracle function (the function it checks in brackets):
  field mul/add/sub/inv      Python big-int closed forms + reference KATs
                             (tests/test_field.cu:46-130) + reference code
  omega / omega_inv          5^((r-1)/2^28) powers, w^n = 1, w*w^-1 = 1
  ntt_radix2                 naive DFT (oracle and Python), NTT([1,2,3,4]),
                             round trip (tests/test_ntt.cu:19-161)
  G1/G2 scalar mul, add      Python affine formulas + reference code,
                             r*G = O
  msm (Pippenger, naive)     closed form (sum k_i s_i)*G, reference small-n
                             path, n=0, infinity points, zero scalars
  compute_h                  A(t)B(t)-C(t) = h(t)(t^n-1) at random t, h[n-1]=0
  setup + prove              proof verifies under the reference verifier,
                             wrong public input rejected
  ZKMLPK3 / VK / proof I/O   T4 golden files: reference verifier accepts the
                             T4 proofs; PK parse equals an independent parser
The oracle/_ref comparisons run the reference's host code compiled in place
with the reference's own CUDA-runtime test shim (tests/host/shim).  They are
cross-checks and pin nothing by themselves: every oracle function also has a
pin that needs no reference code (closed forms, KATs, T4 golden files).
"""
import os
import random
import struct

import numpy as np
import pytest

import zkpy as Z
from bindings import OracleR1CS, oracle, ptr, ref, ref_available, words
from groth16_closed_form import parse_zkmlpk3
from r1cs_gen import mul_circuit, random_r1cs

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
needs_ref = pytest.mark.skipif(not ref_available(), reason="oracle/_ref not built (reference absent)")


def w4(x):
    return np.array(Z.limbs(x), dtype=np.uint64)


def call2(fn, a, b):
    o = np.zeros(4, dtype=np.uint64)
    fn(ptr(a), ptr(b), ptr(o))
    return Z.from_limbs(o)


# ------------------------------------------------------------------ fields
@pytest.mark.parametrize("mod,name", [(Z.P, "fq"), (Z.R, "fr")])
def test_field_closed_form(mod, name):
    lib = oracle()
    mul, add, sub, inv = (getattr(lib, f"orc_{name}_{op}") for op in ("mul", "add", "sub", "inv"))
    rng = random.Random(7)
    vals = [0, 1, 2, mod - 1, mod - 2, (mod + 1) // 2] + [rng.randrange(mod) for _ in range(200)]
    for _ in range(300):
        a, b = rng.choice(vals), rng.choice(vals)
        am, bm = w4(Z.to_mont(a, mod)), w4(Z.to_mont(b, mod))
        assert Z.from_mont(call2(mul, am, bm), mod) == a * b % mod
        assert Z.from_mont(call2(add, am, bm), mod) == (a + b) % mod
        assert Z.from_mont(call2(sub, am, bm), mod) == (a - b) % mod
        # outputs canonical
        assert call2(mul, am, bm) < mod
        if a:
            o = np.zeros(4, dtype=np.uint64)
            inv(ptr(am), ptr(o))
            assert Z.from_mont(Z.from_limbs(o), mod) == pow(a, -1, mod)


def test_field_reference_kats():
    """KATs of tests/test_field.cu:46-130 (Fp) and 224-252 (Fr)."""
    lib = oracle()

    def fq(v):
        return w4(Z.to_mont(v, Z.P))

    def std(m):
        o = np.zeros(4, dtype=np.uint64)
        lib.orc_fq_to_std(ptr(m), ptr(o))
        return Z.from_limbs(o)

    assert std(fq(42)) == 42
    assert std(np.array(Z.limbs(call2(lib.orc_fq_add, fq(1), fq(1))), dtype=np.uint64)) == 2
    assert std(np.array(Z.limbs(call2(lib.orc_fq_sub, fq(0), fq(1))), dtype=np.uint64)) == Z.P - 1
    assert std(np.array(Z.limbs(call2(lib.orc_fq_mul, fq(3), fq(7))), dtype=np.uint64)) == 21
    assert std(np.array(Z.limbs(call2(lib.orc_fq_mul, fq(42), fq(58))), dtype=np.uint64)) == 2436
    # Montgomery constants quoted by the reference (montgomery.cuh:44-60, fp.cuh:338-349)
    assert Z.to_mont(1, Z.P) == 0x0E0A77C19A07DF2F666EA36F7879462C0A78EB28F5C70B3DD35D438DC58F0D9D
    assert pow(2, 512, Z.P) == 0x06D89F71CAB8351F47AB1EFF0A417FF6B5E71911D44501FBF32CFC5B538AFA89
    assert Z.to_mont(1, Z.R) == 0x0E0A77C19A07DF2F666EA36F7879462E36FC76959F60CD29AC96341C4FFFFFFB
    assert pow(2, 512, Z.R) == 0x0216D0B17F4E44A58C49833D53BB808553FE3AB1E35C59E31BB8E645AE216DA7
    assert (-pow(Z.P, -1, 1 << 64)) % (1 << 64) == 0x87D20782E4866389
    assert (-pow(Z.R, -1, 1 << 64)) % (1 << 64) == 0xC2E1F593EFFFFFFF


@needs_ref
@pytest.mark.parametrize("mod,name", [(Z.P, "fq"), (Z.R, "fr")])
def test_field_matches_reference_code(mod, name):
    o, r = oracle(), ref()
    rng = random.Random(11)
    for _ in range(200):
        a, b = w4(rng.randrange(mod)), w4(rng.randrange(mod))
        assert call2(getattr(o, f"orc_{name}_mul"), a, b) == call2(getattr(r, f"ref_{name}_mul"), a, b)


# ------------------------------------------------------------------ NTT
def test_omega_constants():
    lib = oracle()
    for log_n in (1, 2, 10, 16, 20, 22, 28):
        o = np.zeros(4, dtype=np.uint64)
        lib.orc_omega(log_n, 0, ptr(o))
        w = Z.from_mont(Z.from_limbs(o), Z.R)
        assert w == Z.omega(log_n)
        assert pow(w, 1 << log_n, Z.R) == 1 and pow(w, 1 << (log_n - 1), Z.R) != 1
        lib.orc_omega(log_n, 1, ptr(o))
        assert Z.from_mont(Z.from_limbs(o), Z.R) * w % Z.R == 1
    assert Z.OMEGA28 == 0x2A3C09F0A58A7E8500E0A7EB8EF62ABC402D111E41112ED49BD61B6E725B19F0


def fr_array(vals):
    return np.array([Z.fr_words(v) for v in vals], dtype=np.uint64).reshape(-1, 4)


def fr_list(arr):
    return [Z.fr_from_words(r) for r in arr]


def test_ntt_kat_1234():
    """tests/test_ntt.cu:65-93: NTT([1,2,3,4])[0] = 10, plus the full vector."""
    lib = oracle()
    a = fr_array([1, 2, 3, 4])
    lib.orc_ntt(ptr(a), 2, 0, 1)
    out = fr_list(a)
    assert out[0] == 10
    assert out == Z.dft([1, 2, 3, 4], Z.omega(2))
    lib.orc_ntt(ptr(a), 2, 1, 1)
    assert fr_list(a) == [1, 2, 3, 4]


@pytest.mark.parametrize("log_n", [1, 3, 5, 8, 10])
def test_ntt_vs_naive_dft(log_n):
    lib = oracle()
    rng = random.Random(log_n)
    vals = [rng.randrange(Z.R) for _ in range(1 << log_n)]
    ninv = pow(1 << log_n, -1, Z.R)
    for inv in (0, 1):
        a = fr_array(vals)
        b = np.zeros_like(a)
        lib.orc_dft_naive(ptr(a), ptr(b), log_n, inv)
        lib.orc_ntt(ptr(a), log_n, inv, 2)
        naive = fr_list(b)
        if inv:  # the naive DFT with w^-1 is unscaled; the iNTT scales by 1/n
            naive = [v * ninv % Z.R for v in naive]
        assert fr_list(a) == naive
        if log_n <= 5:
            w = Z.omega(log_n)
            if inv:
                w = pow(w, -1, Z.R)
            expect = Z.dft(vals, w)
            if inv:
                ninv = pow(1 << log_n, -1, Z.R)
                expect = [e * ninv % Z.R for e in expect]
                assert fr_list(a) == expect
            else:
                assert fr_list(a) == expect


def test_ntt_round_trip_4096():
    lib = oracle()
    rng = np.random.default_rng(3)
    vals = [int(x) for x in rng.integers(0, 2**62, size=4096)]
    a = fr_array(vals)
    a0 = a.copy()
    lib.orc_ntt(ptr(a), 12, 0, 4)
    assert not np.array_equal(a, a0)
    lib.orc_ntt(ptr(a), 12, 1, 4)
    assert np.array_equal(a, a0)


# ------------------------------------------------------------------ curves
def test_generators():
    lib = oracle()
    g1 = np.zeros(8, dtype=np.uint64)
    g2 = np.zeros(16, dtype=np.uint64)
    lib.orc_g1_generator(ptr(g1))
    lib.orc_g2_generator(ptr(g2))
    assert Z.g1_from_words(g1) == Z.G1
    assert Z.g2_from_words(g2) == Z.G2
    # reference raw Montgomery limbs of the G2 generator (src/curve/g2.cuh:47-65)
    assert int(g2[0]) == 0x8E83B5D102BC2026 and int(g2[15]) == 0x0DA4A0E693FD6482
    if ref_available():
        r1 = np.zeros(8, dtype=np.uint64)
        r2 = np.zeros(16, dtype=np.uint64)
        ref().ref_g1_generator(ptr(r1))
        ref().ref_g2_generator(ptr(r2))
        assert np.array_equal(r1, g1) and np.array_equal(r2, g2)


def test_scalar_mul_closed_form():
    lib = oracle()
    rng = random.Random(5)
    g1 = np.array(Z.g1_to_words(Z.G1), dtype=np.uint64)
    g2 = np.array(Z.g2_to_words(Z.G2), dtype=np.uint64)
    for k in [0, 1, 2, 5, Z.R - 1, Z.R - 2] + [rng.randrange(Z.R) for _ in range(6)]:
        km = w4(Z.to_mont(k, Z.R))
        o1 = np.zeros(8, dtype=np.uint64)
        lib.orc_g1_mul(ptr(g1), ptr(km), ptr(o1))
        assert Z.g1_from_words(o1) == Z.g1.pmul(Z.G1, k)
        o2 = np.zeros(16, dtype=np.uint64)
        lib.orc_g2_mul(ptr(g2), ptr(km), ptr(o2))
        assert Z.g2_from_words(o2) == Z.g2.pmul(Z.G2, k)
        if ref_available():
            r1 = np.zeros(8, dtype=np.uint64)
            r2 = np.zeros(16, dtype=np.uint64)
            ref().ref_g1_mul(ptr(g1), ptr(km), ptr(r1))
            ref().ref_g2_mul(ptr(g2), ptr(km), ptr(r2))
            assert np.array_equal(r1, o1) and np.array_equal(r2, o2)
    # (r-1)*G + G = O : order r
    km = w4(Z.to_mont(Z.R - 1, Z.R))
    o = np.zeros(16, dtype=np.uint64)
    lib.orc_g2_mul(ptr(g2), ptr(km), ptr(o))
    s = np.zeros(16, dtype=np.uint64)
    lib.orc_g2_add(ptr(o), ptr(g2), ptr(s))
    assert not s.any()


def test_fixed_base_batch_matches_scalar_mul():
    lib = oracle()
    rng = random.Random(9)
    ks = [0, 1, Z.R - 1] + [rng.randrange(Z.R) for _ in range(13)]
    km = fr_array(ks)
    out = np.zeros((len(ks), 8), dtype=np.uint64)
    lib.orc_g1_gen_batch(ptr(km), len(ks), ptr(out), 2)
    for k, o in zip(ks, out):
        assert Z.g1_from_words(o) == Z.g1.pmul(Z.G1, k)
    out2 = np.zeros((4, 16), dtype=np.uint64)
    lib.orc_g2_gen_batch(ptr(km[:4].copy()), 4, ptr(out2), 2)
    for k, o in zip(ks[:4], out2):
        assert Z.g2_from_words(o) == Z.g2.pmul(Z.G2, k)


# ------------------------------------------------------------------ MSM
def msm_inputs(n, seed, g2=False):
    lib = oracle()
    rng = random.Random(seed)
    ks = [rng.randrange(1, Z.R) for _ in range(n)]
    ss = [rng.randrange(Z.R) for _ in range(n)]
    pts = np.zeros((n, 16 if g2 else 8), dtype=np.uint64)
    (lib.orc_g2_gen_batch if g2 else lib.orc_g1_gen_batch)(ptr(fr_array(ks)), n, ptr(pts), 4)
    return ks, ss, pts


@pytest.mark.parametrize("n", [0, 1, 2, 64, 300, 1500])
def test_msm_g1_closed_form(n):
    lib = oracle()
    ks, ss, pts = msm_inputs(n, n)
    sc = fr_array(ss) if n else np.zeros((0, 4), dtype=np.uint64)
    expect = Z.g1.pmul(Z.G1, sum(k * s for k, s in zip(ks, ss)) % Z.R)
    for mode in (0, 1) if n <= 300 else (0,):
        o = np.zeros(8, dtype=np.uint64)
        lib.orc_msm_g1(ptr(pts), ptr(sc), n, mode, 4, ptr(o))
        assert Z.g1_from_words(o) == expect


def test_msm_g1_special_cases():
    """Infinity points and zero digits are skipped (msm.cu:114-148)."""
    lib = oracle()
    ks, ss, pts = msm_inputs(400, 4)
    ss[3] = 0
    ss[7] = 1
    ss[8] = Z.R - 1
    pts[10] = 0
    ks[10] = 0
    sc = fr_array(ss)
    expect = Z.g1.pmul(Z.G1, sum(k * s for k, s in zip(ks, ss)) % Z.R)
    o = np.zeros(8, dtype=np.uint64)
    lib.orc_msm_g1(ptr(pts), ptr(sc), 400, 0, 4, ptr(o))
    assert Z.g1_from_words(o) == expect


@pytest.mark.parametrize("n", [1, 16, 200])
def test_msm_g2_closed_form(n):
    lib = oracle()
    ks, ss, pts = msm_inputs(n, 100 + n, g2=True)
    sc = fr_array(ss)
    expect = Z.g2.pmul(Z.G2, sum(k * s for k, s in zip(ks, ss)) % Z.R)
    for mode in (0, 2):  # Jacobian G2; the reference's affine-inversion G2
        o = np.zeros(16, dtype=np.uint64)
        lib.orc_msm_g2(ptr(pts), ptr(sc), n, mode, 4, ptr(o))
        assert Z.g2_from_words(o) == expect, mode


def test_msm_g2_affine_ref_special_cases():
    """The reference's affine-inversion G2 (g2.cuh:103-146) through the
    Pippenger path (n > 128) with a repeated point (bucket sums P + P take the
    tangent), a negated point (P + -P gives infinity), an infinity point and
    zero, one and r - 1 scalars: equal to the closed form and to Jacobian G2."""
    lib = oracle()
    n = 300
    ks, ss, pts = msm_inputs(n, 9, g2=True)
    ks[5], ks[6] = ks[4], Z.R - ks[4]
    ss[5] = ss[4]
    ss[6] = ss[4]
    ks[10] = 0
    ss[3], ss[7], ss[8] = 0, 1, Z.R - 1
    ss[20] = ss[21] = ss[22] = 12345  # one bucket, three different points
    fresh = np.zeros((3, 16), dtype=np.uint64)
    lib.orc_g2_gen_batch(ptr(fr_array([ks[4], Z.R - ks[4], 1])), 3, ptr(fresh), 1)
    pts[5], pts[6] = fresh[0], fresh[1]
    pts[10] = 0
    sc = fr_array(ss)
    expect = Z.g2.pmul(Z.G2, sum(k * s for k, s in zip(ks, ss)) % Z.R)
    got = {}
    for mode in (0, 2):
        o = np.zeros(16, dtype=np.uint64)
        lib.orc_msm_g2(ptr(pts), ptr(sc), n, mode, 4, ptr(o))
        got[mode] = o
        assert Z.g2_from_words(o) == expect, mode
    assert np.array_equal(got[0], got[2])


@needs_ref
def test_msm_matches_reference_small_path():
    lib, r = oracle(), ref()
    ks, ss, pts = msm_inputs(64, 77)
    sc = fr_array(ss)
    a = np.zeros(8, dtype=np.uint64)
    b = np.zeros(8, dtype=np.uint64)
    lib.orc_msm_g1(ptr(pts), ptr(sc), 64, 0, 2, ptr(a))
    r.ref_msm_g1_small(ptr(pts), ptr(sc), 64, ptr(b))
    assert np.array_equal(a, b)
    ks, ss, pts = msm_inputs(6, 78, g2=True)
    sc = fr_array(ss)
    a = np.zeros(16, dtype=np.uint64)
    b = np.zeros(16, dtype=np.uint64)
    lib.orc_msm_g2(ptr(pts), ptr(sc), 6, 0, 2, ptr(a))
    r.ref_msm_g2_small(ptr(pts), ptr(sc), 6, ptr(b))
    assert np.array_equal(a, b)


# ------------------------------------------------------------------ compute_h
def check_quotient(circ, h_words, seed=0):
    n = len(h_words)
    log_n = n.bit_length() - 1
    h = fr_list(h_words)
    assert h[n - 1] == 0
    A, B, C = circ.row_values(n)
    w = Z.omega(log_n)
    tau = random.Random(seed).randrange(2, Z.R)
    zt = (pow(tau, n, Z.R) - 1) % Z.R
    ninv = pow(n, -1, Z.R)

    def at_tau(vals):
        acc = 0
        wj = 1
        for v in vals:
            if v:
                acc += v * wj * pow(tau - wj, -1, Z.R)
            wj = wj * w % Z.R
        return acc * zt * ninv % Z.R

    lhs = (at_tau(A) * at_tau(B) - at_tau(C)) % Z.R
    assert lhs == Z.poly_eval(h, tau) * zt % Z.R


def test_oracle_dot_product_closed_form():
    """orc_fr_dot_std: sum a_i b_i mod r in standard form (the closed-form
    MSM scalar), against Python big integers, edge values included."""
    rng = random.Random(77)
    vals_a = [0, 1, Z.R - 1, Z.R - 1] + [rng.randrange(Z.R) for _ in range(996)]
    vals_b = [Z.R - 1, Z.R - 1, Z.R - 1, 1] + [rng.randrange(Z.R) for _ in range(996)]
    a = np.array([Z.limbs(v) for v in vals_a], dtype=np.uint64)
    b = np.array([Z.limbs(v) for v in vals_b], dtype=np.uint64)
    out = np.zeros(4, dtype=np.uint64)
    oracle().orc_fr_dot_std(ptr(a), ptr(b), len(vals_a), ptr(out))
    assert Z.from_limbs(out) == sum(x * y for x, y in zip(vals_a, vals_b)) % Z.R


@pytest.mark.parametrize("log_n,g", [(3, 5), (8, 7)])
def test_oracle_coset_scale_evaluates_on_the_coset(log_n, g):
    """orc_coset_scale then orc_ntt gives the polynomial at g w^j (Horner),
    and the inverse order (iNTT, then g^-i) undoes it."""
    n = 1 << log_n
    rng = random.Random(log_n)
    coeffs = [rng.randrange(Z.R) for _ in range(n)]
    a = np.array([Z.fr_words(c) for c in coeffs], dtype=np.uint64)
    lib = oracle()
    b = np.ascontiguousarray(a.copy())
    lib.orc_coset_scale(ptr(b), log_n, g, 0)
    lib.orc_ntt(ptr(b), log_n, 0, 2)
    w = Z.omega(log_n)
    assert [Z.fr_from_words(r) for r in b] == [Z.poly_eval(coeffs, g * pow(w, j, Z.R) % Z.R) for j in range(n)]
    lib.orc_ntt(ptr(b), log_n, 1, 2)
    lib.orc_coset_scale(ptr(b), log_n, g, 1)
    assert np.array_equal(b, a)


@pytest.mark.parametrize("rows", [2, 37, 200])
def test_compute_h_quotient_identity(rows):
    circ = random_r1cs(rows, seed=rows) if rows > 2 else mul_circuit()
    oc = OracleR1CS(circ.nc, circ.nv, circ.npub, circ.npriv, circ.mats())
    w = circ.witness_words()
    assert oc.verify(w)
    check_quotient(circ, oc.compute_h(w), seed=rows)
    bad = w.copy()
    bad[-1] = np.array(Z.fr_words(12345), dtype=np.uint64)
    assert not oc.verify(bad)


# ------------------------------------------------------------------ Groth16 end to end
def write_public(path, vals):
    with open(path, "wb") as f:
        f.write(struct.pack("<i", len(vals)))
        for v in vals:
            f.write(v.to_bytes(32, "little"))


@needs_ref
@pytest.mark.parametrize("kind", ["mul", "random"])
def test_oracle_groth16_verifies_with_reference(kind, tmp_path):
    circ = mul_circuit(7, 9) if kind == "mul" else random_r1cs(60, seed=42)
    oc = OracleR1CS(circ.nc, circ.nv, circ.npub, circ.npriv, circ.mats())
    pk, vk = str(tmp_path / "pk.bin"), str(tmp_path / "vk.bin")
    oc.setup(0xDEADBEEF42, pk, vk)
    rc, proof, _ = oc.prove(pk, circ.witness_words(), 0xCAFEBABE)
    assert rc == 0
    pf = tmp_path / "proof.bin"
    pf.write_bytes(proof)
    pub = tmp_path / "pub.bin"
    write_public(pub, circ.public())
    assert ref().ref_verify_files(vk.encode(), str(pf).encode(), str(pub).encode()) == 1
    bad = list(circ.public())
    bad[0] = (bad[0] + 1) % Z.R
    write_public(pub, bad)
    assert ref().ref_verify_files(vk.encode(), str(pf).encode(), str(pub).encode()) == 0
    # determinism: same seed, same bytes
    rc2, proof2, _ = oc.prove(pk, circ.witness_words(), 0xCAFEBABE)
    assert proof2 == proof
    rc3, proof3, _ = oc.prove(pk, circ.witness_words(), 0xCAFEBABF)
    assert proof3 != proof


def test_oracle_prove_affine_g2_same_bytes(tmp_path):
    """The oracle's prove with B on the reference's affine-inversion G2 (the
    timed CPU baseline's arithmetic) gives the same 256 bytes as with
    Jacobian G2 (whose proofs the seed pins check against closed forms)."""
    circ = random_r1cs(300, npub=3, seed=8)
    oc = OracleR1CS(circ.nc, circ.nv, circ.npub, circ.npriv, circ.mats())
    pk, vk = str(tmp_path / "pk.bin"), str(tmp_path / "vk.bin")
    oc.setup(0xDEADBEEF42, pk, vk)
    rc, proof, _ = oc.prove(pk, circ.witness_words(), 0xCAFEBABE)
    rc2, proof2, _ = oc.prove(pk, circ.witness_words(), 0xCAFEBABE, g2_affine_ref=True)
    assert rc == 0 and rc2 == 0 and proof == proof2


# ------------------------------------------------------------------ T4 golden artefacts
def t4_files():
    out = []
    for d in ("t4_p16", "t4_p160"):
        base = os.path.join(GOLD, d)
        for f in sorted(os.listdir(base)):
            if f.endswith(".proof.bin"):
                out.append((os.path.join(base, "vk.bin"), os.path.join(base, f),
                            os.path.join(base, f.replace(".proof.bin", ".public.bin"))))
    return out


@needs_ref
def test_t4_golden_proofs_verify_with_reference():
    files = t4_files()
    assert len(files) >= 8
    for vk, pf, pub in files:
        assert ref().ref_verify_files(vk.encode(), pf.encode(), pub.encode()) == 1, pf


@needs_ref
def test_t4_tampered_proof_rejected(tmp_path):
    vk, pf, pub = t4_files()[0]
    data = bytearray(open(pf, "rb").read())
    # swap A and C
    data[0:64], data[192:256] = data[192:256], data[0:64]
    bad = tmp_path / "bad.proof.bin"
    bad.write_bytes(bytes(data))
    assert ref().ref_verify_files(vk.encode(), str(bad).encode(), pub.encode()) == 0


def test_t4_pk_parse_matches_independent_parser():
    lib = oracle()
    path = os.path.join(GOLD, "t4_p16", "pk.bin")
    hdr, fixed, vecs = parse_zkmlpk3(path)
    assert (hdr["ver"], hdr["n"], hdr["m"], hdr["npub"]) == (3, 128, 140, 75)
    h = np.zeros(3, dtype=np.int32)
    s = np.zeros(7, dtype=np.int32)
    assert lib.orc_pk_read(path.encode(), ptr(h), ptr(s), None, None, None, None, None, None) == 0
    assert list(h) == [128, 140, 75]
    assert list(s) == [len(v) for v in vecs]
    A = np.zeros((s[2], 8), dtype=np.uint64)
    H = np.zeros((s[6], 8), dtype=np.uint64)
    B2 = np.zeros((s[4], 16), dtype=np.uint64)
    fx = np.zeros(24 + 48, dtype=np.uint64)
    lib.orc_pk_read(path.encode(), ptr(h), ptr(s), ptr(fx), ptr(A), None, ptr(B2), None, ptr(H))
    assert [Z.g1_from_words(r) for r in A] == vecs[2]
    assert [Z.g1_from_words(r) for r in H] == vecs[6]
    assert [Z.g2_from_words(r) for r in B2] == vecs[4]
    assert all(Z.g1_on_curve(p) for p in vecs[2] + vecs[3] + vecs[5] + vecs[6])
