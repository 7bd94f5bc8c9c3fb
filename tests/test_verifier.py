"""CPU tests of the host pairing and Groth16 verifier of the product library
(zk_pairing, zk_verify, zk_verify_files; cuda-zkml_amd/csrc/pairing_host.hpp,
verifier.cpp) and of the zkml-verify command line.

Pins:
  pairing      equal, coefficient by coefficient, to the reference's own
               bn254::pairing (src/curve/pairing.cuh, compiled in oracle/_ref)
               on random points; e(aP, Q) = e(P, aQ); e(P1 + P2, Q) =
               e(P1, Q) e(P2, Q) (Fq12 product written here in Python from
               the tower definition); e(O, Q) = 1; e(P, Q) != 1.
  verify       the reference verifier's verdicts on the T4 golden proofs
               (all valid), a tampered proof, a wrong public input and a
               wrong public-input count; .json public inputs; a proof made by
               the oracle's restatement of the reference prover.
The oracle/_ref comparisons run the reference's host code compiled in place
with the reference's own CUDA-runtime test shim (tests/host/shim).  They are
cross-checks and pin nothing by themselves: the pairing is pinned by bilinearity,
non-degeneracy and e(O, Q) = 1, the verifier by the T4 golden proofs.
"""
import json
import os
import random
import subprocess

import numpy as np
import pytest

import zkml_amd
from bindings import OracleR1CS, ref, ref_available
from r1cs_gen import random_r1cs
from zkpy import G1, G2, P as Q, R as ORDER, f2_mul, g1, g2

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
GOLD = os.path.join(ROOT, "tests", "golden")
CLI = os.path.join(ROOT, "cuda-zkml_amd", "zkml-verify")
MONT = 1 << 256
needs_ref = pytest.mark.skipif(not ref_available(), reason="oracle/_ref not built (needs /root/reference)")


def std_words(vals):
    return np.array([(v >> (64 * i)) & ((1 << 64) - 1) for v in vals for i in range(4)], dtype=np.uint64)


def g1_words(pt):
    return std_words([0, 0] if pt is None else [pt[0], pt[1]])


def g2_words(pt):
    return std_words([0] * 4 if pt is None else [pt[0][0], pt[0][1], pt[1][0], pt[1][1]])


def fq12_ints(w):
    return [int(sum(int(w[4 * i + k]) << (64 * k) for k in range(4))) for i in range(12)]


# Fq12 = Fq6[w]/(w^2 - v), Fq6 = Fq2[v]/(v^3 - (9 + u)); element as 6 Fq2 pairs
# (c0.c0, c0.c1, c0.c2, c1.c0, c1.c1, c1.c2), reference order.
def _f2(a, b):
    return ((a[0] + b[0]) % Q, (a[1] + b[1]) % Q)


def _xi(a):
    return ((9 * a[0] - a[1]) % Q, (a[0] + 9 * a[1]) % Q)


def _f6mul(a, b):
    c = [(0, 0)] * 5
    for i in range(3):
        for j in range(3):
            c[i + j] = _f2(c[i + j], f2_mul(a[i], b[j]))
    return [_f2(c[0], _xi(c[3])), _f2(c[1], _xi(c[4])), c[2]]


def fq12_mul(x, y):
    X = [(x[2 * i], x[2 * i + 1]) for i in range(6)]
    Y = [(y[2 * i], y[2 * i + 1]) for i in range(6)]
    a0, a1, b0, b1 = X[:3], X[3:], Y[:3], Y[3:]
    t0, t1 = _f6mul(a0, b0), _f6mul(a1, b1)
    t1v = [_xi(t1[2]), t1[0], t1[1]]
    c0 = [_f2(t0[i], t1v[i]) for i in range(3)]
    m1, m2 = _f6mul(a0, b1), _f6mul(a1, b0)
    c1 = [_f2(m1[i], m2[i]) for i in range(3)]
    return [v for pair in c0 + c1 for v in pair]


ONE12 = [1] + [0] * 11


def rand_points(rng, k):
    return [(g1.pmul(G1, rng.randrange(1, ORDER)), g2.pmul(G2, rng.randrange(1, ORDER))) for _ in range(k)]


@needs_ref
def test_pairing_equals_reference_pairing():
    rng = random.Random(11)
    lib = ref()
    lib.ref_pairing.argtypes = [ctypes_vp()] * 3
    for P, Qp in [(G1, G2)] + rand_points(rng, 3):
        ours = fq12_ints(zkml_amd.pairing(g1_words(P), g2_words(Qp)))
        pm = std_words([P[0] * MONT % Q, P[1] * MONT % Q])
        qm = std_words([Qp[0][0] * MONT % Q, Qp[0][1] * MONT % Q, Qp[1][0] * MONT % Q, Qp[1][1] * MONT % Q])
        out = np.zeros(48, dtype=np.uint64)
        lib.ref_pairing(pm.ctypes.data, qm.ctypes.data, out.ctypes.data)
        theirs = [v * pow(MONT, -1, Q) % Q for v in fq12_ints(out)]
        assert ours == theirs


def ctypes_vp():
    import ctypes
    return ctypes.c_void_p


def test_pairing_bilinear_and_nondegenerate():
    rng = random.Random(12)
    P, Qp = G1, G2
    a = rng.randrange(2, ORDER)
    e = fq12_ints(zkml_amd.pairing(g1_words(P), g2_words(Qp)))
    assert e != ONE12
    assert fq12_ints(zkml_amd.pairing(g1_words(g1.pmul(P, a)), g2_words(Qp))) == \
        fq12_ints(zkml_amd.pairing(g1_words(P), g2_words(g2.pmul(Qp, a))))
    P1, P2 = g1.pmul(P, rng.randrange(1, ORDER)), g1.pmul(P, rng.randrange(1, ORDER))
    lhs = fq12_ints(zkml_amd.pairing(g1_words(g1.padd(P1, P2)), g2_words(Qp)))
    rhs = fq12_mul(fq12_ints(zkml_amd.pairing(g1_words(P1), g2_words(Qp))),
                   fq12_ints(zkml_amd.pairing(g1_words(P2), g2_words(Qp))))
    assert lhs == rhs
    # e(P, Q) e(-P, Q) = 1, and the point at infinity pairs to 1
    assert fq12_mul(e, fq12_ints(zkml_amd.pairing(g1_words(g1.pneg(P)), g2_words(Qp)))) == ONE12
    assert fq12_ints(zkml_amd.pairing(g1_words(None), g2_words(Qp))) == ONE12


def t4_files():
    out = []
    for d in ("t4_p16", "t4_p160"):
        base = os.path.join(GOLD, d)
        for f in sorted(os.listdir(base)):
            if f.endswith(".proof.bin"):
                out.append((os.path.join(base, "vk.bin"), os.path.join(base, f),
                            os.path.join(base, f.replace(".proof.bin", ".public.bin"))))
    return out


def test_t4_golden_proofs_verify():
    files = t4_files()
    assert len(files) >= 8
    for vk, pf, pub in files:
        assert zkml_amd.verify_files(vk, pf, pub), pf
        if ref_available():
            assert ref().ref_verify_files(vk.encode(), pf.encode(), pub.encode()) == 1


def test_rejections_match_reference(tmp_path):
    vk, pf, pub = t4_files()[0]
    proof = open(pf, "rb").read()
    pubdata = open(pub, "rb").read()
    cases = {}
    swapped = bytearray(proof)
    swapped[0:64], swapped[192:256] = proof[192:256], proof[0:64]
    cases["swap_A_C"] = (bytes(swapped), pubdata)
    wrong = bytearray(pubdata)
    wrong[4] ^= 1  # first public input + 1 (or - 1)
    cases["wrong_public"] = (proof, bytes(wrong))
    n = int.from_bytes(pubdata[:4], "little")
    fewer = (n - 1).to_bytes(4, "little") + pubdata[4:4 + 32 * (n - 1)]
    cases["short_public"] = (proof, fewer)
    for name, (pbytes, ubytes) in cases.items():
        p2, u2 = tmp_path / f"{name}.proof.bin", tmp_path / f"{name}.public.bin"
        p2.write_bytes(pbytes)
        u2.write_bytes(ubytes)
        assert not zkml_amd.verify_files(vk, str(p2), str(u2)), name
        if ref_available():
            assert ref().ref_verify_files(vk.encode(), str(p2).encode(), str(u2).encode()) == 0, name


def test_json_public_inputs(tmp_path):
    vk, pf, pub = t4_files()[0]
    d = open(pub, "rb").read()
    n = int.from_bytes(d[:4], "little")
    vals = [int.from_bytes(d[4 + 32 * i:36 + 32 * i], "little") for i in range(n)]
    # the largest value as a negative number (-x = r - x), the rest decimal
    k = max(range(n), key=lambda i: vals[i])
    toks = [str(v) for v in vals]
    toks[k] = str(-(ORDER - vals[k]))
    pj = tmp_path / "public.json"
    pj.write_text(json.dumps([int(t) for t in toks]))
    assert zkml_amd.verify_files(vk, pf, str(pj))


def test_oracle_proof_verifies(tmp_path):
    circ = random_r1cs(120, npub=3, seed=5)
    oc = OracleR1CS(circ.nc, circ.nv, circ.npub, circ.npriv, circ.mats())
    pk, vk = str(tmp_path / "pk.bin"), str(tmp_path / "vk.bin")
    oc.setup(0xDEADBEEF42, pk, vk)
    rc, proof, _ = oc.prove(pk, circ.witness_words(), 0xCAFEBABE)
    assert rc == 0
    w = circ.witness_words()
    pub = np.array([[0] * 4] * circ.npub, dtype=np.uint64)
    for i in range(circ.npub):  # public inputs w[1..npub] in standard form
        x = sum(int(w[1 + i][k]) << (64 * k) for k in range(4)) * pow(MONT, -1, ORDER) % ORDER
        pub[i] = [(x >> (64 * k)) & ((1 << 64) - 1) for k in range(4)]
    vkb = open(vk, "rb").read()
    assert zkml_amd.verify(vkb, proof, pub)
    bad = pub.copy()
    bad[0, 0] ^= 1
    assert not zkml_amd.verify(vkb, proof, bad)


def test_cli_exit_codes(tmp_path):
    assert os.path.exists(CLI), "run __graft_entry__.build() first"
    vk, pf, pub = t4_files()[0]
    ok = subprocess.run([CLI, "--vk", vk, "--proof", pf, "--public-inputs", pub], capture_output=True, text=True)
    assert ok.returncode == 0 and "PROOF VALID" in ok.stdout
    data = bytearray(open(pf, "rb").read())
    data[40] ^= 1
    bad = tmp_path / "bad.proof.bin"
    bad.write_bytes(bytes(data))
    no = subprocess.run([CLI, "--vk", vk, "--proof", str(bad), "--public-inputs", pub], capture_output=True, text=True)
    assert no.returncode == 1
    missing = subprocess.run([CLI, "--vk", vk], capture_output=True, text=True)
    assert missing.returncode == 1
