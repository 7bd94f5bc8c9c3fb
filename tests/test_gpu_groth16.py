"""GPU quotient polynomial, trusted setup and prove through the C ABI.

Pins:
  * h (zk_quotient_h) bit-exact against the oracle's compute_h
    (groth16.cu:263-390) and the quotient identity at a random point;
  * proving and verification key files byte-identical to the oracle's
    restatement of Groth16Prover::setup (groth16.cu:446-642) for the same
    R1CS and toxic-waste seed;
  * 256-byte proofs byte-identical to the oracle's restatement of prove
    (groth16.cu:655-920) for the same key, witness and blinding seed;
  * every key point and proof element equal to s * G for the scalar the
    Groth16 equations give for the reference's seeds (closed forms of
    tests/groth16_closed_form.py, no reference code involved);
  * every proof accepted by the product's verifier (itself pinned by the
    reference's T4 golden proofs) and, where oracle/_ref is built, by the
    reference's own verifier code; a wrong public input rejected, an
    unsatisfying witness refused;
  * the reference's own T4 proving keys load with the reference checks.
The oracle/_ref comparisons run the reference's host code compiled in place
with the reference's own CUDA-runtime test shim (tests/host/shim).  They are
cross-checks and pin nothing by themselves: the proofs are pinned by the oracle (itself
pinned by closed forms) and the scalar-domain closed forms above.
"""
import os
import struct

import numpy as np
import pytest

import zkpy as Z
from bindings import OracleR1CS, ref, ref_available
from r1cs_gen import mul_circuit, random_r1cs
from test_oracle import check_quotient

pytestmark = pytest.mark.gpu
GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
SETUP_SEED = 0xDEADBEEF42
PROVE_SEED = 0xCAFEBABE


@pytest.fixture(scope="module")
def ctx():
    import zkml_amd
    c = zkml_amd.Context(0)
    yield c
    c.close()


def gpu_r1cs(ctx, circ):
    return ctx.r1cs(circ.nc, circ.nv, circ.npub, *circ.mats())


def write_public(path, vals):
    with open(path, "wb") as f:
        f.write(struct.pack("<i", len(vals)))
        for v in vals:
            f.write(v.to_bytes(32, "little"))


@pytest.mark.parametrize("rows", [2, 100, 1000, 5000])
def test_quotient_h_matches_oracle(ctx, rows):
    circ = mul_circuit() if rows == 2 else random_r1cs(rows, seed=rows)
    r = gpu_r1cs(ctx, circ)
    n = 1 << r.log_n
    w = circ.witness_words()
    dw = ctx.upload(w)
    dh = ctx.alloc(n * 32)
    ctx.quotient_h(r, dw, circ.nv, dh)
    got = ctx.d2h(dh, (n, 4))
    oc = OracleR1CS(circ.nc, circ.nv, circ.npub, circ.npriv, circ.mats())
    assert np.array_equal(got, oc.compute_h(w, threads=8))
    if rows <= 1000:
        check_quotient(circ, got, seed=rows)


@pytest.mark.parametrize("kind", ["mul", "r300", "r3000"])
def test_setup_and_prove_match_oracle_and_verify(ctx, tmp_path, kind):
    circ = {"mul": lambda: mul_circuit(7, 9), "r300": lambda: random_r1cs(300, npub=3, seed=5),
            "r3000": lambda: random_r1cs(3000, npub=6, seed=6, small_frac=0.7)}[kind]()
    r = gpu_r1cs(ctx, circ)
    oc = OracleR1CS(circ.nc, circ.nv, circ.npub, circ.npriv, circ.mats())
    pk_g, vk_g = tmp_path / "pk_gpu.bin", tmp_path / "vk_gpu.bin"
    pk_o, vk_o = str(tmp_path / "pk_orc.bin"), str(tmp_path / "vk_orc.bin")
    ctx.setup(r, SETUP_SEED, pk_g, vk_g)
    oc.setup(SETUP_SEED, pk_o, vk_o, threads=8)
    assert pk_g.read_bytes() == open(pk_o, "rb").read()
    assert vk_g.read_bytes() == open(vk_o, "rb").read()
    pk = ctx.load_pk(pk_g)
    assert (pk.n, pk.m, pk.npub) == (1 << r.log_n, circ.nv, circ.npub)
    proof, t = ctx.prove(pk, r, circ.witness_words(), circ.npub, PROVE_SEED)
    rc, proof_o, _ = oc.prove(pk_o, circ.witness_words(), PROVE_SEED, threads=8)
    assert rc == 0
    assert proof == proof_o
    # phase timings: the total by the host clock, the GPU phases by events
    # inside it (a small allowance for the two clocks)
    assert t["total"] > 0 and all(v >= 0 for v in t.values())
    assert max(t[k] for k in ("quotient", "A", "B_g2", "L", "H", "B_g1")) <= t["total"] + 0.05
    pf = tmp_path / "proof.bin"
    pf.write_bytes(proof)
    pub = tmp_path / "pub.bin"
    write_public(pub, circ.public())
    import zkml_amd
    assert zkml_amd.verify_files(str(vk_g), str(pf), str(pub))
    if ref_available():
        assert ref().ref_verify_files(str(vk_g).encode(), str(pf).encode(), str(pub).encode()) == 1
        bad = list(circ.public())
        bad[-1] = (bad[-1] + 1) % Z.R
        write_public(pub, bad)
        assert ref().ref_verify_files(str(vk_g).encode(), str(pf).encode(), str(pub).encode()) == 0


@pytest.mark.parametrize("kind,seeds", [("mul", (SETUP_SEED, PROVE_SEED)), ("r50", (SETUP_SEED, PROVE_SEED)),
                                        ("r50", (7, 11))])
def test_keys_and_proof_equal_closed_form(ctx, tmp_path, kind, seeds):
    """zk_setup / zk_prove against the scalar-domain closed forms: toxic waste
    and blinding from std::mt19937_64 (groth16.cu:48-58, 462-472, 712-715),
    the QAP over the domain {w^j} (groth16.cu:97-189), C = L + H + sA + rB1."""
    import groth16_closed_form as CF
    circ = mul_circuit(7, 9) if kind == "mul" else random_r1cs(50, npub=3, seed=5)
    setup_seed, prove_seed = seeds
    r = gpu_r1cs(ctx, circ)
    ctx.setup(r, setup_seed, tmp_path / "pk.bin", tmp_path / "vk.bin")
    tw = CF.toxic_waste(setup_seed)
    parsed = CF.parse_zkmlpk3(str(tmp_path / "pk.bin"))
    assert CF.check_keys(circ, parsed, (tmp_path / "vk.bin").read_bytes(), tw) == []
    pk = ctx.load_pk(tmp_path / "pk.bin")
    proof, _ = ctx.prove(pk, r, circ.witness_words(), circ.npub, prove_seed)
    rr, ss = CF.blinding(prove_seed)
    assert CF.check_proof(circ, proof, tw, rr, ss) == []


def test_prove_rejects_bad_witness_and_sizes(ctx, tmp_path):
    import zkml_amd
    circ = random_r1cs(64, seed=9)
    r = gpu_r1cs(ctx, circ)
    ctx.setup(r, SETUP_SEED, tmp_path / "pk.bin", tmp_path / "vk.bin")
    pk = ctx.load_pk(tmp_path / "pk.bin")
    w = circ.witness_words()
    bad = w.copy()
    bad[-1] = np.array(Z.fr_words(3), dtype=np.uint64)
    with pytest.raises(zkml_amd.ZkError, match="satisfy"):
        ctx.prove(pk, r, bad, circ.npub, PROVE_SEED)
    with pytest.raises(zkml_amd.ZkError):
        ctx.prove(pk, r, w[:-1], circ.npub, PROVE_SEED)
    with pytest.raises(zkml_amd.ZkError):
        ctx.prove(pk, r, w, circ.npub + 1, PROVE_SEED)
    # ZKML_SKIP_WITNESS_CHECK path: proof produced, but it does not verify
    proof, _ = ctx.prove(pk, r, bad, circ.npub, PROVE_SEED, check_witness=False)
    assert len(proof) == 256


def test_loads_reference_t4_proving_keys(ctx):
    import zkml_amd
    for d, (n, m, npub) in (("t4_p16", (128, 140, 75)), ("t4_p160", (1024, 716, 75))):
        pk = ctx.load_pk(os.path.join(GOLD, d, "pk.bin"))
        assert (pk.n, pk.m, pk.npub) == (n, m, npub)
        pk.close()
    with pytest.raises(zkml_amd.ZkError):
        ctx.load_pk(os.path.join(GOLD, "t4_p16", "vk.bin"))


def test_truncated_pk_rejected(ctx, tmp_path):
    import zkml_amd
    data = open(os.path.join(GOLD, "t4_p16", "pk.bin"), "rb").read()
    p = tmp_path / "trunc.bin"
    p.write_bytes(data[: len(data) // 2])
    with pytest.raises(zkml_amd.ZkError):
        ctx.load_pk(p)


def test_prove_2_16_matches_oracle(ctx, tmp_path):
    """Full-size parity: 2^16-domain synthetic R1CS (BASELINE config-5 shape),
    GPU setup and prove against the oracle on the same key."""
    circ = random_r1cs((1 << 16) - 40, inputs=16, npub=4, seed=16, small_frac=0.7)
    r = gpu_r1cs(ctx, circ)
    assert r.log_n == 16
    pk_path, vk_path = tmp_path / "pk.bin", tmp_path / "vk.bin"
    ctx.setup(r, SETUP_SEED, pk_path, vk_path)
    pk = ctx.load_pk(pk_path)
    proof, t = ctx.prove(pk, r, circ.witness_words(), circ.npub, PROVE_SEED)
    oc = OracleR1CS(circ.nc, circ.nv, circ.npub, circ.npriv, circ.mats())
    rc, proof_o, _ = oc.prove(str(pk_path), circ.witness_words(), PROVE_SEED, threads=16)
    assert rc == 0 and proof == proof_o
    if ref_available():
        pf = tmp_path / "proof.bin"
        pf.write_bytes(proof)
        pub = tmp_path / "pub.bin"
        write_public(pub, circ.public())
        assert ref().ref_verify_files(str(vk_path).encode(), str(pf).encode(), str(pub).encode()) == 1


@pytest.mark.parametrize("nc", [(1 << 14) - 8, (1 << 18) - 64, (1 << 18) + 64])
def test_prove_window_table_shapes(ctx, tmp_path, nc):
    """Proofs whose MSMs run on the proving key's window tables at each shape
    boundary (m = nc + 21 variables): 2^14..2^15 (20 windows of 13 bits for
    every query, a 2^14 domain),
    up to 2^18 (16-bit windows for the witness sets, 13-bit for B2 and H;
    sub-windows of 2^10 and 2^8 buckets) and just above 2^18 (13 windows of
    19-20 bits through the two-level wide sort, 2^15-bucket sub-windows).
    Byte-identical to the oracle's prove on the same key and seed."""
    import zkml_amd
    npub = 4
    A, B, C, w = zkml_amd.synthetic_r1cs(nc, npub, 16, nc % 97)
    r = ctx.r1cs(nc, w.shape[0], npub, A, B, C)
    pk_path, vk_path = tmp_path / "pk.bin", tmp_path / "vk.bin"
    print(f"[prove tables] nc={nc} m={w.shape[0]} domain 2^{r.log_n}", flush=True)
    ctx.setup(r, SETUP_SEED, pk_path, vk_path)
    pk = ctx.load_pk(pk_path)
    proof, _ = ctx.prove(pk, r, w, npub, PROVE_SEED)
    oc = _oracle_of(A, B, C, nc, w.shape[0], npub)
    rc, proof_o, _ = oc.prove(str(pk_path), w, PROVE_SEED, threads=16)
    assert rc == 0 and proof == proof_o
    pub = [Z.from_mont(Z.from_limbs([int(x) for x in w[1 + i]]), Z.R) for i in range(npub)]
    pub_words = np.array([Z.limbs(v) for v in pub], dtype=np.uint64)
    assert zkml_amd.verify(vk_path.read_bytes(), proof, pub_words)
    pk.close()
    r.close()


def _oracle_of(A, B, C, nc, nv, npub):
    mats = [(M["row"], M["col"], np.ascontiguousarray(M["value"])) for M in (A, B, C)]
    return OracleR1CS(nc, nv, npub, nv - 1 - npub, mats)


def test_quotient_h_2_22_matches_oracle(ctx):
    """zk_quotient_h at BASELINE config 5's 2^22 constraints, bit-exact against
    the oracle's compute_h (groth16.cu:263-390) on the box's host threads."""
    import zkml_amd
    nc, npub = 1 << 22, 4
    A, B, C, w = zkml_amd.synthetic_r1cs(nc, npub, 16, 23)
    r = ctx.r1cs(nc, w.shape[0], npub, A, B, C)
    assert r.log_n == 22
    dw = ctx.upload(w)
    dh = ctx.alloc(nc * 32)
    ctx.quotient_h(r, dw, w.shape[0], dh)
    got = ctx.d2h(dh, (nc, 4))
    print("[quotient 2^22] oracle compute_h", flush=True)
    oc = _oracle_of(A, B, C, nc, w.shape[0], npub)
    assert np.array_equal(got, oc.compute_h(w, threads=16))
    assert not got[-1].any()  # h has degree < n - 1
    r.close()


def test_prove_2_22_config5_verifies(ctx, tmp_path):
    """BASELINE config 5 at its full 2^22 constraints (3 nonzeros per A and B
    row, C the fresh product variable): the proof is byte-identical to the
    oracle's prove with the same key, witness and seed; it is accepted by the
    product's verifier (and by the reference's own code in oracle/_ref where
    built), a changed public input is rejected, and a second prove with the
    same seed, its MSM jobs run on the calling thread (thread starts refused
    by the test hook), gives the same bytes."""
    import zkml_amd
    nc, npub = 1 << 22, 4
    A, B, C, w = zkml_amd.synthetic_r1cs(nc, npub, 16, 22)
    r = ctx.r1cs(nc, w.shape[0], npub, A, B, C)
    assert r.log_n == 22
    pk_path, vk_path = tmp_path / "pk.bin", tmp_path / "vk.bin"
    print("[prove 2^22] setup", flush=True)
    ctx.setup(r, SETUP_SEED, pk_path, vk_path)
    pk = ctx.load_pk(pk_path)
    print("[prove 2^22] prove", flush=True)
    proof, _ = ctx.prove(pk, r, w, npub, PROVE_SEED)
    # again with every job thread refused: the jobs run on the calling thread
    # after the quotient (the gated G1 job of this size would otherwise wait
    # for a gate that only that thread opens)
    print("[prove 2^22] prove with the job threads refused", flush=True)
    assert zkml_amd.lib().zk_debug_fail_thread_start(3) == 0
    try:
        again, _ = ctx.prove(pk, r, w, npub, PROVE_SEED)
    finally:
        zkml_amd.lib().zk_debug_fail_thread_start(0)
    assert proof == again
    print("[prove 2^22] oracle prove", flush=True)
    oc = _oracle_of(A, B, C, nc, w.shape[0], npub)
    del A, B, C
    rc, proof_o, _ = oc.prove(str(pk_path), w, PROVE_SEED, threads=16)
    del oc
    os.remove(pk_path)
    assert rc == 0 and proof == proof_o
    pub = [Z.from_mont(Z.from_limbs([int(x) for x in w[1 + i]]), Z.R) for i in range(npub)]
    pub_words = np.array([Z.limbs(v) for v in pub], dtype=np.uint64)
    vk = vk_path.read_bytes()
    assert zkml_amd.verify(vk, proof, pub_words)
    bad = pub_words.copy()
    bad[0, 0] ^= 1
    assert not zkml_amd.verify(vk, proof, bad)
    if ref_available():
        pf = tmp_path / "proof.bin"
        pf.write_bytes(proof)
        pubf = tmp_path / "pub.bin"
        write_public(pubf, pub)
        assert ref().ref_verify_files(str(vk_path).encode(), str(pf).encode(), str(pubf).encode()) == 1
    pk.close()
    r.close()
