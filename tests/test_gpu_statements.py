"""GPU proofs of the BASELINE config 1 and config 4 statements (config 1 and
the reference's variant B built by the reference's own statement builder and
committed as iden3 fixtures; config 4's network as written built by the
product's builder):
  * GPU setup, then a prove whose 256 bytes equal the oracle's restatement of
    the reference prover for the same key, witness and seed;
  * the proof verifies under the product's verifier and the reference's;
  * a wrong public input is rejected.
The oracle/_ref comparisons run the reference's host code compiled in place
with the reference's own CUDA-runtime test shim (tests/host/shim).  They are
cross-checks and pin nothing by themselves: the proofs are pinned by the oracle
and the statements by tests/test_statement_pins.py.
"""
import os
import time

import numpy as np
import pytest

from bindings import OracleR1CS, ref, ref_available
from statements import load

pytestmark = pytest.mark.gpu
MONT = 1 << 256
R_ORDER = 0x30644E72E131A029B85045B68181585D2833E84879B9709143E1F593F0000001


@pytest.fixture(scope="module")
def ctx():
    import zkml_amd
    c = zkml_amd.Context(0)
    yield c
    c.close()


def publics_std(w, npub):
    pub = np.zeros((npub, 4), dtype=np.uint64)
    for i in range(npub):
        x = sum(int(w[1 + i][k]) << (64 * k) for k in range(4)) * pow(MONT, -1, R_ORDER) % R_ORDER
        pub[i] = [(x >> (64 * k)) & (2**64 - 1) for k in range(4)]
    return pub


@pytest.mark.parametrize("name", ["config1", "config4"])
def test_prove_statement(ctx, tmp_path, name):
    import zkml_amd
    print(f"[statement] {name}", flush=True)
    nc, nv, npub, npriv, A, B, C, w = load(name)
    r = ctx.r1cs(nc, nv, npub, A, B, C)
    pk_path, vk_path = str(tmp_path / "pk.bin"), str(tmp_path / "vk.bin")
    ctx.setup(r, 0xDEADBEEF42, pk_path, vk_path)
    pk = ctx.load_pk(pk_path)
    ctx.prove(pk, r, w, npub, 0xCAFEBABE)
    t0 = time.perf_counter()
    proof, parts = ctx.prove(pk, r, w, npub, 0xCAFEBABE)
    ms = (time.perf_counter() - t0) * 1e3
    print(f"[statement] {name}: {nc} constraints, domain 2^{r.log_n}, prove {ms:.2f} ms {parts}", flush=True)
    mats = [(M["row"], M["col"], M["value"].reshape(-1, 4)) for M in (A, B, C)]
    oc = OracleR1CS(nc, nv, npub, npriv, mats)
    rc, proof_o, _ = oc.prove(pk_path, w, 0xCAFEBABE, threads=8)
    assert rc == 0 and proof == proof_o
    pub = publics_std(w, npub)
    vk = open(vk_path, "rb").read()
    assert zkml_amd.verify(vk, proof, pub)
    bad = pub.copy()
    bad[0, 0] ^= 1
    assert not zkml_amd.verify(vk, proof, bad)
    if ref_available():
        pp, up = tmp_path / "p.bin", tmp_path / "pub.bin"
        pp.write_bytes(proof)
        up.write_bytes(np.int32(npub).tobytes() + pub.tobytes())
        assert ref().ref_verify_files(vk_path.encode(), str(pp).encode(), str(up).encode()) == 1


def test_prove_config4_named(ctx, tmp_path):
    """BASELINE config 4's network as written (1x8x8 input, four 3x3 filters,
    MLP 144 -> 32 -> 10, private model and input under Poseidon, routing):
    707,395 constraints on a 2^20 domain, built by the product's statement
    builder (its size pinned by the gadget closed forms); GPU proof
    byte-identical to the oracle's prove with the same key, and verified."""
    import zkml_amd
    import statement_models as sm
    st = sm.config4_named()
    r = ctx.r1cs(st.nc, st.nv, st.npub, st.A, st.B, st.C)
    assert r.log_n == 20
    pk_path, vk_path = str(tmp_path / "pk.bin"), str(tmp_path / "vk.bin")
    print("[config4 named] setup", flush=True)
    ctx.setup(r, 0xDEADBEEF42, pk_path, vk_path)
    pk = ctx.load_pk(pk_path)
    ctx.prove(pk, r, st.w, st.npub, 0xCAFEBABE)
    t0 = time.perf_counter()
    proof, parts = ctx.prove(pk, r, st.w, st.npub, 0xCAFEBABE)
    print(f"[config4 named] {st.nc} constraints: prove {(time.perf_counter() - t0) * 1e3:.2f} ms {parts}",
          flush=True)
    mats = [(M["row"], M["col"], M["value"].reshape(-1, 4)) for M in (st.A, st.B, st.C)]
    oc = OracleR1CS(st.nc, st.nv, st.npub, st.npriv, mats)
    print("[config4 named] oracle prove", flush=True)
    rc, proof_o, _ = oc.prove(pk_path, st.w, 0xCAFEBABE, threads=16)
    assert rc == 0 and proof == proof_o
    pub = publics_std(st.w, st.npub)
    vk = open(vk_path, "rb").read()
    assert zkml_amd.verify(vk, proof, pub)
    bad = pub.copy()
    bad[0, 0] ^= 1
    assert not zkml_amd.verify(vk, proof, bad)
    pk.close()
    r.close()
