"""GPU runs of the zkml-prove / zkml-verify command lines (cuda-zkml_amd/cli).

Pins:
  * a synthetic config-5 statement proved through zkml-prove (GPU setup +
    prove, deterministic seeds) gives a proof that zkml-verify, the product's
    zk_verify and the reference's own verifier (oracle/_ref) accept;
  * the same statement exported with --export-r1cs/--export-wtns and proved
    again from those iden3 files with --pk-load gives the same 256 bytes;
  * the oracle's restatement of the reference prover gives the same 256 bytes
    for the same R1CS, witness, key and seed;
  * exit code 1 and no proof acceptance for a tampered witness;
  * the setup seed contract of the reference (groth16.cu:455-462): without
    ZKML_DETERMINISTIC_SETUP two setups of one statement give different keys,
    with ZKML_DETERMINISTIC_SETUP=1 the keys are byte-identical to the
    oracle's setup at 0xDEADBEEF42, and --toxic-seed S to the oracle's at S.
The oracle/_ref comparisons run the reference's host code compiled in place
with the reference's own CUDA-runtime test shim (tests/host/shim).  They are
cross-checks and pin nothing by themselves: the proofs are pinned by the oracle
(same bytes) and verify under the product verifier.
"""
import os
import subprocess

import numpy as np
import pytest

import zkml_amd
from bindings import OracleR1CS, ref, ref_available

pytestmark = pytest.mark.gpu
ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PROVE = os.path.join(ROOT, "cuda-zkml_amd", "zkml-prove")
VERIFY = os.path.join(ROOT, "cuda-zkml_amd", "zkml-verify")
ENV = dict(os.environ, ZKML_DETERMINISTIC_PROVE="1")
ENV.pop("ZKML_DETERMINISTIC_SETUP", None)


def run(args, env=None, **kw):
    print("[cli]", " ".join(os.path.basename(a) if a.startswith("/") else a for a in args), flush=True)
    return subprocess.run(args, capture_output=True, text=True, env=env or ENV, timeout=240, **kw)


def test_cli_synthetic_then_files(tmp_path):
    assert os.path.exists(PROVE) and os.path.exists(VERIFY), "run __graft_entry__.build() first"
    t = lambda name: str(tmp_path / name)
    r = run([PROVE, "--synthetic", "3000", "--synthetic-seed", "9", "--pk-save", t("pk.bin"), "--vk", t("vk.bin"),
             "--output", t("p1.bin"), "--public-inputs", t("pub.bin"), "--export-r1cs", t("s.r1cs"),
             "--export-wtns", t("s.wtns")])
    assert r.returncode == 0, r.stdout + r.stderr
    assert "Proving time:" in r.stdout and "VALID" in r.stdout
    v = run([VERIFY, "--vk", t("vk.bin"), "--proof", t("p1.bin"), "--public-inputs", t("pub.bin")])
    assert v.returncode == 0, v.stdout + v.stderr
    if ref_available():
        assert ref().ref_verify_files(t("vk.bin").encode(), t("p1.bin").encode(), t("pub.bin").encode()) == 1
    # the same statement from the exported iden3 files and the saved key
    r2 = run([PROVE, "--r1cs", t("s.r1cs"), "--wtns", t("s.wtns"), "--pk-load", t("pk.bin"), "--vk", t("vk.bin"),
              "--output", t("p2.bin"), "--public-inputs", t("pub.json")])
    assert r2.returncode == 0, r2.stdout + r2.stderr
    p1 = open(t("p1.bin"), "rb").read()
    assert open(t("p2.bin"), "rb").read() == p1
    assert zkml_amd.verify_files(t("vk.bin"), t("p2.bin"), t("pub.json"))
    # the oracle's prover gives the same bytes
    nc, nv, npub, npriv, A, B, C = zkml_amd.iden3_r1cs_read(t("s.r1cs"))
    w = zkml_amd.wtns_read(t("s.wtns"))
    oc = OracleR1CS(nc, nv, npub, npriv, [(M["row"], M["col"], M["value"].reshape(-1, 4)) for M in (A, B, C)])
    rc, proof_o, _ = oc.prove(t("pk.bin"), w, 0xCAFEBABE)
    assert rc == 0 and proof_o == p1


def test_cli_rejects_bad_witness(tmp_path):
    t = lambda name: str(tmp_path / name)
    A, B, C, w = zkml_amd.synthetic_r1cs(500, 2, 4, 3)
    nv = w.shape[0]
    zkml_amd.iden3_r1cs_write(t("s.r1cs"), 500, nv, 2, 4, A, B, C)
    w_bad = w.copy()
    w_bad[-1, 0] ^= 1
    zkml_amd.wtns_write(t("bad.wtns"), w_bad)
    r = run([PROVE, "--r1cs", t("s.r1cs"), "--wtns", t("bad.wtns"), "--pk-save", t("pk.bin"), "--vk", t("vk.bin"),
             "--output", t("p.bin")])
    assert r.returncode == 1
    assert "witness" in (r.stdout + r.stderr).lower()


def test_cli_statement_v2_end_to_end(tmp_path):
    """zkml-prove --statement-v2 on the config-4-shaped CNN with a context and
    routing: proof verifies (zkml-verify, reference verifier), the public
    inputs carry the scores / tag / context, the metadata JSON equals the
    reference front end's, and a changed context is rejected."""
    import json
    from cli_models import digits_cnn, ref_cli_available, ref_statement, write_model, write_sample
    t = lambda name: str(tmp_path / name)
    layers, params = digits_cnn()
    arch, model = write_model(str(tmp_path), layers, params)
    x = write_sample(t("x.npy"), np.random.default_rng(7).integers(0, 17, 64))
    r = run([PROVE, "--statement-v2", "--integer-model", "--integer-input", "--model", model, "--arch", arch,
             "--input", x, "--context", "0x1234abcd", "--route-threshold", "3", "--output", t("proof.bin"),
             "--vk", t("vk.bin"), "--public-inputs", t("public.json"), "--statement-meta", t("meta.json")])
    assert r.returncode == 0, r.stdout + r.stderr
    assert "Proving time:" in r.stdout and "Statement mode: PCANI v2" in r.stdout
    v = run([VERIFY, "--vk", t("vk.bin"), "--proof", t("proof.bin"), "--public-inputs", t("public.json")])
    assert v.returncode == 0, v.stdout + v.stderr
    meta = json.load(open(t("meta.json")))
    pub = json.load(open(t("public.json")))
    assert len(pub) == meta["num_public"]
    assert pub[meta["context_public_index"]] == 0x1234abcd
    assert pub[meta["model_tag_public_index"]] == int(meta["model_tag64"], 16)
    if ref_cli_available():
        rc, info, tag, ref_meta = ref_statement(arch, model, [x], t("ref.r1cs"), t("ref.wtns"), context="0x1234abcd",
                                                route_threshold=3)
        assert rc == 0 and open(t("meta.json")).read() == ref_meta
    bad = list(pub)
    bad[meta["context_public_index"]] += 1
    json.dump(bad, open(t("bad.json"), "w"))
    v2 = run([VERIFY, "--vk", t("vk.bin"), "--proof", t("proof.bin"), "--public-inputs", t("bad.json")])
    assert v2.returncode == 1


def test_cli_setup_seed_contract(tmp_path):
    t = lambda name: str(tmp_path / name)
    stmt = ["--synthetic", "400", "--synthetic-seed", "5"]

    def setup(tag, env=None, extra=()):
        r = run([PROVE, *stmt, "--pk-save", t(tag + ".pk"), "--vk", t(tag + ".vk"), "--output", t(tag + ".proof"),
                 "--public-inputs", t(tag + ".pub"), "--export-r1cs", t("s.r1cs"), *extra], env=env)
        assert r.returncode == 0, r.stdout + r.stderr
        return r.stdout, open(t(tag + ".pk"), "rb").read(), open(t(tag + ".vk"), "rb").read()

    out1, pk1, vk1 = setup("rand1")
    out2, pk2, vk2 = setup("rand2")
    assert "randomized" in out1 and "randomized" in out2
    assert "DEADBEEF42" not in out1.upper()
    assert vk1 != vk2 and pk1 != pk2, "two setups without ZKML_DETERMINISTIC_SETUP gave the same key"
    outd, pkd, vkd = setup("det", env=dict(ENV, ZKML_DETERMINISTIC_SETUP="1"))
    assert "0x000000deadbeef42 (deterministic)" in outd
    oute, pke, vke = setup("explicit", extra=("--toxic-seed", "77"))
    assert "(explicit)" in oute
    # the oracle's setup of the same statement at the same seeds
    nc, nv, npub, npriv, A, B, C = zkml_amd.iden3_r1cs_read(t("s.r1cs"))
    oc = OracleR1CS(nc, nv, npub, npriv, [(M["row"], M["col"], M["value"].reshape(-1, 4)) for M in (A, B, C)])
    for seed, pk, vk in ((0xDEADBEEF42, pkd, vkd), (77, pke, vke)):
        oc.setup(seed, t("o.pk"), t("o.vk"))
        assert open(t("o.vk"), "rb").read() == vk and open(t("o.pk"), "rb").read() == pk, hex(seed)
    assert vk1 not in (vkd, vke) and vk2 not in (vkd, vke)
    # every key gives a proof that verifies
    for tag in ("rand1", "rand2", "det", "explicit"):
        v = run([VERIFY, "--vk", t(tag + ".vk"), "--proof", t(tag + ".proof"), "--public-inputs", t(tag + ".pub")])
        assert v.returncode == 0, tag + v.stdout + v.stderr
