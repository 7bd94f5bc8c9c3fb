"""Pins of the seed-derived scalars of setup and prove, with no reference code.

* std::mt19937_64 (tests/mt64.py) against the C++ standard's required value:
  the 10000th output of a default-constructed engine is 9981545732273789042
  ([rand.predef]).
* The oracle's setup and prove (oracle/zk_oracle.cpp) against the
  scalar-domain closed forms of tests/groth16_closed_form.py: every key point
  and every proof element equals s * G for the scalar the Groth16 equations
  give for the reference's seeds (groth16.cu:48-58, 462-472, 712-715) and QAP
  convention (groth16.cu:97-189).  The GPU path gets the same check in
  tests/test_gpu_groth16.py.
* The check is not vacuous: a swapped draw order, raw (non-Montgomery)
  from_uint words, a domain of w^-j instead of w^j and r/s exchanged each make
  it fail.
"""
import pytest

import groth16_closed_form as CF
import zkpy as Z
from bindings import OracleR1CS
from mt64 import MT19937_64
from r1cs_gen import mul_circuit, random_r1cs

SETUP_SEED, PROVE_SEED = 0xDEADBEEF42, 0xCAFEBABE


def test_mt19937_64_standard_value():
    g = MT19937_64()
    for _ in range(9999):
        g()
    assert g() == 9981545732273789042


def test_reference_seed_draws():
    """The deterministic seeds' draws (values < 2^64, as Fr::from_uint takes a u64)."""
    tw = CF.toxic_waste(SETUP_SEED)
    r, s = CF.blinding(PROVE_SEED)
    g = MT19937_64(SETUP_SEED)
    assert [tw[k] for k in ("tau", "alpha", "beta", "gamma", "delta")] == [g() for _ in range(5)]
    g = MT19937_64(PROVE_SEED)
    assert (r, s) == (g(), g())
    assert all(0 < v < 1 << 64 for v in list(tw.values()) + [r, s])


def test_closed_form_quotient_identity():
    """The Lagrange basis behind the QAP scalars: it sums to 1, interpolates
    x, and u_i(tau) summed with the witness equals the row values weighted by
    L_j(tau); the rows are satisfied, so A(x) B(x) - C(x) vanishes on the
    domain and h(tau) Z(tau) = A_w B_w - C_w (the C scalar's identity)."""
    circ = random_r1cs(12, seed=4)
    tau = CF.toxic_waste(SETUP_SEED)["tau"]
    u, v, wt, n, zt = CF.qap_at(circ, tau)
    L, _ = CF.lagrange_at(CF.domain_log(circ.nc), tau)
    # Lagrange basis sums to 1 and interpolates x: sum_j w^j L_j(tau) = tau
    assert sum(L) % Z.R == 1
    w = Z.omega(CF.domain_log(circ.nc))
    assert sum(pow(w, j, Z.R) * L[j] for j in range(n)) % Z.R == tau
    # per-row values at the domain points give the same A_w as u_i(tau)
    a_rows, b_rows, c_rows = circ.row_values(n)
    Aw = sum(circ.w[i] * u[i] for i in range(circ.nv)) % Z.R
    assert Aw == sum(a * l for a, l in zip(a_rows, L)) % Z.R
    # the rows are satisfied, so A(x) B(x) - C(x) vanishes on the domain
    assert all((a * b - c) % Z.R == 0 for a, b, c in zip(a_rows, b_rows, c_rows))


@pytest.mark.parametrize("kind,seeds", [("mul", (SETUP_SEED, PROVE_SEED)), ("random", (SETUP_SEED, PROVE_SEED)),
                                        ("random", (7, 11))])
def test_oracle_keys_and_proof_equal_closed_form(kind, seeds, tmp_path):
    circ = mul_circuit(7, 9) if kind == "mul" else random_r1cs(50, npub=3, seed=5)
    setup_seed, prove_seed = seeds
    oc = OracleR1CS(circ.nc, circ.nv, circ.npub, circ.npriv, circ.mats())
    pk, vk = str(tmp_path / "pk.bin"), str(tmp_path / "vk.bin")
    oc.setup(setup_seed, pk, vk)
    tw = CF.toxic_waste(setup_seed)
    assert CF.check_keys(circ, CF.parse_zkmlpk3(pk), open(vk, "rb").read(), tw) == []
    rc, proof, _ = oc.prove(pk, circ.witness_words(), prove_seed)
    assert rc == 0
    r, s = CF.blinding(prove_seed)
    assert CF.check_proof(circ, proof, tw, r, s) == []


def test_closed_form_detects_plausible_mistakes(tmp_path):
    """Each mistake the pin is meant to catch changes what it expects."""
    circ = mul_circuit(7, 9)
    oc = OracleR1CS(circ.nc, circ.nv, circ.npub, circ.npriv, circ.mats())
    pk, vk = str(tmp_path / "pk.bin"), str(tmp_path / "vk.bin")
    oc.setup(SETUP_SEED, pk, vk)
    parsed, vkd = CF.parse_zkmlpk3(pk), open(vk, "rb").read()
    tw = CF.toxic_waste(SETUP_SEED)
    # tau and alpha drawn in the other order
    swapped = dict(tw, tau=tw["alpha"], alpha=tw["tau"])
    assert CF.check_keys(circ, parsed, vkd, swapped) != []
    # from_uint taken as raw Montgomery words: value v * 2^-256
    rinv = pow(1 << 256, -1, Z.R)
    raw = {k: v * rinv % Z.R for k, v in tw.items()}
    assert CF.check_keys(circ, parsed, vkd, raw) != []
    # the domain {w^-j} instead of {w^j}
    orig = Z.omega
    try:
        Z.omega = lambda log_n: pow(orig(log_n), -1, Z.R)
        assert CF.check_keys(circ, parsed, vkd, tw) != []
    finally:
        Z.omega = orig
    rc, proof, _ = oc.prove(pk, circ.witness_words(), PROVE_SEED)
    r, s = CF.blinding(PROVE_SEED)
    assert CF.check_proof(circ, proof, tw, r, s) == []
    assert CF.check_proof(circ, proof, tw, s, r) != []
