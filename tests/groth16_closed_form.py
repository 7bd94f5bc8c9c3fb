"""Groth16 keys and proofs in the scalar domain (Python big integers).

Independent pin of the seed-derived scalars of setup and prove: given a
circuit and the two seeds, every proving-key, verification-key and proof
point is s * G for a scalar s that this module computes from first
principles, with no C code involved:

* toxic waste (tau, alpha, beta, gamma, delta) = the first five nonzero
  Fr::from_uint(std::mt19937_64(setup_seed)()) values, blinding (r, s) the
  first two of std::mt19937_64(prove_seed)
  (reference src/prover/groth16.cu:48-58, 462-472, 712-715).  Fr::from_uint(v)
  is the Montgomery form of the integer v (fp.cuh:487-492), i.e. the field
  element v itself; std::mt19937_64 is the C++ standard's engine
  (tests/mt64.py, pinned by the standard's 10000th-output requirement).
* QAP at tau: u_i(tau) = sum_j A[j][i] L_j(tau) with the Lagrange basis of the
  domain {w^j} (w = the NTT's 2^log_n-th root of unity),
  L_j(tau) = (tau^n - 1) w^j / (n (tau - w^j))  (groth16.cu:97-189); the
  domain is the power of two >= #constraints, at least 4 (groth16.cu:225-242).
* PK / VK (groth16.cu:480-625): alpha, beta, delta in G1; beta, gamma, delta
  in G2; tau powers in G2 [1, tau]; A_i = u_i, B1_i = B2_i = v_i;
  L_i = (beta u_v + alpha v_v + w_v) / delta for v = i + 1 + npub;
  H_i = tau^i (tau^n - 1) / delta; IC_i = (beta u_i + alpha v_i + w_i) / gamma.
* proof (groth16.cu:769-840): A = alpha + A_w + r delta,
  B = beta + B_w + s delta, C = sum_{i > npub} w_i L_i + h(tau) Z(tau) / delta
  + s A + r (beta + B_w), with h(tau) Z(tau) = A_w B_w - C_w for a satisfying
  witness (the quotient identity), A_w = sum_i w_i u_i(tau) and so on.

The mirror of the reference's own scalar-domain diagnostic
(groth16.cu:843-912), but written from the Groth16 equations, not from the
code under test.
"""
from mt64 import MT19937_64
import zkpy as Z

R, P = Z.R, Z.P


# ------------------------------------------------------------------ seeds
def nonzero_draws(seed, count):
    """The first `count` nonzero Fr::from_uint(mt19937_64(seed)()) values."""
    g = MT19937_64(seed)
    out = []
    while len(out) < count:
        v = g() % R
        if v:
            out.append(v)
    return out


def toxic_waste(seed=0xDEADBEEF42):
    tau, alpha, beta, gamma, delta = nonzero_draws(seed, 5)
    return dict(tau=tau, alpha=alpha, beta=beta, gamma=gamma, delta=delta)


def blinding(seed=0xCAFEBABE):
    r, s = nonzero_draws(seed, 2)
    return r, s


# ------------------------------------------------------------------ QAP at tau
def domain_log(num_constraints):
    n, log_n = 1, 0
    while n < num_constraints:
        n <<= 1
        log_n += 1
    if n < 4:
        n, log_n = 4, 2
    return log_n


def lagrange_at(log_n, tau):
    n = 1 << log_n
    w = Z.omega(log_n)
    zt = (pow(tau, n, R) - 1) % R
    ninv = pow(n, -1, R)
    out, wj = [], 1
    for _ in range(n):
        out.append(zt * wj % R * ninv % R * pow((tau - wj) % R, -1, R) % R)
        wj = wj * w % R
    return out, zt


def qap_at(circ, tau):
    """(u, v, wt, n, Z(tau)): the A, B, C polynomials of each variable at tau."""
    log_n = domain_log(circ.nc)
    n = 1 << log_n
    L, zt = lagrange_at(log_n, tau)
    u, v, wt = [0] * circ.nv, [0] * circ.nv, [0] * circ.nv
    for M, acc in ((circ.A, u), (circ.B, v), (circ.C, wt)):
        for row, col, c in M:
            if row < n and col < circ.nv:
                acc[col] = (acc[col] + c * L[row]) % R
    return u, v, wt, n, zt


# ------------------------------------------------------------------ expected scalars
def key_scalars(circ, tw):
    """Scalars of every PK / VK point, in file order."""
    tau, al, be, ga, de = tw["tau"], tw["alpha"], tw["beta"], tw["gamma"], tw["delta"]
    u, v, wt, n, zt = qap_at(circ, tau)
    dinv, ginv = pow(de, -1, R), pow(ga, -1, R)
    npub, m = circ.npub, circ.nv
    lq = [(be * u[k] + al * v[k] + wt[k]) * dinv % R for k in range(1 + npub, m)]
    hq, t = [], zt * dinv % R
    for _ in range(n):
        hq.append(t)
        t = t * tau % R
    ic = [(be * u[k] + al * v[k] + wt[k]) * ginv % R if k < m else 0 for k in range(npub + 1)]
    return dict(n=n, alpha_g1=al, beta_g1=be, delta_g1=de, beta_g2=be, gamma_g2=ga, delta_g2=de,
                tau_g2=[1, tau], A=u, B1=v, B2=v, L=lq, H=hq, ic=ic)


def proof_scalars(circ, tw, r, s):
    """(A, B, C) scalars of the proof for the circuit's witness."""
    al, be, de = tw["alpha"], tw["beta"], tw["delta"]
    u, v, wt, n, zt = qap_at(circ, tw["tau"])
    w = circ.w
    m = circ.nv
    Aw = sum(w[i] * u[i] for i in range(m)) % R
    Bw = sum(w[i] * v[i] for i in range(m)) % R
    Cw = sum(w[i] * wt[i] for i in range(m)) % R
    dinv = pow(de, -1, R)
    a = (al + Aw + r * de) % R
    b = (be + Bw + s * de) % R
    priv = sum(w[i] * (be * u[i] + al * v[i] + wt[i]) for i in range(1 + circ.npub, m)) * dinv % R
    hz = (Aw * Bw - Cw) * dinv % R
    c = (priv + hz + s * a + r * (be + Bw)) % R
    return a, b, c


# ------------------------------------------------------------------ fast scalar multiples
# Jacobian coordinates over Fq (G1) and Fq2 (G2), y^2 = x^3 + b, a = 0:
# dbl-2009-l and add-2007-bl; one inversion at the end.
class _Field:
    def __init__(self, add, sub, mul, inv, zero, one):
        self.add, self.sub, self.mul, self.inv, self.zero, self.one = add, sub, mul, inv, zero, one


_FQ = _Field(lambda a, b: (a + b) % P, lambda a, b: (a - b) % P, lambda a, b: a * b % P,
             lambda a: pow(a, P - 2, P), 0, 1)
_FQ2 = _Field(Z.f2_add, Z.f2_sub, Z.f2_mul, Z.f2_inv, (0, 0), (1, 0))


def _jdbl(F, p):
    X, Y, Zc = p
    if Zc == F.zero:
        return p
    A = F.mul(X, X)
    B = F.mul(Y, Y)
    C = F.mul(B, B)
    t = F.add(X, B)
    D = F.sub(F.sub(F.mul(t, t), A), C)
    D = F.add(D, D)
    E = F.add(F.add(A, A), A)
    Fv = F.mul(E, E)
    X3 = F.sub(Fv, F.add(D, D))
    C8 = F.add(C, C)
    C8 = F.add(C8, C8)
    C8 = F.add(C8, C8)
    Y3 = F.sub(F.mul(E, F.sub(D, X3)), C8)
    Z3 = F.mul(Y, Zc)
    Z3 = F.add(Z3, Z3)
    return (X3, Y3, Z3)


def _jadd(F, p, q):
    if p[2] == F.zero:
        return q
    if q[2] == F.zero:
        return p
    X1, Y1, Z1 = p
    X2, Y2, Z2 = q
    Z1Z1, Z2Z2 = F.mul(Z1, Z1), F.mul(Z2, Z2)
    U1, U2 = F.mul(X1, Z2Z2), F.mul(X2, Z1Z1)
    S1 = F.mul(F.mul(Y1, Z2), Z2Z2)
    S2 = F.mul(F.mul(Y2, Z1), Z1Z1)
    H = F.sub(U2, U1)
    rr = F.sub(S2, S1)
    if H == F.zero:
        if rr == F.zero:
            return _jdbl(F, p)
        return (F.one, F.one, F.zero)
    I = F.add(H, H)
    I = F.mul(I, I)
    J = F.mul(H, I)
    rr = F.add(rr, rr)
    V = F.mul(U1, I)
    X3 = F.sub(F.sub(F.mul(rr, rr), J), F.add(V, V))
    S1J = F.mul(S1, J)
    Y3 = F.sub(F.mul(rr, F.sub(V, X3)), F.add(S1J, S1J))
    t = F.add(Z1, Z2)
    Z3 = F.mul(F.sub(F.sub(F.mul(t, t), Z1Z1), Z2Z2), H)
    return (X3, Y3, Z3)


def _mul(F, base, k):
    k %= R
    if k == 0:
        return None
    acc = (F.one, F.one, F.zero)
    pt = (base[0], base[1], F.one)
    for bit in bin(k)[2:]:
        acc = _jdbl(F, acc)
        if bit == "1":
            acc = _jadd(F, acc, pt)
    if acc[2] == F.zero:
        return None
    zi = F.inv(acc[2])
    zi2 = F.mul(zi, zi)
    return (F.mul(acc[0], zi2), F.mul(acc[1], F.mul(zi2, zi)))


def g1(k):
    """k * G1 in affine standard form (None = infinity)."""
    return _mul(_FQ, Z.G1, k)


def g2(k):
    """k * G2 (EIP-197 generator) in affine standard form (None = infinity)."""
    return _mul(_FQ2, Z.G2, k)


# ------------------------------------------------------------------ file images
def _g1_std(d, off):
    x = int.from_bytes(d[off:off + 32], "little")
    y = int.from_bytes(d[off + 32:off + 64], "little")
    return None if x == 0 and y == 0 else (x, y)


def _g2_std(d, off):
    v = [int.from_bytes(d[off + 32 * i:off + 32 * i + 32], "little") for i in range(4)]
    return None if not any(v) else ((v[0], v[1]), (v[2], v[3]))


def parse_proof(data):
    """256-byte proof: A.x, A.y, B.x.c0, B.x.c1, B.y.c0, B.y.c1, C.x, C.y
    (src/verifier/verifier.cu:13-45)."""
    assert len(data) == 256
    return _g1_std(data, 0), _g2_std(data, 64), _g1_std(data, 192)


def parse_zkmlpk3(path):
    """Independent Python parser of the ZKMLPK3 layout (groth16.cu:1104-1188)."""
    import struct
    d = open(path, "rb").read()
    assert d[:7] == b"ZKMLPK3"
    ver, n, m, npub = struct.unpack_from("<Iiii", d, 8)
    off = 24
    def g1():
        nonlocal off
        inf = d[off]
        x = int.from_bytes(d[off + 1:off + 33], "little")
        y = int.from_bytes(d[off + 33:off + 65], "little")
        off += 65
        return None if inf else (x, y)
    def g2():
        nonlocal off
        inf = d[off]
        v = [int.from_bytes(d[off + 1 + 32 * i:off + 33 + 32 * i], "little") for i in range(4)]
        off += 129
        return None if inf else ((v[0], v[1]), (v[2], v[3]))
    def vec(f):
        nonlocal off
        (k,) = struct.unpack_from("<i", d, off)
        off += 4
        return [f() for _ in range(k)]
    hdr = dict(ver=ver, n=n, m=m, npub=npub)
    fixed = [g1(), g1(), g1(), g2(), g2(), g2()]
    vecs = [vec(g1), vec(g2), vec(g1), vec(g1), vec(g2), vec(g1), vec(g1)]
    assert off == len(d)
    return hdr, fixed, vecs


def parse_vk(data):
    """VK file (src/verifier/verifier.cu:103-148)."""
    import struct
    (npub,) = struct.unpack_from("<i", data, 0)
    off = 4
    alpha = _g1_std(data, off)
    off += 64
    g2s = []
    for _ in range(3):
        g2s.append(_g2_std(data, off))
        off += 128
    (nic,) = struct.unpack_from("<i", data, off)
    off += 4
    ic = []
    for _ in range(nic):
        ic.append(_g1_std(data, off))
        off += 64
    assert off == len(data)
    return dict(num_public=npub, alpha_g1=alpha, beta_g2=g2s[0], gamma_g2=g2s[1], delta_g2=g2s[2], ic=ic)


def check_keys(circ, pk_parsed, vk_data, tw):
    """Compare a parsed ZKMLPK3 key and a VK image with the closed forms.
    pk_parsed = (hdr, fixed, vecs) as tests/test_oracle.py's parse_zkmlpk3.
    Returns the list of mismatching entry names (empty when all agree)."""
    ks = key_scalars(circ, tw)
    hdr, fixed, vecs = pk_parsed
    bad = []
    if (hdr["n"], hdr["m"], hdr["npub"]) != (ks["n"], circ.nv, circ.npub):
        bad.append("header")
    want_fixed = [g1(ks["alpha_g1"]), g1(ks["beta_g1"]), g1(ks["delta_g1"]), g2(ks["beta_g2"]),
                  g2(ks["gamma_g2"]), g2(ks["delta_g2"])]
    for name, got, want in zip(("alpha_g1", "beta_g1", "delta_g1", "beta_g2", "gamma_g2", "delta_g2"),
                               fixed, want_fixed):
        if got != want:
            bad.append(name)
    tau_g1, tau_g2, A, B1, B2, L, H = vecs
    if tau_g1 != []:
        bad.append("tau_g1")
    if tau_g2 != [g2(k) for k in ks["tau_g2"]]:
        bad.append("tau_g2")
    for name, got, scal, mul in (("A", A, ks["A"], g1), ("B1", B1, ks["B1"], g1), ("B2", B2, ks["B2"], g2),
                                 ("L", L, ks["L"], g1), ("H", H, ks["H"], g1)):
        if len(got) != len(scal):
            bad.append(name + " length")
            continue
        for i, (p, k) in enumerate(zip(got, scal)):
            if p != mul(k):
                bad.append(f"{name}[{i}]")
                break
    vk = parse_vk(vk_data)
    if vk["num_public"] != circ.npub:
        bad.append("vk npub")
    if vk["alpha_g1"] != want_fixed[0] or vk["beta_g2"] != want_fixed[3]:
        bad.append("vk alpha/beta")
    if vk["gamma_g2"] != want_fixed[4] or vk["delta_g2"] != want_fixed[5]:
        bad.append("vk gamma/delta")
    if vk["ic"] != [g1(k) for k in ks["ic"]]:
        bad.append("vk ic")
    return bad


def check_proof(circ, proof, tw, r, s):
    """Mismatching proof elements (empty list when A, B, C equal the closed forms)."""
    a, b, c = proof_scalars(circ, tw, r, s)
    A, B, C = parse_proof(proof)
    bad = []
    if A != g1(a):
        bad.append("A")
    if B != g2(b):
        bad.append("B")
    if C != g1(c):
        bad.append("C")
    return bad
