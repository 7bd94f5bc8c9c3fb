"""Pure-Python BN254 arithmetic used by the tests to pin the oracle and the
GPU path with closed forms (Python big integers, independent of any C code).

Only small amounts of work go through here (a few hundred group operations):
it is the mathematics, not a third implementation to race against.
"""
import random

P = 0x30644E72E131A029B85045B68181585D97816A916871CA8D3C208C16D87CFD47
R = 0x30644E72E131A029B85045B68181585D2833E84879B9709143E1F593F0000001
MONT = 1 << 256

# EIP-197 generator of G2 (standard form), G1 generator (1, 2)
G1 = (1, 2)
G2 = ((10857046999023057135944570762232829481370756359578518086990519993285655852781,
       11559732032986387107991004021392285783925812861821192530917403151452391805634),
      (8495653923123431417604973247489272438418190587263600148770280649306958101930,
       4082367875863433681332203403145435568316851327593401208105741076214120093531))


def to_mont(x, m):
    return x * MONT % m


def from_mont(x, m):
    return x * pow(MONT, -1, m) % m


def limbs(x, n=4):
    return [(x >> (64 * i)) & ((1 << 64) - 1) for i in range(n)]


def from_limbs(ws):
    return sum(int(w) << (64 * i) for i, w in enumerate(ws))


# ----------------------------------------------------------------- Fq2
def f2_add(a, b):
    return ((a[0] + b[0]) % P, (a[1] + b[1]) % P)


def f2_sub(a, b):
    return ((a[0] - b[0]) % P, (a[1] - b[1]) % P)


def f2_mul(a, b):
    return ((a[0] * b[0] - a[1] * b[1]) % P, (a[0] * b[1] + a[1] * b[0]) % P)


def f2_inv(a):
    n = pow((a[0] * a[0] + a[1] * a[1]) % P, P - 2, P)
    return (a[0] * n % P, (-a[1]) * n % P)


# ----------------------------------------------------------------- affine groups
# Points are tuples (x, y) in standard form, None = infinity.
class _G:
    def __init__(self, add, sub, mul, inv, zero, three):
        self.add, self.sub, self.mul, self.inv, self.zero, self.three = add, sub, mul, inv, zero, three

    def padd(self, p, q):
        if p is None:
            return q
        if q is None:
            return p
        if p[0] == q[0]:
            if p[1] == q[1] and p[1] != self.zero:
                lam = self.mul(self.mul(self.three, self.mul(p[0], p[0])), self.inv(self.add(p[1], p[1])))
            else:
                return None
        else:
            lam = self.mul(self.sub(q[1], p[1]), self.inv(self.sub(q[0], p[0])))
        x3 = self.sub(self.sub(self.mul(lam, lam), p[0]), q[0])
        y3 = self.sub(self.mul(lam, self.sub(p[0], x3)), p[1])
        return (x3, y3)

    def pmul(self, p, k):
        k %= R
        acc = None
        while k:
            if k & 1:
                acc = self.padd(acc, p)
            p = self.padd(p, p)
            k >>= 1
        return acc

    def pneg(self, p):
        if p is None:
            return None
        return (p[0], self.sub(self.zero, p[1]))


g1 = _G(lambda a, b: (a + b) % P, lambda a, b: (a - b) % P, lambda a, b: a * b % P,
        lambda a: pow(a, P - 2, P), 0, 3)
g2 = _G(f2_add, f2_sub, f2_mul, f2_inv, (0, 0), (3, 0))


def g1_on_curve(p):
    return p is None or (p[1] * p[1] - p[0] ** 3 - 3) % P == 0


# ----------------------------------------------------------------- layouts
# Interchange layout (the reference's in-memory form without the bool flag):
#   Fr/Fq: 4 x u64 LE Montgomery (R = 2^256); G1 affine 8 u64; G2 16 u64;
#   infinity = all-zero words.
def g1_to_words(p):
    if p is None:
        return [0] * 8
    return limbs(to_mont(p[0], P)) + limbs(to_mont(p[1], P))


def g1_from_words(w):
    w = [int(x) for x in w]
    if not any(w):
        return None
    return (from_mont(from_limbs(w[:4]), P), from_mont(from_limbs(w[4:8]), P))


def g2_to_words(p):
    if p is None:
        return [0] * 16
    return (limbs(to_mont(p[0][0], P)) + limbs(to_mont(p[0][1], P)) +
            limbs(to_mont(p[1][0], P)) + limbs(to_mont(p[1][1], P)))


def g2_from_words(w):
    w = [int(x) for x in w]
    if not any(w):
        return None
    v = [from_mont(from_limbs(w[4 * i:4 * i + 4]), P) for i in range(4)]
    return ((v[0], v[1]), (v[2], v[3]))


def fr_words(x):
    return limbs(to_mont(x % R, R))


def fr_from_words(w):
    return from_mont(from_limbs([int(v) for v in w]), R)


# ----------------------------------------------------------------- NTT closed forms
OMEGA28 = pow(5, (R - 1) >> 28, R)


def omega(log_n):
    return pow(OMEGA28, 1 << (28 - log_n), R)


def dft(vals, w):
    n = len(vals)
    return [sum(v * pow(w, i * j, R) for j, v in enumerate(vals)) % R for i in range(n)]


def poly_eval(coeffs, x):
    acc = 0
    for c in reversed(coeffs):
        acc = (acc * x + c) % R
    return acc


def rand_fr(rng: random.Random):
    return rng.randrange(R)
