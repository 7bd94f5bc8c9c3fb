"""Seeded R1CS + witness generators for the tests (Python big integers).

* mul_circuit(x, y): the reference's own Groth16 test circuit
  (tests/test_groth16.cu:19-56): witness [1, z(public), x, y], a dummy
  constraint w0*w0 = w0 and x*y = z.
* random_r1cs(rows, inputs, npub, seed): the BASELINE config-5 shape at small
  scale -- each row i has <= 3 random-coefficient terms in A and B over earlier
  variables and C = one fresh variable set to (A.w)(B.w), so the witness
  satisfies the system row by row.

Matrices are returned as (rows, cols, values-as-Montgomery-words) triples.
"""
import random

import numpy as np

from zkpy import R, fr_words


class Circuit:
    def __init__(self, nc, nv, npub, npriv, A, B, C, w):
        self.nc, self.nv, self.npub, self.npriv = nc, nv, npub, npriv
        self.A, self.B, self.C = A, B, C
        self.w = w  # list of ints (standard form)

    def mats(self):
        out = []
        for M in (self.A, self.B, self.C):
            rows = np.array([e[0] for e in M], dtype=np.int32)
            cols = np.array([e[1] for e in M], dtype=np.int32)
            vals = np.array([fr_words(e[2]) for e in M], dtype=np.uint64).reshape(-1, 4)
            out.append((rows, cols, vals))
        return out

    def witness_words(self):
        return np.array([fr_words(v) for v in self.w], dtype=np.uint64).reshape(-1, 4)

    def public(self):
        return self.w[1:1 + self.npub]

    def row_values(self, n):
        """(A.w, B.w, C.w) per row, zero-padded to n rows."""
        out = []
        for M in (self.A, self.B, self.C):
            v = [0] * n
            for r, c, a in M:
                if r < n:
                    v[r] = (v[r] + a * self.w[c]) % R
            out.append(v)
        return out


def mul_circuit(x=7, y=9):
    z = x * y % R
    A = [(0, 0, 1), (1, 2, 1)]
    B = [(0, 0, 1), (1, 3, 1)]
    C = [(0, 0, 1), (1, 1, 1)]
    return Circuit(2, 4, 1, 2, A, B, C, [1, z, x, y])


def random_r1cs(rows, inputs=8, npub=3, seed=1, small_frac=0.0):
    """small_frac: fraction of input values drawn below 2^16 (witness-like)."""
    rng = random.Random(seed)
    w = [1]
    for _ in range(inputs):
        w.append(rng.randrange(1 << 16) if rng.random() < small_frac else rng.randrange(R))
    A, B, C = [], [], []
    for i in range(rows):
        nvars = len(w)
        a_terms = [(rng.randrange(nvars), rng.randrange(1, R)) for _ in range(rng.randint(1, 3))]
        b_terms = [(rng.randrange(nvars), rng.randrange(1, R)) for _ in range(rng.randint(1, 3))]
        av = sum(c * w[v] for v, c in a_terms) % R
        bv = sum(c * w[v] for v, c in b_terms) % R
        out = len(w)
        w.append(av * bv % R)
        A += [(i, v, c) for v, c in a_terms]
        B += [(i, v, c) for v, c in b_terms]
        C.append((i, out, 1))
    nv = len(w)
    return Circuit(rows, nv, npub, inputs - npub, A, B, C, w)
