// Host BN254 optimal ate pairing and the Groth16 verification equation.
//
// Replaces bn254::pairing / verify_pairing_product (reference
// src/curve/pairing.cuh:198-282) and Groth16Verifier::verify
// (src/prover/groth16.cu:967-1022).  Same tower as the reference
// (src/field/fp6.cuh, fp12.cuh): Fq6 = Fq2[v]/(v^3 - xi), xi = 9 + u,
// Fq12 = Fq6[w]/(w^2 - v), so a value of e(P, Q) can be compared
// coefficient by coefficient.
//
// Own construction, from the mathematics:
//  - Miller loop over the binary expansion of 6x + 2 (x = 4965661367192848881)
//    with affine line functions on the D-type twist E': y^2 = x^3 + 3/xi.  The
//    untwist psi(x', y') = (x' w^2, y' w^3) turns the line through T, Q with
//    slope l (on E') evaluated at P = (xP, yP) into
//        yP - l xP w + (l xT - yT) w^3,
//    a sparse Fq12 element.  Vertical lines lie in Fq6 and are dropped
//    (the final exponentiation maps Fq6* to 1).
//  - the two extra optimal-ate lines with pi(Q) and -pi^2(Q), where the
//    Frobenius on the twist is (x', y') -> (conj(x') g^2, conj(y') g^3),
//    g = xi^((p-1)/6), computed at first use.
//  - final exponentiation (p^12 - 1)/r as the easy part
//    (p^6 - 1)(p^2 + 1) (conjugation, one inversion, Frobenius) times a plain
//    square-and-multiply by (p^4 - p^2 + 1)/r.
// Any correct evaluation of the reduced optimal ate pairing gives the same
// element of GT, since line scalings by subfield elements and vertical lines
// vanish under the final exponentiation.
//
// Host code: a verification is a few thousand Fq12 operations, serial.
#pragma once
#include <stdint.h>
#include <string.h>

#include <vector>

#include "host_bn254.hpp"

namespace zkh {

// ------------------------------------------------------------------ Fq2 extras
inline Fq2 f2_conj(const Fq2& a) { return Fq2{a.c0, -a.c1}; }
inline Fq2 f2_mul_fq(const Fq2& a, const Fq& s) { return Fq2{a.c0 * s, a.c1 * s}; }
// (9 + u) a
inline Fq2 f2_mul_xi(const Fq2& a) {
  const Fq nine = Fq::from_u64(9);
  return Fq2{nine * a.c0 - a.c1, a.c0 + nine * a.c1};
}
inline Fq2 f2_pow(const Fq2& a, const uint64_t* e, int words) {
  Fq2 r = Fq2::one();
  for (int i = words * 64 - 1; i >= 0; i--) {
    r = r.sqr();
    if ((e[i >> 6] >> (i & 63)) & 1) r = r * a;
  }
  return r;
}

// ------------------------------------------------------------------ Fq6
struct Fq6 {
  Fq2 c0, c1, c2;
  static Fq6 zero() { return Fq6{Fq2::zero(), Fq2::zero(), Fq2::zero()}; }
  static Fq6 one() { return Fq6{Fq2::one(), Fq2::zero(), Fq2::zero()}; }
  bool operator==(const Fq6& o) const { return c0 == o.c0 && c1 == o.c1 && c2 == o.c2; }
  Fq6 operator+(const Fq6& o) const { return Fq6{c0 + o.c0, c1 + o.c1, c2 + o.c2}; }
  Fq6 operator-(const Fq6& o) const { return Fq6{c0 - o.c0, c1 - o.c1, c2 - o.c2}; }
  Fq6 operator-() const { return Fq6{-c0, -c1, -c2}; }
  Fq6 operator*(const Fq6& o) const {
    const Fq2 t0 = c0 * o.c0, t1 = c1 * o.c1, t2 = c2 * o.c2;
    return Fq6{t0 + f2_mul_xi((c1 + c2) * (o.c1 + o.c2) - t1 - t2),
               (c0 + c1) * (o.c0 + o.c1) - t0 - t1 + f2_mul_xi(t2),
               (c0 + c2) * (o.c0 + o.c2) - t0 - t2 + t1};
  }
  // times v: (c0 + c1 v + c2 v^2) v = xi c2 + c0 v + c1 v^2
  Fq6 mul_v() const { return Fq6{f2_mul_xi(c2), c0, c1}; }
  Fq6 inv() const {
    const Fq2 A = c0.sqr() - f2_mul_xi(c1 * c2);
    const Fq2 B = f2_mul_xi(c2.sqr()) - c0 * c1;
    const Fq2 C = c1.sqr() - c0 * c2;
    const Fq2 Fi = (c0 * A + f2_mul_xi(c2 * B + c1 * C)).inv();
    return Fq6{A * Fi, B * Fi, C * Fi};
  }
};

// ------------------------------------------------------------------ Fq12
struct Fq12 {
  Fq6 c0, c1;
  static Fq12 one() { return Fq12{Fq6::one(), Fq6::zero()}; }
  bool operator==(const Fq12& o) const { return c0 == o.c0 && c1 == o.c1; }
  Fq12 operator*(const Fq12& o) const {
    const Fq6 t0 = c0 * o.c0, t1 = c1 * o.c1;
    return Fq12{t0 + t1.mul_v(), (c0 + c1) * (o.c0 + o.c1) - t0 - t1};
  }
  Fq12 sqr() const { return *this * *this; }
  Fq12 conj() const { return Fq12{c0, -c1}; }
  Fq12 inv() const {
    const Fq6 n = (c0 * c0 - (c1 * c1).mul_v()).inv();
    return Fq12{c0 * n, -(c1 * n)};
  }
};

// g^k for g = xi^((p-1)/6), k = 0..5 (Frobenius on Fq12 and on the twist)
struct FrobConsts {
  Fq2 g[6];
  FrobConsts() {
    // (p - 1) / 6
    static const uint64_t e[4] = {0x34B017592414D4E1ULL, 0xEE9591C2E6BDA1C2ULL, 0xF40D60F3C0403964ULL,
                                  0x0810B7BDD032F006ULL};
    const Fq2 xi{Fq::from_u64(9), Fq::from_u64(1)};
    g[0] = Fq2::one();
    g[1] = f2_pow(xi, e, 4);
    for (int k = 2; k < 6; k++) g[k] = g[k - 1] * g[1];
  }
};
inline const FrobConsts& frob_consts() {
  static const FrobConsts c;
  return c;
}

// f^p: every Fq2 coefficient of w^k is conjugated and multiplied by g^k
// (w^p = w * xi^((p-1)/6) since w^6 = xi).
inline Fq12 frobenius(const Fq12& f) {
  const FrobConsts& k = frob_consts();
  return Fq12{Fq6{f2_conj(f.c0.c0), f2_conj(f.c0.c1) * k.g[2], f2_conj(f.c0.c2) * k.g[4]},
              Fq6{f2_conj(f.c1.c0) * k.g[1], f2_conj(f.c1.c1) * k.g[3], f2_conj(f.c1.c2) * k.g[5]}};
}

// ------------------------------------------------------------------ Miller loop
struct G1A {
  Fq x, y;
  bool inf;
};
struct G2A {
  Fq2 x, y;
  bool inf;
};

// line with slope l through (xT, yT) on E', evaluated at P:
// yP - l xP w + (l xT - yT) w^3
inline Fq12 line_at(const Fq2& l, const Fq2& xT, const Fq2& yT, const G1A& P) {
  return Fq12{Fq6{Fq2{P.y, Fq::zero()}, Fq2::zero(), Fq2::zero()},
              Fq6{-f2_mul_fq(l, P.x), l * xT - yT, Fq2::zero()}};
}

// f *= line through T and Q (tangent when T == Q); T = T + Q.  Affine
// coordinates on the twist.
inline void miller_add(Fq12& f, G2A& T, const G2A& Q, const G1A& P) {
  if (T.inf) {
    T = Q;
    return;
  }
  if (Q.inf) return;
  Fq2 l;
  if (T.x == Q.x) {
    if (!(T.y == Q.y) || T.y.is_zero()) {  // vertical line: drop it, T + Q = O
      T.inf = true;
      return;
    }
    const Fq2 x2 = T.x.sqr();
    l = (x2 + x2 + x2) * (T.y + T.y).inv();
  } else {
    l = (Q.y - T.y) * (Q.x - T.x).inv();
  }
  f = f * line_at(l, T.x, T.y, P);
  const Fq2 x3 = l.sqr() - T.x - Q.x;
  const Fq2 y3 = l * (T.x - x3) - T.y;
  T.x = x3;
  T.y = y3;
}

inline Fq12 miller_loop(const G1A& P, const G2A& Q) {
  if (P.inf || Q.inf) return Fq12::one();
  const uint64_t ate = 0x9D797039BE763BA8ULL;  // 6x + 2 = 0x1_9D797039BE763BA8 (65 bits)
  Fq12 f = Fq12::one();
  G2A T = Q;
  for (int i = 63; i >= 0; i--) {  // bit 64 is the leading one
    f = f.sqr();
    G2A T0 = T;
    miller_add(f, T, T0, P);
    if ((ate >> i) & 1) miller_add(f, T, Q, P);
  }
  const FrobConsts& k = frob_consts();
  G2A q1{f2_conj(Q.x) * k.g[2], f2_conj(Q.y) * k.g[3], false};
  G2A q2{f2_conj(q1.x) * k.g[2], f2_conj(q1.y) * k.g[3], false};
  q2.y = -q2.y;
  miller_add(f, T, q1, P);
  miller_add(f, T, q2, P);
  return f;
}

inline Fq12 final_exponentiation(const Fq12& f) {
  // easy part: f^((p^6 - 1)(p^2 + 1))
  Fq12 t = f.conj() * f.inv();
  t = frobenius(frobenius(t)) * t;
  // hard part: (p^4 - p^2 + 1) / r, 761 bits, little-endian words
  static const uint64_t h[12] = {0xE81BB482CCDF42B1ULL, 0x5ABF5CC4F49C36D4ULL, 0xF1154E7E1DA014FDULL,
                                 0xDCC7B44C87CDBACFULL, 0xAAA441E3954BCF8AULL, 0x6B887D56D5095F23ULL,
                                 0x79581E16F3FD90C6ULL, 0x3B1B1355D189227DULL, 0x4E529A5861876F6BULL,
                                 0x6C0EB522D5B12278ULL, 0x331EC15183177FAFULL, 0x01BAAA710B0759ADULL};
  Fq12 r = Fq12::one();
  for (int i = 12 * 64 - 1; i >= 0; i--) {
    r = r.sqr();
    if ((h[i >> 6] >> (i & 63)) & 1) r = r * t;
  }
  return r;
}

inline Fq12 pairing(const G1A& P, const G2A& Q) { return final_exponentiation(miller_loop(P, Q)); }

// ------------------------------------------------------------------ checks
inline bool g1_on_curve(const G1A& P) {
  return P.inf || P.y.sqr() == P.x.sqr() * P.x + Fq::from_u64(3);
}
inline Fq2 twist_b() {  // 3 / (9 + u)
  return f2_mul_fq(Fq2{Fq::from_u64(9), Fq::from_u64(1)}.inv(), Fq::from_u64(3));
}
inline bool g2_on_curve(const G2A& Q) { return Q.inf || Q.y.sqr() == Q.x.sqr() * Q.x + twist_b(); }

// r * Q == O (the proof's B must lie in the order-r subgroup of E'(Fq2)).
inline bool g2_in_subgroup(const G2A& Q) {
  if (Q.inf) return true;
  Jac<Fq2> J = Jac<Fq2>::affine(Q.x, Q.y);
  uint64_t rr[4];
  memcpy(rr, RMod::M, 32);
  return J.mul_std(rr).is_inf();
}

// ------------------------------------------------------------------ Groth16
struct VerifyingKey {
  int npub = 0;
  G1A alpha;
  G2A beta, gamma, delta;
  std::vector<G1A> ic;
};

// e(-A, B) e(alpha, beta) e(vk_x, gamma) e(C, delta) == 1 with
// vk_x = IC[0] + sum_i pub_i IC[i + 1] (groth16.cu:967-1022).  pub: standard
// form scalars.  A wrong public-input count rejects, as in the reference.
inline bool groth16_verify(const VerifyingKey& vk, const G1A& A, const G2A& B, const G1A& C,
                           const std::vector<std::vector<uint64_t>>& pub) {
  if ((int)pub.size() != vk.npub || vk.ic.empty()) return false;
  if (!g1_on_curve(A) || !g1_on_curve(C) || !g2_on_curve(B) || !g2_in_subgroup(B)) return false;
  G1 acc = vk.ic[0].inf ? G1::inf() : G1::affine(vk.ic[0].x, vk.ic[0].y);
  for (size_t i = 0; i < pub.size(); i++) {
    if (i + 1 >= vk.ic.size() || vk.ic[i + 1].inf) continue;
    acc = acc.add(G1::affine(vk.ic[i + 1].x, vk.ic[i + 1].y).mul_std(pub[i].data()));
  }
  G1A vkx;
  vkx.inf = acc.is_inf();
  if (!vkx.inf) acc.to_affine(vkx.x, vkx.y);
  const G1A negA{A.x, -A.y, A.inf};
  Fq12 f = miller_loop(negA, B) * miller_loop(vk.alpha, vk.beta) * miller_loop(vkx, vk.gamma) *
           miller_loop(C, vk.delta);
  return final_exponentiation(f) == Fq12::one();
}

}  // namespace zkh
