// Host-side BN254 arithmetic for the serial tails of the prover: MSM window
// combination (W*c doublings), affine conversion, the r/s blinding scalar
// multiplications of Groth16Prover::prove (reference src/prover/groth16.cu:
// 769-840) and file encodings.  A CPU core finishes a serial field multiply
// far sooner than a single wave64, so these chains stay on the host.
//
// Representation: the reference's 4 x u64 Montgomery form (R = 2^256),
// multiplied with CIOS and one conditional subtraction, as in
// src/field/montgomery.cuh:330-368.  Values are always canonical.
#pragma once
#include <stdint.h>
#include <string.h>
#include <x86intrin.h>

namespace zkh {

typedef unsigned __int128 u128;

struct QMod {
  static constexpr uint64_t M[4] = {0x3C208C16D87CFD47ULL, 0x97816A916871CA8DULL, 0xB85045B68181585DULL,
                                    0x30644E72E131A029ULL};
  static constexpr uint64_t INV = 0x87D20782E4866389ULL;
  static constexpr uint64_t ONE[4] = {0xD35D438DC58F0D9DULL, 0x0A78EB28F5C70B3DULL, 0x666EA36F7879462CULL,
                                      0x0E0A77C19A07DF2FULL};
  static constexpr uint64_t R2[4] = {0xF32CFC5B538AFA89ULL, 0xB5E71911D44501FBULL, 0x47AB1EFF0A417FF6ULL,
                                     0x06D89F71CAB8351FULL};
};
struct RMod {
  static constexpr uint64_t M[4] = {0x43E1F593F0000001ULL, 0x2833E84879B97091ULL, 0xB85045B68181585DULL,
                                    0x30644E72E131A029ULL};
  static constexpr uint64_t INV = 0xC2E1F593EFFFFFFFULL;
  static constexpr uint64_t ONE[4] = {0xAC96341C4FFFFFFBULL, 0x36FC76959F60CD29ULL, 0x666EA36F7879462EULL,
                                      0x0E0A77C19A07DF2FULL};
  static constexpr uint64_t R2[4] = {0x1BB8E645AE216DA7ULL, 0x53FE3AB1E35C59E3ULL, 0x8C49833D53BB8085ULL,
                                     0x0216D0B17F4E44A5ULL};
};

template <class M>
struct F {
  uint64_t v[4];

  static F zero() { return F{{0, 0, 0, 0}}; }
  static F one() { return F{{M::ONE[0], M::ONE[1], M::ONE[2], M::ONE[3]}}; }
  static F raw(const void* p) {
    F r;
    memcpy(r.v, p, 32);
    return r;
  }
  bool is_zero() const { return (v[0] | v[1] | v[2] | v[3]) == 0; }
  bool operator==(const F& o) const { return memcmp(v, o.v, 32) == 0; }

  // r = t - m when t >= m, else t: a carry chain and a mask select (the
  // outcome is data dependent, so a branch would mispredict half the time).
  static inline void csub(uint64_t* r, uint64_t t0, uint64_t t1, uint64_t t2, uint64_t t3) {
    unsigned long long s0, s1, s2, s3;
    unsigned char b = _subborrow_u64(0, t0, M::M[0], &s0);
    b = _subborrow_u64(b, t1, M::M[1], &s1);
    b = _subborrow_u64(b, t2, M::M[2], &s2);
    b = _subborrow_u64(b, t3, M::M[3], &s3);
    const uint64_t keep = 0 - (uint64_t)b;  // all ones when t < m
    r[0] = (t0 & keep) | (s0 & ~keep);
    r[1] = (t1 & keep) | (s1 & ~keep);
    r[2] = (t2 & keep) | (s2 & ~keep);
    r[3] = (t3 & keep) | (s3 & ~keep);
  }
  // Montgomery product a b 2^-256 mod m, CIOS without the extra carry word:
  // both moduli have a top limb below 2^62, so the running value stays
  // below 2m < 2^256 after every outer step (Gautam, Kumar, Tomescu et al.,
  // "Faster Montgomery multiplication ... for SNARKs", 2023, the "no-carry"
  // condition).  One conditional subtraction at the end.
  static inline void mont(uint64_t* r, const uint64_t* a, const uint64_t* b) {
    uint64_t t0 = 0, t1 = 0, t2 = 0, t3 = 0;
    for (int i = 0; i < 4; i++) {
      const uint64_t bi = b[i];
      u128 x = (u128)a[0] * bi + t0;
      const uint64_t lo = (uint64_t)x;
      uint64_t A = (uint64_t)(x >> 64);
      const uint64_t m = lo * M::INV;
      u128 y = (u128)m * M::M[0] + lo;
      uint64_t C = (uint64_t)(y >> 64);
      x = (u128)a[1] * bi + t1 + A;
      A = (uint64_t)(x >> 64);
      y = (u128)m * M::M[1] + (uint64_t)x + C;
      C = (uint64_t)(y >> 64);
      t0 = (uint64_t)y;
      x = (u128)a[2] * bi + t2 + A;
      A = (uint64_t)(x >> 64);
      y = (u128)m * M::M[2] + (uint64_t)x + C;
      C = (uint64_t)(y >> 64);
      t1 = (uint64_t)y;
      x = (u128)a[3] * bi + t3 + A;
      A = (uint64_t)(x >> 64);
      y = (u128)m * M::M[3] + (uint64_t)x + C;
      C = (uint64_t)(y >> 64);
      t2 = (uint64_t)y;
      t3 = C + A;
    }
    csub(r, t0, t1, t2, t3);
  }
  F operator*(const F& o) const {
    F r;
    mont(r.v, v, o.v);
    return r;
  }
  F sqr() const { return *this * *this; }
  // sums stay below 2^256 since 2m < 2^255
  F operator+(const F& o) const {
    unsigned long long s0, s1, s2, s3;
    unsigned char c = _addcarry_u64(0, v[0], o.v[0], &s0);
    c = _addcarry_u64(c, v[1], o.v[1], &s1);
    c = _addcarry_u64(c, v[2], o.v[2], &s2);
    (void)_addcarry_u64(c, v[3], o.v[3], &s3);
    F r;
    csub(r.v, s0, s1, s2, s3);
    return r;
  }
  F operator-(const F& o) const {
    unsigned long long d0, d1, d2, d3, r0, r1, r2, r3;
    unsigned char b = _subborrow_u64(0, v[0], o.v[0], &d0);
    b = _subborrow_u64(b, v[1], o.v[1], &d1);
    b = _subborrow_u64(b, v[2], o.v[2], &d2);
    b = _subborrow_u64(b, v[3], o.v[3], &d3);
    const uint64_t mask = 0 - (uint64_t)b;  // add m back after a borrow
    unsigned char c = _addcarry_u64(0, d0, M::M[0] & mask, &r0);
    c = _addcarry_u64(c, d1, M::M[1] & mask, &r1);
    c = _addcarry_u64(c, d2, M::M[2] & mask, &r2);
    (void)_addcarry_u64(c, d3, M::M[3] & mask, &r3);
    return F{{r0, r1, r2, r3}};
  }
  F operator-() const { return zero() - *this; }
  F dbl() const { return *this + *this; }
  static F from_std(const uint64_t* s) {
    F r;
    mont(r.v, s, M::R2);
    return r;
  }
  // The integer of nine 29-bit limbs (the device kernels' form of an element,
  // x 2^261 mod m, below 2^261) reduced mod m, taken as this type's
  // Montgomery word: it stands for x 2^5.  A ratio of two such values
  // (X / ZZ, Y / ZZZ of an XYZZ point) is then exact with no radix
  // conversion, the 2^5 cancelling.
  static F from_limbs29_scaled(const uint32_t* l) {
    uint64_t w[5] = {0, 0, 0, 0, 0};
    for (int i = 0; i < 9; i++) {
      const int bit = 29 * i, wd = bit >> 6, sh = bit & 63;
      w[wd] |= (uint64_t)l[i] << sh;
      if (sh > 64 - 29) w[wd + 1] |= (uint64_t)l[i] >> (64 - sh);
    }
    // below 2^261 < 256 m: subtract m 2^k where it fits, k = 7 .. 0
    for (int k = 7; k >= 0; k--) {
      uint64_t mk[5], d[5];
      mk[4] = k ? M::M[3] >> (64 - k) : 0;
      for (int j = 3; j >= 1; j--) mk[j] = k ? (M::M[j] << k) | (M::M[j - 1] >> (64 - k)) : M::M[j];
      mk[0] = M::M[0] << k;
      unsigned char b = 0;
      for (int j = 0; j < 5; j++) {
        unsigned long long t;
        b = _subborrow_u64(b, w[j], mk[j], &t);
        d[j] = t;
      }
      if (!b) memcpy(w, d, sizeof(d));
    }
    F r;
    memcpy(r.v, w, 32);
    return r;
  }
  static F from_u64(uint64_t x) {
    uint64_t s[4] = {x, 0, 0, 0};
    return from_std(s);
  }
  void to_std(uint64_t* out) const {
    uint64_t one[4] = {1, 0, 0, 0};
    mont(out, v, one);
  }
  F pow(const uint64_t* e) const {
    F r = one();
    for (int i = 255; i >= 0; i--) {
      r = r.sqr();
      if ((e[i >> 6] >> (i & 63)) & 1) r = r * *this;
    }
    return r;
  }
  F inv() const {
    uint64_t e[4] = {M::M[0] - 2, M::M[1], M::M[2], M::M[3]};
    return pow(e);
  }
};

typedef F<QMod> Fq;
typedef F<RMod> Fr;

struct Fq2 {
  Fq c0, c1;
  static Fq2 zero() { return Fq2{Fq::zero(), Fq::zero()}; }
  static Fq2 one() { return Fq2{Fq::one(), Fq::zero()}; }
  bool is_zero() const { return c0.is_zero() && c1.is_zero(); }
  bool operator==(const Fq2& o) const { return c0 == o.c0 && c1 == o.c1; }
  Fq2 operator+(const Fq2& o) const { return Fq2{c0 + o.c0, c1 + o.c1}; }
  Fq2 operator-(const Fq2& o) const { return Fq2{c0 - o.c0, c1 - o.c1}; }
  Fq2 operator-() const { return Fq2{-c0, -c1}; }
  Fq2 operator*(const Fq2& o) const {
    Fq a = c0 * o.c0, b = c1 * o.c1;
    return Fq2{a - b, (c0 + c1) * (o.c0 + o.c1) - a - b};
  }
  // (a + b u)^2 = (a + b)(a - b) + 2ab u  (u^2 = -1)
  Fq2 sqr() const {
    const Fq ab = c0 * c1;
    return Fq2{(c0 + c1) * (c0 - c1), ab + ab};
  }
  Fq2 dbl() const { return *this + *this; }
  Fq2 inv() const {
    Fq n = (c0.sqr() + c1.sqr()).inv();
    return Fq2{c0 * n, -(c1 * n)};
  }
};

// Jacobian point (x = X/Z^2, y = Y/Z^3), Z = 0 at infinity.
template <class E>
struct Jac {
  E x, y, z;
  static Jac inf() { return Jac{E::zero(), E::one(), E::zero()}; }
  bool is_inf() const { return z.is_zero(); }
  static Jac affine(const E& x, const E& y) { return Jac{x, y, E::one()}; }
  Jac dbl() const {
    if (is_inf()) return *this;
    E a = x.sqr(), b = y.sqr(), c = b.sqr();
    E d = ((x + b).sqr() - a - c).dbl();
    E e = a.dbl() + a;
    E f = e.sqr();
    Jac r;
    r.x = f - d.dbl();
    r.y = e * (d - r.x) - c.dbl().dbl().dbl();
    r.z = (y * z).dbl();
    return r;
  }
  // Sum with a point whose z is one (an affine point): z2 = 1 drops three
  // multiplications and a squaring from the general formula below.
  Jac add_mixed(const Jac& o) const {
    if (is_inf()) return o;
    const E z1z1 = z.sqr();
    const E u2 = o.x * z1z1, s2 = o.y * (z * z1z1);
    const E h = u2 - x, rr = s2 - y;
    if (h.is_zero()) return rr.is_zero() ? dbl() : inf();
    const E hh = h.sqr(), hhh = hh * h, v = x * hh;
    Jac r;
    r.x = rr.sqr() - hhh - v.dbl();
    r.y = rr * (v - r.x) - y * hhh;
    r.z = z * h;
    return r;
  }
  Jac add(const Jac& o) const {
    if (is_inf()) return o;
    if (o.is_inf()) return *this;
    if (o.z == E::one()) return add_mixed(o);
    if (z == E::one()) return o.add_mixed(*this);
    E z1z1 = z.sqr(), z2z2 = o.z.sqr();
    E u1 = x * z2z2, u2 = o.x * z1z1;
    E s1 = y * o.z * z2z2, s2 = o.y * z * z1z1;
    E h = u2 - u1, rr = s2 - s1;
    if (h.is_zero()) return rr.is_zero() ? dbl() : inf();
    E hh = h.sqr(), hhh = hh * h, v = u1 * hh;
    Jac r;
    r.x = rr.sqr() - hhh - v.dbl();
    r.y = rr * (v - r.x) - s1 * hhh;
    r.z = z * o.z * h;
    return r;
  }
  Jac neg() const { return Jac{x, -y, z}; }
  // k given as 4 little-endian u64 words in standard form
  Jac mul_std(const uint64_t* k) const {
    Jac r = inf();
    int top = -1;
    for (int i = 255; i >= 0; i--)
      if ((k[i >> 6] >> (i & 63)) & 1) {
        top = i;
        break;
      }
    for (int i = top; i >= 0; i--) {
      r = r.dbl();
      if ((k[i >> 6] >> (i & 63)) & 1) r = r.add(*this);
    }
    return r;
  }
  Jac mul(const Fr& k) const {
    uint64_t s[4];
    k.to_std(s);
    return mul_std(s);
  }
  // a P + b Q with one chain of doublings (Shamir's trick): each bit
  // position adds P, Q or the precomputed P + Q.
  static Jac mul2(const Jac& P, const Fr& a, const Jac& Q, const Fr& b) {
    uint64_t ka[4], kb[4];
    a.to_std(ka);
    b.to_std(kb);
    const Jac PQ = P.add(Q);
    Jac r = inf();
    int top = -1;
    for (int i = 255; i >= 0 && top < 0; i--)
      if (((ka[i >> 6] | kb[i >> 6]) >> (i & 63)) & 1) top = i;
    for (int i = top; i >= 0; i--) {
      r = r.dbl();
      const int ba = (int)((ka[i >> 6] >> (i & 63)) & 1), bb = (int)((kb[i >> 6] >> (i & 63)) & 1);
      if (ba && bb) r = r.add(PQ);
      else if (ba) r = r.add(P);
      else if (bb) r = r.add(Q);
    }
    return r;
  }
  // canonical affine; returns false for infinity (x = y = 0 then)
  bool to_affine(E& ax, E& ay) const {
    if (is_inf()) {
      ax = E::zero();
      ay = E::zero();
      return false;
    }
    E zi = z.inv(), zi2 = zi.sqr();
    ax = x * zi2;
    ay = y * zi2 * zi;
    return true;
  }
};

typedef Jac<Fq> G1;
typedef Jac<Fq2> G2;

}  // namespace zkh
