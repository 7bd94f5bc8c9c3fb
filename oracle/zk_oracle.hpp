// TEST INFRASTRUCTURE ONLY -- CPU oracle for the Groth16 hot path.
//
// A from-scratch CPU restatement of the reference prover's algorithms
// (gdtsitlauri/cuda-zkml, paths relative to the reference root).  Only tests/,
// __graft_entry__.smoke() and bench.py's cpu_baseline leg may load it, and only
// as the checker or as the timed CPU baseline; the product never links it.
//
// Arithmetic follows the reference exactly in representation: 4 x 64-bit
// little-endian limbs, Montgomery form with R = 2^256, CIOS multiplication
// with a single conditional subtraction (src/field/montgomery.cuh:330-368,
// src/field/fp.cuh:363-427).  Every value it hands out is canonical (< m), so
// "bit-exact with the reference" is "mathematically equal".
#pragma once
#include <stdint.h>
#include <string.h>

#include <random>
#include <string>
#include <vector>

namespace orc {

typedef unsigned __int128 u128;

// ---------------------------------------------------------------- fields
struct QParams {  // base field (src/field/montgomery.cuh:33-60)
  static constexpr uint64_t M[4] = {0x3C208C16D87CFD47ULL, 0x97816A916871CA8DULL, 0xB85045B68181585DULL,
                                    0x30644E72E131A029ULL};
  static constexpr uint64_t INV = 0x87D20782E4866389ULL;
  static constexpr uint64_t ONE[4] = {0xD35D438DC58F0D9DULL, 0x0A78EB28F5C70B3DULL, 0x666EA36F7879462CULL,
                                      0x0E0A77C19A07DF2FULL};
  static constexpr uint64_t R2[4] = {0xF32CFC5B538AFA89ULL, 0xB5E71911D44501FBULL, 0x47AB1EFF0A417FF6ULL,
                                     0x06D89F71CAB8351FULL};
};
struct RParams {  // scalar field (src/field/fp.cuh:329-349)
  static constexpr uint64_t M[4] = {0x43E1F593F0000001ULL, 0x2833E84879B97091ULL, 0xB85045B68181585DULL,
                                    0x30644E72E131A029ULL};
  static constexpr uint64_t INV = 0xC2E1F593EFFFFFFFULL;
  static constexpr uint64_t ONE[4] = {0xAC96341C4FFFFFFBULL, 0x36FC76959F60CD29ULL, 0x666EA36F7879462EULL,
                                      0x0E0A77C19A07DF2FULL};
  static constexpr uint64_t R2[4] = {0x1BB8E645AE216DA7ULL, 0x53FE3AB1E35C59E3ULL, 0x8C49833D53BB8085ULL,
                                     0x0216D0B17F4E44A5ULL};
};

template <class P>
struct F {
  uint64_t v[4];

  static F zero() { return F{{0, 0, 0, 0}}; }
  static F one() { return F{{P::ONE[0], P::ONE[1], P::ONE[2], P::ONE[3]}}; }
  static F raw(const uint64_t* w) {
    F r;
    memcpy(r.v, w, 32);
    return r;
  }
  bool is_zero() const { return (v[0] | v[1] | v[2] | v[3]) == 0; }
  bool operator==(const F& o) const { return memcmp(v, o.v, 32) == 0; }
  bool operator!=(const F& o) const { return !(*this == o); }

  // CIOS, 4 x 64 (src/field/montgomery.cuh:330-368)
  static void mont(uint64_t* r, const uint64_t* a, const uint64_t* b) {
    uint64_t T[5] = {0, 0, 0, 0, 0};
    for (int i = 0; i < 4; i++) {
      u128 c = 0;
      for (int j = 0; j < 4; j++) {
        c += (u128)a[i] * b[j] + T[j];
        T[j] = (uint64_t)c;
        c >>= 64;
      }
      c = (u128)T[4] + (uint64_t)c;
      T[4] = (uint64_t)c;
      uint64_t m = T[0] * P::INV;
      c = ((u128)T[0] + (u128)m * P::M[0]) >> 64;
      for (int j = 1; j < 4; j++) {
        c += (u128)T[j] + (u128)m * P::M[j];
        T[j - 1] = (uint64_t)c;
        c >>= 64;
      }
      c += T[4];
      T[3] = (uint64_t)c;
      T[4] = (uint64_t)(c >> 64);
    }
    uint64_t t[4];
    uint64_t br = sub4(t, T, P::M);
    if (!br) memcpy(r, t, 32);
    else memcpy(r, T, 32);
  }
  static uint64_t add4(uint64_t* r, const uint64_t* a, const uint64_t* b) {
    u128 c = 0;
    for (int i = 0; i < 4; i++) {
      c += (u128)a[i] + b[i];
      r[i] = (uint64_t)c;
      c >>= 64;
    }
    return (uint64_t)c;
  }
  static uint64_t sub4(uint64_t* r, const uint64_t* a, const uint64_t* b) {
    uint64_t br = 0;
    for (int i = 0; i < 4; i++) {
      u128 d = (u128)a[i] - b[i] - br;
      r[i] = (uint64_t)d;
      br = (uint64_t)(d >> 127) & 1;
    }
    return br;
  }
  F operator*(const F& o) const {
    F r;
    mont(r.v, v, o.v);
    return r;
  }
  F sqr() const { return *this * *this; }
  // fp.cuh:84-113 / 435-453
  F operator+(const F& o) const {
    F r, t;
    uint64_t c = add4(r.v, v, o.v);
    uint64_t b = sub4(t.v, r.v, P::M);
    if (c || !b) return t;
    return r;
  }
  F operator-(const F& o) const {
    F r;
    if (sub4(r.v, v, o.v)) add4(r.v, r.v, P::M);
    return r;
  }
  F operator-() const {
    if (is_zero()) return *this;
    F r;
    sub4(r.v, P::M, v);
    return r;
  }
  F dbl() const { return *this + *this; }
  static F from_uint(uint64_t x) {
    uint64_t p[4] = {x, 0, 0, 0};
    F r;
    mont(r.v, p, P::R2);
    return r;
  }
  static F from_std(const uint64_t* s) {
    F r;
    mont(r.v, s, P::R2);
    return r;
  }
  void to_std(uint64_t* out) const {
    uint64_t one[4] = {1, 0, 0, 0};
    mont(out, v, one);
  }
  F pow(const uint64_t* e) const {
    F r = one();
    int top = -1;
    for (int i = 255; i >= 0; i--)
      if ((e[i >> 6] >> (i & 63)) & 1) {
        top = i;
        break;
      }
    for (int i = top; i >= 0; i--) {
      r = r.sqr();
      if ((e[i >> 6] >> (i & 63)) & 1) r = r * *this;
    }
    return r;
  }
  F inv() const {  // Fermat, fp.cuh:240 / 547
    uint64_t e[4];
    memcpy(e, P::M, 32);
    e[0] -= 2;
    return pow(e);
  }
};

typedef F<QParams> Fq;
typedef F<RParams> Fr;

// Fp2 = Fp[u]/(u^2+1), Karatsuba (src/field/fp2.cuh:22-134)
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
    Fq ac = c0 * o.c0, bd = c1 * o.c1;
    Fq s = (c0 + c1) * (o.c0 + o.c1);
    return Fq2{ac - bd, s - ac - bd};
  }
  Fq2 sqr() const {
    Fq ab = c0 * c1;
    return Fq2{(c0 + c1) * (c0 - c1), ab + ab};
  }
  Fq2 dbl() const { return *this + *this; }
  Fq2 inv() const {
    Fq n = (c0.sqr() + c1.sqr()).inv();
    return Fq2{c0 * n, -(c1 * n)};
  }
};

// ---------------------------------------------------------------- curves
// Jacobian formulas of src/curve/g1.cuh:89-187 (dbl-2009-l, 12M+4S add,
// 8M+3S mixed add).  The G2 group reuses them over Fq2; the reference's G2
// routes every operation through affine coordinates (src/curve/g2.cuh:103-146)
// but both produce the same canonical affine output.
template <class E>
struct Aff {
  E x, y;
  bool inf;
};
template <class E>
struct Jac {
  E x, y, z;
  static Jac identity() {
    Jac r;
    r.x = E::zero();
    r.y = E::one();
    r.z = E::zero();
    return r;
  }
  static Jac from_affine(const Aff<E>& p) {
    if (p.inf) return identity();
    Jac r;
    r.x = p.x;
    r.y = p.y;
    r.z = E::one();
    return r;
  }
  bool is_inf() const { return z.is_zero(); }
  Jac dbl() const {
    if (is_inf()) return *this;
    E A = x.sqr(), B = y.sqr(), C = B.sqr();
    E D = (x + B).sqr() - A - C;
    D = D + D;
    E Ee = A + A + A;
    E Ff = Ee.sqr();
    Jac r;
    r.x = Ff - D - D;
    E C8 = C.dbl().dbl().dbl();
    r.y = Ee * (D - r.x) - C8;
    r.z = (y + z).sqr() - B - z.sqr();
    return r;
  }
  Jac add(const Jac& o) const {
    if (is_inf()) return o;
    if (o.is_inf()) return *this;
    E Z1Z1 = z.sqr(), Z2Z2 = o.z.sqr();
    E U1 = x * Z2Z2, U2 = o.x * Z1Z1;
    E S1 = y * o.z * Z2Z2, S2 = o.y * z * Z1Z1;
    E H = U2 - U1, R = S2 - S1;
    if (H.is_zero()) {
      if (R.is_zero()) return dbl();
      return identity();
    }
    E HH = H.sqr(), HHH = HH * H, V = U1 * HH;
    Jac r;
    r.x = R.sqr() - HHH - V - V;
    r.y = R * (V - r.x) - S1 * HHH;
    r.z = z * o.z * H;
    return r;
  }
  Jac add_affine(const Aff<E>& o) const {
    if (o.inf) return *this;
    if (is_inf()) return from_affine(o);
    E Z1Z1 = z.sqr();
    E U2 = o.x * Z1Z1, S2 = o.y * z * Z1Z1;
    E H = U2 - x, R = S2 - y;
    if (H.is_zero()) {
      if (R.is_zero()) return dbl();
      return identity();
    }
    E HH = H.sqr(), HHH = HH * H, V = x * HH;
    Jac r;
    r.x = R.sqr() - HHH - V - V;
    r.y = R * (V - r.x) - y * HHH;
    r.z = z * H;
    return r;
  }
  Jac neg() const {
    Jac r = *this;
    r.y = -y;
    return r;
  }
  Aff<E> to_affine() const {
    Aff<E> a;
    if (is_inf()) {
      a.x = E::zero();
      a.y = E::zero();
      a.inf = true;
      return a;
    }
    E zi = z.inv(), zi2 = zi.sqr(), zi3 = zi2 * zi;
    a.x = x * zi2;
    a.y = y * zi3;
    a.inf = false;
    return a;
  }
  // MSB-first double-and-add over the standard-form scalar (g1.cuh:197-240)
  Jac mul(const Fr& k) const {
    uint64_t s[4];
    k.to_std(s);
    return mul_std(s);
  }
  Jac mul_std(const uint64_t* s) const {
    Jac r = identity();
    int top = -1;
    for (int i = 255; i >= 0; i--)
      if ((s[i >> 6] >> (i & 63)) & 1) {
        top = i;
        break;
      }
    for (int i = top; i >= 0; i--) {
      r = r.dbl();
      if ((s[i >> 6] >> (i & 63)) & 1) r = r.add(*this);
    }
    return r;
  }
};

typedef Aff<Fq> G1A;
typedef Jac<Fq> G1J;
typedef Aff<Fq2> G2A;
typedef Jac<Fq2> G2J;

// The reference's own G2 arithmetic (src/curve/g2.cuh:88-146): Jacobian
// storage, but every group operation converts its operands to affine (one
// Fq2 inversion per operand, z = 1 included, as G2Jacobian::to_affine does)
// and applies the affine chord/tangent formulas, whose slope is one more
// inversion.  Same canonical affine results as Jac<Fq2>, at the reference's
// cost; used for the timed CPU baseline of the reference's host algorithm.
struct G2Ref {
  Fq2 x, y, z;
  static G2Ref identity() { return G2Ref{Fq2::zero(), Fq2::one(), Fq2::zero()}; }
  static G2Ref from_affine(const G2A& p) {  // g2.cuh:90-93
    if (p.inf) return identity();
    return G2Ref{p.x, p.y, Fq2::one()};
  }
  bool is_inf() const { return z.is_zero(); }
  G2A to_affine() const {  // g2.cuh:95-101
    G2A a;
    if (is_inf()) {
      a.x = Fq2::zero();
      a.y = Fq2::zero();
      a.inf = true;
      return a;
    }
    Fq2 zi = z.inv(), zi2 = zi.sqr(), zi3 = zi2 * zi;
    a.x = x * zi2;
    a.y = y * zi3;
    a.inf = false;
    return a;
  }
  static G2A inf_point() {
    G2A a;
    a.x = Fq2::zero();
    a.y = Fq2::zero();
    a.inf = true;
    return a;
  }
  static G2A dbl_aff(const G2A& p) {  // g2.cuh:103-115: lambda = 3x^2 / 2y
    if (p.inf || p.y.is_zero()) return inf_point();
    Fq2 lambda = (p.x.sqr() + p.x.sqr() + p.x.sqr()) * (p.y + p.y).inv();
    G2A r;
    r.x = lambda.sqr() - p.x - p.x;
    r.y = lambda * (p.x - r.x) - p.y;
    r.inf = false;
    return r;
  }
  static G2A add_aff(const G2A& p, const G2A& q) {  // g2.cuh:117-132
    if (p.inf) return q;
    if (q.inf) return p;
    if (p.x == q.x) {
      if (!(p.y == q.y)) return inf_point();
      return dbl_aff(p);
    }
    Fq2 lambda = (q.y - p.y) * (q.x - p.x).inv();
    G2A r;
    r.x = lambda.sqr() - p.x - q.x;
    r.y = lambda * (p.x - r.x) - p.y;
    r.inf = false;
    return r;
  }
  G2Ref dbl() const { return from_affine(dbl_aff(to_affine())); }                       // g2.cuh:134-136
  G2Ref add(const G2Ref& o) const { return from_affine(add_aff(to_affine(), o.to_affine())); }  // :139-141
  G2Ref add_affine(const G2A& o) const { return from_affine(add_aff(to_affine(), o)); }  // :144-146
  // MSB-first double-and-add over the standard-form scalar (g2.cuh:153-190)
  G2Ref mul(const Fr& k) const {
    uint64_t s[4];
    k.to_std(s);
    G2Ref r = identity();
    int top = -1;
    for (int i = 255; i >= 0; i--)
      if ((s[i >> 6] >> (i & 63)) & 1) {
        top = i;
        break;
      }
    for (int i = top; i >= 0; i--) {
      r = r.dbl();
      if ((s[i >> 6] >> (i & 63)) & 1) r = r.add(*this);
    }
    return r;
  }
};

G1A g1_generator();  // (1, 2)            g1.cuh:40
G2A g2_generator();  // EIP-197           g2.cuh:47-65

// Batch conversion of Jacobian points to affine with one inversion.
template <class E>
void batch_to_affine(const std::vector<Jac<E>>& in, std::vector<Aff<E>>& out);

// ---------------------------------------------------------------- NTT
Fr omega(int log_n);      // ntt.cu:64-87
Fr omega_inv(int log_n);  // ntt.cu:89-111
void ntt_radix2(std::vector<Fr>& a, int log_n, bool inverse, int threads);  // ntt.cu:354-465
void dft_naive(const std::vector<Fr>& in, std::vector<Fr>& out, const Fr& w);  // tests/test_ntt.cu:19-37

// ---------------------------------------------------------------- MSM
struct MsmConfig {  // src/msm/msm.cuh:40-64
  int c, windows, buckets;
  static MsmConfig for_size(int n, bool g2);
};
G1J msm_g1(const G1A* pts, const Fr* sc, int n, int threads);  // msm.cu:320-442
G2J msm_g2(const G2A* pts, const Fr* sc, int n, int threads);  // msm.cu:526-598
G1J msm_g1_naive(const G1A* pts, const Fr* sc, int n);        // tests/test_msm.cu:20-28
G2J msm_g2_naive(const G2A* pts, const Fr* sc, int n);
// msm_g2 on the reference's affine-inversion arithmetic (G2Ref)
G2Ref msm_g2_affine_ref(const G2A* pts, const Fr* sc, int n, int threads);

// ---------------------------------------------------------------- R1CS / Groth16
struct Entry {  // src/prover/circuit.cuh:32-36
  int row, col;
  Fr value;
};
struct R1CS {  // circuit.cuh:39-124
  int num_constraints = 0, num_variables = 0, num_public = 0, num_private = 0;
  std::vector<Entry> A, B, C;
  bool verify_witness(const std::vector<Fr>& w) const;
};

struct ProvingKey {  // groth16.cuh:74-159
  int num_constraints = 0, num_variables = 0, num_public = 0;
  G1A alpha_g1, beta_g1, delta_g1;
  G2A beta_g2, gamma_g2, delta_g2;
  std::vector<G1A> tau_g1;
  std::vector<G2A> tau_g2;
  std::vector<G1A> A_query, B_g1_query, L_query, H_query;
  std::vector<G2A> B_g2_query;
  bool save(const char* path) const;   // groth16.cu:1104-1188
  bool load(const char* path);         // groth16.cu:1190-1314
};
struct VerifyingKey {  // groth16.cuh:164-174
  int num_public = 0;
  G1A alpha_g1;
  G2A beta_g2, gamma_g2, delta_g2;
  std::vector<G1A> ic;
  bool save(const char* path) const;  // src/verifier/verifier.cu:103-148
  bool load(const char* path);        // verifier.cu:150-195
};
struct Proof {
  G1A A;
  G2A B;
  G1A C;
  bool valid = false;
  void serialize(uint8_t out[256]) const;  // groth16.cu:1058-1074
};

int qap_log_n(int num_constraints);  // groth16.cu:225-242
std::vector<Fr> compute_h(const R1CS& c, const std::vector<Fr>& w, int threads);  // groth16.cu:263-390
void setup(const R1CS& c, uint64_t seed, ProvingKey& pk, VerifyingKey& vk, int threads);  // groth16.cu:446-642
// g2_affine_ref: B's MSM and s*delta2 on G2Ref (the reference's G2 cost)
// instead of Jac<Fq2>; the proof is the same either way
Proof prove(const ProvingKey& pk, const R1CS& c, const std::vector<Fr>& w, uint64_t seed, int threads,
            double* ms_breakdown, bool g2_affine_ref = false);  // groth16.cu:655-920

}  // namespace orc
