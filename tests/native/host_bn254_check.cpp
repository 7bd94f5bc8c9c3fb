// C shim over cuda-zkml_amd/csrc/host_bn254.hpp (the host arithmetic of the
// proof assembly, the MSM window combination and the verifier) for
// tests/test_host_bn254.py.  Points cross in the interchange layout
// (Montgomery words, all zero = infinity); an optional z word vector
// re-expresses an affine input in Jacobian coordinates (x z^2, y z^3, z), so
// that both the mixed (z = 1) and the general addition are reached.
#include <stdint.h>
#include <string.h>

#include "host_bn254.hpp"

using namespace zkh;

namespace {

bool all_zero(const uint64_t* w, int n) {
  for (int i = 0; i < n; i++)
    if (w[i]) return false;
  return true;
}

G1 g1_in(const uint64_t* w, const uint64_t* z) {
  if (all_zero(w, 8)) return G1::inf();
  G1 p = G1::affine(Fq::raw(w), Fq::raw(w + 4));
  if (z) {
    const Fq zs = Fq::raw(z), z2 = zs.sqr();
    p = G1{p.x * z2, p.y * (z2 * zs), zs};
  }
  return p;
}

void g1_out(const G1& p, uint64_t* w) {
  Fq x, y;
  memset(w, 0, 64);
  if (!p.to_affine(x, y)) return;
  memcpy(w, x.v, 32);
  memcpy(w + 4, y.v, 32);
}

G2 g2_in(const uint64_t* w, const uint64_t* z) {
  if (all_zero(w, 16)) return G2::inf();
  G2 p = G2::affine(Fq2{Fq::raw(w), Fq::raw(w + 4)}, Fq2{Fq::raw(w + 8), Fq::raw(w + 12)});
  if (z) {
    const Fq2 zs{Fq::raw(z), Fq::raw(z + 4)}, z2 = zs.sqr();
    p = G2{p.x * z2, p.y * (z2 * zs), zs};
  }
  return p;
}

void g2_out(const G2& p, uint64_t* w) {
  Fq2 x, y;
  memset(w, 0, 128);
  if (!p.to_affine(x, y)) return;
  memcpy(w, x.c0.v, 32);
  memcpy(w + 4, x.c1.v, 32);
  memcpy(w + 8, y.c0.v, 32);
  memcpy(w + 12, y.c1.v, 32);
}

}  // namespace

extern "C" {

int hb_g1_add(const uint64_t* p, const uint64_t* zp, const uint64_t* q, const uint64_t* zq, uint64_t* out) {
  g1_out(g1_in(p, zp).add(g1_in(q, zq)), out);
  return 0;
}

int hb_g1_mul(const uint64_t* p, const uint64_t* k, uint64_t* out) {
  g1_out(g1_in(p, nullptr).mul(Fr::raw(k)), out);
  return 0;
}

int hb_g1_mul2(const uint64_t* p, const uint64_t* a, const uint64_t* q, const uint64_t* b, uint64_t* out) {
  g1_out(G1::mul2(g1_in(p, nullptr), Fr::raw(a), g1_in(q, nullptr), Fr::raw(b)), out);
  return 0;
}

int hb_g2_add(const uint64_t* p, const uint64_t* zp, const uint64_t* q, const uint64_t* zq, uint64_t* out) {
  g2_out(g2_in(p, zp).add(g2_in(q, zq)), out);
  return 0;
}

int hb_g2_mul(const uint64_t* p, const uint64_t* k, uint64_t* out) {
  g2_out(g2_in(p, nullptr).mul(Fr::raw(k)), out);
  return 0;
}

}  // extern "C"

extern "C" int hb_fq_from_limbs29_scaled(const uint32_t* limbs, uint64_t* out) {
  const Fq r = Fq::from_limbs29_scaled(limbs);
  memcpy(out, r.v, 32);
  return 0;
}
