// Host build of the device field / curve headers (cuda-zkml_amd/csrc/field.hpp,
// curve.hpp) for CPU unit tests: the same source that the kernels inline,
// compiled by g++ and driven from Python with big-integer expectations.
#include <stdint.h>
#include <string.h>

#include "curve.hpp"

using namespace zk;

static fq ld(const uint32_t* p) {
  fq r;
  memcpy(r.l, p, sizeof(r.l));
  return r;
}
static void st(uint32_t* p, const fq& a) { memcpy(p, a.l, sizeof(a.l)); }
static fq2 ld2(const uint32_t* p) { return fq2{ld(p), ld(p + NL)}; }
static void st2(uint32_t* p, const fq2& a) {
  st(p, a.c0);
  st(p + NL, a.c1);
}

extern "C" {

// Field operations on 9-limb Fq elements.
int fh_op(int op, const uint32_t* a, const uint32_t* b, const uint32_t* c, const uint32_t* d, uint32_t* out) {
  fq A = ld(a), B = ld(b), C = ld(c), D = ld(d), r;
  switch (op) {
    case 0: r = fmul(A, B); break;
    case 1: r = fsqr(A); break;
    case 2: r = fmul2(A, B, C, D); break;
    case 3: r = fsub_lazy(A, B); break;
    case 4: r = fneg_lazy(A); break;
    case 5: r = fadd(A, B); break;
    case 6: r = fsub(A, B); break;
    case 7: r = fmul_sub(A, B, C, D); break;
    case 9: r = fsub3<FqP>(A, B, C); break;
    case 10: r = fsub_lazy4<FqP>(A, B); break;
    case 11: r = fneg_lazy4<FqP>(A); break;
    case 12: r = fe_zero<FqP>(); r.l[0] = fis_zero<FqP>(A) ? 1u : 0u; break;
    case 13: r = fe_zero<FqP>(); r.l[0] = fis_zero4<FqP>(A) ? 1u : 0u; break;
    case 14: r = fadd_wide(A, B); break;
    case 15: r = fcsub(A, FqP::MOD2); break;
    case 8: {  // four products: a*b + c*d + a*d + c*b
      const fq x[4] = {A, C, A, C}, y[4] = {B, D, D, B};
      r = fmul_sum<FqP, 4>(x, y);
      break;
    }
    default: return -1;
  }
  st(out, r);
  return 0;
}

// The NTT butterfly's Fr operations (the same templates over the scalar
// field): 0 fmul, 1 fadd_wide, 2 fcsub(a, 2r), 3 fsub_lazy (a + 2r - b),
// 4 / 5 / 7: a - b + 4r / 8r / 2r, 6 freduce (canonical value).
int fh_fr_op(int op, const uint32_t* a, const uint32_t* b, uint32_t* out) {
  fr A, B, r;
  memcpy(A.l, a, sizeof(A.l));
  memcpy(B.l, b, sizeof(B.l));
  switch (op) {
    case 0: r = fmul(A, B); break;
    case 1: r = fadd_wide(A, B); break;
    case 2: r = fcsub(A, FrP::MOD2); break;
    case 3: r = fsub_lazy(A, B); break;
    case 4: r = fsub_off<4>(A, B); break;
    case 5: r = fsub_off<8>(A, B); break;
    case 6: r = freduce(A); break;
    case 7: r = fsub_off<2>(A, B); break;
    default: return -1;
  }
  memcpy(out, r.l, sizeof(r.l));
  return 0;
}

// XYZZ operations; G1 points are 36 words (x, y, zz, zzz), G2 points 72.
// op 0: p += (qx, qy) affine   1: p += q   2: p = 2p   3: p = 2 (qx, qy)
int fh_xyzz(int g2, int op, const uint32_t* p, const uint32_t* q, uint32_t* out) {
  if (!g2) {
    xyzz<fq> P{ld(p), ld(p + 9), ld(p + 18), ld(p + 27)}, Q{ld(q), ld(q + 9), ld(q + 18), ld(q + 27)};
    switch (op) {
      case 0: xyzz_madd(P, Q.x, Q.y); break;
      case 1: xyzz_add(P, Q); break;
      case 2: xyzz_dbl(P); break;
      case 3: xyzz_mdbl(P, Q.x, Q.y); break;
      default: return -1;
    }
    st(out, P.x);
    st(out + 9, P.y);
    st(out + 18, P.zz);
    st(out + 27, P.zzz);
  } else {
    xyzz<fq2> P{ld2(p), ld2(p + 18), ld2(p + 36), ld2(p + 54)}, Q{ld2(q), ld2(q + 18), ld2(q + 36), ld2(q + 54)};
    switch (op) {
      case 0: xyzz_madd(P, Q.x, Q.y); break;
      case 1: xyzz_add(P, Q); break;
      case 2: xyzz_dbl(P); break;
      case 3: xyzz_mdbl(P, Q.x, Q.y); break;
      default: return -1;
    }
    st2(out, P.x);
    st2(out + 18, P.y);
    st2(out + 36, P.zz);
    st2(out + 54, P.zzz);
  }
  return 0;
}
}
