// BN254 G1 (over Fq) and G2 (over Fq2 = Fq[u]/(u^2+1)) group arithmetic for
// the MSM kernels, in XYZZ coordinates: (X, Y, ZZ, ZZZ) with x = X/ZZ,
// y = Y/ZZZ, ZZ^3 = ZZZ^2; ZZ = 0 encodes the point at infinity.  Formulas are
// the a = 0 cases of the EFD "xyzz" family: madd-2008-s (8M+2S),
// add-2008-s (12M+2S), dbl-2008-s-1 (6M+3S) and mdbl-2008-s-1.  The reference
// uses Jacobian coordinates (src/curve/g1.cuh:89-187) and affine G2 formulas
// (src/curve/g2.cuh:103-146); every one of them computes the same group law,
// and results leave the device as canonical affine points.
//
// All functions are generic over the coordinate field F (fq or fq2) through
// the overloads fmul/fsqr/fadd/fsub/fis_zero/fdbl below.
#pragma once
#include "field.hpp"

namespace zk {

// ------------------------------------------------------------------ Fq2
struct fq2 {
  fq c0, c1;
};

ZK_HD fq2 fadd(const fq2& a, const fq2& b) { return fq2{fadd(a.c0, b.c0), fadd(a.c1, b.c1)}; }
ZK_HD fq2 fsub(const fq2& a, const fq2& b) { return fq2{fsub(a.c0, b.c0), fsub(a.c1, b.c1)}; }
ZK_HD fq2 fdbl(const fq2& a) { return fq2{fdbl(a.c0), fdbl(a.c1)}; }
ZK_HD fq2 fneg(const fq2& a) { return fq2{fneg(a.c0), fneg(a.c1)}; }
ZK_HD fq fneg_canon_if(const fq& a, bool neg) { return fneg_canon_if<FqP>(a, neg); }
ZK_HD fq2 fneg_canon_if(const fq2& a, bool neg) { return fq2{fneg_canon_if(a.c0, neg), fneg_canon_if(a.c1, neg)}; }
// (a0 + a1 u)(b0 + b1 u) = (a0 b0 - a1 b1) + (a0 b1 + a1 b0) u, each
// coordinate one fmul_sum (4 limb products, 2 reductions; the reference uses
// Karatsuba, src/field/fp2.cuh:73-78: 3 multiplies, each with its own
// reduction).  -a1 enters as 2q - a1, so a must be reduced (< 2q); b may be a
// lazy difference (< 4q).
ZK_HD fq2 fmul(const fq2& a, const fq2& b) {
  const fq x0[2] = {a.c0, fneg_lazy(a.c1)}, y0[2] = {b.c0, b.c1};
  const fq x1[2] = {a.c0, a.c1}, y1[2] = {b.c1, b.c0};
  return fq2{fmul_sum<FqP, 2>(x0, y0), fmul_sum<FqP, 2>(x1, y1)};
}
// (a + bu)^2 = (a+b)(a-b) + 2ab u; a may be a lazy value (< 4q).
ZK_HD fq2 fsqr(const fq2& a) {
  fq ab = fmul(a.c0, a.c1);
  return fq2{fmul(fadd_lazy(a.c0, a.c1), fsub_lazy4(a.c0, a.c1)), fdbl(ab)};
}
ZK_HD bool fis_zero(const fq2& a) { return fis_zero(a.c0) && fis_zero(a.c1); }
ZK_HD bool fis_zero4(const fq& a) { return fis_zero4<FqP>(a); }
ZK_HD bool fis_zero4(const fq2& a) { return fis_zero4<FqP>(a.c0) && fis_zero4<FqP>(a.c1); }
ZK_HD fq fsub3(const fq& a, const fq& b, const fq& c) { return fsub3<FqP>(a, b, c); }
ZK_HD fq2 fsub3(const fq2& a, const fq2& b, const fq2& c) {
  return fq2{fsub3<FqP>(a.c0, b.c0, c.c0), fsub3<FqP>(a.c1, b.c1, c.c1)};
}

ZK_HD void fset_zero(fq& a) { a = fe_zero<FqP>(); }
ZK_HD void fset_zero(fq2& a) { a = fq2{fe_zero<FqP>(), fe_zero<FqP>()}; }
ZK_HD void fset_one(fq& a) { a = fe_one<FqP>(); }
ZK_HD void fset_one(fq2& a) { a = fq2{fe_one<FqP>(), fe_zero<FqP>()}; }

// a*b - c*d with one Montgomery reduction per coordinate (fmul_sum, the
// subtracted products entering as (km - x) * y).  a and b may be lazy values
// (< 4m: fsub_m, fsub_r); c and d are reduced (< 2m).
ZK_HD fq fmul_sub(const fq& a, const fq& b, const fq& c, const fq& d) { return fmul2(a, b, c, fneg_lazy(d)); }
ZK_HD fq2 fmul_sub(const fq2& a, const fq2& b, const fq2& c, const fq2& d) {
  // real: a0 b0 - a1 b1 - c0 d0 + c1 d1, imaginary: a0 b1 + a1 b0 - c0 d1 - c1 d0
  const fq na1 = fneg_lazy4(a.c1), nc0 = fneg_lazy(c.c0), nc1 = fneg_lazy(c.c1);
  const fq x0[4] = {a.c0, na1, nc0, c.c1}, y0[4] = {b.c0, b.c1, d.c0, d.c1};
  const fq x1[4] = {a.c0, a.c1, nc0, nc1}, y1[4] = {b.c1, b.c0, d.c1, d.c0};
  return fq2{fmul_sum<FqP, 4>(x0, y0), fmul_sum<FqP, 4>(x1, y1)};
}
// a - b left in (0, 4m) for reduced a, b: only as an fmul_sub factor or an
// fsqr input.
ZK_HD fq fsub_m(const fq& a, const fq& b) { return fsub_lazy(a, b); }
ZK_HD fq2 fsub_m(const fq2& a, const fq2& b) { return fq2{fsub_lazy(a.c0, b.c0), fsub_lazy(a.c1, b.c1)}; }

// ------------------------------------------------------------------ XYZZ
template <class F>
struct xyzz {
  F x, y, zz, zzz;
};

template <class F>
ZK_HD void xyzz_set_inf(xyzz<F>& p) {
  fset_zero(p.x);
  fset_zero(p.y);
  fset_zero(p.zz);
  fset_zero(p.zzz);
}

template <class F>
ZK_HD bool xyzz_is_inf(const xyzz<F>& p) {
  return fis_zero(p.zz);
}

template <class F>
ZK_HD void xyzz_set_affine(xyzz<F>& p, const F& x, const F& y) {
  p.x = x;
  p.y = y;
  fset_one(p.zz);
  fset_one(p.zzz);
}

// p = 2 * (x, y) for an affine point (mdbl-2008-s-1)
template <class F>
ZK_HD void xyzz_mdbl(xyzz<F>& p, const F& x, const F& y) {
  F u = fdbl(y);
  F v = fsqr(u);
  F w = fmul(u, v);
  F s = fmul(x, v);
  F x2 = fsqr(x);
  F m = fadd(fdbl(x2), x2);
  F zero;
  fset_zero(zero);
  F x3 = fsub3(fsqr(m), zero, s);
  F y3 = fmul_sub(m, fsub_m(s, x3), w, y);
  p.x = x3;
  p.y = y3;
  p.zz = v;
  p.zzz = w;
}

// p = 2p (dbl-2008-s-1)
template <class F>
ZK_HD void xyzz_dbl(xyzz<F>& p) {
  if (xyzz_is_inf(p)) return;
  F u = fdbl(p.y);
  F v = fsqr(u);
  F w = fmul(u, v);
  F s = fmul(p.x, v);
  F x2 = fsqr(p.x);
  F m = fadd(fdbl(x2), x2);
  F zero;
  fset_zero(zero);
  F x3 = fsub3(fsqr(m), zero, s);
  F y3 = fmul_sub(m, fsub_m(s, x3), w, p.y);
  p.x = x3;
  p.y = y3;
  p.zz = fmul(v, p.zz);
  p.zzz = fmul(w, p.zzz);
}

// p += (x2, y2) affine, finite (madd-2008-s)
// p += (x2, y2) for a finite p; returns true when the sum is the point at
// infinity (then p is set to it).
template <class F>
ZK_HD bool xyzz_madd_fin(xyzz<F>& p, const F& x2, const F& y2) {
  F u2 = fmul(x2, p.zz);
  F s2 = fmul(y2, p.zzz);
  F P = fsub_m(u2, p.x);  // lazy, (0, 4m): only squared, multiplied as the lazy operand and tested
  F R = fsub_m(s2, p.y);  // lazy, (0, 4m)
  if (fis_zero4(P)) {
    if (fis_zero4(R)) {
      xyzz_mdbl(p, x2, y2);
      return false;
    }
    xyzz_set_inf(p);
    return true;
  }
  F pp = fsqr(P);
  F ppp = fmul(pp, P);
  F q = fmul(p.x, pp);
  F x3 = fsub3(fsqr(R), ppp, q);
  F y3 = fmul_sub(R, fsub_m(q, x3), p.y, ppp);
  p.x = x3;
  p.y = y3;
  p.zz = fmul(p.zz, pp);
  p.zzz = fmul(p.zzz, ppp);
  return false;
}

template <class F>
ZK_HD void xyzz_madd(xyzz<F>& p, const F& x2, const F& y2) {
  if (xyzz_is_inf(p)) {
    xyzz_set_affine(p, x2, y2);
    return;
  }
  (void)xyzz_madd_fin(p, x2, y2);
}

// p += q (add-2008-s)
template <class F>
ZK_HD void xyzz_add(xyzz<F>& p, const xyzz<F>& q) {
  if (xyzz_is_inf(q)) return;
  if (xyzz_is_inf(p)) {
    p = q;
    return;
  }
  F u1 = fmul(p.x, q.zz);
  F u2 = fmul(q.x, p.zz);
  F s1 = fmul(p.y, q.zzz);
  F s2 = fmul(q.y, p.zzz);
  F P = fsub_m(u2, u1);  // lazy, (0, 4m)
  F R = fsub_m(s2, s1);  // lazy, (0, 4m)
  if (fis_zero4(P)) {
    if (fis_zero4(R)) xyzz_dbl(p);
    else xyzz_set_inf(p);
    return;
  }
  F pp = fsqr(P);
  F ppp = fmul(pp, P);
  F qq = fmul(u1, pp);
  F x3 = fsub3(fsqr(R), ppp, qq);
  F y3 = fmul_sub(R, fsub_m(qq, x3), s1, ppp);
  p.x = x3;
  p.y = y3;
  p.zz = fmul(fmul(p.zz, q.zz), pp);
  p.zzz = fmul(fmul(p.zzz, q.zzz), ppp);
}

template <class F>
ZK_HD void xyzz_neg(xyzz<F>& p) {
  p.y = fneg(p.y);
}

// p = k * p for a small non-negative integer k (double-and-add, MSB first).
template <class F>
ZK_HD void xyzz_mul_small(xyzz<F>& p, uint32_t k) {
  xyzz<F> acc;
  xyzz_set_inf(acc);
  if (k == 0 || xyzz_is_inf(p)) {
    p = acc;
    return;
  }
  int top = 31 - __builtin_clz(k);
  acc = p;
  for (int i = top - 1; i >= 0; i--) {
    xyzz_dbl(acc);
    if ((k >> i) & 1u) xyzz_add(acc, p);
  }
  p = acc;
}

// a^-1 = a^(q-2) (Fermat); Fq2 through the norm: (c0 - c1 u) / (c0^2 + c1^2)
ZK_HD fq finv(const fq& a) {
  const uint32_t qm2[8] = {0xd87cfd45u, 0x3c208c16u, 0x6871ca8du, 0x97816a91u,
                           0x8181585du, 0xb85045b6u, 0xe131a029u, 0x30644e72u};  // q - 2
  return fpow(a, qm2);
}
ZK_HD fq2 finv(const fq2& a) {
  fq n = finv(fadd(fsqr(a.c0), fsqr(a.c1)));
  return fq2{fmul(a.c0, n), fneg(fmul(a.c1, n))};
}

// Affine forms x = X / ZZ, y = Y / ZZZ of PER points with one inversion of
// the product of every ZZ * ZZZ (Montgomery's trick); inf[j] marks the point
// at infinity (x, y then unset).
template <class F, int PER>
ZK_HD void xyzz_to_affine_batch(const xyzz<F> (&p)[PER], F (&x)[PER], F (&y)[PER], bool (&inf)[PER]) {
  F pre[PER], d[PER];
  F prod;
  fset_one(prod);
  for (int j = 0; j < PER; j++) {
    pre[j] = prod;
    inf[j] = xyzz_is_inf(p[j]);
    if (!inf[j]) {
      d[j] = fmul(p[j].zz, p[j].zzz);
      prod = fmul(prod, d[j]);
    }
  }
  F inv = finv(prod);
  for (int j = PER - 1; j >= 0; j--) {
    if (inf[j]) continue;
    F di = fmul(inv, pre[j]);  // 1 / (ZZ_j ZZZ_j)
    inv = fmul(inv, d[j]);
    x[j] = fmul(p[j].x, fmul(di, p[j].zzz));
    y[j] = fmul(p[j].y, fmul(di, p[j].zz));
  }
}

}  // namespace zk
