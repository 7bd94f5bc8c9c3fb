// Fq2 split over a lane pair, for the latency-bound G2 kernels (chunk
// combine, bucket reduction).  There a few waves each run a long chain of
// dependent point additions, so the chain's length in instructions is the
// time.  With fq2h the two coordinates of every Fq2 value live in two
// adjacent lanes (even lane: c0, odd lane: c1): additions are one Fq
// operation per lane, and a product takes the partner's coordinates through a
// DPP lane swap and then needs a single fmul_sum per lane instead of two.
// The XYZZ formulas of curve.hpp run unchanged on fq2h.
//
// Both lanes of a pair must execute together: every branch inside these
// operations is taken on values both lanes agree on (fis_zero combines the
// two halves), and the kernels index work by pair.
#pragma once
#include "curve.hpp"

namespace zk {

struct fq2h {
  fq c;  // this lane's coordinate: c0 (even lane) or c1 (odd lane)
};

__device__ __forceinline__ bool lane_odd() { return (threadIdx.x & 1) != 0; }

// the partner lane's value (DPP quad_perm [1, 0, 3, 2])
__device__ __forceinline__ uint32_t swap_pair(uint32_t v) {
  return (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0xB1, 0xF, 0xF, false);
}
__device__ __forceinline__ fq swap_pair(const fq& a) {
  fq r;
#pragma unroll
  for (int i = 0; i < NL; i++) r.l[i] = swap_pair(a.l[i]);
  return r;
}
__device__ __forceinline__ fq fsel(bool odd, const fq& a, const fq& b) {
  fq r;
#pragma unroll
  for (int i = 0; i < NL; i++) r.l[i] = odd ? a.l[i] : b.l[i];
  return r;
}

__device__ __forceinline__ fq2h fadd(const fq2h& a, const fq2h& b) { return fq2h{fadd(a.c, b.c)}; }
__device__ __forceinline__ fq2h fsub(const fq2h& a, const fq2h& b) { return fq2h{fsub(a.c, b.c)}; }
__device__ __forceinline__ fq2h fdbl(const fq2h& a) { return fq2h{fdbl(a.c)}; }
__device__ __forceinline__ fq2h fneg(const fq2h& a) { return fq2h{fneg(a.c)}; }
__device__ __forceinline__ fq2h fneg_canon_if(const fq2h& a, bool neg) { return fq2h{fneg_canon_if(a.c, neg)}; }
__device__ __forceinline__ fq2h fsub3(const fq2h& a, const fq2h& b, const fq2h& c) {
  return fq2h{fsub3<FqP>(a.c, b.c, c.c)};
}
__device__ __forceinline__ fq2h fsub_m(const fq2h& a, const fq2h& b) { return fq2h{fsub_lazy(a.c, b.c)}; }

__device__ __forceinline__ bool fis_zero(const fq2h& a) {
  const uint32_t z = fis_zero(a.c) ? 1u : 0u;
  return (z & swap_pair(z)) != 0;
}
__device__ __forceinline__ bool fis_zero4(const fq2h& a) {
  const uint32_t z = fis_zero4<FqP>(a.c) ? 1u : 0u;
  return (z & swap_pair(z)) != 0;
}
__device__ __forceinline__ void fset_zero(fq2h& a) { a.c = fe_zero<FqP>(); }
__device__ __forceinline__ void fset_one(fq2h& a) { a.c = lane_odd() ? fe_zero<FqP>() : fe_one<FqP>(); }

// (a0 + a1 u)(b0 + b1 u): even lane a0 b0 + (-a1) b1, odd lane a1 b0 + a0 b1
// (the pairs of the fq2 fmul of curve.hpp, with the same operand bounds).
__device__ __forceinline__ fq2h fmul(const fq2h& a, const fq2h& b) {
  const bool odd = lane_odd();
  const fq pa = swap_pair(a.c), pb = swap_pair(b.c);
  const fq x[2] = {fsel(odd, pa, a.c), fsel(odd, a.c, fneg_lazy(pa))};
  const fq y[2] = {b.c, pb};
  return fq2h{fmul_sum<FqP, 2>(x, y)};
}

// (a + bu)^2: even lane (a0 + a1)(a0 - a1), odd lane 2 a0 a1
__device__ __forceinline__ fq2h fsqr(const fq2h& a) {
  const bool odd = lane_odd();
  const fq pa = swap_pair(a.c);
  const fq t = fmul(fsel(odd, pa, fadd_lazy(a.c, pa)), fsel(odd, a.c, fsub_lazy4(a.c, pa)));
  return fq2h{fsel(odd, fdbl(t), t)};
}

// a b - c d (fq2 fmul_sub of curve.hpp): even lane a0 b0 - a1 b1 - c0 d0 +
// c1 d1, odd lane a1 b0 + a0 b1 - c1 d0 - c0 d1.
__device__ __forceinline__ fq2h fmul_sub(const fq2h& a, const fq2h& b, const fq2h& c, const fq2h& d) {
  const bool odd = lane_odd();
  const fq pa = swap_pair(a.c), pb = swap_pair(b.c), pc = swap_pair(c.c), pd = swap_pair(d.c);
  const fq nc = fneg_lazy(c.c), npc = fneg_lazy(pc);
  const fq x[4] = {fsel(odd, pa, a.c), fsel(odd, a.c, fneg_lazy4(pa)), fsel(odd, npc, nc), fsel(odd, nc, pc)};
  const fq y[4] = {b.c, pb, d.c, pd};
  return fq2h{fmul_sum<FqP, 4>(x, y)};
}

// Point loads and stores between the fq2 memory layout (c0 then c1 for each
// coordinate) and the lane-pair registers: each lane moves its half.
__device__ __forceinline__ xyzz<fq2h> load_half(const xyzz<fq2>& p) {
  const int r = lane_odd() ? 1 : 0;
  const fq* w = (const fq*)&p;
  return xyzz<fq2h>{fq2h{w[0 + r]}, fq2h{w[2 + r]}, fq2h{w[4 + r]}, fq2h{w[6 + r]}};
}
__device__ __forceinline__ void store_half(xyzz<fq2>& p, const xyzz<fq2h>& v) {
  const int r = lane_odd() ? 1 : 0;
  fq* w = (fq*)&p;
  w[0 + r] = v.x.c;
  w[2 + r] = v.y.c;
  w[4 + r] = v.zz.c;
  w[6 + r] = v.zzz.c;
}

// Register form of the latency-bound kernels: fq stays one lane per point,
// fq2 becomes a lane pair.
template <class F>
struct Lanes {
  typedef F R;
  static constexpr int N = 1;
  __device__ static xyzz<F> load(const xyzz<F>& p) { return p; }
  __device__ static void store(xyzz<F>& p, const xyzz<F>& v) { p = v; }
};
template <>
struct Lanes<fq2> {
  typedef fq2h R;
  static constexpr int N = 2;
  __device__ static xyzz<fq2h> load(const xyzz<fq2>& p) { return load_half(p); }
  __device__ static void store(xyzz<fq2>& p, const xyzz<fq2h>& v) { store_half(p, v); }
};

}  // namespace zk

namespace zk {

// ------------------------------------------------------------------ split point operations
// One point operation of a latency-bound chain dealt to two lane groups
// ("roles"): G1 to a lane pair (E = fq, role = lane bit 0), G2 to two lane
// pairs (E = fq2h, role = lane bit 1, each pair holding the two Fq2 halves).
// Both roles hold the whole point.  The formulas' independent products are
// split between the roles, each role computing one of them with operands it
// selects by its role, and the results are exchanged through DPP lane swaps:
// an addition's chain of 12 multiplications, 2 squarings and one two-product
// sum becomes about 7.5 multiplications deep.  The roles branch together
// (every branch tests values both hold).  Worth it where a chain runs alone
// on its SIMD; beside other waves the extra selects and swaps cost issue
// slots.
template <class E>
struct split {
  E v;
};

template <class E>
struct SplitRole;
template <>
struct SplitRole<fq> {
  static constexpr uint32_t BIT = 1;
  static constexpr int DPP = 0xB1;  // quad_perm [1, 0, 3, 2]: the other lane of the pair
};
template <>
struct SplitRole<fq2h> {
  static constexpr uint32_t BIT = 2;
  static constexpr int DPP = 0x4E;  // quad_perm [2, 3, 0, 1]: the same half in the other pair
};

template <class E>
__device__ __forceinline__ bool split_role1() {
  return (threadIdx.x & SplitRole<E>::BIT) != 0;
}

template <int CTRL>
__device__ __forceinline__ fq dpp_fq(const fq& a) {
  fq r;
#pragma unroll
  for (int i = 0; i < NL; i++) r.l[i] = (uint32_t)__builtin_amdgcn_mov_dpp((int)a.l[i], CTRL, 0xF, 0xF, false);
  return r;
}
__device__ __forceinline__ fq other_role(const fq& a) { return dpp_fq<SplitRole<fq>::DPP>(a); }
__device__ __forceinline__ fq2h other_role(const fq2h& a) { return fq2h{dpp_fq<SplitRole<fq2h>::DPP>(a.c)}; }
__device__ __forceinline__ fq pick(bool c, const fq& a, const fq& b) { return fsel(c, a, b); }
__device__ __forceinline__ fq2h pick(bool c, const fq2h& a, const fq2h& b) { return fq2h{fsel(c, a.c, b.c)}; }

template <class E>
__device__ __forceinline__ void fset_zero(split<E>& a) {
  fset_zero(a.v);
}
template <class E>
__device__ __forceinline__ void fset_one(split<E>& a) {
  fset_one(a.v);
}
template <class E>
__device__ __forceinline__ bool fis_zero(const split<E>& a) {
  return fis_zero(a.v);
}
template <class E>
__device__ __forceinline__ split<E> fneg(const split<E>& a) {
  return split<E>{fneg(a.v)};
}

// p = 2p (dbl-2008-s-1): V = U^2 | X^2, then W = U V | S = X V, then M^2 |
// V ZZ, then W ZZZ | Y3 = M (S - X3) - W Y.
template <class E>
__device__ __forceinline__ void xyzz_dbl(xyzz<split<E>>& p) {
  if (fis_zero(p.zz.v)) return;
  const bool r1 = split_role1<E>();
  const E U = fdbl(p.y.v);
  const E a = fsqr(pick(r1, p.x.v, U));  // V | X^2
  const E ao = other_role(a);
  const E V = pick(r1, ao, a), X2 = pick(r1, a, ao);
  const E b = fmul(pick(r1, p.x.v, U), V);  // W | S
  const E bo = other_role(b);
  const E W = pick(r1, bo, b), S = pick(r1, b, bo);
  const E M = fadd(fdbl(X2), X2);
  const E c = fmul(pick(r1, V, M), pick(r1, p.zz.v, M));  // M^2 | ZZ3 = V ZZ
  const E co = other_role(c);
  const E MM = pick(r1, co, c), ZZ3 = pick(r1, c, co);
  E zero;
  fset_zero(zero);
  const E X3 = fsub3(MM, zero, S);
  // W ZZZ - 0 | M (S - X3) - W Y
  const E d = fmul_sub(pick(r1, M, W), pick(r1, fsub_m(S, X3), p.zzz.v), pick(r1, W, zero), pick(r1, p.y.v, zero));
  const E dd = other_role(d);
  p.x.v = X3;
  p.y.v = pick(r1, d, dd);
  p.zz.v = ZZ3;
  p.zzz.v = pick(r1, dd, d);
}

// p += q (add-2008-s): U1 | U2, S1 | S2, ZZ1 ZZ2 | ZZZ1 ZZZ2; then PP | RR;
// then PPP | Q and ZZ3 on both; then ZZZ3 | Y3.
template <class E>
__device__ __forceinline__ void xyzz_add(xyzz<split<E>>& p, const xyzz<split<E>>& q) {
  if (fis_zero(q.zz.v)) return;
  if (fis_zero(p.zz.v)) {
    p = q;
    return;
  }
  const bool r1 = split_role1<E>();
  const E a = fmul(pick(r1, q.x.v, p.x.v), pick(r1, p.zz.v, q.zz.v));     // U1 = X1 ZZ2 | U2 = X2 ZZ1
  const E b = fmul(pick(r1, q.y.v, p.y.v), pick(r1, p.zzz.v, q.zzz.v));   // S1 = Y1 ZZZ2 | S2 = Y2 ZZZ1
  const E c = fmul(pick(r1, p.zzz.v, p.zz.v), pick(r1, q.zzz.v, q.zz.v)); // ZZ1 ZZ2 | ZZZ1 ZZZ2
  const E ao = other_role(a), bo = other_role(b), co = other_role(c);
  const E U1 = pick(r1, ao, a), U2 = pick(r1, a, ao);
  const E S1 = pick(r1, bo, b), S2 = pick(r1, b, bo);
  const E ZZ12 = pick(r1, co, c), ZZZ12 = pick(r1, c, co);
  const E P = fsub_m(U2, U1);  // lazy, (0, 4m)
  const E R = fsub_m(S2, S1);  // lazy, (0, 4m)
  if (fis_zero4(P)) {
    if (fis_zero4(R)) xyzz_dbl(p);
    else xyzz_set_inf(p);
    return;
  }
  const E t = fsqr(pick(r1, R, P));  // PP | RR
  const E to = other_role(t);
  const E PP = pick(r1, to, t), RR = pick(r1, t, to);
  const E v = fmul(PP, pick(r1, U1, P));  // PPP | Q (P lazy: the second factor)
  const E ZZ3 = fmul(ZZ12, PP);
  const E vo = other_role(v);
  const E PPP = pick(r1, vo, v), Q = pick(r1, v, vo);
  const E X3 = fsub3(RR, PPP, Q);
  E zero;
  fset_zero(zero);
  // ZZZ12 PPP - 0 | R (Q - X3) - S1 PPP
  const E d = fmul_sub(pick(r1, R, ZZZ12), pick(r1, fsub_m(Q, X3), PPP), pick(r1, S1, zero), pick(r1, PPP, zero));
  const E dd = other_role(d);
  p.x.v = X3;
  p.y.v = pick(r1, d, dd);
  p.zz.v = ZZ3;
  p.zzz.v = pick(r1, dd, d);
}

// Register forms of the latency-bound kernels with the operations split
// over two roles: a G1 point on a lane pair, a G2 point on four lanes.  Only
// role 0 stores (both hold the same point).
template <class F>
struct SplitLanes;
template <>
struct SplitLanes<fq> {
  typedef split<fq> R;
  static constexpr int N = 2;
  __device__ static xyzz<R> load(const xyzz<fq>& p) { return xyzz<R>{R{p.x}, R{p.y}, R{p.zz}, R{p.zzz}}; }
  __device__ static void store(xyzz<fq>& p, const xyzz<R>& v) {
    if (!split_role1<fq>()) p = xyzz<fq>{v.x.v, v.y.v, v.zz.v, v.zzz.v};
  }
};
template <>
struct SplitLanes<fq2> {
  typedef split<fq2h> R;
  static constexpr int N = 4;
  __device__ static xyzz<R> load(const xyzz<fq2>& p) {
    const xyzz<fq2h> h = load_half(p);
    return xyzz<R>{R{h.x}, R{h.y}, R{h.zz}, R{h.zzz}};
  }
  __device__ static void store(xyzz<fq2>& p, const xyzz<R>& v) {
    if (!split_role1<fq2h>()) store_half(p, xyzz<fq2h>{v.x.v, v.y.v, v.zz.v, v.zzz.v});
  }
};

}  // namespace zk
