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
