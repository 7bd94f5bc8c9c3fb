// BN254 base field Fq and scalar field Fr for gfx950.
//
// Representation (device and host-math builds alike)
// ---------------------------------------------------
// An element is 9 limbs of 29 bits (uint32 each, limb < 2^29), little endian,
// holding a value in the lazy range [0, 2m) for modulus m.  The Montgomery
// radix inside kernels is R' = 2^261 (= 2^(29*9)), not the reference's 2^256:
// with 29-bit limbs every limb product is one v_mad_u64_u32 into a 64-bit
// column accumulator and no carry has to be propagated until the column is
// finished (18 products of < 2^60 plus a 2^35 carry stay below 2^64).  On
// gfx950 the 32x32->64 mad issues at full rate, so the instruction count of
// the multiply is what matters; this layout needs 162 mads and 42 other ops
// (a square 126 and 50) against ~560 instructions for a compiler-lowered
// 8x32-bit CIOS.
//
// At the memory boundary elements are the reference's 32-byte little-endian
// form (4 x u64 = 8 x u32 words), Montgomery form with R = 2^256
// (reference: src/field/montgomery.cuh:33-60, src/field/fp.cuh:322-349).
// from_mont256/to_mont256 convert between the two radices with one multiply
// by a constant (2^266 mod m in, 2^256 mod m out).  For maps that are linear
// over the field (NTT, scaling by a constant prepared in the internal radix)
// the radix cancels and a plain limb repack suffices (repack_in/repack_out).
#pragma once
#include <stdint.h>

#if defined(__HIPCC__)
#include <hip/hip_runtime.h>
#include <utility>
#include "mad_chain.hpp"
#define ZK_HD __host__ __device__ __forceinline__
#else
#define ZK_HD static inline
#endif

namespace zk {

constexpr int NL = 9;
constexpr uint32_t LMASK = (1u << 29) - 1u;

// BN254 base field q = 0x30644e72e131a029b85045b68181585d97816a916871ca8d3c208c16d87cfd47
// (reference src/field/montgomery.cuh:33-38).
struct FqP {
  static constexpr uint32_t MOD[9] = {0x187cfd47u, 0x010460b6u, 0x1c72a34fu, 0x02d522d0u, 0x1585d978u,
                                      0x02db40c0u, 0x00a6e141u, 0x0e5c2634u, 0x0030644eu};
  static constexpr uint32_t MOD2[9] = {0x10f9fa8eu, 0x0208c16du, 0x18e5469eu, 0x05aa45a1u, 0x0b0bb2f0u,
                                       0x05b68181u, 0x014dc282u, 0x1cb84c68u, 0x0060c89cu};
  static constexpr uint32_t MOD3[9] = {0x0976f7d5u, 0x030d2224u, 0x1557e9edu, 0x087f6872u, 0x00918c68u,
                                       0x0891c242u, 0x01f4a3c3u, 0x0b14729cu, 0x00912cebu};
  static constexpr uint32_t MOD4[9] = {0x01f3f51cu, 0x041182dbu, 0x11ca8d3cu, 0x0b548b43u, 0x161765e0u,
                                       0x0b6d0302u, 0x029b8504u, 0x197098d0u, 0x00c19139u};
  static constexpr uint32_t MOD6[9] = {0x12edefaau, 0x061a4448u, 0x0aafd3dau, 0x10fed0e5u, 0x012318d0u,
                                       0x11238484u, 0x03e94786u, 0x1628e538u, 0x012259d6u};
  static constexpr uint32_t MOD8[9] = {0x03e7ea38u, 0x082305b6u, 0x03951a78u, 0x16a91687u, 0x0c2ecbc0u,
                                       0x16da0605u, 0x05370a08u, 0x12e131a0u, 0x01832273u};
  static constexpr uint32_t INV = 0x04866389u;  // -q^-1 mod 2^29
  static constexpr uint32_t ONE[9] = {0x157ccc21u, 0x141c2758u, 0x185230d3u, 0x014c0419u, 0x0aa36fb9u,
                                      0x1d4240ceu, 0x11d54c07u, 0x052ac7a8u, 0x000dc836u};  // 2^261 mod q
  static constexpr uint32_t R2[9] = {0x059bac10u, 0x0d1503a3u, 0x018016b8u, 0x10ab0ca8u, 0x02632639u,
                                     0x02c0169fu, 0x169bfd53u, 0x11869d4cu, 0x002a11a6u};  // 2^522 mod q
  static constexpr uint32_t K_IN[9] = {0x13349ca1u, 0x1a5d84a8u, 0x0a3e5cacu, 0x100249e0u, 0x12b951e8u,
                                       0x0e92d304u, 0x14cb95b3u, 0x041b9d3du, 0x00058003u};  // 2^266 mod q
  static constexpr uint32_t K_OUT[9] = {0x058f0d9du, 0x1aea1c6eu, 0x11c2cf74u, 0x11d651ebu, 0x1462c0a7u,
                                        0x11b7bc3cu, 0x1cbd99bau, 0x183340fbu, 0x000e0a77u};  // 2^256 mod q
};

// BN254 scalar field r = 0x30644e72e131a029b85045b68181585d2833e84879b9709143e1f593f0000001
// (reference src/field/fp.cuh:329-335).
struct FrP {
  static constexpr uint32_t MOD[9] = {0x10000001u, 0x1f0fac9fu, 0x0e5c2450u, 0x07d090f3u, 0x1585d283u,
                                      0x02db40c0u, 0x00a6e141u, 0x0e5c2634u, 0x0030644eu};
  static constexpr uint32_t MOD2[9] = {0x00000002u, 0x1e1f593fu, 0x1cb848a1u, 0x0fa121e6u, 0x0b0ba506u,
                                       0x05b68181u, 0x014dc282u, 0x1cb84c68u, 0x0060c89cu};
  static constexpr uint32_t MOD3[9] = {0x10000003u, 0x1d2f05deu, 0x0b146cf2u, 0x1771b2dau, 0x00917789u,
                                       0x0891c242u, 0x01f4a3c3u, 0x0b14729cu, 0x00912cebu};
  static constexpr uint32_t MOD4[9] = {0x00000004u, 0x1c3eb27eu, 0x19709143u, 0x1f4243cdu, 0x16174a0cu,
                                       0x0b6d0302u, 0x029b8504u, 0x197098d0u, 0x00c19139u};
  static constexpr uint32_t MOD6[9] = {0x00000006u, 0x1a5e0bbdu, 0x1628d9e5u, 0x0ee365b4u, 0x0122ef13u,
                                       0x11238484u, 0x03e94786u, 0x1628e538u, 0x012259d6u};
  static constexpr uint32_t MOD8[9] = {0x00000008u, 0x187d64fcu, 0x12e12287u, 0x1e84879bu, 0x0c2e9419u,
                                       0x16da0605u, 0x05370a08u, 0x12e131a0u, 0x01832273u};
  static constexpr uint32_t INV = 0x0fffffffu;  // -r^-1 mod 2^29
  static constexpr uint32_t ONE[9] = {0x0fffff57u, 0x1ea70ab4u, 0x052c068bu, 0x17504f49u, 0x0aa8075bu,
                                      0x1d4240ceu, 0x11d54c07u, 0x052ac7a8u, 0x000dc836u};  // 2^261 mod r
  static constexpr uint32_t R2[9] = {0x05b69bd4u, 0x06170a5au, 0x020cddceu, 0x1db6310bu, 0x0e54d0ffu,
                                     0x1cf855e3u, 0x1c15e103u, 0x07d09161u, 0x000a054au};  // 2^522 mod r
  static constexpr uint32_t K_IN[9] = {0x0fffead7u, 0x1d5444f4u, 0x04438aa5u, 0x03b4d096u, 0x134c84dau,
                                       0x0e92d304u, 0x14cb95b3u, 0x041b9d3du, 0x00058003u};  // 2^266 mod r
  static constexpr uint32_t K_OUT[9] = {0x0ffffffbu, 0x04b1a0e2u, 0x18334a6bu, 0x18ed2b3eu, 0x1462e36fu,
                                        0x11b7bc3cu, 0x1cbd99bau, 0x183340fbu, 0x000e0a77u};  // 2^256 mod r
};

template <class P>
struct fe {
  uint32_t l[NL];
};

using fq = fe<FqP>;
using fr = fe<FrP>;

template <class P>
ZK_HD fe<P> fe_zero() {
  fe<P> r;
#pragma unroll
  for (int i = 0; i < NL; i++) r.l[i] = 0;
  return r;
}

template <class P>
ZK_HD fe<P> fe_const(const uint32_t (&c)[NL]) {
  fe<P> r;
#pragma unroll
  for (int i = 0; i < NL; i++) r.l[i] = c[i];
  return r;
}

template <class P>
ZK_HD fe<P> fe_one() {
  return fe_const<P>(P::ONE);
}

#if defined(__HIP_DEVICE_COMPILE__)
// Device columns of the Montgomery products below: the same terms in the
// same columns, each column one serial multiply-add chain seeded with the
// incoming carry (mad_chain.hpp).  Every partial sum is a prefix of the
// column's sum, so the bounds stated for the products hold at every step.
//
// Reduction part of column K: q_i m_(K-i) for i < K, 1 <= K - i <= 8, then
// the column's own quotient (K < 9) or output limb (K >= 9), then the carry.
template <class P, int K>
__device__ __forceinline__ void mont_col_reduce(uint64_t& acc, uint32_t* q, fe<P>& r) {
  constexpr int rlo = K > NL - 1 ? K - (NL - 1) : 0;
  constexpr int nr = (K < NL ? K : NL) - rlo;
  if constexpr (nr > 0) {
    uint32_t x[nr], y[nr];
#pragma unroll
    for (int u = 0; u < nr; u++) {
      x[u] = q[rlo + u];
      y[u] = P::MOD[K - rlo - u];
    }
    mad_vs<nr>(acc, x, y);
  }
  if constexpr (K < NL) {
    q[K] = ((uint32_t)acc * P::INV) & LMASK;
    const uint32_t x[1] = {q[K]}, y[1] = {P::MOD[0]};
    mad_vs<1>(acc, x, y);
  } else {
    r.l[K - NL] = (uint32_t)acc & LMASK;
  }
  acc >>= 29;
}

// Column K of sum_t a[t]*b[t]: the products a[t]_i b[t]_(K-i), then the reduction.
template <class P, int N, int K>
__device__ __forceinline__ void mont_col(uint64_t& acc, const fe<P>* a, const fe<P>* b, uint32_t* q, fe<P>& r) {
  constexpr int ilo = K < NL ? 0 : K - NL + 1;
  constexpr int np = (K < NL ? K : NL - 1) - ilo + 1;
  uint32_t x[N * np], y[N * np];
#pragma unroll
  for (int t = 0; t < N; t++) {
#pragma unroll
    for (int u = 0; u < np; u++) {
      x[t * np + u] = a[t].l[ilo + u];
      y[t * np + u] = b[t].l[K - ilo - u];
    }
  }
  mad_vv<N * np>(acc, x, y);
  mont_col_reduce<P, K>(acc, q, r);
}

template <class P, int N, int... K>
__device__ __forceinline__ fe<P> mont_product(const fe<P>* a, const fe<P>* b, std::integer_sequence<int, K...>) {
  uint32_t q[NL];
  fe<P> r;
  uint64_t acc = 0;
  (mont_col<P, N, K>(acc, a, b, q, r), ...);
  r.l[NL - 1] = (uint32_t)acc;
  return r;
}

// Column K of a^2: cross products a_i (2 a_j), i < j, and the square of
// a_(K/2) for even K.  With limbs below 2^30 the largest column (K = 8: four
// cross products below 2^61, a square below 2^60, nine reduction products
// below 2^58, a carry below 2^35) stays below 1.41 * 2^63.
template <class P, int K>
__device__ __forceinline__ void sqr_col(uint64_t& acc, const fe<P>& a, const uint32_t* a2, uint32_t* q, fe<P>& r) {
  constexpr int ilo = K < NL ? 0 : K - NL + 1;
  constexpr int ihi = K >= 1 ? (K - 1) / 2 : -1;  // i < K - i
  constexpr int nc = ihi >= ilo ? ihi - ilo + 1 : 0;
  constexpr int nd = (K % 2 == 0) ? 1 : 0;
  uint32_t x[nc + nd], y[nc + nd];
#pragma unroll
  for (int u = 0; u < nc; u++) {
    x[u] = a.l[ilo + u];
    y[u] = a2[K - ilo - u];
  }
  if constexpr (nd) {
    x[nc] = a.l[K / 2];
    y[nc] = a.l[K / 2];
  }
  mad_vv<nc + nd>(acc, x, y);
  mont_col_reduce<P, K>(acc, q, r);
}

template <class P, int... K>
__device__ __forceinline__ fe<P> mont_square(const fe<P>& a, std::integer_sequence<int, K...>) {
  uint32_t q[NL], a2[NL];
  fe<P> r;
#pragma unroll
  for (int i = 0; i < NL; i++) a2[i] = a.l[i] << 1;
  uint64_t acc = 0;
  (sqr_col<P, K>(acc, a, a2, q, r), ...);
  r.l[NL - 1] = (uint32_t)acc;
  return r;
}
#endif

// Montgomery product a*b*2^-261 mod m, column (product-scanning) order with the
// reduction interleaved per column.  Inputs: limbs < 2^30.  Output: limbs
// < 2^29, value < a*b/2^261 + m, so below 2m for values < 8m, and also when
// one operand is below m and the other anywhere below 2^261.
template <class P>
ZK_HD fe<P> fmul(const fe<P>& a, const fe<P>& b) {
#if defined(__HIP_DEVICE_COMPILE__)
  return mont_product<P, 1>(&a, &b, std::make_integer_sequence<int, 2 * NL - 1>{});
#else
  uint32_t q[NL];
  fe<P> r;
  uint64_t acc = 0;
#pragma unroll
  for (int k = 0; k < 2 * NL - 1; k++) {
#pragma unroll
    for (int i = 0; i < NL; i++) {
      const int j = k - i;
      if (j >= 0 && j < NL) acc += (uint64_t)a.l[i] * b.l[j];
    }
#pragma unroll
    for (int i = 0; i < NL; i++) {
      const int j = k - i;
      if (i < k && j >= 1 && j < NL) acc += (uint64_t)q[i] * P::MOD[j];
    }
    if (k < NL) {
      q[k] = ((uint32_t)acc * P::INV) & LMASK;
      acc += (uint64_t)q[k] * P::MOD[0];
    } else {
      r.l[k - NL] = (uint32_t)acc & LMASK;
    }
    acc >>= 29;
  }
  r.l[NL - 1] = (uint32_t)acc;
  return r;
#endif
}

// sum_t a[t]*b[t] * 2^-261 mod m, N <= 4, with one Montgomery reduction for
// all products.  Inputs: normalized limbs (< 2^29), values <= 4m.  Every
// column then holds at most 9N + 9 terms below 2^58 plus a carry below 2^35,
// which stays below 2^64, and the result is below 64m^2 / 2^261 + m < 1.4m.
template <class P, int N>
ZK_HD fe<P> fmul_sum(const fe<P> (&a)[N], const fe<P> (&b)[N]) {
  static_assert(N >= 1 && N <= 4, "column accumulator bound");
#if defined(__HIP_DEVICE_COMPILE__)
  return mont_product<P, N>(a, b, std::make_integer_sequence<int, 2 * NL - 1>{});
#else
  uint32_t q[NL];
  fe<P> r;
  uint64_t acc = 0;
#pragma unroll
  for (int k = 0; k < 2 * NL - 1; k++) {
#pragma unroll
    for (int i = 0; i < NL; i++) {
      const int j = k - i;
      if (j >= 0 && j < NL) {
#pragma unroll
        for (int t = 0; t < N; t++) acc += (uint64_t)a[t].l[i] * b[t].l[j];
      }
    }
#pragma unroll
    for (int i = 0; i < NL; i++) {
      const int j = k - i;
      if (i < k && j >= 1 && j < NL) acc += (uint64_t)q[i] * P::MOD[j];
    }
    if (k < NL) {
      q[k] = ((uint32_t)acc * P::INV) & LMASK;
      acc += (uint64_t)q[k] * P::MOD[0];
    } else {
      r.l[k - NL] = (uint32_t)acc & LMASK;
    }
    acc >>= 29;
  }
  r.l[NL - 1] = (uint32_t)acc;
  return r;
#endif
}

// (a*b + c*e) * 2^-261 mod m: fmul_sum of two products (values < 4m).
template <class P>
ZK_HD fe<P> fmul2(const fe<P>& a, const fe<P>& b, const fe<P>& c, const fe<P>& e) {
  const fe<P> x[2] = {a, c}, y[2] = {b, e};
  return fmul_sum<P, 2>(x, y);
}

// Squaring: cross products are summed once and doubled per column.
template <class P>
ZK_HD fe<P> fsqr(const fe<P>& a) {
#if defined(__HIP_DEVICE_COMPILE__)
  return mont_square<P>(a, std::make_integer_sequence<int, 2 * NL - 1>{});
#else
  uint32_t q[NL];
  fe<P> r;
  uint64_t acc = 0;
#pragma unroll
  for (int k = 0; k < 2 * NL - 1; k++) {
    uint64_t cross = 0;
#pragma unroll
    for (int i = 0; i < NL; i++) {
      const int j = k - i;
      if (j > i && j < NL) cross += (uint64_t)a.l[i] * a.l[j];
    }
    acc += cross << 1;
    if ((k & 1) == 0 && k / 2 < NL) acc += (uint64_t)a.l[k / 2] * a.l[k / 2];
#pragma unroll
    for (int i = 0; i < NL; i++) {
      const int j = k - i;
      if (i < k && j >= 1 && j < NL) acc += (uint64_t)q[i] * P::MOD[j];
    }
    if (k < NL) {
      q[k] = ((uint32_t)acc * P::INV) & LMASK;
      acc += (uint64_t)q[k] * P::MOD[0];
    } else {
      r.l[k - NL] = (uint32_t)acc & LMASK;
    }
    acc >>= 29;
  }
  r.l[NL - 1] = (uint32_t)acc;
  return r;
#endif
}

// (a + b) mod m into [0, 2m).  Inputs normalized, values < 2m.
template <class P>
ZK_HD fe<P> fadd(const fe<P>& a, const fe<P>& b) {
  fe<P> s, t;
  uint32_t c = 0;
#pragma unroll
  for (int i = 0; i < NL; i++) {
    uint32_t v = a.l[i] + b.l[i] + c;
    c = v >> 29;
    s.l[i] = v & LMASK;
  }
  int32_t br = 0;
#pragma unroll
  for (int i = 0; i < NL; i++) {
    int32_t v = (int32_t)s.l[i] - (int32_t)P::MOD2[i] + br;
    br = v >> 29;
    t.l[i] = (uint32_t)v & LMASK;
  }
  // br == -1: s < 2m, keep s.
#pragma unroll
  for (int i = 0; i < NL; i++) s.l[i] = br ? s.l[i] : t.l[i];
  return s;
}

// (a - b) mod m into [0, 2m).  Inputs normalized, values < 2m.
template <class P>
ZK_HD fe<P> fsub(const fe<P>& a, const fe<P>& b) {
  fe<P> d;
  int32_t br = 0;
#pragma unroll
  for (int i = 0; i < NL; i++) {
    int32_t v = (int32_t)a.l[i] - (int32_t)b.l[i] + br;
    br = v >> 29;
    d.l[i] = (uint32_t)v & LMASK;
  }
  const uint32_t mask = (uint32_t)br;  // all ones when a < b
  uint32_t c = 0;
#pragma unroll
  for (int i = 0; i < NL; i++) {
    uint32_t v = d.l[i] + (P::MOD2[i] & mask) + c;
    c = v >> 29;
    d.l[i] = v & LMASK;
  }
  return d;
}

// a - b + 2m without the final correction: value in (0, 4m) for a, b in
// [0, 2m), normalized limbs.  Valid only as a multiplication input.
template <class P>
ZK_HD fe<P> fsub_lazy(const fe<P>& a, const fe<P>& b) {
  fe<P> d;
  int32_t c = 0;
#pragma unroll
  for (int i = 0; i < NL; i++) {
    int32_t v = (int32_t)a.l[i] + (int32_t)P::MOD2[i] - (int32_t)b.l[i] + c;
    c = v >> 29;
    d.l[i] = (uint32_t)v & LMASK;
  }
  return d;
}

// 2m - a for a in [0, 2m]: value in [0, 2m], normalized limbs (congruent to
// -a; not reduced, so a valid multiplication input only).
template <class P>
ZK_HD fe<P> fneg_lazy(const fe<P>& a) {
  fe<P> d;
  int32_t c = 0;
#pragma unroll
  for (int i = 0; i < NL; i++) {
    int32_t v = (int32_t)P::MOD2[i] - (int32_t)a.l[i] + c;
    c = v >> 29;
    d.l[i] = (uint32_t)v & LMASK;
  }
  return d;
}

// neg ? m - a : a for a canonical (in [0, m)); m - a is in (0, m], a valid
// value of the lazy range [0, 2m).
template <class P>
ZK_HD fe<P> fneg_canon_if(const fe<P>& a, bool neg) {
  fe<P> d;
  int32_t br = 0;
#pragma unroll
  for (int i = 0; i < NL; i++) {
    int32_t v = (int32_t)P::MOD[i] - (int32_t)a.l[i] + br;
    br = v >> 29;
    d.l[i] = (uint32_t)v & LMASK;
  }
#pragma unroll
  for (int i = 0; i < NL; i++) d.l[i] = neg ? d.l[i] : a.l[i];
  return d;
}

template <class P>
ZK_HD fe<P> fneg(const fe<P>& a) {
  return fsub(fe_zero<P>(), a);
}

template <class P>
ZK_HD fe<P> fdbl(const fe<P>& a) {
  return fadd(a, a);
}

// a + b with carries and no reduction: normalized limbs, value in [0, 4m) for
// a, b in [0, 2m).
template <class P>
ZK_HD fe<P> fadd_wide(const fe<P>& a, const fe<P>& b) {
  fe<P> s;
  uint32_t c = 0;
#pragma unroll
  for (int i = 0; i < NL; i++) {
    uint32_t v = a.l[i] + b.l[i] + c;
    c = v >> 29;
    s.l[i] = v & LMASK;
  }
  return s;
}

// Limb-wise sum without normalization: limbs < 2^30, value < 4m.  Valid only
// as a direct input of fmul/fsqr.
template <class P>
ZK_HD fe<P> fadd_lazy(const fe<P>& a, const fe<P>& b) {
  fe<P> s;
#pragma unroll
  for (int i = 0; i < NL; i++) s.l[i] = a.l[i] + b.l[i];
  return s;
}

// Reduce [0, 2m) to the canonical [0, m).
template <class P>
ZK_HD fe<P> fcanon(const fe<P>& a) {
  fe<P> t;
  int32_t br = 0;
#pragma unroll
  for (int i = 0; i < NL; i++) {
    int32_t v = (int32_t)a.l[i] - (int32_t)P::MOD[i] + br;
    br = v >> 29;
    t.l[i] = (uint32_t)v & LMASK;
  }
  fe<P> r;
#pragma unroll
  for (int i = 0; i < NL; i++) r.l[i] = br ? a.l[i] : t.l[i];
  return r;
}

// a == 0 mod m for a in [0, 2m): a is 0 or m.
template <class P>
ZK_HD bool fis_zero(const fe<P>& a) {
  uint32_t z = 0, e = 0;
#pragma unroll
  for (int i = 0; i < NL; i++) {
    z |= a.l[i];
    e |= a.l[i] ^ P::MOD[i];
  }
  return z == 0 || e == 0;
}

// a == 0 mod m for a in [0, 4m): a is 0, m, 2m or 3m.
template <class P>
ZK_HD bool fis_zero4(const fe<P>& a) {
  uint32_t z = 0, e1 = 0, e2 = 0, e3 = 0;
#pragma unroll
  for (int i = 0; i < NL; i++) {
    z |= a.l[i];
    e1 |= a.l[i] ^ P::MOD[i];
    e2 |= a.l[i] ^ P::MOD2[i];
    e3 |= a.l[i] ^ P::MOD3[i];
  }
  return z == 0 || e1 == 0 || e2 == 0 || e3 == 0;
}

// t - K if t >= K (K normalized limbs), else t.
template <class P>
ZK_HD fe<P> fcsub(const fe<P>& t, const uint32_t (&K)[NL]) {
  fe<P> u;
  int32_t br = 0;
#pragma unroll
  for (int i = 0; i < NL; i++) {
    int32_t v = (int32_t)t.l[i] - (int32_t)K[i] + br;
    br = v >> 29;
    u.l[i] = (uint32_t)v & LMASK;
  }
  fe<P> r;
#pragma unroll
  for (int i = 0; i < NL; i++) r.l[i] = br ? t.l[i] : u.l[i];
  return r;
}

// (a - b - 2c) mod m into [0, 2m) for a, b, c in [0, 2m): one pass forms
// a + 6m - b - 2c in (0, 8m), then two conditional subtractions of 4m, 2m.
template <class P>
ZK_HD fe<P> fsub3(const fe<P>& a, const fe<P>& b, const fe<P>& c) {
  fe<P> t;
  int32_t cy = 0;
#pragma unroll
  for (int i = 0; i < NL; i++) {
    int32_t v = (int32_t)a.l[i] + (int32_t)P::MOD6[i] - (int32_t)b.l[i] - 2 * (int32_t)c.l[i] + cy;
    cy = v >> 29;
    t.l[i] = (uint32_t)v & LMASK;
  }
  return fcsub(fcsub(t, P::MOD4), P::MOD2);
}

// a - b + 4m for a in [0, 4m), b in [0, 4m]: value in (0, 8m), normalized
// limbs.  Valid only as an fmul / fsqr input.
template <class P>
ZK_HD fe<P> fsub_lazy4(const fe<P>& a, const fe<P>& b) {
  fe<P> d;
  int32_t c = 0;
#pragma unroll
  for (int i = 0; i < NL; i++) {
    int32_t v = (int32_t)a.l[i] + (int32_t)P::MOD4[i] - (int32_t)b.l[i] + c;
    c = v >> 29;
    d.l[i] = (uint32_t)v & LMASK;
  }
  return d;
}

// 4m - a for a in [0, 4m]: value in [0, 4m], normalized limbs.
template <class P>
ZK_HD fe<P> fneg_lazy4(const fe<P>& a) {
  fe<P> d;
  int32_t c = 0;
#pragma unroll
  for (int i = 0; i < NL; i++) {
    int32_t v = (int32_t)P::MOD4[i] - (int32_t)a.l[i] + c;
    c = v >> 29;
    d.l[i] = (uint32_t)v & LMASK;
  }
  return d;
}

// a - b + KM*m with carries (KM in {2, 4, 8}): for b < KM*m the value is
// a - b + KM*m > 0 with normalized limbs (valid while below 2^261).
template <int KM, class P>
ZK_HD fe<P> fsub_off(const fe<P>& a, const fe<P>& b) {
  static_assert(KM == 2 || KM == 4 || KM == 8, "offset multiple");
  const uint32_t(&K)[NL] = KM == 2 ? P::MOD2 : KM == 4 ? P::MOD4 : P::MOD8;
  fe<P> d;
  int32_t c = 0;
#pragma unroll
  for (int i = 0; i < NL; i++) {
    int32_t v = (int32_t)a.l[i] + (int32_t)K[i] - (int32_t)b.l[i] + c;
    c = v >> 29;
    d.l[i] = (uint32_t)v & LMASK;
  }
  return d;
}

// Canonical value of x (normalized limbs, any value below 2^261).  Both
// moduli have top limb M8 = 0x30644e; q = (l8 * floor(2^40 / (M8 + 1))) >> 40
// never exceeds floor(x / m) and falls short of it by at most 2, so
// x - q m < 3m and two conditional subtractions finish.
template <class P>
ZK_HD fe<P> freduce(const fe<P>& x) {
  static_assert(P::MOD[NL - 1] == 0x0030644eu, "quotient estimate assumes the BN254 top limb");
  const uint32_t q = (uint32_t)(((uint64_t)x.l[NL - 1] * 346695ull) >> 40);
  fe<P> r;
  int64_t c = 0;
#pragma unroll
  for (int i = 0; i < NL; i++) {
    const int64_t t = (int64_t)x.l[i] - (int64_t)q * (int64_t)P::MOD[i] + c;
    r.l[i] = (uint32_t)t & LMASK;
    c = t >> 29;
  }
  return fcsub(fcsub(r, P::MOD2), P::MOD);
}

template <class P>
ZK_HD bool feq(const fe<P>& a, const fe<P>& b) {
  return fis_zero(fsub(a, b));
}

// Bit repack of a 256-bit little-endian word array into 29-bit limbs (no change
// of value).
template <class P>
ZK_HD fe<P> repack_in(const uint32_t w[8]) {
  fe<P> r;
#pragma unroll
  for (int i = 0; i < NL; i++) {
    const int bit = 29 * i;
    const int wd = bit >> 5;
    const int sh = bit & 31;
    uint64_t v = w[wd];
    if (wd + 1 < 8) v |= (uint64_t)w[wd + 1] << 32;
    r.l[i] = (uint32_t)(v >> sh) & LMASK;
  }
  return r;
}

// Canonicalize and repack into 8 little-endian 32-bit words.
template <class P>
ZK_HD void repack_out(const fe<P>& a, uint32_t w[8]) {
  fe<P> c = fcanon(a);
#pragma unroll
  for (int j = 0; j < 8; j++) {
    const int bit = 32 * j;
    const int i = bit / 29;
    const int sh = bit % 29;
    uint64_t v = c.l[i];
    if (i + 1 < NL) v |= (uint64_t)c.l[i + 1] << 29;
    if (i + 2 < NL && sh > 26) v |= (uint64_t)c.l[i + 2] << 58;
    w[j] = (uint32_t)(v >> sh);
  }
}

// Reference Montgomery form (R = 2^256) <-> internal form (R' = 2^261).
template <class P>
ZK_HD fe<P> from_mont256(const uint32_t w[8]) {
  return fmul(repack_in<P>(w), fe_const<P>(P::K_IN));
}

template <class P>
ZK_HD void to_mont256(const fe<P>& a, uint32_t w[8]) {
  repack_out(fmul(a, fe_const<P>(P::K_OUT)), w);
}

// Plain integer (standard form) <-> internal form.
template <class P>
ZK_HD fe<P> from_std(const uint32_t w[8]) {
  return fmul(repack_in<P>(w), fe_const<P>(P::R2));
}

template <class P>
ZK_HD void to_std(const fe<P>& a, uint32_t w[8]) {
  fe<P> one_plain = fe_zero<P>();
  one_plain.l[0] = 1;
  repack_out(fmul(a, one_plain), w);
}

// Square-and-multiply with a 256-bit plain exponent (little-endian words).
template <class P>
ZK_HD fe<P> fpow(const fe<P>& a, const uint32_t e[8]) {
  fe<P> r = fe_one<P>();
  for (int bit = 255; bit >= 0; bit--) {
    r = fsqr(r);
    if ((e[bit >> 5] >> (bit & 31)) & 1u) r = fmul(r, a);
  }
  return r;
}

}  // namespace zk
