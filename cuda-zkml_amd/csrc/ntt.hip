// BN254 Fr NTT, inverse NTT and coset NTT for gfx950.
//
// Replaces bn254::ntt_gpu (reference src/ntt/ntt.cu:354-465): a bit-reversal
// kernel, a shared-memory kernel for the first ten stages and one HBM pass per
// remaining stage with host-built twiddles.  Here a transform of n = 2^L is a
// four-step (Bailey) decomposition n = R_0 * ... * R_{P-1} with P <= 3 passes
// over HBM and R_p <= 256:
//
//   digits of the input index (most significant first) i_0 .. i_{P-1};
//   pass p < P-1: DFT of size R_p over digit i_p for every setting of the
//     other digits, result k_p written back to the same positions, then
//     multiplied by w_{R_p S_p}^(k_p * m) with m the index formed by the lower
//     digits (S_p = R_{p+1} * ... * R_{P-1});
//   pass P-1: DFT over the last digit and a digit-reversed store, so that the
//     output index is k_0 + R_0 k_1 + R_0 R_1 k_2 (natural order).
//
// A pass works on tiles of R rows (the DFT's length) x T columns (T
// neighbouring transforms, adjacent in HBM for the first passes).  Each
// thread owns 2^KMAX elements of a column and runs the DFT as radix-2^KMAX
// decimation-in-time steps held in registers:
//   * the first step reads its elements straight from HBM at bit-reversed
//     rows (so no bit-reversal pass exists) and its twiddles are the same for
//     every thread (w_2, w_4, w_8 powers, several of them 1);
//   * the steps in between exchange elements through LDS (nine 29-bit limb
//     planes, rows XOR-swizzled against bank conflicts) with per-thread
//     twiddles w_R^e from an LDS copy of the pass's table;
//   * the last step writes its outputs straight to HBM, multiplied by the
//     inter-pass twiddle (or the coset / 1/n factor of the last pass).
//
// Butterflies are lazy: u + w v and u - w v + 2m with carries normalised but
// no modular reduction, so a value grows by at most 2m per stage (w v is a
// Montgomery product, below 2m).  After the eight stages of a pass it is
// below 26m, far inside the 2^261 range of nine 29-bit limbs; the pass's
// output multiply brings it back below 2m, and the last pass reduces to the
// canonical range.  The inverse transform's 1/n rides in the first
// inter-pass table, so it costs no multiply.
//
// Radix bookkeeping: the NTT is linear, so the kernels run directly on the
// 256-bit words of the reference's Montgomery form (repack only); twiddles and
// scale tables are prepared in the internal 2^261 radix so that each fmul
// multiplies the stored integers by the intended field constant.
#include <string.h>

#include <utility>

#include "zk_internal.hpp"

namespace zk {

constexpr int NTT_MAX_LOG = 24;
constexpr int NTT_MAX_LOGR = 8;

// Table of internal-form field elements.  Twiddles of a DFT step (copied to
// LDS planes) are limb-major: limb l of entry i at l*count + i.  Tables read
// per element from HBM (inter-pass twiddles, coset factors) are packed like
// the elements, 8 words per entry: a tile row of T columns then reads T * 32
// contiguous bytes, where nine limb planes would read nine runs of T * 4
// bytes, each a fraction of a cache line (measured at 2^22: the first pass
// fetched 0.74 GB for 0.28 GB of elements and table).
constexpr int PACKED_WORDS = 8;
struct FrTable {
  uint32_t* d = nullptr;
  size_t count = 0;
};

struct NttPlan {
  int log_n = 0, P = 0;
  int logR[3] = {0, 0, 0};
  FrTable twr[3][2];  // [pass][direction]: w_{R_p}^e, e < R_p / 2
  FrTable twp[2][2];  // [pass < P-1][direction]: w_{R_p S_p}^(k m); the inverse pass-0 table carries 1/n
  uint32_t ninv[NL];  // n^-1 in internal form
};

// Per (log_n, g): g^i (forward coset pre-multiply), g^-i / n^[P == 1]
// (inverse coset post-multiply) and g^i / n^[P == 1] (an inverse transform
// whose output goes on to a coset transform).
struct CosetTables {
  FrTable pre, post_inv, post_fold;
};

__device__ __forceinline__ void store_table(uint32_t* __restrict__ t, size_t count, size_t i, const fr& x) {
  fr c = fcanon(x);
#pragma unroll
  for (int l = 0; l < NL; l++) t[l * count + i] = c.l[l];
}

__device__ __forceinline__ fr load_elem(const uint4* __restrict__ p, size_t i) {
  uint4 a = p[2 * i], b = p[2 * i + 1];
  uint32_t w[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
  return repack_in<FrP>(w);
}

// Pack nine limbs of a value below 2^256 into eight words (no reduction).
__device__ __forceinline__ void store_elem_raw(uint4* __restrict__ p, size_t i, const fr& x) {
  uint32_t w[8];
#pragma unroll
  for (int j = 0; j < 8; j++) {
    const int bit = 32 * j;
    const int k = bit / 29;
    const int sh = bit % 29;
    uint64_t v = x.l[k];
    if (k + 1 < NL) v |= (uint64_t)x.l[k + 1] << 29;
    if (k + 2 < NL && sh > 26) v |= (uint64_t)x.l[k + 2] << 58;
    w[j] = (uint32_t)(v >> sh);
  }
  p[2 * i] = make_uint4(w[0], w[1], w[2], w[3]);
  p[2 * i + 1] = make_uint4(w[4], w[5], w[6], w[7]);
}

// Packed tables: canonical values (below m < 2^256) in the element layout.
__device__ __forceinline__ fr load_packed(const uint32_t* __restrict__ t, size_t i) {
  return load_elem((const uint4*)t, i);
}
__device__ __forceinline__ void store_packed(uint32_t* __restrict__ t, size_t i, const fr& x) {
  store_elem_raw((uint4*)t, i, fcanon(x));
}

__device__ __forceinline__ uint32_t bitrev(uint32_t x, int bits) { return bits ? __brev(x) >> (32 - bits) : 0; }

// ------------------------------------------------------------------ pass kernel
enum { PRE_NONE = 0, PRE_TABLE = 1, PRE_QUOTIENT = 2 };
enum { POST_NONE = 0, POST_SCALE = 1, POST_TABLE = 2 };

struct PassGeo {
  uint32_t logR, logT;  // DFT length and tile columns
  uint32_t logS;        // middle pass: stride of this digit
  uint32_t logR0, logS0, logS1, logNR;  // last pass: first-digit count and stride, middle-digit stride, log(n/R)
  uint64_t n;
};

struct PassIO {
  const uint4* src;
  uint4* dst;
  const uint32_t* twr;   // w_R^e, e < R/2 (R/2 entries)
  const uint32_t* twp;   // middle pass: inter-pass table, R * S entries
  const uint32_t* pre;   // PRE_TABLE: n entries by input position
  const uint32_t* post;  // POST_TABLE: n entries by output position
  int pre_mode, post_mode;
  fr scale;              // POST_SCALE
  fr kc, zk;             // PRE_QUOTIENT: h = (a b - c kc) zk
};

// LDS word of (row p, column c) in a plane: rows swizzled so that the 32/T
// rows a half-wave touches at once (T < 32) fall in different banks.
__device__ __forceinline__ uint32_t lds_ix(uint32_t p, uint32_t c, uint32_t logT, uint32_t smask) {
  return ((p ^ ((p >> 3) & smask)) << logT) + c;
}

__device__ __forceinline__ fr lds_get(const uint32_t* s, uint32_t E, uint32_t ix) {
  fr x;
#pragma unroll
  for (int l = 0; l < NL; l++) x.l[l] = s[l * E + ix];
  return x;
}

__device__ __forceinline__ void lds_put(uint32_t* s, uint32_t E, uint32_t ix, const fr& x) {
#pragma unroll
  for (int l = 0; l < NL; l++) s[l * E + ix] = x.l[l];
}

__device__ __forceinline__ fr tw_get(const uint32_t* tw, uint32_t half, uint32_t e) {
  fr x;
#pragma unroll
  for (int l = 0; l < NL; l++) x.l[l] = tw[l * half + e];
  return x;
}

// f(integral_constant<int, I>) for I = 0 .. N-1, expanded at compile time so
// that every register-array index inside is a constant.
template <class F, int... I>
__device__ __forceinline__ void unroll_seq(F&& f, std::integer_sequence<int, I...>) {
  (f(std::integral_constant<int, I>{}), ...);
}
template <int N, class F>
__device__ __forceinline__ void unroll(F&& f) {
  unroll_seq(f, std::make_integer_sequence<int, N>{});
}

// One lazy DIT butterfly with a twiddle: (u + w v, u - w v + 2m).
__device__ __forceinline__ void bfly(fr& u, fr& v, const fr& w) {
  const fr t = fmul(v, w);
  v = fsub_off<2>(u, t);
  u = fadd_wide(u, t);
}

// Index of the p-th pair's lower element at sub-stage i (bit i clear).
template <int I, int P>
constexpr int pair_lo() {
  return ((P >> I) << (I + 1)) | (P & ((1 << I) - 1));
}

// First step of a tile: K radix-2 stages (h = 1 .. 2^(K-1)) whose twiddles
// w_{2^(i+1)}^(t mod 2^i) are the same for every group; index 0 is 1 and is
// skipped (the subtraction then adds the bound of its operand: inputs below
// 2m give at most 2^(i+2) m after sub-stage i).
template <int K>
__device__ __forceinline__ void first_step(fr (&x)[1 << K], const uint32_t* tw, uint32_t half, uint32_t logR) {
  unroll<K>([&](auto I) {
    constexpr int i = decltype(I)::value, hi = 1 << i;
    unroll<(1 << K) / 2>([&](auto Pp) {
      constexpr int t = pair_lo<i, decltype(Pp)::value>();
      constexpr int lo = t & (hi - 1);
      if constexpr (lo == 0) {
        const fr u = x[t], v = x[t + hi];
        x[t] = fadd_wide(u, v);
        x[t + hi] = fsub_off<(i == 0 ? 2 : i == 1 ? 4 : 8)>(u, v);
      } else {
        bfly(x[t], x[t + hi], tw_get(tw, half, (uint32_t)lo << (logR - 1 - i)));
      }
    });
  });
}

// A step of K stages starting at stage s (h = 2^s) on the group
// {j0 + t h : t < 2^K}, jl = j0 mod h: sub-stage i pairs t, t + 2^i with
// twiddle w_{2 h 2^i}^(jl + (t mod 2^i) h) = w_R^((jl + (t mod 2^i) h) << (logR-1-s-i)).
template <int K>
__device__ __forceinline__ void mid_step(fr (&x)[1 << K], const uint32_t* tw, uint32_t half, uint32_t logR,
                                         uint32_t s, uint32_t jl) {
  unroll<K>([&](auto I) {
    constexpr int i = decltype(I)::value, hi = 1 << i;
    unroll<(1 << K) / 2>([&](auto Pp) {
      constexpr int t = pair_lo<i, decltype(Pp)::value>();
      const uint32_t e = (jl + ((uint32_t)(t & (hi - 1)) << s)) << (logR - 1 - s - i);
      bfly(x[t], x[t + hi], tw_get(tw, half, e));
    });
  });
}
// Tile origin of a pass: middle passes read and write (row r, column c) at
// base + (r << logS) + c, base = u R S + m0 (m0 = the tile's first column);
// the last pass reads (k0s + c) S0 + v S1 + r and writes output index
// (k0s + c) + v R0 + k n / R.
struct TileOrigin {
  size_t base;
  uint32_t m0, k0s, v;
};

template <bool LAST>
__device__ __forceinline__ size_t in_pos(const PassGeo& g, const TileOrigin& o, uint32_t r, uint32_t c) {
  if (LAST) return ((size_t)(o.k0s + c) << g.logS0) + o.base + r;
  return o.base + ((size_t)r << g.logS) + c;
}

// (a b - c kc) zk: the quotient's pointwise step on the three transforms'
// values at position pos (a, b, c canonical; result below 2m).
__device__ __forceinline__ fr quotient_in(const PassGeo& g, const PassIO& io, const uint4* src, size_t pos) {
  const fr a = load_elem(src, pos), b = load_elem(src + 2 * g.n, pos), c = load_elem(src + 4 * g.n, pos);
  return fmul(fsub(fmul(a, b), fmul(c, io.kc)), io.zk);
}

// Last step of a pass, output row (digit) k of column c: the pass's
// multiply and its HBM position.  Middle passes multiply by the inter-pass
// twiddle (result below 2m < 2^256, stored as is); the last pass multiplies
// by its post table or constant and canonicalises, or reduces the lazy
// value when there is no multiply.
template <bool LAST>
__device__ __forceinline__ fr finish(const PassGeo& g, const PassIO& io, const TileOrigin& o, uint32_t k, uint32_t c,
                                     const fr& x, size_t& pos) {
  if (!LAST) {
    const size_t rel = ((size_t)k << g.logS) + o.m0 + c;
    pos = o.base + ((size_t)k << g.logS) + c;
    return fmul(x, load_packed(io.twp, rel));
  }
  pos = (size_t)(o.k0s + c) + ((size_t)o.v << g.logR0) + ((size_t)k << g.logNR);
  if (io.post_mode == POST_NONE) return freduce(x);
  const fr m = io.post_mode == POST_TABLE ? load_packed(io.post, pos) : io.scale;
  return fcanon(fmul(x, m));
}

// Everything a step of a tile needs.
struct TileCtx {
  uint32_t* s;           // LDS planes
  const uint32_t* tw;    // LDS twiddles w_R^e
  uint32_t E, half, logR, logT, smask, cmask, tid, nthr;
};

// First step of K stages: each group (q, c) loads rows bitrev(q) +
// bitrev(t) R / 2^K (t < 2^K), optionally pre-multiplied, and leaves the DIT
// positions (q << K) + t in LDS.
template <int K, int EPT, bool LAST>
__device__ __forceinline__ void tile_first(const TileCtx& tc, const PassGeo& g, const PassIO& io, const uint4* src,
                                           const TileOrigin& o) {
  for (uint32_t gi = 0; gi < (uint32_t)(EPT >> K); gi++) {
    const uint32_t grp = tc.tid + gi * tc.nthr;
    const uint32_t q = grp >> tc.logT, c = grp & tc.cmask;
    const uint32_t rq = bitrev(q, tc.logR - K);
    fr x[1 << K];
    auto row = [&](int t) { return in_pos<LAST>(g, o, rq + (bitrev(t, K) << (tc.logR - K)), c); };
    if (io.pre_mode == PRE_QUOTIENT) {
      unroll<(1 << K)>([&](auto T) { x[T] = quotient_in(g, io, src, row(T)); });
    } else {
      unroll<(1 << K)>([&](auto T) { x[T] = load_elem(src, row(T)); });
      if (io.pre_mode == PRE_TABLE)
        unroll<(1 << K)>([&](auto T) { x[T] = fmul(x[T], load_packed(io.pre, row(T))); });
    }
    first_step<K>(x, tc.tw, tc.half, tc.logR);
    unroll<(1 << K)>([&](auto T) { lds_put(tc.s, tc.E, lds_ix((q << K) + T, c, tc.logT, tc.smask), x[T]); });
  }
}

// A later step of K stages starting at stage s: group (q, c) holds rows
// j0 + t 2^s; results back to LDS (OUT = false) or out of the pass (OUT =
// true).  The groups of a step are disjoint, so each thread reads and
// writes back its own rows and only the barrier between steps is needed.
template <int K, int EPT, bool LAST, bool OUT>
__device__ __forceinline__ void tile_step(const TileCtx& tc, const PassGeo& g, const PassIO& io, uint4* dst,
                                          const TileOrigin& o, uint32_t s) {
  const uint32_t h = 1u << s;
  for (uint32_t gi = 0; gi < (uint32_t)(EPT >> K); gi++) {
    const uint32_t grp = tc.tid + gi * tc.nthr;
    const uint32_t q = grp >> tc.logT, c = grp & tc.cmask;
    const uint32_t jl = q & (h - 1);
    const uint32_t j0 = ((q >> s) << (s + K)) | jl;
    fr x[1 << K];
    unroll<(1 << K)>([&](auto T) { x[T] = lds_get(tc.s, tc.E, lds_ix(j0 + ((uint32_t)T << s), c, tc.logT, tc.smask)); });
    mid_step<K>(x, tc.tw, tc.half, tc.logR, s, jl);
    if constexpr (OUT) {
      unroll<(1 << K)>([&](auto T) {
        size_t pos;
        const fr y = finish<LAST>(g, io, o, j0 + ((uint32_t)T << s), c, x[T], pos);
        store_elem_raw(dst, pos, y);
      });
    } else {
      unroll<(1 << K)>([&](auto T) { lds_put(tc.s, tc.E, lds_ix(j0 + ((uint32_t)T << s), c, tc.logT, tc.smask), x[T]); });
    }
  }
}

// All rows of a tile from LDS straight out (a single-step DFT).
template <int EPT, bool LAST>
__device__ __forceinline__ void tile_copy_out(const TileCtx& tc, const PassGeo& g, const PassIO& io, uint4* dst,
                                              const TileOrigin& o) {
  for (uint32_t e = tc.tid; e < tc.E; e += tc.nthr) {
    const uint32_t q = e >> tc.logT, c = e & tc.cmask;
    size_t pos;
    const fr y = finish<LAST>(g, io, o, q, c, lds_get(tc.s, tc.E, lds_ix(q, c, tc.logT, tc.smask)), pos);
    store_elem_raw(dst, pos, y);
  }
}

// ---- fixed-geometry tiles: the elements stay in registers between steps
// and move through LDS in two halves (limbs 0-4, then 5-8) over five planes,
// so a 2048-element tile takes 45 KB of LDS instead of 78 KB and three
// blocks (three waves per SIMD) fit on a CU where two did.
constexpr int NTT_XPLANES = 5;

// LDS rows of a step of K stages starting at stage s: group gi of the
// thread holds rows j0 + t 2^s (t < 2^K) of column c; element e = gi 2^K + t.
template <int EPT, int K>
__device__ __forceinline__ void step_rows(const TileCtx& tc, uint32_t s, uint32_t (&row)[EPT], uint32_t (&col)[EPT],
                                          uint32_t (&jl)[EPT >> K]) {
  const uint32_t h = 1u << s;
  unroll<(EPT >> K)>([&](auto GI) {
    const uint32_t grp = tc.tid + (uint32_t)GI * tc.nthr;
    const uint32_t q = grp >> tc.logT, c = grp & tc.cmask;
    const uint32_t l = q & (h - 1);
    jl[GI] = l;
    const uint32_t j0 = ((q >> s) << (s + K)) | l;
    unroll<(1 << K)>([&](auto T) {
      row[GI * (1 << K) + T] = j0 + ((uint32_t)T << s);
      col[GI * (1 << K) + T] = c;
    });
  });
}

// Registers x (at LDS index ixo of each element) to the elements at ixi.
template <int EPT>
__device__ __forceinline__ void xchg_halves(const TileCtx& tc, fr (&x)[EPT], const uint32_t (&ixo)[EPT],
                                            const uint32_t (&ixi)[EPT]) {
  uint32_t* s = tc.s;
  const uint32_t E = tc.E;
  uint32_t lo[EPT][NTT_XPLANES];
  __syncthreads();
  unroll<EPT>([&](auto e) { unroll<NTT_XPLANES>([&](auto l) { s[l * E + ixo[e]] = x[e].l[l]; }); });
  __syncthreads();
  unroll<EPT>([&](auto e) { unroll<NTT_XPLANES>([&](auto l) { lo[e][l] = s[l * E + ixi[e]]; }); });
  __syncthreads();
  unroll<EPT>([&](auto e) { unroll<NL - NTT_XPLANES>([&](auto l) { s[l * E + ixo[e]] = x[e].l[NTT_XPLANES + l]; }); });
  __syncthreads();
  unroll<EPT>([&](auto e) {
    unroll<NL - NTT_XPLANES>([&](auto l) { x[e].l[NTT_XPLANES + l] = s[l * E + ixi[e]]; });
    unroll<NTT_XPLANES>([&](auto l) { x[e].l[l] = lo[e][l]; });
  });
}

// A whole pass over one tile of R = 2^LR rows (LR > KMAX) with the tile's
// elements in registers: first step from HBM, middle steps of KMAX stages,
// the last step of the remaining stages straight to HBM.
template <int KMAX, bool LAST, int LR>
__device__ __forceinline__ void tile_fixed(const TileCtx& tc, const PassGeo& g, const PassIO& io, const uint4* src,
                                           uint4* dst, const TileOrigin& o) {
  constexpr int EPT = 1 << KMAX;
  constexpr int NSTEPS = (LR + KMAX - 1) / KMAX;
  constexpr int KLAST = LR - KMAX * (NSTEPS - 1);
  static_assert(NSTEPS >= 2, "fixed tiles take at least two steps");
  fr x[EPT];
  uint32_t ixo[EPT], ixi[EPT];
  {
    const uint32_t q = tc.tid >> tc.logT, c = tc.tid & tc.cmask;
    const uint32_t rq = bitrev(q, LR - KMAX);
    auto rowp = [&](int t) { return in_pos<LAST>(g, o, rq + (bitrev(t, KMAX) << (LR - KMAX)), c); };
    if (io.pre_mode == PRE_QUOTIENT) {
      unroll<EPT>([&](auto T) { x[T] = quotient_in(g, io, src, rowp(T)); });
    } else {
      unroll<EPT>([&](auto T) { x[T] = load_elem(src, rowp(T)); });
      if (io.pre_mode == PRE_TABLE) unroll<EPT>([&](auto T) { x[T] = fmul(x[T], load_packed(io.pre, rowp(T))); });
    }
    first_step<KMAX>(x, tc.tw, tc.half, LR);
    unroll<EPT>([&](auto T) { ixo[T] = lds_ix((q << KMAX) + T, c, tc.logT, tc.smask); });
  }
  uint32_t stage = KMAX;
  unroll<NSTEPS - 2>([&](auto) {
    uint32_t row[EPT], col[EPT], jl[1];
    step_rows<EPT, KMAX>(tc, stage, row, col, jl);
    unroll<EPT>([&](auto e) { ixi[e] = lds_ix(row[e], col[e], tc.logT, tc.smask); });
    xchg_halves<EPT>(tc, x, ixo, ixi);
    mid_step<KMAX>(x, tc.tw, tc.half, LR, stage, jl[0]);
    unroll<EPT>([&](auto e) { ixo[e] = ixi[e]; });
    stage += KMAX;
  });
  uint32_t row[EPT], col[EPT], jl[EPT >> KLAST];
  step_rows<EPT, KLAST>(tc, stage, row, col, jl);
  unroll<EPT>([&](auto e) { ixi[e] = lds_ix(row[e], col[e], tc.logT, tc.smask); });
  xchg_halves<EPT>(tc, x, ixo, ixi);
  unroll<(EPT >> KLAST)>([&](auto GI) {
    fr y[1 << KLAST];
    unroll<(1 << KLAST)>([&](auto T) { y[T] = x[GI * (1 << KLAST) + T]; });
    mid_step<KLAST>(y, tc.tw, tc.half, LR, stage, jl[GI]);
    unroll<(1 << KLAST)>([&](auto T) {
      size_t pos;
      const fr r = finish<LAST>(g, io, o, row[GI * (1 << KLAST) + T], col[GI * (1 << KLAST) + T], y[T], pos);
      store_elem_raw(dst, pos, r);
    });
  });
}

// One pass over tiles of R = 2^logR rows and T = 2^logT columns; block =
// T*R / 2^min(KMAX, logR) threads; grid = (tiles, batch).  Dynamic LDS: nine
// planes of T*R words plus nine planes of R/2 twiddles.  Inputs below 2m
// (canonical words, or the previous pass's outputs).  The DFT runs in steps
// of KMAX stages, the remainder in the last step.
//
// LR > 0 fixes the geometry at compile time: R = 2^LR rows in tiles of
// NTT_TILE_FIXED elements (the large transforms' shape).  The LDS plane and
// twiddle strides are then constants, so the nine limb accesses of an element
// share one address register and differ by immediate offsets, where runtime
// strides cost an address computation per limb.  LR = 0 reads the geometry
// from g.
constexpr uint32_t NTT_TILE_FIXED_LOG = 11;

// Occupancy: the fixed-geometry passes target 3 waves per SIMD, the runtime-
// geometry radix-8 passes 2.  The small transforms' radix-4 passes (KMAX 2)
// target 4: they then fit in 96 VGPRs without spills, so in a proof the
// quotient's passes find room on a SIMD beside three MSM accumulation waves
// (128 VGPRs each) instead of waiting for one to end (at 3 waves they took
// 132 VGPRs; config 1 proof 0.543-0.548 -> 0.528-0.536 ms, standalone
// transforms of 2^12-2^18 points unchanged).
template <int KMAX, bool LAST, int LR = 0>
__global__ __launch_bounds__(256)
__attribute__((amdgpu_waves_per_eu(LR > 0 ? 3 : KMAX != 3 ? 4 : 2))) void k_ntt_pass(PassGeo g, PassIO io) {
  quotient_priority();
  extern __shared__ uint32_t smem[];
  constexpr int EPT = 1 << KMAX;
  TileCtx tc;
  if constexpr (LR > 0) {
    tc.logR = LR;
    tc.logT = NTT_TILE_FIXED_LOG - LR;
    tc.nthr = 1u << (NTT_TILE_FIXED_LOG - KMAX);
  } else {
    tc.logR = g.logR;
    tc.logT = g.logT;
    tc.nthr = blockDim.x;
  }
  tc.E = 1u << (tc.logR + tc.logT);
  tc.half = 1u << (tc.logR - 1);
  tc.smask = tc.logT >= 5 ? 0u : (tc.logT >= 3 ? (32u >> tc.logT) - 1u : 7u);
  tc.cmask = (1u << tc.logT) - 1;
  tc.s = smem;
  tc.tw = smem + (LR > 0 ? NTT_XPLANES : NL) * tc.E;
  tc.tid = threadIdx.x;

  const size_t boff = (size_t)blockIdx.y * g.n;
  const uint4* src = io.src + 2 * boff;
  uint4* dst = io.dst + 2 * boff;

  TileOrigin o{};
  if (!LAST) {
    const uint32_t lt = g.logS - tc.logT;  // tiles per block of R*S elements (log)
    const size_t u = blockIdx.x >> lt;
    o.m0 = (blockIdx.x & ((1u << lt) - 1)) << tc.logT;
    o.base = (u << (tc.logR + g.logS)) + o.m0;
  } else {
    const uint32_t lt = g.logR0 - tc.logT;
    o.v = blockIdx.x >> lt;
    o.k0s = (blockIdx.x & ((1u << lt) - 1)) << tc.logT;
    o.base = (size_t)o.v << g.logS1;
  }

  uint32_t* twl = (uint32_t*)tc.tw;
  for (uint32_t e = tc.tid; e < tc.half; e += tc.nthr) {
#pragma unroll
    for (int l = 0; l < NL; l++) twl[l * tc.half + e] = io.twr[l * tc.half + e];
  }
  __syncthreads();
  if constexpr (LR > 0) {
    tile_fixed<KMAX, LAST, LR>(tc, g, io, src, dst, o);
    return;
  }

  const uint32_t nsteps = (tc.logR + KMAX - 1) / KMAX;
  const uint32_t klast = tc.logR - KMAX * (nsteps - 1);
  if (nsteps == 1) {
    // a single step (R <= 2^KMAX): the whole DFT in the first step, then out
    switch (klast) {
      case 1: tile_first<1, EPT, LAST>(tc, g, io, src, o); break;
      case 2: if constexpr (KMAX >= 2) tile_first<2, EPT, LAST>(tc, g, io, src, o); break;
      case 3: if constexpr (KMAX >= 3) tile_first<3, EPT, LAST>(tc, g, io, src, o); break;
      default: break;
    }
    __syncthreads();
    tile_copy_out<EPT, LAST>(tc, g, io, dst, o);
    return;
  }
  tile_first<KMAX, EPT, LAST>(tc, g, io, src, o);
  uint32_t stage = KMAX;
  for (uint32_t st = 1; st + 1 < nsteps; st++) {
    __syncthreads();
    tile_step<KMAX, EPT, LAST, false>(tc, g, io, dst, o, stage);
    stage += KMAX;
  }
  __syncthreads();
  switch (klast) {
    case 1: tile_step<1, EPT, LAST, true>(tc, g, io, dst, o, stage); break;
    case 2: if constexpr (KMAX >= 2) tile_step<2, EPT, LAST, true>(tc, g, io, dst, o, stage); break;
    case 3: if constexpr (KMAX >= 3) tile_step<3, EPT, LAST, true>(tc, g, io, dst, o, stage); break;
    default: break;
  }
}

// ------------------------------------------------------------------ tables
// Packed table[e] = base^(e_hi * e_lo) * mul with (e_hi, e_lo) = (e >> log_cols,
// e mod 2^log_cols), the exponent reduced mod 2^log_order; base and mul in
// internal form.  log_cols = 0 gives base^e (e_lo = 0 would give base^0: handled by
// the linear variant below).
__global__ void k_fill_pow_table(uint32_t* __restrict__ t, size_t count, uint32_t log_cols, fr base, int log_order,
                                 fr mul) {
  size_t e = blockIdx.x * (size_t)blockDim.x + threadIdx.x;
  if (e >= count) return;
  uint64_t ex = (uint64_t)(e >> log_cols) * (uint64_t)(e & (((size_t)1 << log_cols) - 1));
  if (log_order < 64) ex &= ((uint64_t)1 << log_order) - 1;
  fr r = fe_one<FrP>(), b = base;
  while (ex) {
    if (ex & 1) r = fmul(r, b);
    b = fsqr(b);
    ex >>= 1;
  }
  store_packed(t, e, fmul(r, mul));
}

// table[e] = base^e * mul, limb-major or packed.
__global__ void k_fill_pow_linear(uint32_t* __restrict__ t, size_t count, fr base, fr mul, int packed) {
  size_t e = blockIdx.x * (size_t)blockDim.x + threadIdx.x;
  if (e >= count) return;
  uint64_t ex = e;
  fr r = fe_one<FrP>(), b = base;
  while (ex) {
    if (ex & 1) r = fmul(r, b);
    b = fsqr(b);
    ex >>= 1;
  }
  if (packed)
    store_packed(t, e, fmul(r, mul));
  else
    store_table(t, count, e, fmul(r, mul));
}

// h = (a*b - c) * zinv on the reference's Montgomery words (kept for callers
// that need H itself; the prover fuses it into the last transform).  With raw
// words A = a 2^256, fmul(A,B) = ab 2^251, fmul(C, 2^256) = c 2^251 and
// fmul(., z 2^266) = (ab - c) z 2^256: three multiplies per element.
__global__ void k_quotient_pointwise(uint4* __restrict__ h, const uint4* __restrict__ A, const uint4* __restrict__ B,
                                     const uint4* __restrict__ C, size_t n, fr kc, fr zk) {
  quotient_priority();
  size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x;
  if (i >= n) return;
  fr t = fmul(load_elem(A, i), load_elem(B, i));
  fr u = fmul(load_elem(C, i), kc);
  store_elem_raw(h, i, fcanon(fmul(fsub(t, u), zk)));
}

// ------------------------------------------------------------------ host side
static fr fr_from_mont256_words(const uint64_t w[4]) {
  uint32_t v[8];
  memcpy(v, w, 32);
  return from_mont256<FrP>(v);
}

static fr fr_small(uint64_t x) {  // plain integer -> internal form
  uint32_t w[8] = {(uint32_t)x, (uint32_t)(x >> 32), 0, 0, 0, 0, 0, 0};
  return from_std<FrP>(w);
}

// w_{2^28} = 5^((r-1)/2^28) (reference ntt.cu:53-62), internal form.
static fr omega_int(int log_n, bool inverse) {
  static const uint64_t W28[4] = {0x636E735580D13D9CULL, 0xA22BF3742445FFD6ULL, 0x56452AC01EB203D8ULL,
                                  0x1860EF942963F9E7ULL};
  static const uint64_t W28I[4] = {0x89BCC016584BB683ULL, 0xE8D9887F0164A50CULL, 0x755E95CB795EDA3DULL,
                                   0x0F572B871323B130ULL};
  fr w = fr_from_mont256_words(inverse ? W28I : W28);
  for (int i = 0; i < 28 - log_n; i++) w = fsqr(w);
  return w;
}

static fr fr_inv_host(const fr& x) {
  uint32_t e[8] = {0xeffffffful, 0x43e1f593u, 0x79b97091u, 0x2833e848u,
                   0x8181585du, 0xb85045b6u, 0xe131a029u, 0x30644e72u};  // r - 2
  return fpow(x, e);
}

// n^-1 = ((r+1)/2)^log_n (reference ntt.cu:437-458)
static fr ninv_int(int log_n) {
  fr two_inv = fr_inv_host(fr_small(2));
  fr r = fe_one<FrP>();
  for (int i = 0; i < log_n; i++) r = fmul(r, two_inv);
  return fcanon(r);
}

// Pass layout for 2^log_n points: P passes of at most 2^8 points each.
struct PassShape {
  int P;
  int logR[3];
};

static PassShape pass_shape(int log_n) {
  PassShape s{};
  if (log_n <= NTT_MAX_LOGR) {
    s.P = 1;
    s.logR[0] = log_n;
  } else if (log_n <= 2 * NTT_MAX_LOGR) {
    s.P = 2;
    s.logR[0] = (log_n + 1) / 2;
    s.logR[1] = log_n / 2;
  } else {
    s.P = 3;
    s.logR[0] = (log_n + 2) / 3;
    s.logR[1] = (log_n + 1) / 3;
    s.logR[2] = log_n / 3;
  }
  return s;
}

// Device words of the tables of one plan (both directions), for a plan
// placed in caller-provided memory.
static size_t plan_table_words(const PassShape& sh, int log_n) {
  size_t w = 0;
  int below = log_n;
  for (int q = 0; q < sh.P; q++) {
    w += 2 * ((size_t)1 << (sh.logR[q] - 1)) * NL;
    if (q < sh.P - 1) w += 2 * ((size_t)1 << below) * PACKED_WORDS;
    below -= sh.logR[q];
  }
  return w;
}

static int launch_fill_linear(zk_context* ctx, const FrTable& t, const fr& base, const fr& mul, bool packed,
                              hipStream_t st) {
  ZK_LAUNCH(ctx, st, "ntt_twiddle_fill", k_fill_pow_linear, dim3(cdiv(t.count, 256)), dim3(256), 0, t.d, t.count,
            base, mul, packed ? 1 : 0);
  return ZK_OK;
}

static int launch_fill_pow(zk_context* ctx, const FrTable& t, uint32_t log_cols, const fr& base, int log_order,
                           const fr& mul, hipStream_t st) {
  ZK_LAUNCH(ctx, st, "ntt_twiddle_fill", k_fill_pow_table, dim3(cdiv(t.count, 256)), dim3(256), 0, t.d, t.count,
            log_cols, base, log_order, mul);
  return ZK_OK;
}

// Fill every table of plan p (whose FrTable pointers and counts are set) on
// stream st.
static int plan_fill(zk_context* ctx, NttPlan* p, hipStream_t st) {
  const int log_n = p->log_n;
  const fr one = fe_one<FrP>();
  fr ninv;
  memcpy(ninv.l, p->ninv, sizeof(ninv.l));
  for (int d = 0; d < 2; d++) {
    const fr w = omega_int(log_n, d == 1);
    int below = log_n;  // log of R_q * S_q
    for (int q = 0; q < p->P; q++) {
      const int lr = p->logR[q];
      fr wr = w;  // w_{R_q} = w_n^(n / R_q)
      for (int i = 0; i < log_n - lr; i++) wr = fsqr(wr);
      ZK_TRY(launch_fill_linear(ctx, p->twr[q][d], wr, one, false, st));
      if (q < p->P - 1) {
        fr wm = w;  // w_{R_q S_q} = w_n^(n / (R_q S_q)); table over (k, m) in [R_q) x [S_q)
        for (int i = 0; i < log_n - below; i++) wm = fsqr(wm);
        const fr mul = (d == 1 && q == 0) ? ninv : one;
        ZK_TRY(launch_fill_pow(ctx, p->twp[q][d], (uint32_t)(below - lr), wm, below, mul, st));
      }
      below -= lr;
    }
  }
  return ZK_OK;
}

// Carve plan tables out of `words` (device memory of plan_table_words).
static void plan_place(NttPlan* p, uint32_t* words) {
  int below = p->log_n;
  for (int q = 0; q < p->P; q++) {
    for (int d = 0; d < 2; d++) {
      p->twr[q][d].count = (size_t)1 << (p->logR[q] - 1);
      p->twr[q][d].d = words;
      words += p->twr[q][d].count * NL;
      if (q < p->P - 1) {
        p->twp[q][d].count = (size_t)1 << below;
        p->twp[q][d].d = words;
        words += p->twp[q][d].count * PACKED_WORDS;
      }
    }
    below -= p->logR[q];
  }
}

static void plan_init(NttPlan* p, int log_n) {
  const PassShape sh = pass_shape(log_n);
  p->log_n = log_n;
  p->P = sh.P;
  for (int q = 0; q < 3; q++) p->logR[q] = sh.logR[q];
  const fr ninv = ninv_int(log_n);
  memcpy(p->ninv, ninv.l, sizeof(p->ninv));
}

static int plan_get(zk_context* ctx, int log_n, NttPlan** out, hipStream_t st) {
  auto it = ctx->ntt_plans.find(log_n);
  if (it != ctx->ntt_plans.end()) {
    *out = it->second;
    return ZK_OK;
  }
  std::unique_ptr<NttPlan> p(new NttPlan());
  plan_init(p.get(), log_n);
  const size_t words = plan_table_words(pass_shape(log_n), log_n);
  void* mem = nullptr;
  if (dev_malloc(&mem, words * 4) != hipSuccess) return ctx->fail(ZK_ERR_OOM, "NTT table allocation failed");
  plan_place(p.get(), (uint32_t*)mem);
  // Tables are filled on the caller's stream and waited for before the plan
  // is cached, so a later call on any stream finds them complete.
  int rc = plan_fill(ctx, p.get(), st);
  if (rc == ZK_OK && hipStreamSynchronize(st) != hipSuccess) rc = ctx->fail(ZK_ERR_HIP, "NTT table fill failed");
  if (rc != ZK_OK) {
    (void)hipFree(mem);
    return rc;
  }
  NttPlan* raw = p.release();
  ctx->ntt_plans[log_n] = raw;
  *out = raw;
  return ZK_OK;
}

void ntt_plans_free(zk_context* ctx) {
  for (auto& kv : ctx->ntt_plans) {
    NttPlan* p = kv.second;
    if (p->twr[0][0].d) (void)hipFree(p->twr[0][0].d);  // the plan's one allocation starts there
    delete p;
  }
  ctx->ntt_plans.clear();
  for (auto& kv : ctx->coset_tables) {
    CosetTables* c = (CosetTables*)kv.second;
    if (c->pre.d) (void)hipFree(c->pre.d);
    delete c;
  }
  ctx->coset_tables.clear();
}

static int coset_get(zk_context* ctx, int log_n, uint64_t g, const NttPlan* plan, CosetTables** out,
                     hipStream_t st) {
  const uint64_t key = ((uint64_t)log_n << 56) ^ g;
  auto it = ctx->coset_tables.find(key);
  if (it != ctx->coset_tables.end()) {
    *out = (CosetTables*)it->second;
    return ZK_OK;
  }
  const size_t n = (size_t)1 << log_n;
  std::unique_ptr<CosetTables> c(new CosetTables());
  void* mem = nullptr;
  if (dev_malloc(&mem, 3 * n * PACKED_WORDS * 4) != hipSuccess)
    return ctx->fail(ZK_ERR_OOM, "coset table allocation failed");
  uint32_t* w = (uint32_t*)mem;
  c->pre = FrTable{w, n};
  c->post_inv = FrTable{w + n * PACKED_WORDS, n};
  c->post_fold = FrTable{w + 2 * n * PACKED_WORDS, n};
  const fr gi = fr_small(g), ginv = fr_inv_host(gi);
  fr scale = fe_one<FrP>();
  if (plan->P == 1) memcpy(scale.l, plan->ninv, sizeof(scale.l));
  int rc = launch_fill_linear(ctx, c->pre, gi, fe_one<FrP>(), true, st);            // g^i
  if (rc == ZK_OK) rc = launch_fill_linear(ctx, c->post_inv, ginv, scale, true, st);  // g^-i (/ n when P == 1)
  if (rc == ZK_OK) rc = launch_fill_linear(ctx, c->post_fold, gi, scale, true, st);   // g^i (/ n when P == 1)
  if (rc == ZK_OK && hipStreamSynchronize(st) != hipSuccess) rc = ctx->fail(ZK_ERR_HIP, "coset table fill failed");
  if (rc != ZK_OK) {
    (void)hipFree(mem);
    return rc;
  }
  CosetTables* raw = c.release();
  ctx->coset_tables[key] = raw;
  *out = raw;
  return ZK_OK;
}

// One transform (or a batch of them) over prepared tables.
//   src -> dst; mid: n*batch elements for the passes before the last (may be
//   src when src is writable and differs from dst; never dst);
//   pre/post modes as in PassIO (PRE_QUOTIENT reads src, src + n, src + 2n).
struct NttCall {
  void* dst;
  const void* src;
  void* mid;
  int log_n, inverse, batch;
  int pre_mode, post_mode;
  const uint32_t* pre;
  const uint32_t* post;
  fr kc, zk;
  int kmax;  // 2 or 3: elements per thread 4 or 8
};

// Tiles of 2048 elements take 78 KB of LDS: above the 64 KB a launch may
// request by default.
static void ntt_lds_limits() {
  static std::once_flag once;
  std::call_once(once, [] {
    const int bytes = 160 * 1024;
    (void)hipFuncSetAttribute((const void*)k_ntt_pass<3, true>, hipFuncAttributeMaxDynamicSharedMemorySize, bytes);
    (void)hipFuncSetAttribute((const void*)k_ntt_pass<3, true, 8>, hipFuncAttributeMaxDynamicSharedMemorySize, bytes);
    (void)hipFuncSetAttribute((const void*)k_ntt_pass<3, false, 8>, hipFuncAttributeMaxDynamicSharedMemorySize, bytes);
    (void)hipFuncSetAttribute((const void*)k_ntt_pass<3, true, 7>, hipFuncAttributeMaxDynamicSharedMemorySize, bytes);
    (void)hipFuncSetAttribute((const void*)k_ntt_pass<3, false, 7>, hipFuncAttributeMaxDynamicSharedMemorySize, bytes);
    (void)hipFuncSetAttribute((const void*)k_ntt_pass<3, true, 6>, hipFuncAttributeMaxDynamicSharedMemorySize, bytes);
    (void)hipFuncSetAttribute((const void*)k_ntt_pass<3, false, 6>, hipFuncAttributeMaxDynamicSharedMemorySize, bytes);
    (void)hipFuncSetAttribute((const void*)k_ntt_pass<3, false>, hipFuncAttributeMaxDynamicSharedMemorySize, bytes);
    (void)hipFuncSetAttribute((const void*)k_ntt_pass<2, true>, hipFuncAttributeMaxDynamicSharedMemorySize, bytes);
    (void)hipFuncSetAttribute((const void*)k_ntt_pass<2, false>, hipFuncAttributeMaxDynamicSharedMemorySize, bytes);
  });
}

static int ntt_exec(zk_context* ctx, const NttPlan* plan, const NttCall& c, hipStream_t st) {
  ntt_lds_limits();
  const int d = c.inverse ? 1 : 0;
  const int L = c.log_n, P = plan->P;
  const size_t n = (size_t)1 << L;
  const int kmax = c.kmax;
  const int logE = std::min(L, kmax == 3 ? 11 : 10);
  int logS[3];
  {
    int s = L;
    for (int q = 0; q < P; q++) {
      s -= plan->logR[q];
      logS[q] = s;
    }
  }
  for (int q = 0; q < P; q++) {
    const bool last = q == P - 1;
    PassGeo g{};
    g.logR = (uint32_t)plan->logR[q];
    g.n = n;
    PassIO io{};
    io.twr = plan->twr[q][d].d;
    io.src = (const uint4*)(q == 0 ? c.src : c.mid);
    io.dst = (uint4*)(last ? c.dst : c.mid);
    io.pre_mode = q == 0 ? c.pre_mode : PRE_NONE;
    io.pre = c.pre;
    io.kc = c.kc;
    io.zk = c.zk;
    if (!last) {
      g.logS = (uint32_t)logS[q];
      g.logT = (uint32_t)std::min(logE - plan->logR[q], logS[q]);
      io.twp = plan->twp[q][d].d;
    } else {
      g.logR0 = P == 1 ? 0 : (uint32_t)plan->logR[0];
      g.logS0 = P == 1 ? 0 : (uint32_t)logS[0];
      g.logS1 = P == 3 ? (uint32_t)logS[1] : 0;
      g.logNR = (uint32_t)(L - plan->logR[q]);
      g.logT = P == 1 ? 0 : (uint32_t)std::min(logE - plan->logR[q], (int)g.logR0);
      io.post_mode = c.post_mode;
      io.post = c.post;
      if (c.post_mode == POST_SCALE) memcpy(io.scale.l, plan->ninv, sizeof(io.scale.l));
    }
    const uint32_t E = 1u << (g.logR + g.logT);
    const uint32_t kk = std::min<uint32_t>((uint32_t)kmax, g.logR);
    const uint32_t threads = std::max<uint32_t>(1, E >> kk);
    const uint32_t tiles = (uint32_t)(n / E);
    const bool fixed = kmax == 3 && E == (1u << NTT_TILE_FIXED_LOG) && threads == (E >> 3) && g.logR >= 6 &&
                       g.logR <= 8;
    const size_t lds = (size_t)4 * ((fixed ? NTT_XPLANES : NL) * E + NL * (1u << (g.logR - 1)));
    const dim3 grid(tiles, c.batch), block(threads);
    if (fixed && g.logR == 8) {
      if (last)
        ZK_LAUNCH(ctx, st, "ntt_pass", (k_ntt_pass<3, true, 8>), grid, block, lds, g, io);
      else
        ZK_LAUNCH(ctx, st, "ntt_pass", (k_ntt_pass<3, false, 8>), grid, block, lds, g, io);
    } else if (fixed && g.logR == 7) {
      if (last)
        ZK_LAUNCH(ctx, st, "ntt_pass", (k_ntt_pass<3, true, 7>), grid, block, lds, g, io);
      else
        ZK_LAUNCH(ctx, st, "ntt_pass", (k_ntt_pass<3, false, 7>), grid, block, lds, g, io);
    } else if (fixed && g.logR == 6) {
      if (last)
        ZK_LAUNCH(ctx, st, "ntt_pass", (k_ntt_pass<3, true, 6>), grid, block, lds, g, io);
      else
        ZK_LAUNCH(ctx, st, "ntt_pass", (k_ntt_pass<3, false, 6>), grid, block, lds, g, io);
    } else if (kmax == 3 && g.logR >= 3) {
      if (last)
        ZK_LAUNCH(ctx, st, "ntt_pass", (k_ntt_pass<3, true>), grid, block, lds, g, io);
      else
        ZK_LAUNCH(ctx, st, "ntt_pass", (k_ntt_pass<3, false>), grid, block, lds, g, io);
    } else if (g.logR >= 2) {
      if (last)
        ZK_LAUNCH(ctx, st, "ntt_pass", (k_ntt_pass<2, true>), grid, block, lds, g, io);
      else
        ZK_LAUNCH(ctx, st, "ntt_pass", (k_ntt_pass<2, false>), grid, block, lds, g, io);
    } else {
      if (last)
        ZK_LAUNCH(ctx, st, "ntt_pass", (k_ntt_pass<1, true>), grid, block, lds, g, io);
      else
        ZK_LAUNCH(ctx, st, "ntt_pass", (k_ntt_pass<1, false>), grid, block, lds, g, io);
    }
  }
  return ZK_OK;
}

// Elements per thread: 8 for large transforms (throughput), 4 below (a
// thread's elements are a serial chain, so small transforms want more
// threads).
#ifndef ZK_NTT_KMAX_LARGE
#define ZK_NTT_KMAX_LARGE 3
#endif
#ifndef ZK_NTT_LARGE_LOG
#define ZK_NTT_LARGE_LOG 19
#endif
static int choose_kmax(int log_n, int batch) {
  return ((size_t)batch << log_n) >= ((size_t)1 << ZK_NTT_LARGE_LOG) ? ZK_NTT_KMAX_LARGE : 2;
}

int ntt_run(zk_context* ctx, void* d_out, const void* d_in, int log_n, int inverse, int batch, uint64_t coset_g,
            hipStream_t st) {
  if (!d_out || !d_in || batch < 1) return ctx->fail(ZK_ERR_INVALID, "ntt: null buffer or batch < 1");
  if (log_n < 1 || log_n > NTT_MAX_LOG) return ctx->fail(ZK_ERR_SIZE, "ntt: log_n outside [1, 24]");
  NttPlan* plan = nullptr;
  ZK_TRY(plan_get(ctx, log_n, &plan, st));
  CosetTables* cos = nullptr;
  if (coset_g) ZK_TRY(coset_get(ctx, log_n, coset_g, plan, &cos, st));
  const size_t n = (size_t)1 << log_n;
  NttCall c{};
  c.dst = d_out;
  c.src = d_in;
  c.log_n = log_n;
  c.inverse = inverse;
  c.batch = batch;
  c.kmax = choose_kmax(log_n, batch);
  if (plan->P > 1) {
    ZK_TRY(ctx->ensure(ctx->scratch_a, n * 32 * (size_t)batch));
    c.mid = ctx->scratch_a.p;
  }
  c.pre_mode = (cos && !inverse) ? PRE_TABLE : PRE_NONE;
  c.pre = cos ? cos->pre.d : nullptr;
  if (inverse) {
    if (cos) {
      c.post_mode = POST_TABLE;
      c.post = cos->post_inv.d;
    } else {
      c.post_mode = plan->P == 1 ? POST_SCALE : POST_NONE;
    }
  }
  return ntt_exec(ctx, plan, c, st);
}

// (kc, zk) of the pointwise quotient step for (g^n - 1)^-1 given in
// Montgomery words: kc = 2^256 mod r as a raw integer, zk = z 2^266.
static void quotient_consts(const uint64_t zinv_mont[4], fr& kc, fr& zk) {
  static const uint32_t K256[8] = {0x4ffffffbu, 0xac96341cu, 0x9f60cd29u, 0x36fc7695u,
                                   0x7879462eu, 0x666ea36fu, 0x9a07df2fu, 0x0e0a77c1u};  // 2^256 mod r
  static const uint32_t K271[8] = {0x2ffd5addu, 0x29ab3316u, 0xf4f5739fu, 0x3b9f942fu,
                                   0x3ca28ff2u, 0x84aad391u, 0xf9a8c5dfu, 0x1ed378c2u};  // 2^271 mod r
  kc = repack_in<FrP>(K256);
  uint32_t zw[8];
  memcpy(zw, zinv_mont, 32);
  zk = fmul(repack_in<FrP>(zw), repack_in<FrP>(K271));
}

int quotient_pointwise(zk_context* ctx, void* d_h, const void* d_a, const void* d_b, const void* d_c, size_t n,
                       const uint64_t zinv_mont[4], hipStream_t st) {
  fr kc, zk;
  quotient_consts(zinv_mont, kc, zk);
  ZK_LAUNCH(ctx, st, "quotient_pointwise", k_quotient_pointwise, dim3(cdiv(n, 256)), dim3(256), 0, (uint4*)d_h,
            (const uint4*)d_a, (const uint4*)d_b, (const uint4*)d_c, n, kc, zk);
  return ZK_OK;
}

// The transforms of the quotient (groth16.cu:321-383) on evaluations
// abc = A | B | C (3n elements, destroyed; work: 3n more elements):
//   3 inverse transforms whose outputs are multiplied by g^i (the coset
//   shift of the next step, with 1/n in the first inter-pass table);
//   3 forward transforms -> A, B, C on the coset g H;
//   one inverse transform whose first pass forms (A B - C) / Z from the three
//   and whose output is multiplied by g^-i -> h.
int quotient_ntts(zk_context* ctx, void* d_h, void* d_abc, void* d_work, int log_n, uint64_t g,
                  const uint64_t zinv_mont[4], hipStream_t st) {
  NttPlan* plan = nullptr;
  ZK_TRY(plan_get(ctx, log_n, &plan, st));
  CosetTables* cos = nullptr;
  ZK_TRY(coset_get(ctx, log_n, g, plan, &cos, st));
  NttCall c{};
  c.log_n = log_n;
  c.batch = 3;
  c.kmax = choose_kmax(log_n, 3);
  // coefficients * g^i: X -> Y (X is writable: the passes before the last run in it)
  c.src = d_abc;
  c.dst = d_work;
  c.mid = d_abc;
  c.inverse = 1;
  c.post_mode = POST_TABLE;
  c.post = cos->post_fold.d;
  ZK_TRY(ntt_exec(ctx, plan, c, st));
  // coset evaluations: Y -> X
  c.src = d_work;
  c.dst = d_abc;
  c.mid = d_work;
  c.inverse = 0;
  c.post_mode = POST_NONE;
  c.post = nullptr;
  ZK_TRY(ntt_exec(ctx, plan, c, st));
  // h: (A B - C) / Z from X, through Y, to d_h
  quotient_consts(zinv_mont, c.kc, c.zk);
  c.batch = 1;
  c.kmax = choose_kmax(log_n, 1);
  c.src = d_abc;
  c.dst = d_h;
  c.mid = d_work;
  c.inverse = 1;
  c.pre_mode = PRE_QUOTIENT;
  c.post_mode = POST_TABLE;
  c.post = cos->post_inv.d;
  return ntt_exec(ctx, plan, c, st);
}

// ------------------------------------------------------------------ no-allocation variant
// zk_ntt_noalloc runs the same kernels with its twiddle tables and its
// pass-to-pass buffer in `scratch`, a fixed device array of this library:
// every GPU holds one copy from module load to process end, and every call
// on that GPU shares it (calls that overlap on one GPU race on the buffer).
// Each log_n has its own table slot, filled by the first call of that size
// and never written with other values, so a call never depends on which
// sizes ran before it; a call on a stream under graph capture always puts
// the (idempotent) fill into the graph, so a replay finds its tables whatever
// ran between capture and replay.  Limits: 2^NTT_NA_MAX_LOG points per
// transform and 2^NTT_NA_MAX_ELEMS_LOG elements per call.
constexpr int NTT_NA_MAX_LOG = 16;
constexpr int NTT_NA_MAX_ELEMS_LOG = 18;
// the table slots of log_n = 1..16: each plan has at most 3 passes of at most
// 2^8 rows (2 * 128 DFT twiddles of NL words per direction and pass) and
// inter-pass tables of at most 2^log_n packed entries per direction; the exact
// layout is checked against this bound at set-up (ntt_scratch_init)
constexpr size_t NTT_NA_TABLE_WORDS =
    NTT_NA_MAX_LOG * 3 * 2 * 128 * NL + 2 * (((size_t)2 << NTT_NA_MAX_LOG) - 2) * PACKED_WORDS;
constexpr size_t NTT_NA_MID_WORDS = ((size_t)1 << NTT_NA_MAX_ELEMS_LOG) * 8;
constexpr size_t NTT_NA_WORDS = NTT_NA_TABLE_WORDS + NTT_NA_MID_WORDS;

static __device__ __align__(256) uint32_t scratch[NTT_NA_WORDS];

constexpr int NTT_NA_DEVICES = 64;
static std::mutex g_na_mu;
static uint32_t* g_na_ptr[NTT_NA_DEVICES];   // device address of `scratch` per GPU
static int g_na_status[NTT_NA_DEVICES];      // 0 not looked up, 1 ok, -1 lookup failed
static uint32_t g_na_filled[NTT_NA_DEVICES]; // bit log_n: that slot's tables are complete
static size_t g_na_slot[NTT_NA_MAX_LOG + 2]; // word offset of the slot of log_n (slot 17: end)

// Word offsets of the per-log_n table slots; false if they overrun the bound.
static bool na_slots_layout() {
  size_t off = 0;
  for (int k = 1; k <= NTT_NA_MAX_LOG; k++) {
    g_na_slot[k] = off;
    off += plan_table_words(pass_shape(k), k);
    off = (off + 63) & ~(size_t)63;  // 256-byte aligned slots
  }
  g_na_slot[NTT_NA_MAX_LOG + 1] = off;
  return off <= NTT_NA_TABLE_WORDS;
}

// Once per device, with that device current (zk_create): the device address
// of `scratch`.  The host-side name `scratch` is no device address; kernels
// and copies get this pointer.
int ntt_scratch_init(int device) {
  if (device < 0 || device >= NTT_NA_DEVICES) return ZK_ERR_INVALID;
  std::lock_guard<std::mutex> lk(g_na_mu);
  if (g_na_status[device] != 0) return g_na_status[device] > 0 ? ZK_OK : ZK_ERR_HIP;
  void* p = nullptr;
  const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
  g_na_status[device] = (e == hipSuccess && p && na_slots_layout()) ? 1 : -1;
  g_na_ptr[device] = g_na_status[device] > 0 ? (uint32_t*)p : nullptr;
  return g_na_status[device] > 0 ? ZK_OK : ZK_ERR_HIP;
}

int ntt_run_noalloc(zk_context* ctx, void* d_out, const void* d_in, int log_n, int inverse, int batch,
                    hipStream_t st) {
  if (!d_out || !d_in || batch < 1) return ctx->fail(ZK_ERR_INVALID, "ntt_noalloc: null buffer or batch < 1");
  if (log_n < 1 || log_n > NTT_NA_MAX_LOG)
    return ctx->fail(ZK_ERR_SIZE, "ntt_noalloc: log_n outside [1, 16] (the fixed scratch holds 2^16-point plans)");
  if (((size_t)batch << log_n) > ((size_t)1 << NTT_NA_MAX_ELEMS_LOG))
    return ctx->fail(ZK_ERR_SIZE, "ntt_noalloc: batch * 2^log_n above 2^18 elements (the fixed scratch's buffer)");
  hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
  if (hipStreamIsCapturing(st, &cap) != hipSuccess) return ctx->fail(ZK_ERR_HIP, "ntt_noalloc: capture status");
  const bool capturing = cap != hipStreamCaptureStatusNone;
  const int dev = ctx->device;
  uint32_t* base;
  bool filled;
  {
    std::lock_guard<std::mutex> lk(g_na_mu);
    if (dev < 0 || dev >= NTT_NA_DEVICES || g_na_status[dev] <= 0)
      return ctx->fail(ZK_ERR_HIP, "ntt_noalloc: scratch address of this device unknown");
    base = g_na_ptr[dev];
    filled = (g_na_filled[dev] >> log_n) & 1u;
  }
  NttPlan plan;
  plan_init(&plan, log_n);
  plan_place(&plan, base + g_na_slot[log_n]);
  if (!filled || capturing) {
    ZK_TRY(plan_fill(ctx, &plan, st));
    // a fill recorded into a graph has not run yet: the slot stays unfilled
    // for eager calls until one of them fills it
    if (!capturing) {
      std::lock_guard<std::mutex> lk(g_na_mu);
      g_na_filled[dev] |= 1u << log_n;
    }
  }
  NttCall c{};
  c.dst = d_out;
  c.src = d_in;
  c.mid = base + NTT_NA_TABLE_WORDS;
  c.log_n = log_n;
  c.inverse = inverse;
  c.batch = batch;
  c.kmax = choose_kmax(log_n, batch);
  if (inverse) c.post_mode = plan.P == 1 ? POST_SCALE : POST_NONE;
  return ntt_exec(ctx, &plan, c, st);
}

}  // namespace zk

extern "C" {

static int zk_ntt_impl(zk_context* ctx, void* d_out, const void* d_in, int log_n, int inverse, int batch,
                       void* stream) {
  if (!ctx) return ZK_ERR_INVALID;
  return zk::ntt_run(ctx, d_out, d_in, log_n, inverse, batch, 0, ctx->s(stream));
}

int zk_ntt(zk_context* ctx, void* d_out, const void* d_in, int log_n, int inverse, int batch, void* stream) {
  return zk::guard(ctx, [&] { return zk_ntt_impl(ctx, d_out, d_in, log_n, inverse, batch, stream); });
}

static int zk_coset_ntt_impl(zk_context* ctx, void* d_out, const void* d_in, int log_n, uint64_t g, int inverse,
                             int batch, void* stream) {
  if (!ctx) return ZK_ERR_INVALID;
  if (g < 2) return ctx->fail(ZK_ERR_INVALID, "coset generator must be >= 2");
  return zk::ntt_run(ctx, d_out, d_in, log_n, inverse, batch, g, ctx->s(stream));
}

int zk_coset_ntt(zk_context* ctx, void* d_out, const void* d_in, int log_n, uint64_t g, int inverse, int batch,
                 void* stream) {
  return zk::guard(ctx, [&] { return zk_coset_ntt_impl(ctx, d_out, d_in, log_n, g, inverse, batch, stream); });
}

int zk_ntt_noalloc(zk_context* ctx, void* d_out, const void* d_in, int log_n, int inverse, int batch, void* stream) {
  if (!ctx) return ZK_ERR_INVALID;
  return zk::guard(ctx, [&] { return zk::ntt_run_noalloc(ctx, d_out, d_in, log_n, inverse, batch, ctx->s(stream)); });
}

}  // extern "C"
