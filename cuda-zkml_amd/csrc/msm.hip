// Pippenger multi-scalar multiplication over BN254 G1 and G2 for gfx950.
//
// Replaces bn254::msm_g1 / msm_g2 (reference src/msm/msm.cu:320-598): one
// thread per point walking all windows with a global spin lock per bucket,
// one thread per window for the bucket reduction and a host combination.
// Here (same mathematical result, canonical affine output):
//
//  1. convert    points -> internal records (29-bit limbs, radix 2^261), once.
//  2. digits     scalar -> standard form; if s > (r-1)/2 use r - s and -P;
//                signed c-bit digits d_w in [-2^(c-1), 2^(c-1)], stored as
//                |d_w| | sign<<31 per (window, point); d_w = 0 is skipped.
//  3. sort       counting sort by bucket (w, |d_w|), per window: LDS
//                histograms per (window, slice of points), a column scan
//                over slices and a per-window scan give every bucket its
//                [start, end) in a window-major array (window w owns the
//                region [w*n_pad, w*n_pad + n_pad)); a scatter pass with LDS
//                cursors writes (bucket, point | sign<<31) pairs.  The order
//                inside a bucket is arbitrary, which cannot change the sum.
//  4. accumulate every thread sums exactly L0 consecutive sorted entries
//                with mixed XYZZ additions (perfect load balance whatever the
//                bucket sizes); runs that cross a chunk edge leave a head /
//                tail partial.
//  5. combine    the chunk partials of each bucket that spans chunks are
//                folded in groups (one launch for ordinary buckets,
//                ~log8(size/L0) for hot buckets such as many scalars equal
//                to 1).
//  6. reduce     sum_b b*S_b per window: G-bucket segments with running sums
//                plus (segment offset)*run, then LDS scans and trees per
//                group of T segments and per window.
//  7. host       remaining per-window partials are summed and combined with
//                W*c doublings on the CPU (serial chain: a CPU core beats a
//                lone wave64 by an order of magnitude on it).
#include <string.h>
#include <stdlib.h>

#include <algorithm>
#include <numeric>
#include <thread>
#include <type_traits>
#include <vector>

#include "curve.hpp"
#include "curve_split.hpp"
#include "host_bn254.hpp"
#include "zk_internal.hpp"

namespace zk {

constexpr uint32_t KEY_INVALID = 0xffffffffu;
constexpr int MSM_L0 = 64;         // sorted entries per accumulation thread (largest)
constexpr int MSM_CMAX = 16;       // widest window: 2^15 LDS counters (128 KB)
constexpr uint32_t MSM_LDS_B = 32768;  // most buckets a window's slice histogram holds in LDS
constexpr int SORT_T = 1024;       // threads of the histogram / scatter blocks
constexpr int SORT_U = 8;          // loads in flight per thread in the sort passes
constexpr int SCAN_T = 128;        // buckets per column-scan block (<= the smallest B)
constexpr int MSM_NCB = 256;       // coarse bins per window of the two-pass placement
constexpr int MSM_BPC_MAX = 128;   // buckets per coarse bin at B = 2^15
constexpr int PLACE_T = 1024;      // threads of a placement block
constexpr uint32_t MSM_SERIAL_SPAN = 8;  // longest serial chunk-partial chain of the one-launch combine
// Partials folded per bucket group by each level of the level combine.  A
// level costs a launch plus S - 1 dependent additions; measured on MI355X
// (G2 2^16 and G1 witness-like 2^20 MSMs, the 2^16 proof) S = 2 beats 4 and 8.
constexpr uint32_t MSM_COMBINE_S = 2;
// Spans above which the tree combine replaces the level combine.
#ifndef ZK_MSM_TREE_SPAN
#define ZK_MSM_TREE_SPAN 512
#endif
constexpr uint32_t MSM_TREE_SPAN = ZK_MSM_TREE_SPAN;
// G2 accumulation tuning: chunk length divided by 2^ZK_MSM_G2_L0_SHIFT (down
// to MSM_L0 / 8), waves per SIMD the register budget is cut to.
#ifndef ZK_MSM_G2_L0_SHIFT
#define ZK_MSM_G2_L0_SHIFT 0
#endif
#ifndef ZK_MSM_G2_ONE_LANE
#define ZK_MSM_G2_ONE_LANE 1
#endif
#ifndef ZK_MSM_G2_ACC_WAVES
#define ZK_MSM_G2_ACC_WAVES 3
#endif
#ifndef ZK_MSM_TAB_SLICE
#define ZK_MSM_TAB_SLICE 8192
#endif
// Bits covered by the windows.  After the optional negation s <= (r-1)/2 <
// 2^253, and signed digits need one more bit for the final carry.
constexpr int MSM_BITS = 254;

// ------------------------------------------------------------------ point records
// One record per point, exactly one 64-byte (G1) / 128-byte (G2) line so that
// a random gather in the accumulation touches a single line: every
// coordinate is the canonical internal-form value (x * 2^261 mod q) packed as
// 8 little-endian 32-bit words; x = y = 0 encodes the point at infinity (no
// finite point of y^2 = x^3 + 3 has x = y = 0).  G1: x, y; G2: x.c0, x.c1,
// y.c0, y.c1.
template <class F>
struct Rec;
template <>
struct Rec<fq> {
  static constexpr int WORDS = 16;
};
template <>
struct Rec<fq2> {
  static constexpr int WORDS = 32;
};

__device__ __forceinline__ void unpack_coord(const uint32_t* p, fq& a) { a = repack_in<FqP>(p); }
__device__ __forceinline__ void unpack_coord(const uint32_t* p, fq2& a) {
  a.c0 = repack_in<FqP>(p);
  a.c1 = repack_in<FqP>(p + 8);
}
__device__ __forceinline__ void pack_coord(uint32_t* p, const fq& a) { repack_out(a, p); }
__device__ __forceinline__ void pack_coord(uint32_t* p, const fq2& a) {
  repack_out(a.c0, p);
  repack_out(a.c1, p + 8);
}

// Record load through 16-byte vector loads; returns true for infinity.
template <class F>
__device__ __forceinline__ bool load_rec(const uint4* __restrict__ recs, uint32_t idx, F& x, F& y) {
  constexpr int W = Rec<F>::WORDS;
  uint32_t w[W];
  const uint4* p = recs + (size_t)idx * (W / 4);
#pragma unroll
  for (int i = 0; i < W / 4; i++) {
    uint4 v = p[i];
    w[4 * i] = v.x;
    w[4 * i + 1] = v.y;
    w[4 * i + 2] = v.z;
    w[4 * i + 3] = v.w;
  }
  uint32_t any = 0;
#pragma unroll
  for (int i = 0; i < W; i++) any |= w[i];
  unpack_coord(w, x);
  unpack_coord(w + W / 2, y);
  return any == 0;
}

// pack_coord stores canonical values (repack_out), so a negative digit's -y
// is the cheap q - y in the accumulation (fneg_canon_if).
template <class F>
__device__ __forceinline__ void store_rec(uint4* __restrict__ recs, size_t idx, const F& x, const F& y, bool inf) {
  constexpr int W = Rec<F>::WORDS;
  uint32_t w[W];
  pack_coord(w, x);
  pack_coord(w + W / 2, y);
  if (inf) {
#pragma unroll
    for (int k = 0; k < W; k++) w[k] = 0;
  }
  uint4* p = recs + idx * (W / 4);
#pragma unroll
  for (int k = 0; k < W / 4; k++) p[k] = make_uint4(w[4 * k], w[4 * k + 1], w[4 * k + 2], w[4 * k + 3]);
}

__device__ __forceinline__ void ext_to_coord(const uint32_t* e, fq& a) { a = from_mont256<FqP>(e); }
__device__ __forceinline__ void ext_to_coord(const uint32_t* e, fq2& a) {
  a.c0 = from_mont256<FqP>(e);
  a.c1 = from_mont256<FqP>(e + 8);
}

__device__ __forceinline__ void std_to_coord(const uint32_t* e, fq& a) { a = from_std<FqP>(e); }
__device__ __forceinline__ void std_to_coord(const uint32_t* e, fq2& a) {
  a.c0 = from_std<FqP>(e);
  a.c1 = from_std<FqP>(e + 8);
}

// External points (zk_g1_affine / zk_g2_affine: Montgomery R = 2^256, x = y =
// 0 for infinity) -> records.
// Issue priority of the MSM's waves.  Inside a proof several MSMs and the
// quotient share the GPU.  The accumulation is throughput-bound and always
// ready to issue; the digit sort and the chunk combine / bucket reduction are
// short or latency-bound and sit on some MSM's critical path.  Those waves
// run at priority 2 so that the SIMD arbiter serves them first and the
// accumulation takes the remaining issue slots (at equal priority a lone
// chain wave would get a fraction of its SIMD; at lower priority next to an
// always-ready accumulation it would starve).
__device__ __forceinline__ void msm_short_priority() { __builtin_amdgcn_s_setprio(2); }
template <class F>
__device__ __forceinline__ void msm_priority() {
  msm_short_priority();
}
// The G2 accumulation is the longest throughput phase of a proof and starts
// its MSM's critical path: priority 1, above the G1 accumulations (0).
template <class F>
__device__ __forceinline__ void msm_accumulate_priority() {
  if constexpr (sizeof(F) == sizeof(fq2)) __builtin_amdgcn_s_setprio(1);
}

template <class F>
__global__ void k_msm_convert(uint4* __restrict__ recs, const uint32_t* __restrict__ ext, size_t n) {
  size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x;
  if (i >= n) return;
  constexpr int EW = Rec<F>::WORDS;  // the external point has the same word count
  uint32_t e[EW];
  uint32_t any = 0;
#pragma unroll
  for (int k = 0; k < EW; k++) {
    e[k] = ext[i * EW + k];
    any |= e[k];
  }
  F x, y;
  ext_to_coord(e, x);
  ext_to_coord(e + EW / 2, y);
  store_rec(recs, i, x, y, any == 0);
}

// ------------------------------------------------------------------ digits
// (r-1)/2, little-endian 32-bit words
__constant__ uint32_t HALF_R[8] = {0xf8000000u, 0xa1f0fac9u, 0x3cdcb848u, 0x9419f424u,
                                   0x40c0ac2eu, 0xdc2822dbu, 0x7098d014u, 0x18322739u};
__constant__ uint32_t R_WORDS[8] = {0xf0000001u, 0x43e1f593u, 0x79b97091u, 0x2833e848u,
                                    0x8181585du, 0xb85045b6u, 0xe131a029u, 0x30644e72u};

// W windows cover MSM_BITS bits; the first MSM_BITS % W are one bit wider than
// the rest, so no window is left with a few top bits only (a window of k bits
// has 2^(k-1) buckets: a narrow top window would pile its entries into few,
// very large buckets).
__host__ __device__ __forceinline__ int window_width(int w, int W) {
  return MSM_BITS / W + (w < MSM_BITS % W ? 1 : 0);
}

__global__ void k_msm_digits(uint32_t* __restrict__ dig, const uint4* __restrict__ scalars, size_t n, int W) {
  msm_short_priority();
  size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x;
  if (i >= n) return;
  uint4 a = scalars[2 * i], b = scalars[2 * i + 1];
  uint32_t sm[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
  // standard form: fmul(raw s 2^256, 32) = s  (radix 2^261)
  fr t = repack_in<FrP>(sm);
  fr k32 = fe_zero<FrP>();
  k32.l[0] = 32;
  uint32_t s[8];
  repack_out(fmul(t, k32), s);
  // negate when s > (r-1)/2
  int gt = 0;
  for (int k = 7; k >= 0; k--) {
    if (s[k] != HALF_R[k]) {
      gt = s[k] > HALF_R[k];
      break;
    }
  }
  uint32_t neg = 0;
  if (gt) {
    uint32_t br = 0;
    for (int k = 0; k < 8; k++) {
      uint64_t d = (uint64_t)R_WORDS[k] - s[k] - br;
      s[k] = (uint32_t)d;
      br = (uint32_t)(d >> 63);
    }
    neg = 1;
  }
  uint32_t carry = 0;
  int bit = 0;
  for (int w = 0; w < W; w++) {
    const int cw = window_width(w, W);
    const uint32_t mask = (1u << cw) - 1u, half = 1u << (cw - 1);
    const int wd = bit >> 5, sh = bit & 31;
    uint64_t v = wd < 8 ? s[wd] : 0;
    if (wd + 1 < 8) v |= (uint64_t)s[wd + 1] << 32;
    uint32_t d = ((uint32_t)(v >> sh) & mask) + carry;
    uint32_t sign = neg;
    if (d > half) {
      d = (1u << cw) - d;
      carry = 1;
      sign ^= 1u;
    } else {
      carry = 0;
    }
    dig[(size_t)w * n + i] = d == 0 ? 0u : (d | (sign << 31));
    bit += cw;
  }
}

// ------------------------------------------------------------------ counting sort
// Bucket b in [0, B) of window w holds the entries with |d_w| = b + 1; its
// global key is w*B + b.  Slices: window w's points are cut into S slices of
// `slice` points; block (s, w) owns one.

// Per-(window, slice) histogram -> H[(w*S + s)*B + b].
template <int BMAX, int TB = SORT_T>
__global__ __launch_bounds__(TB) void k_msm_hist(const uint32_t* __restrict__ dig, size_t n, uint32_t slice,
                                                     uint32_t S, uint32_t B, uint32_t* __restrict__ H) {
  msm_short_priority();
  __shared__ uint32_t h[BMAX];
  const uint32_t s = blockIdx.x, w = blockIdx.y, t = threadIdx.x;
  for (uint32_t i = t; i < B; i += TB) h[i] = 0;
  __syncthreads();
  const size_t lo = (size_t)s * slice, hi = min(n, lo + slice);
  const uint32_t* d = dig + (size_t)w * n;
  for (size_t p0 = lo + t; p0 < hi; p0 += (size_t)TB * SORT_U) {
    uint32_t v[SORT_U];
#pragma unroll
    for (int u = 0; u < SORT_U; u++) {
      const size_t p = p0 + (size_t)u * TB;
      v[u] = p < hi ? d[p] : 0u;
    }
#pragma unroll
    for (int u = 0; u < SORT_U; u++) {
      const uint32_t m = v[u] & 0x7fffffffu;
      if (m) atomicAdd(&h[m - 1], 1u);
    }
  }
  __syncthreads();
  uint32_t* out = H + ((size_t)w * S + s) * B;
  for (uint32_t i = t; i < B; i += TB) out[i] = h[i];
}

// Column scan over slices, one thread per bucket k = w*B + b, blocks of
// SCAN_T consecutive buckets (B >= SCAN_T, so a block never spans windows):
//  - H becomes the exclusive prefix over s of every bucket's counts;
//  - tot[k] = bucket size, lex[k] = exclusive prefix of tot inside the block;
//  - bsum/bmax[block] = the block's entry count and largest bucket.
__global__ __launch_bounds__(SCAN_T) void k_msm_colscan(uint32_t* __restrict__ H, uint32_t S, uint32_t B,
                                                        uint32_t* __restrict__ tot, uint32_t* __restrict__ lex,
                                                        uint32_t* __restrict__ bsum, uint32_t* __restrict__ bmax) {
  msm_short_priority();
  __shared__ uint32_t wsum[SCAN_T / 64], wmx[SCAN_T / 64];
  const uint32_t t = threadIdx.x, lane = t & 63, wv = t >> 6;
  const uint32_t k = blockIdx.x * SCAN_T + t;
  const uint32_t w = k / B, b = k % B;
  uint32_t acc = 0;
  uint32_t* col = H + (size_t)w * S * B + b;
  for (uint32_t s0 = 0; s0 < S; s0 += SORT_U) {
    uint32_t v[SORT_U];
#pragma unroll
    for (int u = 0; u < SORT_U; u++) v[u] = s0 + u < S ? col[(size_t)(s0 + u) * B] : 0u;
#pragma unroll
    for (int u = 0; u < SORT_U; u++)
      if (s0 + u < S) {
        col[(size_t)(s0 + u) * B] = acc;
        acc += v[u];
      }
  }
  tot[k] = acc;
  uint32_t inc = acc, mx = acc;
  for (int off = 1; off < 64; off <<= 1) {
    const uint32_t o = (uint32_t)__shfl_up((int)inc, off);
    if (lane >= (uint32_t)off) inc += o;
  }
  for (int off = 32; off >= 1; off >>= 1) mx = max(mx, (uint32_t)__shfl_xor((int)mx, off));
  if (lane == 63) wsum[wv] = inc;
  if (lane == 0) wmx[wv] = mx;
  __syncthreads();
  uint32_t base = 0, total = 0, m = 0;
#pragma unroll
  for (int v = 0; v < SCAN_T / 64; v++) {
    if ((uint32_t)v < wv) base += wsum[v];
    total += wsum[v];
    m = max(m, wmx[v]);
  }
  lex[k] = base + inc - acc;
  if (t == 0) {
    bsum[blockIdx.x] = total;
    bmax[blockIdx.x] = m;
  }
}

// Per window (one block of nb = B / SCAN_T <= 256 threads): exclusive scan of
// the block sums -> boff; wstat[2w] = entries of window w, wstat[2w+1] = its
// largest bucket.
__global__ __launch_bounds__(256) void k_msm_bscan(const uint32_t* __restrict__ bsum, const uint32_t* __restrict__ bmax,
                                                   uint32_t nb, uint32_t* __restrict__ boff,
                                                   uint32_t* __restrict__ wstat) {
  msm_short_priority();
  __shared__ uint32_t wsum[4], wmx[4];
  const uint32_t w = blockIdx.x, t = threadIdx.x, lane = t & 63, wv = t >> 6;
  const uint32_t v = t < nb ? bsum[w * nb + t] : 0u;
  uint32_t mx = t < nb ? bmax[w * nb + t] : 0u;
  uint32_t inc = v;
  for (int off = 1; off < 64; off <<= 1) {
    const uint32_t o = (uint32_t)__shfl_up((int)inc, off);
    if (lane >= (uint32_t)off) inc += o;
  }
  for (int off = 32; off >= 1; off >>= 1) mx = max(mx, (uint32_t)__shfl_xor((int)mx, off));
  if (lane == 63) wsum[wv] = inc;
  if (lane == 0) wmx[wv] = mx;
  __syncthreads();
  uint32_t base = 0, total = 0, m = 0;
  for (uint32_t u = 0; u < 4; u++) {
    if (u < wv) base += wsum[u];
    total += wsum[u];
    m = max(m, wmx[u]);
  }
  if (t < nb) boff[w * nb + t] = base + inc - v;
  if (t == 0) {
    wstat[2 * w] = total;
    wstat[2 * w + 1] = m;
  }
}

// Scatter: LDS cursors = bucket start + slice prefix, one LDS atomic per
// entry; out[pos] = (key, point | sign<<31).  Bucket start = w*n_pad +
// boff[k / SCAN_T] + lex[k]; the blocks of slice 0 also store start/end.
template <int BMAX, int TB = SORT_T>
__global__ __launch_bounds__(TB) void k_msm_scatter(const uint32_t* __restrict__ dig, size_t n, uint32_t slice,
                                                        uint32_t S, uint32_t B, uint32_t n_pad,
                                                        const uint32_t* __restrict__ H,
                                                        const uint32_t* __restrict__ boff,
                                                        const uint32_t* __restrict__ lex,
                                                        const uint32_t* __restrict__ tot,
                                                        uint32_t* __restrict__ start, uint32_t* __restrict__ end,
                                                        uint2* __restrict__ out) {
  msm_short_priority();
  __shared__ uint32_t cur[BMAX];
  const uint32_t s = blockIdx.x, w = blockIdx.y, t = threadIdx.x;
  const uint32_t* hp = H + ((size_t)w * S + s) * B;
  for (uint32_t i = t; i < B; i += TB) {
    const uint32_t k = w * B + i;
    const uint32_t st = w * n_pad + boff[k / SCAN_T] + lex[k];
    cur[i] = st + hp[i];
    if (s == 0) {
      start[k] = st;
      end[k] = st + tot[k];
    }
  }
  __syncthreads();
  const size_t lo = (size_t)s * slice, hi = min(n, lo + slice);
  const uint32_t* d = dig + (size_t)w * n;
  const uint32_t kb = w * B - 1;
  for (size_t p0 = lo + t; p0 < hi; p0 += (size_t)TB * SORT_U) {
    uint32_t v[SORT_U];
#pragma unroll
    for (int u = 0; u < SORT_U; u++) {
      const size_t p = p0 + (size_t)u * TB;
      v[u] = p < hi ? d[p] : 0u;
    }
#pragma unroll
    for (int u = 0; u < SORT_U; u++) {
      const uint32_t m = v[u] & 0x7fffffffu;
      if (m) {
        const uint32_t pos = atomicAdd(&cur[m - 1], 1u);
        out[pos] = make_uint2(kb + m, (uint32_t)(p0 + (size_t)u * TB) | (v[u] & 0x80000000u));
      }
    }
  }
}

// The lanes of a wave that share `key` take their positions with one atomic
// when all active lanes hold the same key (a hot bucket or bin), else one
// atomic each; returns this lane's position.  KEY_INVALID lanes take none.
__device__ __forceinline__ uint32_t wave_claim(uint32_t* ctr, uint32_t key, uint32_t idx) {
  const uint32_t lead = __builtin_amdgcn_readfirstlane(key);
  const uint64_t same = __ballot(key == lead);
  uint32_t pos = 0;
  if (same == __ballot(1) && lead != KEY_INVALID) {
    const uint32_t rank = __builtin_amdgcn_mbcnt_hi((uint32_t)(same >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)same, 0u));
    if (rank == 0) pos = atomicAdd(&ctr[idx], (uint32_t)__popcll(same));
    pos = __builtin_amdgcn_readfirstlane(pos) + rank;
  } else if (key != KEY_INVALID) {
    pos = atomicAdd(&ctr[idx], 1u);
  }
  return pos;
}

// Tile-sorted writes of the placement.  A block takes its bin's entries in
// tiles of TILE_E; each entry's bucket gives it a rank from LDS counters
// (wave_claim), one wave turns the tile's counts into offsets, the entries are
// staged in LDS in bucket order and written out by consecutive threads, so
// every bucket's share of the tile leaves as one contiguous run (~32 entries
// at 2^15 buckets) where entry-by-entry stores would each touch their own
// cache line.
constexpr int TILE_U = 4;
constexpr int TILE_E = PLACE_T * TILE_U;  // entries per tile

// Wave 0 only (threadIdx.x < 64): toff = exclusive scan of cnt[0, ns) (ns <=
// 256), gbase = the buckets' global write positions for this tile (cur
// advances by the counts), cnt cleared for the next tile, *tot = the tile's
// entry count.
__device__ __forceinline__ void tile_offsets(uint32_t* cnt, uint32_t* toff, uint32_t* gbase, uint32_t* cur,
                                             uint32_t ns, uint32_t* tot) {
  const uint32_t lane = threadIdx.x;
  uint32_t c[4], sum = 0;
#pragma unroll
  for (int i = 0; i < 4; i++) {
    const uint32_t j = lane * 4 + i;
    c[i] = j < ns ? cnt[j] : 0u;
    sum += c[i];
  }
  uint32_t inc = sum;
  for (int off = 1; off < 64; off <<= 1) {
    const uint32_t o = (uint32_t)__shfl_up((int)inc, off, 64);
    if (lane >= (uint32_t)off) inc += o;
  }
  uint32_t ex = inc - sum;
#pragma unroll
  for (int i = 0; i < 4; i++) {
    const uint32_t j = lane * 4 + i;
    if (j < ns) {
      toff[j] = ex;
      gbase[j] = cur[j];
      cur[j] += c[i];
      cnt[j] = 0u;
      ex += c[i];
    }
  }
  if (lane == 63) *tot = inc;
}

// Two-pass placement for wide windows (B >= 2^13 buckets): one-pass random
// 8-byte writes across the whole window region leave every cache line
// partially written by many blocks.
//
// Pass 1 (block per window x slice): entries go to NCB coarse bins of BPC =
// B / NCB consecutive buckets; a bin's region is exactly its buckets' span,
// and each block writes its share of every bin as one contiguous run.  The
// block's run of bin cb starts at start(first bucket of cb) + sum over the
// bin's buckets of their slice prefixes.  Blocks of slice 0 store start/end.
__global__ __launch_bounds__(SORT_T) void k_msm_scatter_coarse(const uint32_t* __restrict__ dig, size_t n,
                                                               uint32_t slice, uint32_t S, uint32_t B, uint32_t BPC,
                                                               uint32_t n_pad, const uint32_t* __restrict__ H,
                                                               const uint32_t* __restrict__ boff,
                                                               const uint32_t* __restrict__ lex,
                                                               const uint32_t* __restrict__ tot,
                                                               uint32_t* __restrict__ start,
                                                               uint32_t* __restrict__ end, uint2* __restrict__ tmp) {
  msm_short_priority();
  __shared__ uint32_t cur[MSM_NCB];
  const uint32_t s = blockIdx.x, w = blockIdx.y, t = threadIdx.x;
  const uint32_t* hp = H + ((size_t)w * S + s) * B;
  if (t < MSM_NCB) {
    const uint32_t k0 = w * B + t * BPC;
    cur[t] = w * n_pad + boff[k0 / SCAN_T] + lex[k0];
  }
  __syncthreads();
  for (uint32_t i = t; i < B; i += SORT_T) {
    const uint32_t k = w * B + i;
    atomicAdd(&cur[i / BPC], hp[i]);
    if (s == 0) {
      const uint32_t st = w * n_pad + boff[k / SCAN_T] + lex[k];
      start[k] = st;
      end[k] = st + tot[k];
    }
  }
  __syncthreads();
  const size_t lo = (size_t)s * slice, hi = min(n, lo + slice);
  const uint32_t* d = dig + (size_t)w * n;
  const uint32_t kb = w * B - 1;
  for (size_t p0 = lo + t; p0 < hi; p0 += (size_t)SORT_T * SORT_U) {
    uint32_t v[SORT_U];
#pragma unroll
    for (int u = 0; u < SORT_U; u++) {
      const size_t p = p0 + (size_t)u * SORT_T;
      v[u] = p < hi ? d[p] : 0u;
    }
#pragma unroll
    for (int u = 0; u < SORT_U; u++) {
      const uint32_t m = v[u] & 0x7fffffffu;
      if (m) {
        const uint32_t pos = atomicAdd(&cur[(m - 1) / BPC], 1u);
        tmp[pos] = make_uint2(kb + m, (uint32_t)(p0 + (size_t)u * SORT_T) | (v[u] & 0x80000000u));
      }
    }
  }
}

// Pass 2 (block per window x coarse bin): LDS cursors for the bin's BPC
// buckets; every write stays inside the bin's region.  A bin whose largest
// bucket holds at least half of its entries (the hot bucket of skewed
// scalars) writes entry by entry: a wave's lanes then mostly share that
// bucket and take consecutive positions with one atomic (wave_claim), so its
// stores are contiguous already and the tile staging would only add barriers
// on the one block that decides the launch's length.  Other bins go through
// the tile-sorted writes above.
__global__ __launch_bounds__(PLACE_T) void k_msm_place(const uint2* __restrict__ tmp, uint32_t B, uint32_t BPC,
                                                       const uint32_t* __restrict__ start,
                                                       const uint32_t* __restrict__ end,
                                                       const uint32_t* __restrict__ bmax, uint2* __restrict__ out) {
  static_assert(MSM_BPC_MAX <= 256 && MSM_BPC_MAX <= SCAN_T, "one wave scans the bin's counters");
  msm_short_priority();
  __shared__ uint32_t cur[MSM_BPC_MAX], cnt[MSM_BPC_MAX], toff[MSM_BPC_MAX], gbase[MSM_BPC_MAX], ttot;
  __shared__ uint2 stg[TILE_E];
  const uint32_t cb = blockIdx.x, w = blockIdx.y, t = threadIdx.x;
  const uint32_t k0 = w * B + cb * BPC;
  const uint32_t lo = start[k0], hi = end[k0 + BPC - 1];
  for (uint32_t j = t; j < BPC; j += PLACE_T) {
    cur[j] = start[k0 + j];
    cnt[j] = 0u;
  }
  // the largest bucket of the column-scan block holding this bin (BPC <=
  // SCAN_T: that block's buckets include the bin's), an upper bound of the
  // bin's own largest bucket
  const bool hot = 2u * bmax[k0 / SCAN_T] >= hi - lo;
  __syncthreads();
  if (hot) {
    for (uint32_t p0 = lo + t; p0 < hi; p0 += PLACE_T * SORT_U) {
      uint2 e[SORT_U];
#pragma unroll
      for (int u = 0; u < SORT_U; u++) {
        const uint32_t p = p0 + u * PLACE_T;
        e[u] = p < hi ? tmp[p] : make_uint2(KEY_INVALID, 0u);
      }
      // When every active lane of a wave holds the same bucket, the wave
      // takes its positions with one atomic (order inside a bucket is free:
      // its points are summed); a hot bucket would otherwise serialize the
      // CU's LDS on one counter.  All eight atomics are issued before any
      // result is read, so their round trips overlap.
      uint32_t pos[SORT_U], rank[SORT_U];
      bool agg[SORT_U];
#pragma unroll
      for (int u = 0; u < SORT_U; u++) {
        const uint32_t key = e[u].x;
        const uint32_t lead = __builtin_amdgcn_readfirstlane(key);
        const uint64_t same = __ballot(key == lead);
        agg[u] = same == __ballot(1) && lead != KEY_INVALID;
        rank[u] = __builtin_amdgcn_mbcnt_hi((uint32_t)(same >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)same, 0u));
        pos[u] = 0;
        if (agg[u]) {
          if (rank[u] == 0) pos[u] = atomicAdd(&cur[lead - k0], (uint32_t)__popcll(same));
        } else if (key != KEY_INVALID) {
          pos[u] = atomicAdd(&cur[key - k0], 1u);
        }
      }
#pragma unroll
      for (int u = 0; u < SORT_U; u++) {
        if (agg[u]) pos[u] = __builtin_amdgcn_readfirstlane(pos[u]) + rank[u];
        if (e[u].x != KEY_INVALID) out[pos[u]] = e[u];
      }
    }
    return;
  }
  for (uint32_t p0 = lo; p0 < hi; p0 += TILE_E) {
    uint2 e[TILE_U];
    uint32_t rank[TILE_U];
#pragma unroll
    for (int u = 0; u < TILE_U; u++) {
      const uint32_t p = p0 + t + u * PLACE_T;
      e[u] = p < hi ? tmp[p] : make_uint2(KEY_INVALID, 0u);
    }
#pragma unroll
    for (int u = 0; u < TILE_U; u++) rank[u] = wave_claim(cnt, e[u].x, e[u].x == KEY_INVALID ? 0 : e[u].x - k0);
    __syncthreads();
    if (t < 64) tile_offsets(cnt, toff, gbase, cur, BPC, &ttot);
    __syncthreads();
#pragma unroll
    for (int u = 0; u < TILE_U; u++)
      if (e[u].x != KEY_INVALID) stg[toff[e[u].x - k0] + rank[u]] = e[u];
    __syncthreads();
    const uint32_t nt = ttot;
    for (uint32_t lp = t; lp < nt; lp += PLACE_T) {
      const uint2 x = stg[lp];
      const uint32_t j = x.x - k0;
      out[gbase[j] + (lp - toff[j])] = x;
    }
  }
}

// ------------------------------------------------------------------ wide sort
// One bucket space of B = 2^b > 2^15 buckets (window tables with windows of
// more than 16 bits): too many counters for a slice histogram in LDS, so the
// entries go first to NB = 1024 coarse bins of BPC = B / NB consecutive
// buckets (slice histograms of NB counters), then each bin is counted,
// scanned and placed by one block with BPC counters in LDS (measured on the
// 2^22 proof: 256 bins of 2048 buckets placed 1.7 ms per MSM).
constexpr int WIDE_NB = 1024;
constexpr int WIDE_LOG_NB = 10;

// Pass 1a: coarse-bin counts of slice s -> cnt[bin * S + s].
__global__ __launch_bounds__(SORT_T) void k_wide_count(const uint32_t* __restrict__ dig, size_t np, uint32_t slice,
                                                      uint32_t S, uint32_t shift, uint32_t* __restrict__ cnt) {
  msm_short_priority();
  __shared__ uint32_t h[WIDE_NB];
  const uint32_t s = blockIdx.x, t = threadIdx.x;
  for (uint32_t i = t; i < WIDE_NB; i += SORT_T) h[i] = 0;
  __syncthreads();
  const size_t lo = (size_t)s * slice, hi = min(np, lo + slice);
  for (size_t p0 = lo + t; p0 < hi; p0 += (size_t)SORT_T * SORT_U) {
    uint32_t v[SORT_U];
#pragma unroll
    for (int u = 0; u < SORT_U; u++) {
      const size_t p = p0 + (size_t)u * SORT_T;
      v[u] = p < hi ? dig[p] & 0x7fffffffu : 0u;
    }
#pragma unroll
    for (int u = 0; u < SORT_U; u++) {
      const uint32_t bin = v[u] ? (v[u] - 1) >> shift : KEY_INVALID;
      (void)wave_claim(h, bin, bin == KEY_INVALID ? 0 : bin);
    }
  }
  __syncthreads();
  for (uint32_t i = t; i < WIDE_NB; i += SORT_T) cnt[(size_t)i * S + s] = h[i];
}

// Pass 1b: per coarse bin (block of 256 threads, up to 4 slices each),
// cnt[bin * S + s] becomes the exclusive prefix over the bin's slices and
// bintot[bin] its entry count.
__global__ __launch_bounds__(256) void k_wide_scan_rows(uint32_t* __restrict__ cnt, uint32_t S,
                                                      uint32_t* __restrict__ bintot) {
  msm_short_priority();
  __shared__ uint32_t wsum[4];
  const uint32_t t = threadIdx.x, lane = t & 63, wv = t >> 6;
  uint32_t* row = cnt + (size_t)blockIdx.x * S;
  const uint32_t PER = (S + 255) / 256;  // S <= 1024
  const uint32_t s0 = min(t * PER, S), s1 = min(s0 + PER, S);
  uint32_t v[4], sum = 0;
  for (uint32_t i = 0; i < 4; i++) {
    v[i] = s0 + i < s1 ? row[s0 + i] : 0u;
    sum += v[i];
  }
  uint32_t inc = sum;
  for (int off = 1; off < 64; off <<= 1) {
    const uint32_t o = (uint32_t)__shfl_up((int)inc, off);
    if (lane >= (uint32_t)off) inc += o;
  }
  if (lane == 63) wsum[wv] = inc;
  __syncthreads();
  uint32_t base = 0, all = 0;
#pragma unroll
  for (int k = 0; k < 4; k++) {
    if ((uint32_t)k < wv) base += wsum[k];
    all += wsum[k];
  }
  base += inc - sum;
  for (uint32_t i = 0; i < 4; i++) {
    if (s0 + i < s1) row[s0 + i] = base;
    base += v[i];
  }
  if (t == 0) bintot[blockIdx.x] = all;
}

// Pass 1c (one block, a thread per bin): binoff[bin] = the bin's first entry,
// binoff[NB] = the entry count (also wstat[0]; wstat[1] = 0 for the
// placement's maximum).
__global__ __launch_bounds__(WIDE_NB) void k_wide_scan_bins(const uint32_t* __restrict__ bintot,
                                                          uint32_t* __restrict__ binoff, uint32_t* __restrict__ wstat) {
  msm_short_priority();
  __shared__ uint32_t wsum[WIDE_NB / 64];
  const uint32_t b = threadIdx.x, lane = b & 63, wv = b >> 6;
  const uint32_t tot = bintot[b];
  uint32_t inc = tot;
  for (int off = 1; off < 64; off <<= 1) {
    const uint32_t o = (uint32_t)__shfl_up((int)inc, off);
    if (lane >= (uint32_t)off) inc += o;
  }
  if (lane == 63) wsum[wv] = inc;
  __syncthreads();
  uint32_t base = 0, all = 0;
#pragma unroll
  for (int v = 0; v < WIDE_NB / 64; v++) {
    if ((uint32_t)v < wv) base += wsum[v];
    all += wsum[v];
  }
  binoff[b] = base + inc - tot;
  if (b == 0) {
    binoff[WIDE_NB] = all;
    wstat[0] = all;
    wstat[1] = 0;
  }
}

// Pass 1d: slice s's entries to their coarse bins: tmp[pos] = (bucket, p | sign).
__global__ __launch_bounds__(SORT_T) void k_wide_scatter(const uint32_t* __restrict__ dig, size_t np, uint32_t slice,
                                                        uint32_t S, uint32_t shift, const uint32_t* __restrict__ cnt,
                                                        const uint32_t* __restrict__ binoff, uint2* __restrict__ tmp) {
  msm_short_priority();
  __shared__ uint32_t cur[WIDE_NB];
  const uint32_t s = blockIdx.x, t = threadIdx.x;
  for (uint32_t i = t; i < WIDE_NB; i += SORT_T) cur[i] = binoff[i] + cnt[(size_t)i * S + s];
  __syncthreads();
  const size_t lo = (size_t)s * slice, hi = min(np, lo + slice);
  for (size_t p0 = lo + t; p0 < hi; p0 += (size_t)SORT_T * SORT_U) {
    uint32_t v[SORT_U];
#pragma unroll
    for (int u = 0; u < SORT_U; u++) {
      const size_t p = p0 + (size_t)u * SORT_T;
      v[u] = p < hi ? dig[p] : 0u;
    }
#pragma unroll
    for (int u = 0; u < SORT_U; u++) {
      const uint32_t m = v[u] & 0x7fffffffu;
      const uint32_t bin = m ? (m - 1) >> shift : KEY_INVALID;
      const uint32_t pos = wave_claim(cur, bin, bin == KEY_INVALID ? 0 : bin);
      if (m) tmp[pos] = make_uint2(m - 1, (uint32_t)(p0 + (size_t)u * SORT_T) | (v[u] & 0x80000000u));
    }
  }
}

// Pass 2 (block per coarse bin, 2^shift buckets): LDS counts, their scan
// (bucket bounds start/end; the largest bucket into wstat[1]), placement.
__global__ __launch_bounds__(PLACE_T) void k_wide_place(const uint2* __restrict__ tmp,
                                                       const uint32_t* __restrict__ binoff, uint32_t shift,
                                                       uint32_t* __restrict__ start, uint32_t* __restrict__ end,
                                                       uint2* __restrict__ out, uint32_t* __restrict__ wstat) {
  msm_short_priority();
  extern __shared__ uint32_t cur[];  // 2^shift counters, then cursors
  __shared__ uint32_t wsum[PLACE_T / 64], wmx[PLACE_T / 64];
  const uint32_t cb = blockIdx.x, t = threadIdx.x, lane = t & 63, wv = t >> 6;
  const uint32_t BPC = 1u << shift, k0 = cb << shift;
  const uint32_t lo = binoff[cb], hi = binoff[cb + 1];
  for (uint32_t j = t; j < BPC; j += PLACE_T) cur[j] = 0;
  __syncthreads();
  for (uint32_t p0 = lo + t; p0 < hi; p0 += PLACE_T * SORT_U) {
    uint32_t key[SORT_U];
#pragma unroll
    for (int u = 0; u < SORT_U; u++) {
      const uint32_t p = p0 + u * PLACE_T;
      key[u] = p < hi ? tmp[p].x : KEY_INVALID;
    }
#pragma unroll
    for (int u = 0; u < SORT_U; u++) (void)wave_claim(cur, key[u], key[u] == KEY_INVALID ? 0 : key[u] - k0);
  }
  __syncthreads();
  // exclusive scan: thread t owns counters [t PER, t PER + PER)
  const uint32_t PER = (BPC + PLACE_T - 1) / PLACE_T;
  const uint32_t j0 = min(t * PER, BPC), j1 = min(j0 + PER, BPC);
  uint32_t sum = 0, mx = 0;
  for (uint32_t j = j0; j < j1; j++) {
    sum += cur[j];
    mx = max(mx, cur[j]);
  }
  uint32_t inc = sum;
  for (int off = 1; off < 64; off <<= 1) {
    const uint32_t o = (uint32_t)__shfl_up((int)inc, off);
    if (lane >= (uint32_t)off) inc += o;
  }
  for (int off = 32; off >= 1; off >>= 1) mx = max(mx, (uint32_t)__shfl_xor((int)mx, off));
  if (lane == 63) wsum[wv] = inc;
  if (lane == 0) wmx[wv] = mx;
  __syncthreads();
  uint32_t base = lo, m = 0;
#pragma unroll
  for (int v = 0; v < PLACE_T / 64; v++) {
    if ((uint32_t)v < wv) base += wsum[v];
    m = max(m, wmx[v]);
  }
  base += inc - sum;
  for (uint32_t j = j0; j < j1; j++) {
    const uint32_t c = cur[j];
    start[k0 + j] = base;
    end[k0 + j] = base + c;
    cur[j] = base;
    base += c;
  }
  if (t == 0 && m) atomicMax(&wstat[1], m);
  __syncthreads();
  for (uint32_t p0 = lo + t; p0 < hi; p0 += PLACE_T * SORT_U) {
    uint2 e[SORT_U];
#pragma unroll
    for (int u = 0; u < SORT_U; u++) {
      const uint32_t p = p0 + u * PLACE_T;
      e[u] = p < hi ? tmp[p] : make_uint2(KEY_INVALID, 0u);
    }
    uint32_t pos[SORT_U];
#pragma unroll
    for (int u = 0; u < SORT_U; u++) pos[u] = wave_claim(cur, e[u].x, e[u].x == KEY_INVALID ? 0 : e[u].x - k0);
#pragma unroll
    for (int u = 0; u < SORT_U; u++)
      if (e[u].x != KEY_INVALID) out[pos[u]] = e[u];
  }
}

// ------------------------------------------------------------------ accumulate

// Chunk partials of buckets that span chunks; base set s uses the slots
// [s * nchunks, (s + 1) * nchunks).
template <class F>
struct ChunkSlots {
  uint32_t* hkey;
  uint32_t* tkey;
  xyzz<F>* hpt;
  xyzz<F>* tpt;
  __device__ ChunkSlots at(uint32_t set, uint32_t nchunks) const {
    const size_t o = (size_t)set * nchunks;
    return ChunkSlots{hkey + o, tkey + o, hpt + o, tpt + o};
  }
};

// Point sets sharing one scalar vector (and so one sorted digit list): set s
// takes the scalars with index i in [lo[s], hi[s]) and the point recs[s][i -
// lo[s]]; entries outside the range add nothing to that set's buckets.
// Window tables (pstride != 0): the sorted entries are positions p = w n + i
// of one bucket space over all windows (n = pstride), and recs[s] holds the
// window multiples 2^(shift of w) P: row w (tstride[s] records) per window.
constexpr int MSM_SETS = 3;
struct BaseSets {
  const uint4* recs[MSM_SETS];
  uint32_t lo[MSM_SETS], hi[MSM_SETS];
  uint32_t pstride;
  uint32_t tstride[MSM_SETS];
};

// Record load into the accumulation's registers: G1 the whole record, G2
// this lane's half of a lane pair (x.c0, y.c0 on even lanes, x.c1, y.c1 on
// odd lanes).  Returns true for the point at infinity (all words zero).
__device__ __forceinline__ bool load_rec_lanes(const uint4* __restrict__ recs, uint32_t idx, fq& x, fq& y) {
  return load_rec(recs, idx, x, y);
}
__device__ __forceinline__ bool load_rec_lanes(const uint4* __restrict__ recs, uint32_t idx, fq2h& x, fq2h& y) {
  const uint4* p = recs + (size_t)idx * (Rec<fq2>::WORDS / 4) + (lane_odd() ? 2 : 0);
  const uint4 a = p[0], b = p[1], c = p[4], d = p[5];
  const uint32_t wx[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
  const uint32_t wy[8] = {c.x, c.y, c.z, c.w, d.x, d.y, d.z, d.w};
  uint32_t any = 0;
#pragma unroll
  for (int k = 0; k < 8; k++) any |= wx[k] | wy[k];
  any |= swap_pair(any);
  x.c = repack_in<FqP>(wx);
  y.c = repack_in<FqP>(wy);
  return any == 0;
}

__device__ __forceinline__ bool load_rec_lanes(const uint4* __restrict__ recs, uint32_t idx, fq2& x, fq2& y) {
  return load_rec(recs, idx, x, y);
}

// One lane per G2 chunk (the whole Fq2 accumulator in one lane): ~14% fewer
// instructions per addition than a lane pair (no lane swaps or selects), but
// 2 waves per SIMD instead of 3.  Used for the largest G2 MSMs, where the
// accumulation is throughput-bound.
template <class F>
struct OneLane {
  typedef F R;
  static constexpr int N = 1;
  __device__ static xyzz<F> load(const xyzz<F>& p) { return p; }
  __device__ static void store(xyzz<F>& p, const xyzz<F>& v) { p = v; }
};

template <class LN>
constexpr int acc_waves() {
  if constexpr (std::is_same_v<typename LN::R, fq>) return 4;  // G1
  else if constexpr (std::is_same_v<typename LN::R, fq2>) return 2;  // G2 on one lane
  else return ZK_MSM_G2_ACC_WAVES;  // G2 on lane pairs
}
// a pair's coordinate type has G1's size: the target must follow the layout
static_assert(acc_waves<Lanes<fq>>() == 4 && acc_waves<Lanes<fq2>>() == ZK_MSM_G2_ACC_WAVES &&
                  acc_waves<OneLane<fq2>>() == 2,
              "accumulation wave targets by lane layout");

// Chunk ch covers sorted positions [ch*L0, ch*L0 + L0) of window
// ch / chunks_per_window; positions past the window's entry count are empty.
// blockIdx.y selects the base set; its buckets start at set * nbuckets.  A
// chunk is one lane (G1) or one lane pair (G2, Lanes<F>): split over a pair
// the G2 accumulator needs half the registers per lane, so that more waves
// fit on a SIMD to cover the gathers' latency.
//
// Waves are scattered over the chunk space: wave v of the grid takes the
// 64 / Lanes<F>::N chunks of chunk-wave (v * wave_mul) mod nwaves (wave_mul
// coprime to nwaves, so every chunk is taken once).  With skewed scalars most entries
// sit in a few windows (small witness values fill the low ones); in chunk
// order those windows' waves would land on a fraction of the CUs, scattered
// they spread over all of them.
template <class F, bool TAB, class LN = Lanes<F>>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(acc_waves<LN>()))) void k_msm_accumulate(const uint2* __restrict__ sorted, BaseSets sets,
                                                        const uint32_t* __restrict__ start,
                                                        const uint32_t* __restrict__ end,
                                                        const uint32_t* __restrict__ wstat, uint32_t nchunks,
                                                        uint32_t chunks_per_window, uint32_t n_pad, uint32_t L0,
                                                        size_t nbuckets, xyzz<F>* __restrict__ buckets,
                                                        ChunkSlots<F> all_slots, uint32_t nwaves,
                                                        uint32_t wave_mul) {
  typedef typename LN::R R;
  constexpr uint32_t PER_WAVE = 64 / LN::N;  // chunks per wave
  msm_accumulate_priority<F>();
  const uint32_t tid = blockIdx.x * blockDim.x + threadIdx.x;
  if ((tid >> 6) >= nwaves) return;
  const uint32_t ch = (uint32_t)((uint64_t)(tid >> 6) * wave_mul % nwaves) * PER_WAVE + (tid & 63) / LN::N;
  if (ch >= nchunks) return;
  const uint32_t set = blockIdx.y;
  const uint4* __restrict__ recs = sets.recs[set];
  const uint32_t ilo = sets.lo[set], ilen = sets.hi[set] - ilo;
  const uint32_t pstride = sets.pstride, tstride = sets.tstride[set];
  buckets += set * nbuckets;
  const ChunkSlots<F> slots = all_slots.at(set, nchunks);
  const uint32_t w = ch / chunks_per_window;
  const uint32_t total = w * n_pad + wstat[2 * w];
  const uint32_t lo = ch * L0;
  uint32_t hk = KEY_INVALID, tk = KEY_INVALID;
  if (lo < total) {
    const uint32_t hi = min(lo + L0, total);
    xyzz<R> acc;
    xyzz_set_inf(acc);
    bool empty = true;  // acc is the point at infinity
    uint32_t cur = sorted[lo].x;
    for (uint32_t p = lo; p < hi; p++) {
      const uint2 e = sorted[p];
      const uint32_t key = e.x;
      if (key != cur) {
        // run `cur` ended inside the chunk; acc holds whatever the last run
        // left while `empty` (the next point overwrites it), so a run that
        // summed to nothing stores the point at infinity explicitly
        if (__builtin_expect(empty, 0)) xyzz_set_inf(acc);
        if (start[cur] < lo) {
          hk = cur;
          LN::store(slots.hpt[ch], acc);
        } else {
          LN::store(buckets[cur], acc);
        }
        cur = key;
        empty = true;
      }
      const uint32_t v = e.y;
      uint32_t i = (v & 0x7fffffffu), row = 0;
      if constexpr (TAB) {
        row = i / pstride;
        i -= row * pstride;
      }
      i -= ilo;  // wraps below lo
      R x, y;
      if (i < ilen && !load_rec_lanes(recs, row * tstride + i, x, y)) {
        y = fneg_canon_if(y, (v >> 31) != 0);  // negative digit: -P
        if (empty) {
          xyzz_set_affine(acc, x, y);
          empty = false;
        } else {
          empty = xyzz_madd_fin(acc, x, y);
        }
      }
    }
    // last run of the chunk
    if (__builtin_expect(empty, 0)) xyzz_set_inf(acc);
    const uint32_t rs = start[cur], re = end[cur];
    if (rs >= lo && re <= lo + L0) {
      LN::store(buckets[cur], acc);
    } else if (rs < lo) {
      hk = cur;
      LN::store(slots.hpt[ch], acc);
    } else {
      tk = cur;
      LN::store(slots.tpt[ch], acc);
    }
  }
  slots.hkey[ch] = hk;
  slots.tkey[ch] = tk;
}

// The chunk combine and the bucket reduction are chains of dependent point
// additions run by comparatively few threads.  They are templated on the
// lane layout LN (curve_split.hpp): Lanes<F> (one lane per G1 point, a lane
// pair per G2 point) or SplitLanes<F> (each point operation dealt to two
// lane groups: 2 lanes per G1 point, 4 per G2 point).  `item` is the point's
// index; all lanes of an item always take the same branches.
template <class LN>
__device__ __forceinline__ uint32_t lane_item() {
  return (blockIdx.x * blockDim.x + threadIdx.x) / LN::N;
}
__device__ __forceinline__ uint32_t cdiv_dev(uint32_t a, uint32_t b) { return (a + b - 1) / b; }

// Chunk combine.  The partials of a bucket whose run spans chunks c0 .. c1
// are the tail partial of c0 and the head partials of c0+1 .. c1 (every chunk
// holds at most one head and one tail partial).
//
// Spans of up to MSM_SERIAL_SPAN + 1 chunks: one launch in which the chunk
// where the run starts adds the head partials of the chunks it covers, in
// order, and stores the bucket.  Longer spans (hot buckets such as many
// scalars equal to 1, or the large buckets of a window-table MSM) are left to
// k_msm_combine_tree, whose fold counters this launch clears.
template <class F, class LN>
__global__ __launch_bounds__(256) void k_msm_combine_serial(ChunkSlots<F> all_slots,
                                                            const uint32_t* __restrict__ end, uint32_t nchunks,
                                                            uint32_t L0, size_t nbuckets,
                                                            xyzz<F>* __restrict__ buckets,
                                                            uint32_t* __restrict__ fold_cnt, uint32_t tb) {
  msm_priority<F>();
  const uint32_t ch = lane_item<LN>();
  if (ch >= nchunks) return;
  if (fold_cnt && ch % tb == 0) fold_cnt[(size_t)blockIdx.y * cdiv_dev(nchunks, tb) + ch / tb] = 0;
  const ChunkSlots<F> slots = all_slots.at(blockIdx.y, nchunks);
  buckets += blockIdx.y * nbuckets;
  const uint32_t tk = slots.tkey[ch];
  if (tk == KEY_INVALID) return;
  const uint32_t c1 = (end[tk] - 1) / L0;
  if (c1 - ch > MSM_SERIAL_SPAN) return;  // a long span: the tree combine
  auto acc = LN::load(slots.tpt[ch]);
  for (uint32_t j = ch + 1; j <= c1; j++) xyzz_add(acc, LN::load(slots.hpt[j]));
  LN::store(buckets[tk], acc);
}

// Longer spans up to MSM_TREE_SPAN chunks: levels with
// step = 1, S, S^2, ... (S = MSM_COMBINE_S) fold the partials in groups of
// S: the chunk at j = ch - c0 with j % (S*step) == 0 adds the partials at
// j + step, ..., j + (S-1) step that exist.  After the level with S*step >=
// c1 - c0 + 1 chunk c0 holds the bucket's sum and stores it.  A chunk has at
// most one active job: a head job needs its bucket to continue past the
// chunk, and then the chunk's last run is that bucket (no tail).
template <class F, class LN>
__global__ __launch_bounds__(256) void k_msm_combine(ChunkSlots<F> all_slots, const uint32_t* __restrict__ start,
                                                     const uint32_t* __restrict__ end, uint32_t nchunks,
                                                     uint32_t L0, uint32_t step, size_t nbuckets,
                                                     xyzz<F>* __restrict__ buckets) {
  constexpr uint32_t S = MSM_COMBINE_S;
  msm_priority<F>();
  const uint32_t ch = lane_item<LN>();
  if (ch >= nchunks) return;
  const ChunkSlots<F> slots = all_slots.at(blockIdx.y, nchunks);
  buckets += blockIdx.y * nbuckets;
  uint32_t key = slots.tkey[ch];
  const bool tail = key != KEY_INVALID;
  if (!tail) {
    key = slots.hkey[ch];
    if (key == KEY_INVALID) return;
  }
  const uint32_t c0 = start[key] / L0, c1 = (end[key] - 1) / L0;
  if ((ch - c0) % (S * step) != 0 || ch + step > c1) return;  // nothing to fold here
  xyzz<F>* self = tail ? &slots.tpt[ch] : &slots.hpt[ch];
  auto acc = LN::load(*self);
  for (uint32_t m = 1; m < S && ch + m * step <= c1; m++) xyzz_add(acc, LN::load(slots.hpt[ch + m * step]));
  if (tail && c1 - c0 + 1 <= S * step) self = &buckets[key];
  LN::store(*self, acc);
}

// Tree combine of the buckets spanning more than MSM_SERIAL_SPAN + 1 chunks,
// in one launch.  Block j covers the TB chunks [j TB, j TB + TB), one item
// per chunk.  Inside a block every long bucket's head partials form one
// segment of consecutive items, summed by a tree over the item's position in
// its segment (log2 of the segment's length levels, all segments at once);
// the item holding the bucket's tail then adds the sum of the heads that
// follow it in the block.  A bucket inside one block is stored there.  A
// bucket crossing blocks j0 .. j1 gets one contribution per block: OUT[j0]
// (the tail plus the heads of block j0) and IN[j] for j0 < j <= j1 (the
// block's leading segment).  Each contribution is written, fenced and
// counted on fold_cnt[j0]; the block that brings the count to j1 - j0 + 1
// folds the contributions with the same tree and stores the bucket.  A block
// has at most one leading (IN) and one trailing (OUT) bucket, so it folds at
// most two.  Point addition is commutative, so the fold order does not change
// the bucket's value.
template <class F, class LN, int TB>
__global__ __launch_bounds__(TB * LN::N) void k_msm_combine_tree(ChunkSlots<F> all_slots,
                                                                 const uint32_t* __restrict__ start,
                                                                 const uint32_t* __restrict__ end,
                                                                 uint32_t nchunks, uint32_t L0, size_t nbuckets,
                                                                 xyzz<F>* __restrict__ buckets,
                                                                 uint32_t* __restrict__ fold_cnt,
                                                                 xyzz<F>* __restrict__ cin, xyzz<F>* __restrict__ cout) {
  typedef typename LN::R R;
  msm_priority<F>();
  __shared__ xyzz<F> V[TB];
  __shared__ uint32_t fold_key[2], fold_j0[2], fold_n[2], maxlen;
  const uint32_t t = threadIdx.x / LN::N;
  const bool lead = threadIdx.x % LN::N == 0;  // the lane of an item that does its atomics
  const uint32_t set = blockIdx.y;
  const uint32_t nblk = cdiv_dev(nchunks, TB);
  const ChunkSlots<F> slots = all_slots.at(set, nchunks);
  buckets += set * nbuckets;
  fold_cnt += (size_t)set * nblk;
  cin += (size_t)set * nblk;
  cout += (size_t)set * nblk;
  const uint32_t j = blockIdx.x, b0 = j * TB, b1 = min(b0 + TB, nchunks);  // the block's chunks [b0, b1)
  const uint32_t ch = b0 + t;
  if (t < 2) fold_key[t] = KEY_INVALID;
  if (t == 0) maxlen = 0;

  // this item's head partial, when it belongs to a long bucket
  uint32_t hk = KEY_INVALID, r = 0, len = 0, hc0 = 0, hc1 = 0;
  if (ch < b1) {
    const uint32_t k = slots.hkey[ch];
    if (k != KEY_INVALID) {
      hc0 = start[k] / L0;
      hc1 = (end[k] - 1) / L0;
      if (hc1 - hc0 > MSM_SERIAL_SPAN) {
        hk = k;
        const uint32_t lo = max(hc0 + 1, b0), hi = min(hc1, b1 - 1);
        r = ch - lo;
        len = hi - lo + 1;
      }
    }
  }
  // this item's tail partial, when it starts a long bucket
  uint32_t tk = KEY_INVALID, tc1 = 0;
  if (ch < b1) {
    const uint32_t k = slots.tkey[ch];
    if (k != KEY_INVALID) {
      tc1 = (end[k] - 1) / L0;
      if (tc1 - ch > MSM_SERIAL_SPAN) tk = k;
    }
  }
  __syncthreads();
  if (!__syncthreads_or(hk != KEY_INVALID || tk != KEY_INVALID)) return;  // no long bucket here
  if (hk != KEY_INVALID && r == 0 && lead) atomicMax(&maxlen, len);
  xyzz<R> v;
  xyzz_set_inf(v);
  if (hk != KEY_INVALID) {
    v = LN::load(slots.hpt[ch]);
    LN::store(V[t], v);
  }
  __syncthreads();
  const uint32_t levels_len = maxlen;
  for (uint32_t d = 1; d < levels_len; d <<= 1) {
    if (hk != KEY_INVALID && r % (2 * d) == 0 && r + d < len) {
      xyzz_add(v, LN::load(V[t + d]));
      LN::store(V[t], v);
    }
    __syncthreads();
  }
  // V[first item of a segment] = the segment's sum.  Contributions:
  if (tk != KEY_INVALID) {
    xyzz<R> acc = LN::load(slots.tpt[ch]);
    if (ch + 1 < b1) xyzz_add(acc, LN::load(V[t + 1]));  // the heads that follow in this block
    if (tc1 < b1) {
      LN::store(buckets[tk], acc);  // the whole bucket is in this block
    } else {
      LN::store(cout[j], acc);
      __threadfence();
      if (lead) {
        const uint32_t j1 = tc1 / TB, need = j1 - j + 1;
        if (atomicAdd(&fold_cnt[j], 1u) == need - 1) {
          fold_key[1] = tk;
          fold_j0[1] = j;
          fold_n[1] = need;
        }
      }
    }
  }
  if (hk != KEY_INVALID && r == 0 && hc0 < b0) {  // the leading segment of a bucket from an earlier block
    LN::store(cin[j], v);
    __threadfence();
    if (lead) {
      const uint32_t j0 = hc0 / TB, j1 = hc1 / TB, need = j1 - j0 + 1;
      if (atomicAdd(&fold_cnt[j0], 1u) == need - 1) {
        fold_key[0] = hk;
        fold_j0[0] = j0;
        fold_n[0] = need;
      }
    }
  }
  __syncthreads();
  // The last contributor of a crossing bucket folds OUT[j0], IN[j0+1 .. j1].
  for (int f = 0; f < 2; f++) {
    const uint32_t key = fold_key[f];
    if (key == KEY_INVALID) continue;  // uniform over the block
    __threadfence();
    const uint32_t j0 = fold_j0[f], n = fold_n[f];
    xyzz<R> a;
    xyzz_set_inf(a);
    for (uint32_t i = t; i < n; i += TB) xyzz_add(a, LN::load(i == 0 ? cout[j0] : cin[j0 + i]));
    __syncthreads();
    LN::store(V[t], a);
    __syncthreads();
    const uint32_t m = min(n, (uint32_t)TB);
    for (uint32_t d = 1; d < m; d <<= 1) {
      if (t % (2 * d) == 0 && t + d < m) {
        xyzz_add(a, LN::load(V[t + d]));
        LN::store(V[t], a);
      }
      __syncthreads();
    }
    if (t == 0) LN::store(buckets[key], a);
    __syncthreads();
  }
}

// ------------------------------------------------------------------ bucket reduction
// Window sum  sum_{b=1..B} b S_b,  B = 2^(c-1).
//
// Bucket b of a window holds digit b + 1.  Level 1: K workgroups per window;
// group k owns the buckets b = k + K p (every K-th bucket, positions
// p = 0 .. T G - 1), its thread t the positions p = t G + i, i < G, forming
//   run_t = sum_i S,  acc_t = sum_i (i+1) S      (2G additions, from the top).
// With the inclusive suffix sums SR_t = sum_{u >= t} run_u (Hillis-Steele scan
// in LDS),  sum_p (p+1) S = sum_t acc_t + G sum_{t >= 1} SR_t,  so each thread
// adds G*SR_t (log2 G doublings) to acc_t and a tree sums the group.  Outputs
// per group: P_k (that sum) and RUN_k = SR_0.
// Level 2 (k_msm_reduce2) weights group k by K and k + 1 - K, so its chain
// holds log2 K doublings where contiguous groups would need log2(T G).
// "Thread" t is an item of the lane layout LN; T = blockDim.x / LN::N.

// Inclusive suffix scan over the T values held by the items of a workgroup;
// returns this item's sum_{u >= t} v_u.
template <class F, class LN, class R>
__device__ __forceinline__ xyzz<R> wg_suffix_scan(xyzz<R> v, xyzz<F>* sh, int T) {
  const int t = threadIdx.x / LN::N;
  LN::store(sh[t], v);
  __syncthreads();
  for (int d = 1; d < T; d <<= 1) {
    xyzz<R> o;
    const bool has = t + d < T;
    if (has) o = LN::load(sh[t + d]);
    __syncthreads();
    if (has) {
      xyzz_add(v, o);
      LN::store(sh[t], v);
    }
    __syncthreads();
  }
  return v;
}

// Sum of the T values of a workgroup (T a power of two), valid in item 0.
template <class F, class LN, class R>
__device__ __forceinline__ xyzz<R> wg_sum(xyzz<R> v, xyzz<F>* sh, int T) {
  const int t = threadIdx.x / LN::N;
  __syncthreads();
  LN::store(sh[t], v);
  __syncthreads();
  for (int h = T / 2; h >= 1; h >>= 1) {
    if (t < h) {
      xyzz_add(v, LN::load(sh[t + h]));
      LN::store(sh[t], v);
    }
    __syncthreads();
  }
  return v;
}

// Level 1: block k of window w (blockIdx.x = w*K + k), T items of G buckets
// each (G = 2^log2g).  Windows of several base sets follow each other (W_set
// windows per set); the sorted-list bounds start/end are those of the window
// within its set.
template <class F, int TMAX, class LN>
__global__ __launch_bounds__(TMAX * LN::N) void k_msm_reduce1(const xyzz<F>* __restrict__ buckets,
                                                              const uint32_t* __restrict__ start,
                                                              const uint32_t* __restrict__ end, uint32_t B1,
                                                              uint32_t K, uint32_t W_set, int log2g,
                                                              xyzz<F>* __restrict__ P, xyzz<F>* __restrict__ RUN) {
  typedef typename LN::R R;
  msm_priority<F>();
  __shared__ xyzz<F> sh[TMAX];
  const int T = blockDim.x / LN::N, G = 1 << log2g;
  const uint32_t w = blockIdx.x / K, k = blockIdx.x % K;
  const uint32_t t = threadIdx.x / LN::N;
  // group k owns buckets k + K p, p = 0, 1, ...; this item the positions
  // p = t G + i, i < G
  const uint32_t kb = w * B1 + k;            // bucket of position 0
  const uint32_t sb = (w % W_set) * B1 + k;  // its key in the sorted list
  xyzz<R> run, acc;
  xyzz_set_inf(run);
  xyzz_set_inf(acc);
  for (int i = G - 1; i >= 0; i--) {
    const uint32_t off = (t * G + i) * K;
    if (end[sb + off] > start[sb + off]) xyzz_add(run, LN::load(buckets[kb + off]));
    xyzz_add(acc, run);
  }
  xyzz<R> sr = wg_suffix_scan<F, LN, R>(run, sh, T);
  if (t >= 1) {
    for (int d = 0; d < log2g; d++) xyzz_dbl(sr);
    xyzz_add(acc, sr);
  } else {
    LN::store(RUN[blockIdx.x], sr);  // item 0 holds the group total
  }
  xyzz<R> tot = wg_sum<F, LN, R>(acc, sh, T);
  if (t == 0) LN::store(P[blockIdx.x], tot);
}

// A point from the lane `lanes` above (ds_bpermute per 32-bit word); every
// lane of the wave must execute it.
template <class R>
__device__ __forceinline__ xyzz<R> shfl_down_pt(const xyzz<R>& p, int lanes) {
  xyzz<R> q;
  const uint32_t* s = reinterpret_cast<const uint32_t*>(&p);
  uint32_t* d = reinterpret_cast<uint32_t*>(&q);
#pragma unroll
  for (int i = 0; i < (int)(sizeof(xyzz<R>) / 4); i++) d[i] = (uint32_t)__shfl_down((int)s[i], lanes, 64);
  return q;
}

// Level 2: one workgroup of two waves per window over its K group results
// (K a power of two, at most one wave of items).  With P_k and RUN_k of the
// strided groups above,
//   sum_b (b+1) S_b = sum_k [(k+1) RUN_k + K (P_k - RUN_k)]
//                   = sum_k [SR_k + K (P_k - RUN_k)],  SR_k = sum_{k' >= k} RUN_k'.
// Wave 1 forms K (P_k - RUN_k) (log2 K doublings) while wave 0 forms the
// suffix sums with lane shuffles; wave 0 then adds them and sums the items.
// plain (when not null) gets the window's plain bucket sum SR_0.
template <class F, class LN>
__global__ __launch_bounds__(128) void k_msm_reduce2(const xyzz<F>* __restrict__ P, const xyzz<F>* __restrict__ RUN,
                                                     uint32_t K, int log2k, xyzz<F>* __restrict__ out,
                                                     xyzz<F>* __restrict__ plain) {
  typedef typename LN::R R;
  msm_priority<F>();
  __shared__ xyzz<F> ku[64];
  const uint32_t w = blockIdx.x;
  const uint32_t t = (threadIdx.x & 63) / LN::N;  // item within its wave
  const bool wave0 = threadIdx.x < 64;
  xyzz<R> v;
  xyzz_set_inf(v);
  if (!wave0) {
    if (t < K) {
      xyzz<R> r = LN::load(RUN[w * K + t]);
      v = LN::load(P[w * K + t]);
      r.y = fneg(r.y);
      xyzz_add(v, r);
      for (int d = 0; d < log2k; d++) xyzz_dbl(v);
      LN::store(ku[t], v);
    }
  } else {
    if (t < K) v = LN::load(RUN[w * K + t]);
    for (uint32_t d = 1; d < K; d <<= 1) {  // inclusive suffix scan
      const xyzz<R> o = shfl_down_pt(v, (int)(d * LN::N));
      if (t + d < K) xyzz_add(v, o);
    }
    if (plain && t == 0) LN::store(plain[w], v);
  }
  __syncthreads();
  if (wave0) {
    if (t < K) xyzz_add(v, LN::load(ku[t]));
    for (uint32_t d = K / 2; d >= 1; d >>= 1) {  // tree sum into item 0
      const xyzz<R> o = shfl_down_pt(v, (int)(d * LN::N));
      if (t < d) xyzz_add(v, o);
    }
    if (t == 0) LN::store(out[w], v);
  }
}

// ------------------------------------------------------------------ workspace
constexpr int MSM_MAX_W = 32;   // windows of the narrowest window (8 bits)
constexpr int MSM_PARTS = 192;  // window (or sub-window) partials of one MSM, all sets

struct MsmWorkspace {
  DevBuf recs, dig, hist, tot, lex, bsum, bmax, boff, tmp, sorted, start, end, wstat, buckets, hkey, tkey, hpt, tpt,
      seg, grp, win, fcnt, fin, fout;
  uint32_t* h_stat = nullptr;  // pinned, 2 words per window
  void* h_parts = nullptr;     // pinned, the per-window partials of every set
  hipEvent_t stat_ready = nullptr;
  MsmGate* gate = nullptr;  // waited for before the accumulation
};

void msm_workspace_gate(MsmWorkspace* ws, MsmGate* wait_before_accumulate) { ws->gate = wait_before_accumulate; }

void msm_workspace_free(MsmWorkspace* ws) {
  if (!ws) return;
  for (DevBuf* b : {&ws->recs, &ws->dig, &ws->hist, &ws->tot, &ws->lex, &ws->bsum, &ws->bmax, &ws->boff, &ws->tmp,
                    &ws->sorted, &ws->start, &ws->end, &ws->wstat, &ws->buckets, &ws->hkey, &ws->tkey, &ws->hpt,
                    &ws->tpt, &ws->seg, &ws->grp, &ws->win, &ws->fcnt, &ws->fin, &ws->fout})
    if (b->p) (void)hipFree(b->p);
  if (ws->h_stat) (void)hipHostFree(ws->h_stat);
  if (ws->h_parts) (void)hipHostFree(ws->h_parts);
  if (ws->stat_ready) (void)hipEventDestroy(ws->stat_ready);
  delete ws;
}

// Multiplier of the accumulation's wave scatter: coprime to nwaves (so
// v -> v * m mod nwaves is a permutation) and near nwaves / golden ratio, so
// that consecutive waves land far apart in the chunk space.
static uint32_t wave_scatter(uint32_t nwaves) {
  if (nwaves <= 2) return 1;
  uint32_t m = (uint32_t)(nwaves * 0.6180339887) | 1u;
  while (std::gcd(m, nwaves) != 1) m += 2;
  return m % nwaves;
}

// Window size by input size (index: ceil(log2 n)), from measurements on
// gfx950 with uniform scalars.  Below ~2^19 points the accumulation and the
// bucket reduction are latency-bound, so fewer buckets pay off well beyond
// what operation counts suggest; G2 operations are ~3x longer still.
static int choose_c(size_t n, bool g2) {
  int lg = 0;
  while (((size_t)1 << lg) < n) lg++;
  static const int g1_table[20] = {8, 8, 8, 8, 8, 8, 8, 8, 8, 8, 8, 8, 8, 9, 9, 10, 11, 12, 13, 14};
  static const int g2_table[20] = {8, 8, 8, 8, 8, 8, 8, 8, 8, 8, 8, 8, 8, 9, 9, 9, 10, 12, 13, 14};
  if (lg >= 20) return MSM_CMAX;
  return g2 ? g2_table[lg] : g1_table[lg];
}

// ------------------------------------------------------------------ host tail
template <class F>
struct HostSide;
// conv takes the device's limbs as they are (zkh::F::from_limbs29_scaled):
// every host use is a ratio X / ZZ or Y / ZZZ, in which the radix factor
// 2^5 cancels, so no conversion multiply is needed.
template <>
struct HostSide<fq> {
  typedef zkh::Fq E;
  static E conv(const fq& a) { return E::from_limbs29_scaled(a.l); }
  static void out(const E& x, const E& y, uint64_t* o) {
    memcpy(o, x.v, 32);
    memcpy(o + 4, y.v, 32);
  }
  static void out_jac(const zkh::Jac<E>& r, uint64_t* o) {
    memcpy(o, r.x.v, 32);
    memcpy(o + 4, r.y.v, 32);
    memcpy(o + 8, r.z.v, 32);
  }
};
template <>
struct HostSide<fq2> {
  typedef zkh::Fq2 E;
  static E conv(const fq2& a) {
    return E{zkh::Fq::from_limbs29_scaled(a.c0.l), zkh::Fq::from_limbs29_scaled(a.c1.l)};
  }
  static void out(const E& x, const E& y, uint64_t* o) {
    memcpy(o, x.c0.v, 32);
    memcpy(o + 4, x.c1.v, 32);
    memcpy(o + 8, y.c0.v, 32);
    memcpy(o + 12, y.c1.v, 32);
  }
  static void out_jac(const zkh::Jac<E>& r, uint64_t* o) {
    const E* c[3] = {&r.x, &r.y, &r.z};
    for (int i = 0; i < 3; i++) {
      memcpy(o + 8 * i, c[i]->c0.v, 32);
      memcpy(o + 8 * i + 4, c[i]->c1.v, 32);
    }
  }
};

// An MSM's result: affine words (x, y), or with jac_out Jacobian words (x, y,
// z) for a caller that adds it to other points before its own affine
// conversion (one inversion fewer).  Infinity is all zeros either way.
template <class F>
static void host_result(const zkh::Jac<typename HostSide<F>::E>& r, bool jac_out, uint64_t* out) {
  typedef typename HostSide<F>::E E;
  if (jac_out) {
    if (r.is_inf()) memset(out, 0, sizeof(E) * 3);
    else HostSide<F>::out_jac(r, out);
    return;
  }
  E ax, ay;
  r.to_affine(ax, ay);
  HostSide<F>::out(ax, ay, out);
}

// XYZZ partials (device layout, copied to the host) -> affine via one batch
// inversion -> per-window sums -> Horner over windows.
template <class F>
static void host_finish(const std::vector<xyzz<F>>& parts, int W, int per_w, uint64_t* out, bool jac_out) {
  typedef typename HostSide<F>::E E;
  typedef zkh::Jac<E> J;
  const size_t m = parts.size();
  std::vector<E> X(m), Y(m), ZZ(m), ZZZ(m), prod(m);
  std::vector<char> inf(m);
  E acc = E::one();
  for (size_t i = 0; i < m; i++) {
    X[i] = HostSide<F>::conv(parts[i].x);
    Y[i] = HostSide<F>::conv(parts[i].y);
    ZZ[i] = HostSide<F>::conv(parts[i].zz);
    ZZZ[i] = HostSide<F>::conv(parts[i].zzz);
    inf[i] = ZZ[i].is_zero();
    prod[i] = acc;
    if (!inf[i]) acc = acc * (ZZ[i] * ZZZ[i]);
  }
  E inv = acc.inv();
  std::vector<J> win(W, J::inf());
  for (size_t i = m; i-- > 0;) {
    if (inf[i]) continue;
    E d = ZZ[i] * ZZZ[i];
    E di = inv * prod[i];
    inv = inv * d;
    E x = X[i] * (di * ZZZ[i]);  // X / ZZ
    E y = Y[i] * (di * ZZ[i]);   // Y / ZZZ
    const int w = (int)(i / per_w);
    win[w] = win[w].add(J::affine(x, y));
  }
  J r = win[W - 1];
  for (int w = W - 2; w >= 0; w--) {
    for (int k = 0; k < window_width(w, W); k++) r = r.dbl();
    r = r.add(win[w]);
  }
  host_result<F>(r, jac_out, out);
}

// Sizes of one MSM: n points, W windows of about c bits, B buckets per window.
struct MsmShape {
  size_t n;
  int W;
  uint32_t B;
  uint32_t n_pad;  // window region of the sorted list, padded to the longest chunk
  uint32_t S;      // slices per window of the sort: about 256 blocks, each slice at least B points
};

// Counting sort of all windows on st.  The windows' entry counts and largest
// buckets are copied to ws.h_stat, and ws.stat_ready is recorded after the
// copy (the scatter is still running then).
static int msm_sort_wide(zk_context* ctx, MsmWorkspace& ws, const MsmShape& sh, hipStream_t st);

static int msm_sort(zk_context* ctx, MsmWorkspace& ws, const MsmShape& sh, bool small_blocks, hipStream_t st) {
  if (sh.B > MSM_LDS_B) return msm_sort_wide(ctx, ws, sh, st);
  const size_t n = sh.n;
  const int W = sh.W;
  const uint32_t B = sh.B, n_pad = sh.n_pad, S = sh.S, nb = B / SCAN_T;  // nb: column-scan blocks per window
  const uint32_t slice = (uint32_t)cdiv(n, S);
  const uint32_t* dig = (const uint32_t*)ws.dig.p;
  uint32_t* hist = (uint32_t*)ws.hist.p;
  uint32_t* tot = (uint32_t*)ws.tot.p;
  uint32_t* lex = (uint32_t*)ws.lex.p;
  uint32_t* bsum = (uint32_t*)ws.bsum.p;
  uint32_t* bmax = (uint32_t*)ws.bmax.p;
  uint32_t* boff = (uint32_t*)ws.boff.p;
  uint32_t* start = (uint32_t*)ws.start.p;
  uint32_t* end = (uint32_t*)ws.end.p;
  uint32_t* wstat = (uint32_t*)ws.wstat.p;
  uint2* sorted = (uint2*)ws.sorted.p;
  // small_blocks: the sort runs while other jobs' accumulations hold the CUs
  // (a proof's H); its small-bucket kernels then take blocks of 256 threads,
  // since a CU holding accumulation waves rarely has room for a 1024-thread
  // block, which waits for one to end (a 2^16 proof's H histogram took 210
  // us instead of 7 in a trace).  Config 4's proof 1.217-1.250 -> 1.213-1.236
  // ms over six runs on one box; for the B2 job, which sorts before the
  // accumulations, small blocks lost (1.23 -> 1.25 ms).
  constexpr int SMALL_T = 256;
  if (B <= 4096 && small_blocks) {
    ZK_LAUNCH(ctx, st, "msm_hist", (k_msm_hist<4096, SMALL_T>), dim3(S, W), dim3(SMALL_T), 0, dig, n, slice, S, B,
              hist);
  } else if (B <= 4096) {
    ZK_LAUNCH(ctx, st, "msm_hist", k_msm_hist<4096>, dim3(S, W), dim3(SORT_T), 0, dig, n, slice, S, B, hist);
  } else {
    ZK_LAUNCH(ctx, st, "msm_hist", k_msm_hist<32768>, dim3(S, W), dim3(SORT_T), 0, dig, n, slice, S, B, hist);
  }
  ZK_LAUNCH(ctx, st, "msm_scan", k_msm_colscan, dim3((uint32_t)W * nb), dim3(SCAN_T), 0, hist, S, B, tot, lex, bsum,
            bmax);
  ZK_LAUNCH(ctx, st, "msm_scan", k_msm_bscan, dim3(W), dim3(256), 0, bsum, bmax, nb, boff, wstat);
  ZK_HIP(ctx, hipMemcpyAsync(ws.h_stat, wstat, (size_t)W * 8, hipMemcpyDeviceToHost, st));
  ZK_HIP(ctx, hipEventRecord(ws.stat_ready, st));
  if (B <= 4096 && small_blocks) {
    ZK_LAUNCH(ctx, st, "msm_scatter", (k_msm_scatter<4096, SMALL_T>), dim3(S, W), dim3(SMALL_T), 0, dig, n, slice, S,
              B, n_pad, hist, boff, lex, tot, start, end, sorted);
  } else if (B <= 4096) {
    ZK_LAUNCH(ctx, st, "msm_scatter", k_msm_scatter<4096>, dim3(S, W), dim3(SORT_T), 0, dig, n, slice, S, B, n_pad,
              hist, boff, lex, tot, start, end, sorted);
  } else {
    const uint32_t BPC = B / MSM_NCB;  // 32..128
    uint2* tmp = (uint2*)ws.tmp.p;
    ZK_LAUNCH(ctx, st, "msm_scatter", k_msm_scatter_coarse, dim3(S, W), dim3(SORT_T), 0, dig, n, slice, S, B, BPC,
              n_pad, hist, boff, lex, tot, start, end, tmp);
    ZK_LAUNCH(ctx, st, "msm_place", k_msm_place, dim3(MSM_NCB, W), dim3(PLACE_T), 0, tmp, B, BPC, start, end, bmax,
              sorted);
  }
  return ZK_OK;
}

// The sort of one wide bucket space (window tables, B > 2^15) on st: coarse
// bins, then per-bin counting and placement; the entry count and largest
// bucket come back after the placement.
static int msm_sort_wide(zk_context* ctx, MsmWorkspace& ws, const MsmShape& sh, hipStream_t st) {
  if (sh.W != 1) return ctx->fail(ZK_ERR_INVALID, "msm: wide sort of several windows");
  int b = 0;
  while ((1u << b) < sh.B) b++;
  const uint32_t shift = (uint32_t)(b - WIDE_LOG_NB);  // log2 of the buckets per coarse bin
  if ((1u << b) != sh.B || b <= WIDE_LOG_NB || shift > 13)
    return ctx->fail(ZK_ERR_INVALID, "msm: wide sort bucket count");
  const size_t np = sh.n;
  const uint32_t S = (uint32_t)std::max<size_t>(1, std::min<size_t>(1024, cdiv(np, 32768)));
  const uint32_t slice = (uint32_t)cdiv(np, S);
  ZK_TRY(ctx->ensure(ws.hist, (size_t)WIDE_NB * S * 4));
  ZK_TRY(ctx->ensure(ws.boff, (size_t)(WIDE_NB + 1) * 4));
  ZK_TRY(ctx->ensure(ws.bsum, (size_t)WIDE_NB * 4));
  const uint32_t* dig = (const uint32_t*)ws.dig.p;
  uint32_t* cnt = (uint32_t*)ws.hist.p;
  uint32_t* binoff = (uint32_t*)ws.boff.p;
  uint32_t* bintot = (uint32_t*)ws.bsum.p;
  uint32_t* wstat = (uint32_t*)ws.wstat.p;
  uint2* tmp = (uint2*)ws.tmp.p;
  ZK_LAUNCH(ctx, st, "msm_hist", k_wide_count, dim3(S), dim3(SORT_T), 0, dig, np, slice, S, shift, cnt);
  ZK_LAUNCH(ctx, st, "msm_scan", k_wide_scan_rows, dim3(WIDE_NB), dim3(256), 0, cnt, S, bintot);
  ZK_LAUNCH(ctx, st, "msm_scan", k_wide_scan_bins, dim3(1), dim3(WIDE_NB), 0, bintot, binoff, wstat);
  ZK_LAUNCH(ctx, st, "msm_scatter", k_wide_scatter, dim3(S), dim3(SORT_T), 0, dig, np, slice, S, shift, cnt, binoff,
            tmp);
  ZK_LAUNCH(ctx, st, "msm_place", k_wide_place, dim3(WIDE_NB), dim3(PLACE_T), (size_t)4 << shift, tmp, binoff,
            shift, (uint32_t*)ws.start.p, (uint32_t*)ws.end.p, (uint2*)ws.sorted.p, wstat);
  ZK_HIP(ctx, hipMemcpyAsync(ws.h_stat, wstat, 8, hipMemcpyDeviceToHost, st));
  ZK_HIP(ctx, hipEventRecord(ws.stat_ready, st));
  return ZK_OK;
}

// Accumulation shape, from the sort statistics.
struct AccPlan {
  uint32_t L0;        // sorted entries per chunk
  uint32_t cpw;       // chunks per window
  uint32_t nchunks;   // chunks of one set
  uint32_t max_span;  // chunks spanned by the largest bucket
};

// Entries per accumulation thread, by the entry count (G1: zero digits are
// no entries, so skewed scalars, such as a witness of small values, count
// for less than W*n): short chunks give small MSMs enough threads (a thread's
// chunk is a serial chain of additions), long chunks keep the chunk-combine
// tree of large ones shallow.  Measured on MI355X over 2^10 .. 2^20 points,
// G1 and G2, uniform and witness-like scalars.  Inside a proof the same
// lengths serve: halving the G1 chunks beside the other jobs once paid (2^16
// proof 1.97 -> 1.87 ms), but with the proof's later host and placement
// work it cost config 4's 2^16 proof 1.26 -> 1.29 ms.
template <class F>
static AccPlan plan_accumulation(const MsmWorkspace& ws, const MsmShape& sh) {
  constexpr bool G2 = sizeof(F) != sizeof(fq);
  size_t entries = 0;
  uint32_t maxrun = 1;
  for (int w = 0; w < sh.W; w++) {
    entries += ws.h_stat[2 * w];
    maxrun = std::max(maxrun, ws.h_stat[2 * w + 1]);
  }
  entries += entries / 32;  // uniform scalars' few zero digits keep their chunk length
  // a G2 chunk combine costs about 3x a G1 one: shorter G2 chunks for skewed
  // scalars lost more there than they gained (2^16 witness-like G2 MSM 1.30 ->
  // 1.35 ms), so G2 keeps the length of W*n entries
  if (G2) entries = (size_t)sh.W * sh.n;
  const uint32_t L0_alone = entries >= ((size_t)1 << 23)   ? MSM_L0
                            : entries >= ((size_t)1 << 20) ? MSM_L0 / 2
                            : entries >= ((size_t)1 << 18) ? MSM_L0 / 4
                                                           : MSM_L0 / 8;
  AccPlan ap;
  ap.L0 = G2 ? std::max<uint32_t>(L0_alone >> ZK_MSM_G2_L0_SHIFT, MSM_L0 / 8) : L0_alone;
  ap.cpw = sh.n_pad / ap.L0;
  ap.nchunks = ap.cpw * (uint32_t)sh.W;
  ap.max_span = (maxrun + ap.L0 - 2) / ap.L0 + 1;
  return ap;
}

// Accumulation and chunk combine of all nsets sets, on st.
template <class F>
static int msm_accumulate(zk_context* ctx, MsmWorkspace& ws, const MsmShape& sh, const BaseSets& sets, int nsets,
                          const AccPlan& ap, bool beside, hipStream_t st) {
  constexpr bool G2 = sizeof(F) != sizeof(fq);
  const size_t nbuckets = (size_t)sh.W * sh.B;  // buckets of one set
  const uint2* sorted = (const uint2*)ws.sorted.p;
  const uint32_t* start = (const uint32_t*)ws.start.p;
  const uint32_t* end = (const uint32_t*)ws.end.p;
  const uint32_t* wstat = (const uint32_t*)ws.wstat.p;
  xyzz<F>* buckets = (xyzz<F>*)ws.buckets.p;
  const uint32_t nchunks = ap.nchunks, L0 = ap.L0;
  ZK_TRY(ctx->ensure(ws.hkey, (size_t)nsets * nchunks * 4));
  ZK_TRY(ctx->ensure(ws.tkey, (size_t)nsets * nchunks * 4));
  ZK_TRY(ctx->ensure(ws.hpt, (size_t)nsets * nchunks * sizeof(xyzz<F>)));
  ZK_TRY(ctx->ensure(ws.tpt, (size_t)nsets * nchunks * sizeof(xyzz<F>)));
  ChunkSlots<F> slots{(uint32_t*)ws.hkey.p, (uint32_t*)ws.tkey.p, (xyzz<F>*)ws.hpt.p, (xyzz<F>*)ws.tpt.p};
  // lanes per chunk: G1 one, G2 a lane pair, or one for the longest chunks
  // (the largest G2 MSMs, throughput-bound)
  const bool one_lane = G2 && ZK_MSM_G2_ONE_LANE && L0 >= (uint32_t)MSM_L0;
  const uint32_t lanes = one_lane ? 1 : Lanes<F>::N;
  const uint32_t gxl = cdiv((size_t)nchunks * lanes, 256);
  const uint32_t nwaves = cdiv((size_t)nchunks * lanes, 64);
  if (one_lane) {
    if constexpr (G2) {
      if (sets.pstride)
        ZK_LAUNCH(ctx, st, "msm_accumulate", (k_msm_accumulate<F, true, OneLane<F>>), dim3(gxl, nsets), dim3(256), 0,
                  sorted, sets, start, end, wstat, nchunks, ap.cpw, sh.n_pad, L0, nbuckets, buckets, slots, nwaves,
                  wave_scatter(nwaves));
      else
        ZK_LAUNCH(ctx, st, "msm_accumulate", (k_msm_accumulate<F, false, OneLane<F>>), dim3(gxl, nsets), dim3(256),
                  0, sorted, sets, start, end, wstat, nchunks, ap.cpw, sh.n_pad, L0, nbuckets, buckets, slots, nwaves,
                  wave_scatter(nwaves));
    }
  } else if (sets.pstride) {
    ZK_LAUNCH(ctx, st, "msm_accumulate", (k_msm_accumulate<F, true>), dim3(gxl, nsets), dim3(256), 0, sorted, sets,
              start, end, wstat, nchunks, ap.cpw, sh.n_pad, L0, nbuckets, buckets, slots, nwaves,
              wave_scatter(nwaves));
  } else {
    ZK_LAUNCH(ctx, st, "msm_accumulate", (k_msm_accumulate<F, false>), dim3(gxl, nsets), dim3(256), 0, sorted, sets,
              start, end, wstat, nchunks, ap.cpw, sh.n_pad, L0, nbuckets, buckets, slots, nwaves,
              wave_scatter(nwaves));
  }
  // The chunk combine and the bucket reduction are chains of dependent
  // additions.  Few of their waves are busy at once (the combine's active
  // chunks are the spanning runs), so they deal each point operation to two
  // lane groups (SplitLanes) wherever the plain layout would leave SIMDs idle.
  // Alone on the GPU a G2 MSM's combine stays on lane pairs (split over four
  // lanes its sparse chains shared SIMDs: G2 2^16 0.12 -> 0.15 ms); beside
  // other MSMs, where the SIMDs are shared anyway, it splits (proofs of 2^13
  // and 2^16 constraints 3-5% shorter).
  typedef SplitLanes<F> SL;
  const bool split_combine = !G2 || beside;
  const uint32_t gxs = cdiv((size_t)nchunks * (split_combine ? SL::N : Lanes<F>::N), 256);
  // The largest bucket decides the combine: spans of up to MSM_SERIAL_SPAN + 1
  // chunks fold serially in one launch; up to MSM_TREE_SPAN chunks, levels
  // folding MSM_COMBINE_S partials each; beyond, the serial launch takes the
  // short spans and the tree combine the long ones in a second launch (its
  // fold counters cleared by the first).
  if (ap.max_span > MSM_SERIAL_SPAN + 1 && ap.max_span <= MSM_TREE_SPAN) {
    for (uint64_t step = 1; step < ap.max_span; step *= MSM_COMBINE_S) {
      if (split_combine)
        ZK_LAUNCH(ctx, st, "msm_combine", (k_msm_combine<F, SL>), dim3(gxs, nsets), dim3(256), 0, slots, start, end,
                  nchunks, L0, (uint32_t)step, nbuckets, buckets);
      else
        ZK_LAUNCH(ctx, st, "msm_combine", (k_msm_combine<F, Lanes<F>>), dim3(gxs, nsets), dim3(256), 0, slots, start,
                  end, nchunks, L0, (uint32_t)step, nbuckets, buckets);
    }
  } else if (ap.max_span > 1) {
    const bool tree = ap.max_span > MSM_SERIAL_SPAN + 1;
    constexpr int TB = G2 ? 128 : 256;  // chunks per tree block (36 KB of LDS points)
    const uint32_t nblk = cdiv(nchunks, TB);
    uint32_t* fcnt = nullptr;
    if (tree) {
      ZK_TRY(ctx->ensure(ws.fcnt, (size_t)nsets * nblk * 4));
      ZK_TRY(ctx->ensure(ws.fin, (size_t)nsets * nblk * sizeof(xyzz<F>)));
      ZK_TRY(ctx->ensure(ws.fout, (size_t)nsets * nblk * sizeof(xyzz<F>)));
      fcnt = (uint32_t*)ws.fcnt.p;
    }
    if (split_combine)
      ZK_LAUNCH(ctx, st, "msm_combine", (k_msm_combine_serial<F, SL>), dim3(gxs, nsets), dim3(256), 0, slots, end,
                nchunks, L0, nbuckets, buckets, fcnt, (uint32_t)TB);
    else
      ZK_LAUNCH(ctx, st, "msm_combine", (k_msm_combine_serial<F, Lanes<F>>), dim3(gxs, nsets), dim3(256), 0, slots,
                end, nchunks, L0, nbuckets, buckets, fcnt, (uint32_t)TB);
    if (tree) {
      xyzz<F>* fin = (xyzz<F>*)ws.fin.p;
      xyzz<F>* fout = (xyzz<F>*)ws.fout.p;
      if (split_combine)
        ZK_LAUNCH(ctx, st, "msm_combine", (k_msm_combine_tree<F, SL, TB>), dim3(nblk, nsets), dim3(TB * SL::N), 0,
                  slots, start, end, nchunks, L0, nbuckets, buckets, fcnt, fin, fout);
      else
        ZK_LAUNCH(ctx, st, "msm_combine", (k_msm_combine_tree<F, Lanes<F>, TB>), dim3(nblk, nsets),
                  dim3(TB * Lanes<F>::N), 0, slots, start, end, nchunks, L0, nbuckets, buckets, fcnt, fin, fout);
    }
  }
  return ZK_OK;
}

// Bucket reduction of Wr windows of Br buckets per set (level 1: T threads
// x G buckets per group, level 2 per window); the window sums sum_b (b+1) S_b
// (set-major) are copied to the pinned ws.h_parts on st, followed, with
// `plain`, by the windows' plain sums sum_b S_b.
template <class F>
static int msm_reduce(zk_context* ctx, MsmWorkspace& ws, int Wr, uint32_t Br, int nsets, bool beside, bool plain,
                      hipStream_t st) {
  typedef SplitLanes<F> SL;
  const uint32_t B = Br;
  // items per workgroup (a G2 item is a lane pair: 256 lanes either way)
  constexpr int TMAX = sizeof(F) == sizeof(fq) ? 256 : 128;
  constexpr int KMAX = 64 / Lanes<F>::N;  // level 2 holds the K groups of a window in one wave
  // Level 1 splits its point operations (SplitLanes) when the plain layout
  // would fill at most half of the SIMDs.  Alone on the GPU a split
  // workgroup takes half the items (256 lanes, one wave per SIMD) and a
  // window twice the groups, so the chains spread over more CUs instead of
  // sharing SIMDs (G1 2^16 0.58 -> 0.53 ms, G2 2^16 1.08 -> 1.00 ms); beside
  // other MSMs it keeps the full items (fewer workgroups find CU slots
  // sooner: proofs 3-5% shorter that way).  At 2^15 buckets per window and
  // one wave per SIMD splitting lost (G1 2^20: 0.28 -> 0.31 ms), and so did
  // G = 4 there (0.37 ms).
  const bool split1 = (size_t)Wr * nsets * B / 4 * Lanes<F>::N <= (size_t)512 * 64;
  const bool half1 = split1 && !beside;
  const int TM = half1 ? TMAX / 2 : TMAX;
  // measured: T = TMAX; G = 8 for 2^15 buckets per window, else 4
  int T1 = TM, log2g = B >= 32768 ? 3 : 2;
  // shrink the group for small windows: T1 * G <= B
  while (log2g > 0 && (T1 << log2g) > (int)B) log2g--;
  while (T1 > 1 && (T1 << log2g) > (int)B) T1 >>= 1;
  uint32_t K = B / ((uint32_t)T1 << log2g);
  while (K > KMAX) {  // too many groups for level 2: widen the groups
    log2g++;
    K >>= 1;
  }
  if (T1 < 1 || T1 > TM || (T1 & (T1 - 1)) || K < 1 || (size_t)K * ((size_t)T1 << log2g) != B)
    return ctx->fail(ZK_ERR_INVALID, "msm: unsupported reduction shape");
  const uint32_t WS = (uint32_t)Wr * nsets;  // windows of all sets
  if (WS > MSM_PARTS) return ctx->fail(ZK_ERR_INVALID, "msm: too many windows");
  ZK_TRY(ctx->ensure(ws.seg, (size_t)K * WS * sizeof(xyzz<F>)));
  ZK_TRY(ctx->ensure(ws.grp, (size_t)K * WS * sizeof(xyzz<F>)));
  ZK_TRY(ctx->ensure(ws.win, (size_t)2 * WS * sizeof(xyzz<F>)));
  const xyzz<F>* buckets = (const xyzz<F>*)ws.buckets.p;
  const uint32_t* start = (const uint32_t*)ws.start.p;
  const uint32_t* end = (const uint32_t*)ws.end.p;
  xyzz<F>* Pk = (xyzz<F>*)ws.seg.p;
  xyzz<F>* RUNk = (xyzz<F>*)ws.grp.p;
  xyzz<F>* win = (xyzz<F>*)ws.win.p;
  xyzz<F>* pln = plain ? win + WS : nullptr;
  if (half1) {
    ZK_LAUNCH(ctx, st, "msm_reduce", (k_msm_reduce1<F, TMAX / 2, SL>), dim3(K * WS), dim3(T1 * SL::N), 0, buckets,
              start, end, B, K, (uint32_t)Wr, log2g, Pk, RUNk);
  } else if (split1) {
    ZK_LAUNCH(ctx, st, "msm_reduce", (k_msm_reduce1<F, TMAX, SL>), dim3(K * WS), dim3(T1 * SL::N), 0, buckets, start,
              end, B, K, (uint32_t)Wr, log2g, Pk, RUNk);
  } else {
    ZK_LAUNCH(ctx, st, "msm_reduce", (k_msm_reduce1<F, TMAX, Lanes<F>>), dim3(K * WS), dim3(T1 * Lanes<F>::N), 0,
              buckets, start, end, B, K, (uint32_t)Wr, log2g, Pk, RUNk);
  }
  int log2k = 0;
  while ((1u << log2k) < K) log2k++;
  // one group per window: its P is the window sum (no level-2 launch, which
  // beside other MSMs would wait for a CU with room for its two waves); level
  // 2 holds a window's K groups in one wave, split when they fit
  if (K > 1 && K * SL::N <= 64) {
    ZK_LAUNCH(ctx, st, "msm_reduce2", (k_msm_reduce2<F, SL>), dim3(WS), dim3(128), 0, Pk, RUNk, K, log2k, win, pln);
  } else if (K > 1) {
    ZK_LAUNCH(ctx, st, "msm_reduce2", (k_msm_reduce2<F, Lanes<F>>), dim3(WS), dim3(128), 0, Pk, RUNk, K, log2k, win,
              pln);
  }
  // pinned destination: a copy to pageable memory costs a staged transfer
  // (measured: G1 2^16 MSM 0.535 -> 0.505 ms, the 2^16 proof 1.70 -> 1.62 ms)
  ZK_HIP(ctx, hipMemcpyAsync(ws.h_parts, K > 1 ? win : Pk, (size_t)WS * sizeof(xyzz<F>), hipMemcpyDeviceToHost, st));
  // with one group per window the plain sum is that group's RUN
  if (plain)
    ZK_HIP(ctx, hipMemcpyAsync((xyzz<F>*)ws.h_parts + WS, K > 1 ? pln : RUNk, (size_t)WS * sizeof(xyzz<F>),
                               hipMemcpyDeviceToHost, st));
  return ZK_OK;
}

// Window-table MSM: one bucket space split into H sub-windows of 2^log_sub
// buckets; P[h] = sum_b (b+1) S_{h,b}, R[h] = sum_b S_{h,b} (device XYZZ).
// The sum over all buckets of (h 2^log_sub + b + 1) S_{h,b} is
//   sum_h P[h] + 2^log_sub sum_h h R[h],
// the second sum as running sums from the top sub-window down.
template <class F>
static void host_finish_sub(const xyzz<F>* P, const xyzz<F>* R, int H, int log_sub, uint64_t* out, bool jac_out) {
  typedef typename HostSide<F>::E E;
  typedef zkh::Jac<E> J;
  const size_t m = 2 * (size_t)H;
  std::vector<E> X(m), Y(m), ZZ(m), ZZZ(m), prod(m);
  std::vector<char> inf(m);
  E acc = E::one();
  for (size_t i = 0; i < m; i++) {
    const xyzz<F>& q = i < (size_t)H ? P[i] : R[i - H];
    X[i] = HostSide<F>::conv(q.x);
    Y[i] = HostSide<F>::conv(q.y);
    ZZ[i] = HostSide<F>::conv(q.zz);
    ZZZ[i] = HostSide<F>::conv(q.zzz);
    inf[i] = ZZ[i].is_zero();
    prod[i] = acc;
    if (!inf[i]) acc = acc * (ZZ[i] * ZZZ[i]);
  }
  E inv = acc.inv();
  std::vector<J> pt(m, J::inf());
  for (size_t i = m; i-- > 0;) {
    if (inf[i]) continue;
    E d = ZZ[i] * ZZZ[i];
    E di = inv * prod[i];
    inv = inv * d;
    pt[i] = J::affine(X[i] * (di * ZZZ[i]), Y[i] * (di * ZZ[i]));
  }
  J run = J::inf(), weighted = J::inf(), sum = J::inf();
  for (int h = H - 1; h >= 1; h--) {
    run = run.add(pt[H + h]);
    weighted = weighted.add(run);
  }
  for (int k = 0; k < log_sub; k++) weighted = weighted.dbl();
  for (int h = 0; h < H; h++) sum = sum.add(pt[h]);
  host_result<F>(sum.add(weighted), jac_out, out);
}

// MSMs of `nsets` point sets over one scalar vector of n entries (see
// BaseSets): one digit sort, then accumulation, chunk combine and bucket
// reduction for all sets in the same launches (the set is a grid dimension),
// so the sets share every latency-bound step.  Point records are in the
// internal form (see Rec<F>): the workspace's conversion buffer or a proving
// key's resident queries.  outs[s] receives set s's affine result.
template <class F>
static int msm_run_sets(zk_context* ctx, MsmWorkspace& ws, const BaseSets& sets_in, int nsets, const void* d_scalars,
                        size_t n, uint64_t* const* outs, hipStream_t st, bool beside = false,
                        const MsmTab* tab = nullptr, bool jac_out = false) {
  const int OUTW = (sizeof(F) == sizeof(fq) ? 4 : 8) * (jac_out ? 3 : 2);
  if (nsets < 1 || nsets > MSM_SETS) return ctx->fail(ZK_ERR_INVALID, "msm: 1 to 3 point sets");
  for (int k = 0; k < nsets; k++) memset(outs[k], 0, OUTW * 8);
  if (n == 0) return ZK_OK;
  if (n > MSM_MAX_N) return ctx->fail(ZK_ERR_SIZE, "msm: n above 2^26");
  constexpr bool G2 = sizeof(F) != sizeof(fq);
  BaseSets sets = sets_in;
  MsmShape sh;
  int Wd;  // digit windows
  if (!tab) {
    const int c = choose_c(n, G2);
    Wd = (MSM_BITS + c - 1) / c;
    sh.n = n;
    sh.W = Wd;
    sh.B = 1u << (c - 1);
    sets.pstride = 0;
  } else {
    // one bucket space for the positions w n + i of all windows
    Wd = tab->W;
    if (Wd < 1 || Wd > MSM_MAX_W || (size_t)Wd * n > MSM_MAX_N)
      return ctx->fail(ZK_ERR_INVALID, "msm: window table shape");
    sh.n = (size_t)Wd * n;
    sh.W = 1;
    sh.B = 1u << (window_width(0, Wd) - 1);
    if (tab->log_sub < 7 || ((size_t)1 << tab->log_sub) > sh.B)
      return ctx->fail(ZK_ERR_INVALID, "msm: window table sub-window size");
    sets.pstride = (uint32_t)n;
  }
  // window regions of the sorted list are padded to the longest chunk, so
  // every chunk length divides them (the length is chosen after the sort's
  // counts are known)
  sh.n_pad = (uint32_t)((sh.n + MSM_L0 - 1) / MSM_L0 * MSM_L0);
  // slices per window: about 256 blocks; each slice at least B points, or,
  // for the one bucket space of a window table, at least ZK_MSM_TAB_SLICE
  // (a slice's histogram of B counters is written and scanned once)
  sh.S = tab ? (uint32_t)std::max<size_t>(1, std::min<size_t>(256, sh.n / ZK_MSM_TAB_SLICE))
             : (uint32_t)std::max<size_t>(1, std::min<size_t>({(size_t)cdiv(256, sh.W), (size_t)64, sh.n / sh.B}));
  const int W = sh.W;
  if (W > MSM_MAX_W) return ctx->fail(ZK_ERR_INVALID, "msm: too many windows");
  const size_t nbuckets = (size_t)W * sh.B;
  ZK_TRY(ctx->ensure(ws.dig, (size_t)W * sh.n * 4));
  ZK_TRY(ctx->ensure(ws.hist, nbuckets * sh.S * 4));
  ZK_TRY(ctx->ensure(ws.tot, nbuckets * 4));
  ZK_TRY(ctx->ensure(ws.lex, nbuckets * 4));
  ZK_TRY(ctx->ensure(ws.bsum, nbuckets / SCAN_T * 4));
  ZK_TRY(ctx->ensure(ws.bmax, nbuckets / SCAN_T * 4));
  ZK_TRY(ctx->ensure(ws.boff, nbuckets / SCAN_T * 4));
  ZK_TRY(ctx->ensure(ws.sorted, (size_t)W * sh.n_pad * 8));
  if (sh.B > 4096) ZK_TRY(ctx->ensure(ws.tmp, (size_t)W * sh.n_pad * 8));
  ZK_TRY(ctx->ensure(ws.start, nbuckets * 4));
  ZK_TRY(ctx->ensure(ws.end, nbuckets * 4));
  ZK_TRY(ctx->ensure(ws.wstat, (size_t)W * 8));
  ZK_TRY(ctx->ensure(ws.buckets, nsets * nbuckets * sizeof(xyzz<F>)));
  if (!ws.h_stat) ZK_HIP(ctx, hipHostMalloc((void**)&ws.h_stat, 2 * MSM_MAX_W * 4, hipHostMallocDefault));
  if (!ws.h_parts)
    ZK_HIP(ctx, hipHostMalloc(&ws.h_parts, 2 * MSM_PARTS * sizeof(xyzz<fq2>), hipHostMallocDefault));
  if (!ws.stat_ready) ZK_HIP(ctx, hipEventCreateWithFlags(&ws.stat_ready, hipEventDisableTiming));

  ZK_LAUNCH(ctx, st, "msm_digits", k_msm_digits, dim3(cdiv(n, 256)), dim3(256), 0, (uint32_t*)ws.dig.p,
            (const uint4*)d_scalars, n, Wd);
  // a single-set G1 table MSM beside other jobs is a proof's H, sorted after
  // the quotient while the other jobs accumulate
  ZK_TRY(msm_sort(ctx, ws, sh, beside && nsets == 1 && tab != nullptr && sizeof(F) == sizeof(fq), st));
  // the windows' entry counts and largest buckets come back while the
  // scatter runs
  ZK_HIP(ctx, hipEventSynchronize(ws.stat_ready));
  const AccPlan ap = plan_accumulation<F>(ws, sh);
  if (ws.gate) {
    int gs;
    while ((gs = ws.gate->state.load()) == 0) std::this_thread::yield();
    if (gs == 1) ZK_HIP(ctx, hipStreamWaitEvent(st, ws.gate->ev, 0));
  }
  ZK_TRY(msm_accumulate<F>(ctx, ws, sh, sets, nsets, ap, beside, st));
  // a window table's bucket space reduces as sub-windows of 2^log_sub buckets
  const int Wr = tab ? (int)(sh.B >> tab->log_sub) : W;
  const uint32_t Br = tab ? 1u << tab->log_sub : sh.B;
  ZK_TRY(msm_reduce<F>(ctx, ws, Wr, Br, nsets, beside, tab != nullptr, st));
  ZK_HIP(ctx, hipStreamSynchronize(st));
  const xyzz<F>* parts = (const xyzz<F>*)ws.h_parts;
  // window combination on the host (W * c doublings per set): one thread per set
  int rc_fin[MSM_SETS] = {ZK_OK, ZK_OK, ZK_OK};
  auto finish = [&](int k) {
    try {
      if (tab)
        host_finish_sub<F>(parts + (size_t)k * Wr, parts + (size_t)(nsets + k) * Wr, Wr, tab->log_sub, outs[k],
                           jac_out);
      else
        host_finish<F>(std::vector<xyzz<F>>(parts + (size_t)k * W, parts + (size_t)(k + 1) * W), W, 1, outs[k],
                       jac_out);
    } catch (...) {
      rc_fin[k] = ZK_ERR_OOM;
    }
  };
  // the other sets on the context's worker threads (run here when none can
  // take them)
  std::vector<WorkerPool::TaskRef> helpers;
  struct Joiner {
    std::vector<WorkerPool::TaskRef>& v;
    ~Joiner() {
      for (const WorkerPool::TaskRef& t : v) WorkerPool::finish(t);
    }
  } joiner{helpers};
  for (int k = 1; k < nsets; k++) {
    WorkerPool::TaskRef t;
    try {
      t = ctx->pool.submit([&finish, k] { finish(k); });
    } catch (...) {
      t = nullptr;
    }
    if (t) helpers.push_back(t);
    else finish(k);
  }
  finish(0);
  for (const WorkerPool::TaskRef& t : helpers) WorkerPool::finish(t);
  for (int k = 0; k < nsets; k++)
    if (rc_fin[k] != ZK_OK) return ctx->fail(rc_fin[k], "msm: host allocation failed");
  return ZK_OK;
}

// One point set over all n scalars.
template <class F>
static int msm_run_recs(zk_context* ctx, MsmWorkspace& ws, const uint4* recs, const void* d_scalars, size_t n,
                        uint64_t* out, hipStream_t st, bool beside = false, bool jac_out = false) {
  BaseSets sets{};
  sets.recs[0] = recs;
  sets.lo[0] = 0;
  sets.hi[0] = (uint32_t)std::min<size_t>(n, 0xffffffffu);
  uint64_t* outs[1] = {out};
  return msm_run_sets<F>(ctx, ws, sets, 1, d_scalars, n, outs, st, beside, nullptr, jac_out);
}

template <class F>
static int msm_run(zk_context* ctx, MsmWorkspace*& wsp, const void* d_points, const void* d_scalars, size_t n,
                   uint64_t* out, hipStream_t st) {
  constexpr int OUTW = sizeof(F) == sizeof(fq) ? 8 : 16;
  memset(out, 0, OUTW * 8);
  if (n == 0) return ZK_OK;
  if (!d_points || !d_scalars) return ctx->fail(ZK_ERR_INVALID, "msm: null buffer");
  if (n > MSM_MAX_N) return ctx->fail(ZK_ERR_SIZE, "msm: n above 2^26");
  if (!wsp) wsp = new MsmWorkspace();
  MsmWorkspace& ws = *wsp;
  ZK_TRY(ctx->ensure(ws.recs, n * Rec<F>::WORDS * 4));
  ZK_LAUNCH(ctx, st, "msm_convert", k_msm_convert<F>, dim3(cdiv(n, 256)), dim3(256), 0, (uint4*)ws.recs.p,
            (const uint32_t*)d_points, n);
  return msm_run_recs<F>(ctx, ws, (const uint4*)ws.recs.p, d_scalars, n, out, st);
}

int msm_g1_run(zk_context* ctx, const void* d_points, const void* d_scalars, size_t n, uint64_t out[8],
               hipStream_t st) {
  return msm_run<fq>(ctx, ctx->msm_ws, d_points, d_scalars, n, out, st);
}

int msm_g2_run(zk_context* ctx, const void* d_points, const void* d_scalars, size_t n, uint64_t out[16],
               hipStream_t st) {
  return msm_run<fq2>(ctx, ctx->msm_ws_g2, d_points, d_scalars, n, out, st);
}

MsmWorkspace* msm_workspace_new() { return new MsmWorkspace(); }

int msm_g1_sets_ws(zk_context* ctx, MsmWorkspace* ws, int nsets, const void* const* recs, const size_t* lo,
                   const size_t* count, const void* d_scalars, size_t n, uint64_t* const* outs, hipStream_t st,
                   bool beside, const MsmTab* tab, const size_t* rows) {
  if (!ws || nsets < 1 || nsets > MSM_SETS) return ctx->fail(ZK_ERR_INVALID, "msm: 1 to 3 point sets");
  if (tab && !rows) return ctx->fail(ZK_ERR_INVALID, "msm: window table without its row length");
  BaseSets sets{};
  for (int k = 0; k < nsets; k++) {
    if (lo[k] + count[k] > n) return ctx->fail(ZK_ERR_INVALID, "msm: point set beyond the scalars");
    if (tab && count[k] > rows[k]) return ctx->fail(ZK_ERR_INVALID, "msm: point set beyond its window table");
    sets.recs[k] = (const uint4*)recs[k];
    sets.lo[k] = (uint32_t)lo[k];
    sets.hi[k] = (uint32_t)(lo[k] + count[k]);
    sets.tstride[k] = tab ? (uint32_t)rows[k] : 0u;
  }
  return msm_run_sets<fq>(ctx, *ws, sets, nsets, d_scalars, n, outs, st, beside, tab);
}

int msm_recs_tab(zk_context* ctx, MsmWorkspace* ws, bool g2, const void* d_table, size_t rows, const MsmTab& tab,
                 const void* d_scalars, size_t n, uint64_t* out, hipStream_t st, bool beside, bool jac_out) {
  if (!ws) return ctx->fail(ZK_ERR_INVALID, "msm: no workspace");
  if (n > rows) return ctx->fail(ZK_ERR_INVALID, "msm: more scalars than window table rows");
  BaseSets sets{};
  sets.recs[0] = (const uint4*)d_table;
  sets.lo[0] = 0;
  sets.hi[0] = (uint32_t)n;
  sets.tstride[0] = (uint32_t)rows;
  uint64_t* outs[1] = {out};
  if (g2) return msm_run_sets<fq2>(ctx, *ws, sets, 1, d_scalars, n, outs, st, beside, &tab, jac_out);
  return msm_run_sets<fq>(ctx, *ws, sets, 1, d_scalars, n, outs, st, beside, &tab, jac_out);
}

// ------------------------------------------------------------------ window tables

// tmp[w count + j] = 2^(bits of the windows below w) P_j, XYZZ.
template <class F>
__global__ void k_msm_tab_double(const uint4* __restrict__ recs, size_t count, int W, xyzz<F>* __restrict__ tmp) {
  const size_t j = blockIdx.x * (size_t)blockDim.x + threadIdx.x;
  if (j >= count) return;
  F x, y;
  xyzz<F> p;
  if (load_rec(recs, (uint32_t)j, x, y))
    xyzz_set_inf(p);
  else
    xyzz_set_affine(p, x, y);
  for (int w = 0; w < W; w++) {
    tmp[(size_t)w * count + j] = p;
    if (w + 1 < W)
      for (int k = 0; k < window_width(w, W); k++) xyzz_dbl(p);
  }
}

// XYZZ -> canonical affine records, PER points per thread sharing one inversion.
template <class F, int PER>
__global__ void k_msm_tab_affine(const xyzz<F>* __restrict__ tmp, size_t total, uint4* __restrict__ out) {
  const size_t base = (blockIdx.x * (size_t)blockDim.x + threadIdx.x) * PER;
  if (base >= total) return;
  xyzz<F> p[PER];
  for (int k = 0; k < PER; k++) {
    if (base + k < total)
      p[k] = tmp[base + k];
    else
      xyzz_set_inf(p[k]);
  }
  F x[PER], y[PER];
  bool inf[PER];
  xyzz_to_affine_batch<F, PER>(p, x, y, inf);
  for (int k = 0; k < PER; k++) {
    if (base + k >= total) continue;
    if (inf[k]) {
      fset_zero(x[k]);
      fset_zero(y[k]);
    }
    store_rec(out, base + k, x[k], y[k], inf[k]);
  }
}

size_t msm_table_bytes(bool g2, size_t count, const MsmTab& t) {
  return (size_t)t.W * count * (g2 ? Rec<fq2>::WORDS : Rec<fq>::WORDS) * 4;
}

template <class F>
static int table_build(zk_context* ctx, const uint4* recs, size_t count, const MsmTab& t, uint4* table,
                       hipStream_t st) {
  if (t.W < 1 || t.W > MSM_MAX_W || (size_t)t.W * count > MSM_MAX_N)
    return ctx->fail(ZK_ERR_INVALID, "msm table: window count");
  if (count == 0) return ZK_OK;
  DevBuf tmp;
  ZK_TRY(ctx->ensure(tmp, (size_t)t.W * count * sizeof(xyzz<F>)));
  int rc = ZK_OK;
  {
    (void)hipGetLastError();
    zk::TimingToken tk = ctx->tic("msm_table", st);
    hipLaunchKernelGGL(k_msm_tab_double<F>, dim3(cdiv(count, 128)), dim3(128), 0, st, recs, count, t.W,
                       (xyzz<F>*)tmp.p);
    constexpr int PER = sizeof(F) == sizeof(fq) ? 4 : 2;
    const size_t total = (size_t)t.W * count;
    hipLaunchKernelGGL((k_msm_tab_affine<F, PER>), dim3(cdiv(cdiv(total, PER), 128)), dim3(128), 0, st,
                       (const xyzz<F>*)tmp.p, total, table);
    if (hipGetLastError() != hipSuccess) rc = ctx->fail(ZK_ERR_HIP, "msm table: launch");
    ctx->toc(tk, st);
  }
  // the temporary goes once the kernels are done
  if (hipStreamSynchronize(st) != hipSuccess && rc == ZK_OK) rc = ctx->fail(ZK_ERR_HIP, "msm table: build");
  (void)hipFree(tmp.p);
  return rc;
}

int msm_table_build(zk_context* ctx, bool g2, const void* d_recs, size_t count, const MsmTab& t, void* d_table,
                    hipStream_t st) {
  if (!d_recs || !d_table) return ctx->fail(ZK_ERR_INVALID, "msm table: null buffer");
  if (g2) return table_build<fq2>(ctx, (const uint4*)d_recs, count, t, (uint4*)d_table, st);
  return table_build<fq>(ctx, (const uint4*)d_recs, count, t, (uint4*)d_table, st);
}

int msm_recs_ws(zk_context* ctx, MsmWorkspace* ws, bool g2, const void* d_recs, const void* d_scalars, size_t n,
                uint64_t* out, hipStream_t st, bool beside, bool jac_out) {
  if (!ws) return ctx->fail(ZK_ERR_INVALID, "msm: no workspace");
  if (g2) return msm_run_recs<fq2>(ctx, *ws, (const uint4*)d_recs, d_scalars, n, out, st, beside, jac_out);
  return msm_run_recs<fq>(ctx, *ws, (const uint4*)d_recs, d_scalars, n, out, st, beside, jac_out);
}

// Records of n points for MSMs over one base set, converted once (the
// conversion k_msm_convert otherwise runs on every standalone MSM call).
int msm_points_to_recs(zk_context* ctx, bool g2, const void* d_points, size_t n, void* d_recs, hipStream_t st) {
  if (n == 0) return ZK_OK;
  if (!d_points || !d_recs) return ctx->fail(ZK_ERR_INVALID, "msm: null buffer");
  if (n > MSM_MAX_N) return ctx->fail(ZK_ERR_SIZE, "msm: n above 2^26");
  const size_t bytes = n * (size_t)(g2 ? Rec<fq2>::WORDS : Rec<fq>::WORDS) * 4;
  const uintptr_t p0 = (uintptr_t)d_points, r0 = (uintptr_t)d_recs;
  if (p0 < r0 + bytes && r0 < p0 + bytes) return ctx->fail(ZK_ERR_INVALID, "msm: records overlap the points");
  if (g2) {
    ZK_LAUNCH(ctx, st, "msm_convert", k_msm_convert<fq2>, dim3(cdiv(n, 256)), dim3(256), 0, (uint4*)d_recs,
              (const uint32_t*)d_points, n);
  } else {
    ZK_LAUNCH(ctx, st, "msm_convert", k_msm_convert<fq>, dim3(cdiv(n, 256)), dim3(256), 0, (uint4*)d_recs,
              (const uint32_t*)d_points, n);
  }
  return ZK_OK;
}

int msm_g1_recs(zk_context* ctx, const void* d_recs, const void* d_scalars, size_t n, uint64_t out[8],
                hipStream_t st) {
  if (!ctx->msm_ws) ctx->msm_ws = new MsmWorkspace();
  return msm_run_recs<fq>(ctx, *ctx->msm_ws, (const uint4*)d_recs, d_scalars, n, out, st);
}

int msm_g2_recs(zk_context* ctx, const void* d_recs, const void* d_scalars, size_t n, uint64_t out[16],
                hipStream_t st) {
  if (!ctx->msm_ws_g2) ctx->msm_ws_g2 = new MsmWorkspace();
  return msm_run_recs<fq2>(ctx, *ctx->msm_ws_g2, (const uint4*)d_recs, d_scalars, n, out, st);
}

// Point records from standard-form coordinates (proving-key files store
// x, y in standard form, src/prover/groth16.cu:1131-1150).  flags[i] != 0
// marks the point at infinity.
template <class F>
__global__ void k_recs_from_std(uint4* __restrict__ recs, const uint32_t* __restrict__ std_words,
                                const uint8_t* __restrict__ flags, size_t n) {
  size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x;
  if (i >= n) return;
  constexpr int EW = Rec<F>::WORDS;
  uint32_t e[EW];
#pragma unroll
  for (int k = 0; k < EW; k++) e[k] = std_words[i * EW + k];
  F x, y;
  std_to_coord(e, x);
  std_to_coord(e + EW / 2, y);
  store_rec(recs, i, x, y, flags[i] != 0);
}

int recs_from_std(zk_context* ctx, bool g2, void* d_recs, const void* d_std, const void* d_flags, size_t n,
                  hipStream_t st) {
  if (n == 0) return ZK_OK;
  if (g2)
    ZK_LAUNCH(ctx, st, "pk_convert", k_recs_from_std<fq2>, dim3(cdiv(n, 256)), dim3(256), 0, (uint4*)d_recs,
              (const uint32_t*)d_std, (const uint8_t*)d_flags, n);
  else
    ZK_LAUNCH(ctx, st, "pk_convert", k_recs_from_std<fq>, dim3(cdiv(n, 256)), dim3(256), 0, (uint4*)d_recs,
              (const uint32_t*)d_std, (const uint8_t*)d_flags, n);
  return ZK_OK;
}

size_t rec_bytes(bool g2) { return g2 ? Rec<fq2>::WORDS * 4 : Rec<fq>::WORDS * 4; }

}  // namespace zk

// ------------------------------------------------------------------ C ABI
extern "C" {

static int zk_msm_g1_impl(zk_context* ctx, const void* d_points, const void* d_scalars, size_t n, void* h_result,
                          void* stream) {
  if (!ctx || !h_result) return ZK_ERR_INVALID;
  return zk::msm_g1_run(ctx, d_points, d_scalars, n, (uint64_t*)h_result, ctx->s(stream));
}

int zk_msm_g1(zk_context* ctx, const void* d_points, const void* d_scalars, size_t n, void* h_result, void* stream) {
  return zk::guard(ctx, [&] { return zk_msm_g1_impl(ctx, d_points, d_scalars, n, h_result, stream); });
}

static int zk_msm_g2_impl(zk_context* ctx, const void* d_points, const void* d_scalars, size_t n, void* h_result,
                          void* stream) {
  if (!ctx || !h_result) return ZK_ERR_INVALID;
  return zk::msm_g2_run(ctx, d_points, d_scalars, n, (uint64_t*)h_result, ctx->s(stream));
}

int zk_msm_g2(zk_context* ctx, const void* d_points, const void* d_scalars, size_t n, void* h_result, void* stream) {
  return zk::guard(ctx, [&] { return zk_msm_g2_impl(ctx, d_points, d_scalars, n, h_result, stream); });
}

size_t zk_msm_record_bytes(int g2) { return (size_t)(g2 ? zk::Rec<zk::fq2>::WORDS : zk::Rec<zk::fq>::WORDS) * 4; }

int zk_msm_prepare_points(zk_context* ctx, const void* d_points, size_t n, int g2, void* d_recs, void* stream) {
  if (!ctx) return ZK_ERR_INVALID;
  return zk::guard(ctx, [&] { return zk::msm_points_to_recs(ctx, g2 != 0, d_points, n, d_recs, ctx->s(stream)); });
}

static int zk_msm_prepared_impl(zk_context* ctx, bool g2, const void* d_recs, const void* d_scalars, size_t n,
                                void* h_result, void* stream) {
  if (!ctx || !h_result) return ZK_ERR_INVALID;
  if (n > 0 && (!d_recs || !d_scalars)) {
    memset(h_result, 0, g2 ? 128 : 64);
    return ctx->fail(ZK_ERR_INVALID, "msm: null buffer");
  }
  if (g2) return zk::msm_g2_recs(ctx, d_recs, d_scalars, n, (uint64_t*)h_result, ctx->s(stream));
  return zk::msm_g1_recs(ctx, d_recs, d_scalars, n, (uint64_t*)h_result, ctx->s(stream));
}

int zk_msm_g1_prepared(zk_context* ctx, const void* d_recs, const void* d_scalars, size_t n, void* h_result,
                       void* stream) {
  return zk::guard(ctx, [&] { return zk_msm_prepared_impl(ctx, false, d_recs, d_scalars, n, h_result, stream); });
}

int zk_msm_g2_prepared(zk_context* ctx, const void* d_recs, const void* d_scalars, size_t n, void* h_result,
                       void* stream) {
  return zk::guard(ctx, [&] { return zk_msm_prepared_impl(ctx, true, d_recs, d_scalars, n, h_result, stream); });
}

int zk_msm_config(size_t n, int g2, int* window_bits, int* windows) {
  if (!window_bits || !windows) return ZK_ERR_INVALID;
  *window_bits = zk::choose_c(n, g2 != 0);
  *windows = (zk::MSM_BITS + *window_bits - 1) / *window_bits;
  return ZK_OK;
}

// Reference host structs: G1Affine = {Fp x, y; bool infinity} (72 bytes),
// G2Affine = {Fp2 x, y; bool infinity} (136 bytes); results as Jacobian with
// z = 1 (or the reference identity (0, 1, 0)).
static int msm_host_common(zk_context* ctx, const void* h_points, const void* h_scalars, int n, void* h_result,
                           bool g2) {
  if (!ctx || !h_result || n < 0 || (n > 0 && (!h_points || !h_scalars))) return ZK_ERR_INVALID;
  const int cw = g2 ? 16 : 8;                 // u64 words of (x, y)
  const size_t rec = g2 ? 136 : 72;           // reference struct size
  uint64_t res[16];
  memset(res, 0, sizeof(res));
  if (n > 0) {
    std::vector<uint64_t> pts((size_t)n * cw);
    for (int i = 0; i < n; i++) {
      const uint8_t* p = (const uint8_t*)h_points + rec * i;
      const bool inf = p[cw * 8] != 0;
      if (inf) memset(&pts[(size_t)i * cw], 0, cw * 8);
      else memcpy(&pts[(size_t)i * cw], p, cw * 8);
    }
    void *dp = nullptr, *ds = nullptr;
    ZK_TRY(zk_dev_alloc(ctx, pts.size() * 8, &dp));
    int stt = zk_dev_alloc(ctx, (size_t)n * 32, &ds);
    if (stt == ZK_OK) stt = zk_memcpy_h2d(ctx, dp, pts.data(), pts.size() * 8);
    if (stt == ZK_OK) stt = zk_memcpy_h2d(ctx, ds, h_scalars, (size_t)n * 32);
    if (stt == ZK_OK)
      stt = g2 ? zk::msm_g2_run(ctx, dp, ds, n, res, ctx->stream) : zk::msm_g1_run(ctx, dp, ds, n, res, ctx->stream);
    zk_dev_free(ctx, dp);
    zk_dev_free(ctx, ds);
    if (stt != ZK_OK) return stt;
  }
  // Jacobian out: x, y, z (each cw/2 words)
  uint64_t* o = (uint64_t*)h_result;
  const int half = cw / 2;
  bool inf = true;
  for (int i = 0; i < cw; i++) inf = inf && res[i] == 0;
  memset(o, 0, 3 * half * 8);
  if (inf) {
    // reference identity: (0, 1, 0) with 1 in Montgomery form
    memcpy(o + half, zkh::QMod::ONE, 32);
  } else {
    memcpy(o, res, cw * 8);
    memcpy(o + cw, zkh::QMod::ONE, 32);
  }
  return ZK_OK;
}

static int zk_msm_g1_host_impl(zk_context* ctx, const void* h_points, const void* h_scalars, int n,
                               void* h_result_jacobian) {
  return msm_host_common(ctx, h_points, h_scalars, n, h_result_jacobian, false);
}

int zk_msm_g1_host(zk_context* ctx, const void* h_points, const void* h_scalars, int n, void* h_result_jacobian) {
  return zk::guard(ctx, [&] { return zk_msm_g1_host_impl(ctx, h_points, h_scalars, n, h_result_jacobian); });
}

static int zk_msm_g2_host_impl(zk_context* ctx, const void* h_points, const void* h_scalars, int n,
                               void* h_result_jacobian) {
  return msm_host_common(ctx, h_points, h_scalars, n, h_result_jacobian, true);
}

int zk_msm_g2_host(zk_context* ctx, const void* h_points, const void* h_scalars, int n, void* h_result_jacobian) {
  return zk::guard(ctx, [&] { return zk_msm_g2_host_impl(ctx, h_points, h_scalars, n, h_result_jacobian); });
}

}  // extern "C"
