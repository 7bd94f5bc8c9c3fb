// Pippenger multi-scalar multiplication over BN254 G1 and G2 for gfx950.
//
// Replaces bn254::msm_g1 / msm_g2 (reference src/msm/msm.cu:320-598): one
// thread per point walking all windows with a global spin lock per bucket,
// one thread per window for the bucket reduction and a host combination.
// Here (same mathematical result, canonical affine output):
//
//  1. convert    points -> internal records (29-bit limbs, radix 2^261), once.
//  2. digits     scalar -> standard form; if s > (r-1)/2 use r - s and -P;
//                signed c-bit digits d_w in [-2^(c-1), 2^(c-1)]; one
//                (key = w<<c | |d_w|, value = point | sign<<31) per window,
//                key SKIP for d_w = 0.
//  3. sort       rocPRIM radix sort of the W*n (key, value) pairs.
//  4. bounds     [start, end) of every key in the sorted order, and the count
//                of real entries (SKIP keys sort last).
//  5. accumulate every thread sums exactly L0 consecutive sorted entries
//                with mixed XYZZ additions (perfect load balance whatever the
//                bucket sizes); runs that cross a chunk edge leave a head /
//                tail partial.
//  6. combine    log-depth tree over the chunk partials of each bucket that
//                spans chunks (one level for ordinary buckets, ~log2(size/L0)
//                levels for hot buckets such as many scalars equal to 1).
//  7. reduce     sum_b b*S_b per window: G-bucket segments with running sums
//                plus (segment offset)*run, then an LDS tree per 256 segments.
//  8. host       remaining per-window partials are summed and combined with
//                W*c doublings on the CPU (serial chain: a CPU core beats a
//                lone wave64 by an order of magnitude on it).
#include <string.h>

#include <algorithm>
#include <vector>

#include "curve.hpp"
#include "host_bn254.hpp"
#include "zk_internal.hpp"

namespace zk {

constexpr uint32_t KEY_INVALID = 0xffffffffu;
constexpr int MSM_L0 = 64;         // sorted entries per accumulation thread
constexpr int MSM_G = 8;           // buckets per reduction thread

// ------------------------------------------------------------------ point records
// G1 record: x[9], y[9], inf, pad  (80 bytes);  G2 record: x0,x1,y0,y1 [9 each],
// inf, pad[3] (160 bytes).  Coordinates in internal form, canonical.
template <class F>
struct Rec;
template <>
struct Rec<fq> {
  static constexpr int WORDS = 20;
  static constexpr int EXT_WORDS = 16;  // 64 external bytes
};
template <>
struct Rec<fq2> {
  static constexpr int WORDS = 40;
  static constexpr int EXT_WORDS = 32;  // 128 external bytes
};

__device__ __forceinline__ fq load_fq9(const uint32_t* p) {
  fq r;
#pragma unroll
  for (int i = 0; i < NL; i++) r.l[i] = p[i];
  return r;
}
__device__ __forceinline__ void store_fq9(uint32_t* p, const fq& a) {
#pragma unroll
  for (int i = 0; i < NL; i++) p[i] = a.l[i];
}

__device__ __forceinline__ void load_coord(const uint32_t* p, fq& a) { a = load_fq9(p); }
__device__ __forceinline__ void load_coord(const uint32_t* p, fq2& a) {
  a.c0 = load_fq9(p);
  a.c1 = load_fq9(p + NL);
}
__device__ __forceinline__ void store_coord(uint32_t* p, const fq& a) { store_fq9(p, a); }
__device__ __forceinline__ void store_coord(uint32_t* p, const fq2& a) {
  store_fq9(p, a.c0);
  store_fq9(p + NL, a.c1);
}
template <class F>
__device__ __forceinline__ constexpr int coord_words() {
  return sizeof(F) / 4;
}

// Record load through 16-byte vector loads (records are 16-byte aligned).
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
  load_coord(w, x);
  load_coord(w + coord_words<F>(), y);
  return w[2 * coord_words<F>()] != 0;  // infinity flag
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
__device__ __forceinline__ fq fcanon_coord(const fq& a) { return fcanon(a); }
__device__ __forceinline__ fq2 fcanon_coord(const fq2& a) { return fq2{fcanon(a.c0), fcanon(a.c1)}; }

template <class F>
__global__ void k_msm_convert(uint4* __restrict__ recs, const uint32_t* __restrict__ ext, size_t n) {
  size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x;
  if (i >= n) return;
  constexpr int EW = Rec<F>::EXT_WORDS, W = Rec<F>::WORDS, CW = coord_words<F>();
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
  uint32_t w[W];
  store_coord(w, x);
  store_coord(w + CW, y);
  w[2 * CW] = any == 0 ? 1u : 0u;
#pragma unroll
  for (int k = 2 * CW + 1; k < W; k++) w[k] = 0;
  uint4* p = recs + i * (W / 4);
#pragma unroll
  for (int k = 0; k < W / 4; k++) p[k] = make_uint4(w[4 * k], w[4 * k + 1], w[4 * k + 2], w[4 * k + 3]);
}

// ------------------------------------------------------------------ digits
// (r-1)/2, little-endian 32-bit words
__constant__ uint32_t HALF_R[8] = {0xf8000000u, 0xa1f0fac9u, 0x3cdcb848u, 0x9419f424u,
                                   0x40c0ac2eu, 0xdc2822dbu, 0x7098d014u, 0x18322739u};
__constant__ uint32_t R_WORDS[8] = {0xf0000001u, 0x43e1f593u, 0x79b97091u, 0x2833e848u,
                                    0x8181585du, 0xb85045b6u, 0xe131a029u, 0x30644e72u};

__global__ void k_msm_digits(uint32_t* __restrict__ keys, uint32_t* __restrict__ vals,
                             const uint4* __restrict__ scalars, size_t n, int c, int W) {
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
  const uint32_t mask = (1u << c) - 1u, half = 1u << (c - 1);
  const uint32_t skip = (uint32_t)W << c;
  uint32_t carry = 0;
  for (int w = 0; w < W; w++) {
    const int bit = w * c, wd = bit >> 5, sh = bit & 31;
    uint64_t v = wd < 8 ? s[wd] : 0;
    if (wd + 1 < 8) v |= (uint64_t)s[wd + 1] << 32;
    uint32_t d = ((uint32_t)(v >> sh) & mask) + carry;
    uint32_t sign = neg;
    if (d > half) {
      d = (1u << c) - d;
      carry = 1;
      sign ^= 1u;
    } else {
      carry = 0;
    }
    const size_t o = (size_t)w * n + i;
    if (d == 0) {
      keys[o] = skip;
      vals[o] = 0;
    } else {
      keys[o] = ((uint32_t)w << c) | d;
      vals[o] = (uint32_t)i | (sign << 31);
    }
  }
}

// ------------------------------------------------------------------ bounds
// stat[0] = number of non-SKIP entries, stat[1] = longest run.
__global__ void k_msm_bounds(const uint32_t* __restrict__ sk, size_t total, uint32_t skip, uint32_t* __restrict__ start,
                             uint32_t* __restrict__ end, uint32_t* __restrict__ stat) {
  size_t p = blockIdx.x * (size_t)blockDim.x + threadIdx.x;
  if (p >= total) return;
  const uint32_t k = sk[p];
  const bool first = p == 0 || sk[p - 1] != k;
  const bool last = p + 1 == total || sk[p + 1] != k;
  if (k == skip) {
    if (first) stat[0] = (uint32_t)p;
    return;
  }
  if (first) start[k] = (uint32_t)p;
  if (last) {
    end[k] = (uint32_t)(p + 1);
    if (p + 1 == total) stat[0] = (uint32_t)total;
  }
}

// longest run, after bounds are complete; one atomic per wave
__global__ void k_msm_maxrun(const uint32_t* __restrict__ start, const uint32_t* __restrict__ end, size_t nkeys,
                             uint32_t* __restrict__ stat) {
  size_t k = blockIdx.x * (size_t)blockDim.x + threadIdx.x;
  uint32_t len = k < nkeys ? end[k] - start[k] : 0;
  for (int off = 32; off >= 1; off >>= 1) len = max(len, (uint32_t)__shfl_xor((int)len, off));
  if ((threadIdx.x & 63) == 0 && len > 1) atomicMax(&stat[1], len);
}

// ------------------------------------------------------------------ accumulate
template <class F>
struct ChunkSlots {
  uint32_t* hkey;
  uint32_t* tkey;
  xyzz<F>* hpt;
  xyzz<F>* tpt;
};

template <class F>
__device__ __forceinline__ uint32_t bucket_id(uint32_t key, int c) {
  return (key >> c) * (1u << (c - 1)) + (key & ((1u << c) - 1u)) - 1u;
}

template <class F>
__global__ __launch_bounds__(256) void k_msm_accumulate(const uint32_t* __restrict__ sk, const uint32_t* __restrict__ sv,
                                                        const uint4* __restrict__ recs,
                                                        const uint32_t* __restrict__ start,
                                                        const uint32_t* __restrict__ end,
                                                        const uint32_t* __restrict__ stat, uint32_t nchunks, int c,
                                                        xyzz<F>* __restrict__ buckets, ChunkSlots<F> slots) {
  const uint32_t ch = blockIdx.x * blockDim.x + threadIdx.x;
  if (ch >= nchunks) return;
  const uint32_t total = stat[0];
  const uint32_t lo = ch * MSM_L0;
  uint32_t hk = KEY_INVALID, tk = KEY_INVALID;
  if (lo < total) {
    const uint32_t hi = min(lo + (uint32_t)MSM_L0, total);
    xyzz<F> acc;
    xyzz_set_inf(acc);
    uint32_t cur = sk[lo];
    for (uint32_t p = lo; p < hi; p++) {
      const uint32_t key = sk[p];
      if (key != cur) {
        // run `cur` ended inside the chunk
        if (start[cur] < lo) {
          hk = cur;
          slots.hpt[ch] = acc;
        } else {
          buckets[bucket_id<F>(cur, c)] = acc;
        }
        cur = key;
        xyzz_set_inf(acc);
      }
      const uint32_t v = sv[p];
      F x, y;
      if (!load_rec(recs, v & 0x7fffffffu, x, y)) {
        if (v >> 31) y = fneg(y);
        xyzz_madd(acc, x, y);
      }
    }
    // last run of the chunk
    const uint32_t rs = start[cur], re = end[cur];
    if (rs >= lo && re <= lo + (uint32_t)MSM_L0) {
      buckets[bucket_id<F>(cur, c)] = acc;
    } else if (rs < lo) {
      hk = cur;
      slots.hpt[ch] = acc;
    } else {
      tk = cur;
      slots.tpt[ch] = acc;
    }
  }
  slots.hkey[ch] = hk;
  slots.tkey[ch] = tk;
}

// One level of the tree over the chunk partials of buckets spanning chunks.
template <class F>
__global__ __launch_bounds__(256) void k_msm_combine(ChunkSlots<F> slots, const uint32_t* __restrict__ start,
                                                     const uint32_t* __restrict__ end, uint32_t nchunks,
                                                     uint32_t step) {
  const uint32_t ch = blockIdx.x * blockDim.x + threadIdx.x;
  if (ch >= nchunks) return;
  const uint32_t tk = slots.tkey[ch];
  if (tk != KEY_INVALID) {
    const uint32_t c1 = (end[tk] - 1) / MSM_L0;
    if (ch + step <= c1) xyzz_add(slots.tpt[ch], slots.hpt[ch + step]);
  }
  const uint32_t hk = slots.hkey[ch];
  if (hk != KEY_INVALID) {
    const uint32_t c0 = start[hk] / MSM_L0, c1 = (end[hk] - 1) / MSM_L0;
    const uint32_t j = ch - c0;
    if ((j % (2 * step)) == 0 && ch + step <= c1) xyzz_add(slots.hpt[ch], slots.hpt[ch + step]);
  }
}

template <class F>
__global__ __launch_bounds__(256) void k_msm_finalize(ChunkSlots<F> slots, uint32_t nchunks, int c,
                                                      xyzz<F>* __restrict__ buckets) {
  const uint32_t ch = blockIdx.x * blockDim.x + threadIdx.x;
  if (ch >= nchunks) return;
  const uint32_t tk = slots.tkey[ch];
  if (tk != KEY_INVALID) buckets[bucket_id<F>(tk, c)] = slots.tpt[ch];
}

// ------------------------------------------------------------------ bucket reduction
// Window sum  sum_{b=1..B} b S_b,  B = 2^(c-1).
//
// Level 1: a workgroup of T threads owns T*G consecutive buckets (base k*T*G);
// thread t owns buckets base + t*G + i, i = 1..G, and forms
//   run_t = sum_i S,  acc_t = sum_i i S      (2G additions, from the top).
// With the inclusive suffix sums SR_t = sum_{u >= t} run_u (Hillis-Steele scan
// in LDS),  sum_{b in group} (b - base) S_b = sum_t acc_t + G sum_{t >= 1} SR_t,
// so each thread adds G*SR_t (log2 G doublings) to acc_t and a tree sums the
// group.  Outputs per group: P_k (that sum) and RUN_k = SR_0.
// Level 2 (one workgroup per window, K groups):
//   sum_b b S_b = sum_k P_k + T G sum_{s >= 1} SRUN_s,  same scan and tree.

// Inclusive suffix scan over the T values held by the threads of a
// workgroup; returns this thread's sum_{u >= t} v_u.
template <class F, int T>
__device__ __forceinline__ xyzz<F> wg_suffix_scan(xyzz<F> v, xyzz<F>* sh) {
  const int t = threadIdx.x;
  sh[t] = v;
  __syncthreads();
  for (int d = 1; d < T; d <<= 1) {
    xyzz<F> o;
    const bool has = t + d < T;
    if (has) o = sh[t + d];
    __syncthreads();
    if (has) {
      xyzz_add(v, o);
      sh[t] = v;
    }
    __syncthreads();
  }
  return v;
}

template <class F, int T>
__device__ __forceinline__ xyzz<F> wg_sum(xyzz<F> v, xyzz<F>* sh) {
  const int t = threadIdx.x;
  __syncthreads();
  sh[t] = v;
  __syncthreads();
  for (int h = T / 2; h >= 1; h >>= 1) {
    if (t < h) {
      xyzz_add(v, sh[t + h]);
      sh[t] = v;
    }
    __syncthreads();
  }
  return v;
}

template <class F, int T>
__global__ __launch_bounds__(T) void k_msm_reduce1(const xyzz<F>* __restrict__ buckets,
                                                   const uint32_t* __restrict__ start,
                                                   const uint32_t* __restrict__ end, int c, uint32_t K,
                                                   xyzz<F>* __restrict__ P, xyzz<F>* __restrict__ RUN) {
  __shared__ xyzz<F> sh[T];
  const uint32_t B1 = 1u << (c - 1);
  const uint32_t w = blockIdx.x / K, k = blockIdx.x % K;
  const uint32_t t = threadIdx.x;
  const uint32_t b0 = k * T * MSM_G + t * MSM_G;  // bucket index offset of this thread
  xyzz<F> run, acc;
  xyzz_set_inf(run);
  xyzz_set_inf(acc);
  for (int i = MSM_G; i >= 1; i--) {
    const uint32_t b = b0 + i;
    const uint32_t key = (w << c) | b;
    if (end[key] > start[key]) xyzz_add(run, buckets[w * B1 + b - 1]);
    xyzz_add(acc, run);
  }
  xyzz<F> sr = wg_suffix_scan<F, T>(run, sh);
  if (t >= 1) {
    for (int d = 1; d < MSM_G; d <<= 1) xyzz_dbl(sr);
    xyzz_add(acc, sr);
  } else {
    RUN[blockIdx.x] = sr;  // thread 0 holds the group total
  }
  xyzz<F> tot = wg_sum<F, T>(acc, sh);
  if (t == 0) P[blockIdx.x] = tot;
}

// One workgroup of K threads per window; log2tg = log2(T*G).
template <class F, int KMAX>
__global__ __launch_bounds__(KMAX) void k_msm_reduce2(const xyzz<F>* __restrict__ P, const xyzz<F>* __restrict__ RUN,
                                                      uint32_t K, int log2tg, xyzz<F>* __restrict__ out) {
  __shared__ xyzz<F> sh[KMAX];
  const uint32_t w = blockIdx.x, t = threadIdx.x;
  xyzz<F> run, acc;
  xyzz_set_inf(run);
  xyzz_set_inf(acc);
  if (t < K) {
    run = RUN[w * K + t];
    acc = P[w * K + t];
  }
  xyzz<F> sr = wg_suffix_scan<F, KMAX>(run, sh);
  if (t >= 1 && t < K) {
    for (int d = 0; d < log2tg; d++) xyzz_dbl(sr);
    xyzz_add(acc, sr);
  }
  xyzz<F> tot = wg_sum<F, KMAX>(acc, sh);
  if (t == 0) out[w] = tot;
}

// ------------------------------------------------------------------ workspace
struct MsmWorkspace {
  DevBuf recs, keys_in, vals_in, keys_out, vals_out, sort_tmp, start, end, stat, buckets, hkey, tkey, hpt, tpt, seg,
      grp, win;
  uint32_t* h_stat = nullptr;  // pinned
};

void msm_workspace_free(MsmWorkspace* ws) {
  if (!ws) return;
  for (DevBuf* b : {&ws->recs, &ws->keys_in, &ws->vals_in, &ws->keys_out, &ws->vals_out, &ws->sort_tmp, &ws->start,
                    &ws->end, &ws->stat, &ws->buckets, &ws->hkey, &ws->tkey, &ws->hpt, &ws->tpt, &ws->seg, &ws->grp,
                    &ws->win})
    if (b->p) (void)hipFree(b->p);
  if (ws->h_stat) (void)hipHostFree(ws->h_stat);
  delete ws;
}

// Window size minimizing W(c) * (n + 1.5 * 2^c) additions (accumulation plus
// bucket reduction), with W(c) = ceil(254 / c) signed windows.
static int choose_c(size_t n) {
  int best = 8;
  double bestv = 1e300;
  for (int c = 8; c <= 18; c++) {
    const int W = (254 + c - 1) / c;
    const double v = (double)W * ((double)n + 1.5 * (double)(1u << c));
    if (v < bestv) {
      bestv = v;
      best = c;
    }
  }
  return best;
}

// ------------------------------------------------------------------ host tail
template <class F>
struct HostSide;
template <>
struct HostSide<fq> {
  typedef zkh::Fq E;
  static E conv(const fq& a) {
    uint32_t w[8];
    to_mont256(a, w);
    return E::raw(w);
  }
  static void out(const E& x, const E& y, uint64_t* o) {
    memcpy(o, x.v, 32);
    memcpy(o + 4, y.v, 32);
  }
};
template <>
struct HostSide<fq2> {
  typedef zkh::Fq2 E;
  static E conv(const fq2& a) {
    uint32_t w0[8], w1[8];
    to_mont256(a.c0, w0);
    to_mont256(a.c1, w1);
    return E{zkh::Fq::raw(w0), zkh::Fq::raw(w1)};
  }
  static void out(const E& x, const E& y, uint64_t* o) {
    memcpy(o, x.c0.v, 32);
    memcpy(o + 4, x.c1.v, 32);
    memcpy(o + 8, y.c0.v, 32);
    memcpy(o + 12, y.c1.v, 32);
  }
};

// XYZZ partials (device layout, copied to the host) -> affine via one batch
// inversion -> per-window sums -> Horner over windows.
template <class F>
static void host_finish(const std::vector<xyzz<F>>& parts, int W, int per_w, int c, uint64_t* out) {
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
  J r = J::inf();
  for (int w = W - 1; w >= 0; w--) {
    for (int k = 0; k < c; k++) r = r.dbl();
    r = r.add(win[w]);
  }
  E ax, ay;
  r.to_affine(ax, ay);
  HostSide<F>::out(ax, ay, out);
}

// MSM over prepared point records (internal form, see Rec<F>).  `recs` may be
// the workspace's own conversion buffer or a proving key's resident queries.
template <class F>
static int msm_run_recs(zk_context* ctx, MsmWorkspace& ws, const uint4* recs, const void* d_scalars, size_t n,
                        uint64_t* out, hipStream_t st) {
  constexpr int OUTW = sizeof(F) == sizeof(fq) ? 8 : 16;
  memset(out, 0, OUTW * 8);
  if (n == 0) return ZK_OK;
  const int c = choose_c(n);
  const int W = (254 + c - 1) / c;
  const size_t total = (size_t)W * n;
  const size_t nkeys = ((size_t)W + 1) << c;
  const size_t nbuckets = (size_t)W << (c - 1);
  const uint32_t nchunks = (uint32_t)((total + MSM_L0 - 1) / MSM_L0);
  ZK_TRY(ctx->ensure(ws.keys_in, total * 4));
  ZK_TRY(ctx->ensure(ws.vals_in, total * 4));
  ZK_TRY(ctx->ensure(ws.keys_out, total * 4));
  ZK_TRY(ctx->ensure(ws.vals_out, total * 4));
  ZK_TRY(ctx->ensure(ws.start, nkeys * 4));
  ZK_TRY(ctx->ensure(ws.end, nkeys * 4));
  ZK_TRY(ctx->ensure(ws.stat, 16));
  ZK_TRY(ctx->ensure(ws.buckets, nbuckets * sizeof(xyzz<F>)));
  ZK_TRY(ctx->ensure(ws.hkey, (size_t)nchunks * 4));
  ZK_TRY(ctx->ensure(ws.tkey, (size_t)nchunks * 4));
  ZK_TRY(ctx->ensure(ws.hpt, (size_t)nchunks * sizeof(xyzz<F>)));
  ZK_TRY(ctx->ensure(ws.tpt, (size_t)nchunks * sizeof(xyzz<F>)));
  if (!ws.h_stat) ZK_HIP(ctx, hipHostMalloc((void**)&ws.h_stat, 16, hipHostMallocDefault));

  uint32_t* kin = (uint32_t*)ws.keys_in.p;
  uint32_t* vin = (uint32_t*)ws.vals_in.p;
  uint32_t* kout = (uint32_t*)ws.keys_out.p;
  uint32_t* vout = (uint32_t*)ws.vals_out.p;
  uint32_t* start = (uint32_t*)ws.start.p;
  uint32_t* end = (uint32_t*)ws.end.p;
  uint32_t* stat = (uint32_t*)ws.stat.p;
  xyzz<F>* buckets = (xyzz<F>*)ws.buckets.p;

  ZK_LAUNCH(ctx, st, "msm_digits", k_msm_digits, dim3(cdiv(n, 256)), dim3(256), 0, kin, vin,
            (const uint4*)d_scalars, n, c, W);

  const unsigned end_bit = 32 - __builtin_clz((unsigned)((W << c) | 1));
  ZK_TRY(sort_pairs_u32(ctx, ws.sort_tmp, kin, kout, vin, vout, total, end_bit, st));

  ZK_HIP(ctx, hipMemsetAsync(start, 0, nkeys * 4, st));
  ZK_HIP(ctx, hipMemsetAsync(end, 0, nkeys * 4, st));
  ZK_HIP(ctx, hipMemsetAsync(stat, 0, 16, st));
  ZK_LAUNCH(ctx, st, "msm_bounds", k_msm_bounds, dim3(cdiv(total, 256)), dim3(256), 0, kout, total,
            (uint32_t)(W << c), start, end, stat);
  ZK_LAUNCH(ctx, st, "msm_bounds", k_msm_maxrun, dim3(cdiv(nkeys, 256)), dim3(256), 0, start, end, nkeys, stat);
  ZK_HIP(ctx, hipMemcpyAsync(ws.h_stat, stat, 8, hipMemcpyDeviceToHost, st));
  ZK_HIP(ctx, hipStreamSynchronize(st));
  const uint32_t real = ws.h_stat[0];
  const uint32_t maxrun = std::max(1u, ws.h_stat[1]);

  ChunkSlots<F> slots{(uint32_t*)ws.hkey.p, (uint32_t*)ws.tkey.p, (xyzz<F>*)ws.hpt.p, (xyzz<F>*)ws.tpt.p};
  const uint32_t used_chunks = std::max(1u, (real + MSM_L0 - 1) / MSM_L0);
  ZK_LAUNCH(ctx, st, "msm_accumulate", k_msm_accumulate<F>, dim3(cdiv(used_chunks, 256)), dim3(256), 0, kout, vout,
            recs, start, end, stat, used_chunks, c, buckets, slots);
  // chunks spanned by the longest run
  const uint32_t max_span = (maxrun + MSM_L0 - 2) / MSM_L0 + 1;
  for (uint32_t step = 1; step < max_span; step <<= 1)
    ZK_LAUNCH(ctx, st, "msm_combine", k_msm_combine<F>, dim3(cdiv(used_chunks, 256)), dim3(256), 0, slots, start,
              end, used_chunks, step);
  ZK_LAUNCH(ctx, st, "msm_combine", k_msm_finalize<F>, dim3(cdiv(used_chunks, 256)), dim3(256), 0, slots,
            used_chunks, c, buckets);

  // bucket reduction: level 1 (T threads x G buckets per group), level 2 per window
  constexpr int T1 = sizeof(F) == sizeof(fq) ? 256 : 128;
  const uint32_t B1 = 1u << (c - 1);
  int t1 = (int)std::min<uint32_t>(T1, B1 / MSM_G);
  const uint32_t K = B1 / (t1 * MSM_G);
  ZK_TRY(ctx->ensure(ws.seg, (size_t)K * W * sizeof(xyzz<F>)));
  ZK_TRY(ctx->ensure(ws.grp, (size_t)K * W * sizeof(xyzz<F>)));
  ZK_TRY(ctx->ensure(ws.win, (size_t)W * sizeof(xyzz<F>)));
  xyzz<F>* Pk = (xyzz<F>*)ws.seg.p;
  xyzz<F>* RUNk = (xyzz<F>*)ws.grp.p;
  xyzz<F>* win = (xyzz<F>*)ws.win.p;
  switch (t1) {
#define ZK_R1(TT)                                                                                              \
  case TT:                                                                                                     \
    ZK_LAUNCH(ctx, st, "msm_reduce", (k_msm_reduce1<F, TT>), dim3(K * W), dim3(TT), 0, buckets, start, end, c, K, \
              Pk, RUNk);                                                                                       \
    break;
    ZK_R1(256)
    ZK_R1(128)
    ZK_R1(64)
    ZK_R1(32)
    ZK_R1(16)
#undef ZK_R1
    default:
      return ctx->fail(ZK_ERR_INVALID, "msm: unsupported reduction shape");
  }
  int log2tg = 0;
  while ((1 << log2tg) < t1 * MSM_G) log2tg++;
  if (K <= 32)
    ZK_LAUNCH(ctx, st, "msm_reduce", (k_msm_reduce2<F, 32>), dim3(W), dim3(32), 0, Pk, RUNk, K, log2tg, win);
  else if (K <= 128)
    ZK_LAUNCH(ctx, st, "msm_reduce", (k_msm_reduce2<F, 128>), dim3(W), dim3(128), 0, Pk, RUNk, K, log2tg, win);
  else
    return ctx->fail(ZK_ERR_INVALID, "msm: too many reduction groups");
  std::vector<xyzz<F>> parts((size_t)W);
  ZK_HIP(ctx, hipMemcpyAsync(parts.data(), win, parts.size() * sizeof(xyzz<F>), hipMemcpyDeviceToHost, st));
  ZK_HIP(ctx, hipStreamSynchronize(st));
  host_finish<F>(parts, W, 1, c, out);
  return ZK_OK;
}

template <class F>
static int msm_run(zk_context* ctx, MsmWorkspace*& wsp, const void* d_points, const void* d_scalars, size_t n,
                   uint64_t* out, hipStream_t st) {
  constexpr int OUTW = sizeof(F) == sizeof(fq) ? 8 : 16;
  memset(out, 0, OUTW * 8);
  if (n == 0) return ZK_OK;
  if (!d_points || !d_scalars) return ctx->fail(ZK_ERR_INVALID, "msm: null buffer");
  if (n > (1u << 28)) return ctx->fail(ZK_ERR_SIZE, "msm: n above 2^28");
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
  constexpr int EW = Rec<F>::EXT_WORDS, W = Rec<F>::WORDS, CW = coord_words<F>();
  uint32_t e[EW];
#pragma unroll
  for (int k = 0; k < EW; k++) e[k] = std_words[i * EW + k];
  const bool inf = flags[i] != 0;
  uint32_t w[W];
#pragma unroll
  for (int k = 0; k < W; k++) w[k] = 0;
  if (!inf) {
    F x, y;
    std_to_coord(e, x);
    std_to_coord(e + EW / 2, y);
    store_coord(w, fcanon_coord(x));
    store_coord(w + CW, fcanon_coord(y));
  }
  w[2 * CW] = inf ? 1u : 0u;
  uint4* p = recs + i * (W / 4);
#pragma unroll
  for (int k = 0; k < W / 4; k++) p[k] = make_uint4(w[4 * k], w[4 * k + 1], w[4 * k + 2], w[4 * k + 3]);
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

int zk_msm_g1(zk_context* ctx, const void* d_points, const void* d_scalars, size_t n, void* h_result, void* stream) {
  if (!ctx || !h_result) return ZK_ERR_INVALID;
  return zk::msm_g1_run(ctx, d_points, d_scalars, n, (uint64_t*)h_result, ctx->s(stream));
}

int zk_msm_g2(zk_context* ctx, const void* d_points, const void* d_scalars, size_t n, void* h_result, void* stream) {
  if (!ctx || !h_result) return ZK_ERR_INVALID;
  return zk::msm_g2_run(ctx, d_points, d_scalars, n, (uint64_t*)h_result, ctx->s(stream));
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

int zk_msm_g1_host(zk_context* ctx, const void* h_points, const void* h_scalars, int n, void* h_result_jacobian) {
  return msm_host_common(ctx, h_points, h_scalars, n, h_result_jacobian, false);
}

int zk_msm_g2_host(zk_context* ctx, const void* h_points, const void* h_scalars, int n, void* h_result_jacobian) {
  return msm_host_common(ctx, h_points, h_scalars, n, h_result_jacobian, true);
}

}  // extern "C"
