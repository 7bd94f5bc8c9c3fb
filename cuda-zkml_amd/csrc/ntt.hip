// BN254 Fr NTT, inverse NTT and coset NTT for gfx950.
//
// Replaces bn254::ntt_gpu (reference src/ntt/ntt.cu:354-465): a bit-reversal
// kernel, a shared-memory kernel for the first ten stages and one HBM pass per
// remaining stage with host-built twiddles.  Here a transform of n = 2^L is a
// four-step (Bailey) decomposition n = R_0 * ... * R_{P-1} with P <= 3 passes
// over HBM and R_p <= 256:
//
//   digits of the input index (most significant first) n_0 .. n_{P-1};
//   pass p < P-1: DFT of size R_p over digit n_p for every setting of the
//     other digits, result k_p written back in place, then multiplied by
//     w_{R_p S_p}^(k_p * m) with m the index formed by the lower digits
//     (S_p = R_{p+1} * ... * R_{P-1});
//   pass P-1: DFT over the last digit and a digit-reversed store so that the
//     output index is k_0 + R_0 k_1 + R_0 R_1 k_2 (natural order).
//
// Every pass works on a tile of 1024 elements (R rows x 1024/R columns) in
// LDS: the 1024/R columns are adjacent in HBM, so each row of the tile is a
// contiguous segment of >= 128 bytes.  The sub-DFT is radix-2 DIT on the
// bit-reversed rows, with w_R^t from a small table.  Field elements live in
// LDS as nine 29-bit limb planes (conflict-free for consecutive lanes).
//
// Radix bookkeeping: the NTT is linear, so the kernels run directly on the
// 256-bit words of the reference's Montgomery form (repack only); twiddles and
// scale tables are prepared in the internal 2^261 radix so that each fmul
// multiplies the stored integers by the intended field constant.
#include <string.h>

#include "zk_internal.hpp"

namespace zk {

constexpr int NTT_TILE = 1024;
constexpr int NTT_THREADS = 256;
constexpr int NTT_MAX_LOG = 24;

// SoA table of internal-form field elements: limb l of entry i at l*count+i.
struct FrTable {
  uint32_t* d = nullptr;
  size_t count = 0;
};

struct NttDir {
  FrTable twr[3];  // w_{R_p}^t, t < R_p/2
  FrTable twp[2];  // w_{R_p S_p}^(k*m) at k*S_p + m, for passes p < P-1
};

struct NttPlan {
  int log_n = 0, P = 0;
  int logR[3] = {0, 0, 0};
  NttDir dir[2];            // [0] forward, [1] inverse
  uint32_t ninv[NL];        // n^-1 in internal form
};

struct CosetTables {
  FrTable fwd;  // g^i
  FrTable inv;  // n^-1 g^-i
};

__device__ __forceinline__ fr load_table(const uint32_t* __restrict__ t, size_t count, size_t i) {
  fr x;
#pragma unroll
  for (int l = 0; l < NL; l++) x.l[l] = t[l * count + i];
  return x;
}

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

__device__ __forceinline__ void store_elem(uint4* __restrict__ p, size_t i, const fr& x) {
  uint32_t w[8];
  repack_out(x, w);
  p[2 * i] = make_uint4(w[0], w[1], w[2], w[3]);
  p[2 * i + 1] = make_uint4(w[4], w[5], w[6], w[7]);
}

__device__ __forceinline__ fr lds_get(const uint32_t* s, int idx) {
  fr x;
#pragma unroll
  for (int l = 0; l < NL; l++) x.l[l] = s[l * NTT_TILE + idx];
  return x;
}

__device__ __forceinline__ void lds_put(uint32_t* s, int idx, const fr& x) {
#pragma unroll
  for (int l = 0; l < NL; l++) s[l * NTT_TILE + idx] = x.l[l];
}

__device__ __forceinline__ uint32_t bitrev(uint32_t x, int bits) { return __brev(x) >> (32 - bits); }

// Twiddles w_R^t, t < R/2: staged in LDS (plane-major) when R/2 <= NTT_TWL
// so the stage loop reads no global memory; the single-pass transforms of
// 2^9 and 2^10 points read the table in place.
constexpr int NTT_TWL = 128;
struct TwView {
  const uint32_t* p;
  int stride;  // words between planes
};

__device__ __forceinline__ TwView stage_twiddles(uint32_t* tw, const uint32_t* __restrict__ twr, int half) {
  if (half > NTT_TWL) return TwView{twr, half};
  for (int e = threadIdx.x; e < half; e += NTT_THREADS) {
#pragma unroll
    for (int l = 0; l < NL; l++) tw[l * NTT_TWL + e] = twr[(size_t)l * half + e];
  }
  return TwView{tw, NTT_TWL};
}

__device__ __forceinline__ fr tw_get(const TwView& tw, int idx) {
  fr x;
#pragma unroll
  for (int l = 0; l < NL; l++) x.l[l] = tw.p[l * tw.stride + idx];
  return x;
}

// In-LDS DIT over the rows of a (R x T) tile stored row-major (index j*T + c);
// rows were stored bit-reversed, results come out natural.  Two radix-2
// stages per LDS round trip (a radix-2^2 step on four rows held in
// registers), a single radix-2 stage first when log2 R is odd.  tw: w_R^t,
// t < R/2, in LDS.
//
// Butterflies are lazy (Harvey's form): a stage's inputs lie in [0, 4m); the
// untwiddled operand X is brought below 2m by one conditional subtraction,
// the twiddled one T is an fmul output (< 2m), and the stage writes X + T and
// X - T + 2m, both in [0, 4m) with normalized limbs.  The first stage's
// inputs are below 2m (canonical loads or fmul outputs) and need no
// subtraction.  Results leave in [0, 4m).
__device__ __forceinline__ void tile_dit(uint32_t* s, const TwView& tw, int logR, int T) {
  const int R = 1 << logR;
  int st = 0;
  if (logR & 1) {  // stage 0: twiddle 1, pairs (2g, 2g + 1)
    for (int b = threadIdx.x; b < (R >> 1) * T; b += NTT_THREADS) {
      const int c = b % T, g = b / T;
      const int i0 = (2 * g) * T + c, i1 = i0 + T;
      const fr x0 = lds_get(s, i0), x1 = lds_get(s, i1);
      lds_put(s, i0, fadd_wide(x0, x1));
      lds_put(s, i1, fsub_lazy(x0, x1));
    }
    __syncthreads();
    st = 1;
  }
  for (; st < logR; st += 2) {
    const int h = 1 << st;
    const int tq = R >> (st + 2);  // twiddle stride of w_{4h} in the w_R table
    for (int b = threadIdx.x; b < (R >> 2) * T; b += NTT_THREADS) {
      const int c = b % T, q = b / T;
      const int k = q & (h - 1);
      const int j0 = ((q >> st) << (st + 2)) + k;
      const int i0 = j0 * T + c, i1 = i0 + h * T, i2 = i1 + h * T, i3 = i2 + h * T;
      fr x0 = lds_get(s, i0), x1 = lds_get(s, i1), x2 = lds_get(s, i2), x3 = lds_get(s, i3);
      fr t1 = x1, t3 = x3;  // h == 1: the first stage, inputs below 2m, twiddle 1
      if (h > 1) {
        const fr w2 = tw_get(tw, 2 * k * tq);  // w_{2h}^k (w^0 is the table's one)
        t1 = fmul(x1, w2);
        t3 = fmul(x3, w2);
        x0 = fcsub(x0, FrP::MOD2);
        x2 = fcsub(x2, FrP::MOD2);
      }
      const fr y0 = fadd_wide(x0, t1), y1 = fsub_lazy(x0, t1);
      const fr y2 = fadd_wide(x2, t3), y3 = fsub_lazy(x2, t3);
      const fr z2 = h > 1 ? fmul(y2, tw_get(tw, k * tq)) : fcsub(y2, FrP::MOD2);  // w_{4h}^k
      const fr z3 = fmul(y3, tw_get(tw, (k + h) * tq));                           // w_{4h}^(k+h)
      const fr u0 = fcsub(y0, FrP::MOD2), u1 = fcsub(y1, FrP::MOD2);
      lds_put(s, i0, fadd_wide(u0, z2));
      lds_put(s, i2, fsub_lazy(u0, z2));
      lds_put(s, i1, fadd_wide(u1, z3));
      lds_put(s, i3, fsub_lazy(u1, z3));
    }
    __syncthreads();
  }
}

struct PassArgs {
  int logR;          // this pass's radix
  int T;             // tile columns = NTT_TILE / R
  uint32_t S;        // stride of this digit
  uint64_t n;        // transform size
  // last pass only
  uint32_t R0, S0;   // first-digit count and stride
  uint32_t R1, S1;   // middle-digit count and stride (P == 3), else R1 = 1
};

// Pass p < P-1: in-place (position-preserving) sub-DFTs with the inter-pass
// twiddle applied on the way out.  pre: optional g^pos table for a forward
// coset transform (first pass only).
__global__ __launch_bounds__(NTT_THREADS) void k_ntt_pass_mid(uint4* __restrict__ dst, const uint4* __restrict__ src,
                                                               PassArgs a, const uint32_t* __restrict__ twr,
                                                               const uint32_t* __restrict__ twp,
                                                               const uint32_t* __restrict__ pre) {
  quotient_priority();
  __shared__ uint32_t s[NL * NTT_TILE];
  __shared__ uint32_t tws[NL * NTT_TWL];
  const int R = 1 << a.logR, T = a.T;
  const size_t boff = (size_t)blockIdx.y * a.n;
  src += 2 * boff;
  dst += 2 * boff;
  const TwView tw = stage_twiddles(tws, twr, R >> 1);
  const uint32_t tiles_per_u = a.S / T;
  const size_t u = blockIdx.x / tiles_per_u;
  const uint32_t m0 = (blockIdx.x % tiles_per_u) * T;
  const size_t ubase = u * (size_t)R * a.S;
  for (int e = threadIdx.x; e < NTT_TILE; e += NTT_THREADS) {
    const int c = e % T, j = e / T;
    const size_t pos = ubase + (size_t)j * a.S + m0 + c;
    fr x = load_elem(src, pos);
    if (pre) x = fmul(x, load_table(pre, a.n, pos));
    lds_put(s, bitrev(j, a.logR) * T + c, x);
  }
  __syncthreads();
  tile_dit(s, tw, a.logR, T);
  const size_t twp_count = (size_t)R * a.S;
  for (int e = threadIdx.x; e < NTT_TILE; e += NTT_THREADS) {
    const int c = e % T, k = e / T;
    const size_t rel = (size_t)k * a.S + m0 + c;
    fr x = lds_get(s, k * T + c);
    if (k != 0 && (m0 + c) != 0) x = fmul(x, load_table(twp, twp_count, rel));
    else x = fcsub(x, FrP::MOD2);
    store_elem(dst, ubase + rel, x);
  }
}

// Last pass: sub-DFT over the last (contiguous) digit for T consecutive
// values of the first digit, digit-reversed store to natural order.
// post: optional per-output-index table (coset iNTT) or, when post is null
// and scale_en is set, the constant `scale` (iNTT 1/n).
__global__ __launch_bounds__(NTT_THREADS) void k_ntt_pass_last(uint4* __restrict__ dst, const uint4* __restrict__ src,
                                                                PassArgs a, const uint32_t* __restrict__ twr,
                                                                const uint32_t* __restrict__ pre,
                                                                const uint32_t* __restrict__ post, fr scale,
                                                                int scale_en) {
  quotient_priority();
  __shared__ uint32_t s[NL * NTT_TILE];
  __shared__ uint32_t tws[NL * NTT_TWL];
  const int R = 1 << a.logR, T = a.T;
  const int E = R * T;
  const size_t boff = (size_t)blockIdx.y * a.n;
  src += 2 * boff;
  dst += 2 * boff;
  const TwView tw = stage_twiddles(tws, twr, R >> 1);
  const uint32_t tiles_per_v = a.R0 / T;
  const uint32_t v = blockIdx.x / tiles_per_v;     // middle digit k_1 (P == 3) or 0
  const uint32_t k0s = (blockIdx.x % tiles_per_v) * T;
  const size_t vpos = (size_t)v * a.S1;
  for (int e = threadIdx.x; e < E; e += NTT_THREADS) {
    const int c = e / R, j = e % R;
    const size_t pos = (size_t)(k0s + c) * a.S0 + vpos + j;
    fr x = load_elem(src, pos);
    if (pre) x = fmul(x, load_table(pre, a.n, pos));
    lds_put(s, bitrev(j, a.logR) * T + c, x);
  }
  __syncthreads();
  tile_dit(s, tw, a.logR, T);
  const size_t kstride = (size_t)a.R0 * a.R1;  // = n / R
  for (int e = threadIdx.x; e < E; e += NTT_THREADS) {
    const int c = e % T, k = e / T;
    const size_t out = (size_t)(k0s + c) + (size_t)a.R0 * v + kstride * k;
    fr x = lds_get(s, k * T + c);
    if (post) x = fmul(x, load_table(post, a.n, out));
    else if (scale_en) x = fmul(x, scale);
    else x = fcsub(x, FrP::MOD2);
    store_elem(dst, out, x);
  }
}

// table[e] = base^(e_hi * e_lo) with (e_hi, e_lo) = (e / cols, e % cols) and
// the exponent reduced mod 2^log_order; base given in internal form.
__global__ void k_fill_pow_table(uint32_t* __restrict__ t, size_t count, uint32_t cols, fr base, int log_order,
                                 fr mul) {
  size_t e = blockIdx.x * (size_t)blockDim.x + threadIdx.x;
  if (e >= count) return;
  uint64_t ex = (uint64_t)(e / cols) * (uint64_t)(e % cols);
  if (log_order < 64) ex &= ((uint64_t)1 << log_order) - 1;
  fr r = fe_one<FrP>(), b = base;
  while (ex) {
    if (ex & 1) r = fmul(r, b);
    b = fsqr(b);
    ex >>= 1;
  }
  r = fmul(r, mul);
  store_table(t, count, e, r);
}

// h = (a*b - c) * zinv on the reference's Montgomery words.  With raw words
// A = a 2^256, fmul(A,B) = ab 2^251, fmul(C, 2^256) = c 2^251 and
// fmul(., z 2^266) = (ab - c) z 2^256: three multiplies per element.
__global__ void k_quotient_pointwise(uint4* __restrict__ h, const uint4* __restrict__ A, const uint4* __restrict__ B,
                                     const uint4* __restrict__ C, size_t n, fr kc, fr zk) {
  quotient_priority();
  size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x;
  if (i >= n) return;
  fr t = fmul(load_elem(A, i), load_elem(B, i));
  fr u = fmul(load_elem(C, i), kc);
  store_elem(h, i, fmul(fsub(t, u), zk));
}

// ------------------------------------------------------------------ host side
// Host copies of field helpers (the device code is ZK_HD so usable here).
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

static int alloc_table(zk_context* ctx, FrTable& t, size_t count) {
  t.count = count;
  if (hipMalloc(&t.d, count * NL * sizeof(uint32_t)) != hipSuccess) {
    t.d = nullptr;
    return ctx->fail(ZK_ERR_OOM, "NTT table allocation failed");
  }
  return ZK_OK;
}

static void free_table(FrTable& t) {
  if (t.d) (void)hipFree(t.d);
  t.d = nullptr;
}

static int fill_pow(zk_context* ctx, FrTable& t, size_t count, uint32_t cols, const fr& base, int log_order,
                    const fr& mul, hipStream_t st) {
  ZK_TRY(alloc_table(ctx, t, count));
  ZK_LAUNCH(ctx, st, "ntt_twiddle_fill", k_fill_pow_table, dim3(cdiv(count, 256)), dim3(256), 0, t.d, count, cols,
            base, log_order, mul);
  return ZK_OK;
}

__global__ void k_fill_pow_linear(uint32_t* __restrict__ t, size_t count, fr base, fr mul) {
  size_t e = blockIdx.x * (size_t)blockDim.x + threadIdx.x;
  if (e >= count) return;
  uint64_t ex = e;
  fr r = fe_one<FrP>(), b = base;
  while (ex) {
    if (ex & 1) r = fmul(r, b);
    b = fsqr(b);
    ex >>= 1;
  }
  store_table(t, count, e, fmul(r, mul));
}

int fill_linear(zk_context* ctx, FrTable& t, const fr& base, const fr& mul, hipStream_t st) {
  ZK_LAUNCH(ctx, st, "ntt_twiddle_fill", k_fill_pow_linear, dim3(cdiv(t.count, 256)), dim3(256), 0, t.d, t.count,
            base, mul);
  return ZK_OK;
}

static int plan_get(zk_context* ctx, int log_n, NttPlan** out, hipStream_t st) {
  auto it = ctx->ntt_plans.find(log_n);
  if (it != ctx->ntt_plans.end()) {
    *out = it->second;
    return ZK_OK;
  }
  NttPlan* p = new NttPlan();
  p->log_n = log_n;
  if (log_n <= 10) {
    p->P = 1;
    p->logR[0] = log_n;
  } else if (log_n <= 16) {
    p->P = 2;
    p->logR[0] = (log_n + 1) / 2;
    p->logR[1] = log_n / 2;
  } else {
    p->P = 3;
    p->logR[0] = (log_n + 2) / 3;
    p->logR[1] = (log_n + 1) / 3;
    p->logR[2] = log_n / 3;
  }
  const fr one = fe_one<FrP>();
  for (int d = 0; d < 2; d++) {
    fr w = omega_int(log_n, d == 1);
    int below = log_n;  // log of R_p * S_p
    for (int q = 0; q < p->P; q++) {
      const int lr = p->logR[q];
      // w_{R_q} = w_n^(n / R_q)
      fr wr = w;
      for (int i = 0; i < log_n - lr; i++) wr = fsqr(wr);
      const size_t half = (size_t)1 << (lr > 0 ? lr - 1 : 0);
      ZK_TRY(alloc_table(ctx, p->dir[d].twr[q], half));
      ZK_TRY(fill_linear(ctx, p->dir[d].twr[q], wr, one, st));
      if (q < p->P - 1) {
        // w_{R_q S_q} = w_n^(n / (R_q S_q)), table over (k, m) in [R_q) x [S_q)
        fr wm = w;
        for (int i = 0; i < log_n - below; i++) wm = fsqr(wm);
        const size_t S = (size_t)1 << (below - lr);
        ZK_TRY(fill_pow(ctx, p->dir[d].twp[q], ((size_t)1 << lr) * S, (uint32_t)S, wm, below, one, st));
      }
      below -= lr;
    }
  }
  // n^-1 = ((r+1)/2)^log_n (reference ntt.cu:437-458)
  fr two_inv = fr_inv_host(fr_small(2));
  fr ninv = one;
  for (int i = 0; i < log_n; i++) ninv = fmul(ninv, two_inv);
  ninv = fcanon(ninv);
  memcpy(p->ninv, ninv.l, sizeof(p->ninv));
  ctx->ntt_plans[log_n] = p;
  *out = p;
  return ZK_OK;
}

void ntt_plans_free(zk_context* ctx) {
  for (auto& kv : ctx->ntt_plans) {
    NttPlan* p = kv.second;
    for (int d = 0; d < 2; d++) {
      for (auto& t : p->dir[d].twr) free_table(t);
      for (auto& t : p->dir[d].twp) free_table(t);
    }
    delete p;
  }
  ctx->ntt_plans.clear();
  for (auto& kv : ctx->coset_tables) {
    CosetTables* c = (CosetTables*)kv.second;
    free_table(c->fwd);
    free_table(c->inv);
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
  CosetTables* c = new CosetTables();
  const size_t n = (size_t)1 << log_n;
  fr gi = fr_small(g);
  fr ginv = fr_inv_host(gi);
  fr ninv;
  memcpy(ninv.l, plan->ninv, sizeof(ninv.l));
  ctx->coset_tables[key] = c;
  ZK_TRY(alloc_table(ctx, c->fwd, n));
  ZK_TRY(alloc_table(ctx, c->inv, n));
  ZK_TRY(fill_linear(ctx, c->fwd, gi, fe_one<FrP>(), st));   // g^i
  ZK_TRY(fill_linear(ctx, c->inv, ginv, ninv, st));          // n^-1 g^-i
  *out = c;
  return ZK_OK;
}

int ntt_run(zk_context* ctx, void* d_out, const void* d_in, int log_n, int inverse, int batch, uint64_t coset_g,
            hipStream_t st) {
  if (!d_out || !d_in || batch < 1) return ctx->fail(ZK_ERR_INVALID, "ntt: null buffer or batch < 1");
  if (log_n < 1 || log_n > NTT_MAX_LOG) return ctx->fail(ZK_ERR_SIZE, "ntt: log_n outside [1, 24]");
  NttPlan* plan = nullptr;
  ZK_TRY(plan_get(ctx, log_n, &plan, st));
  CosetTables* cos = nullptr;
  if (coset_g) ZK_TRY(coset_get(ctx, log_n, coset_g, plan, &cos, st));
  const int d = inverse ? 1 : 0;
  const size_t n = (size_t)1 << log_n;
  const uint32_t* pre = (cos && !inverse) ? cos->fwd.d : nullptr;
  const uint32_t* post = (cos && inverse) ? cos->inv.d : nullptr;
  fr scale;
  memcpy(scale.l, plan->ninv, sizeof(scale.l));
  const int scale_en = inverse ? 1 : 0;
  const int P = plan->P;

  const uint4* src = (const uint4*)d_in;
  uint4* out = (uint4*)d_out;
  if (P > 1) ZK_TRY(ctx->ensure(ctx->scratch_a, n * 32 * (size_t)batch));
  uint4* scr = (uint4*)ctx->scratch_a.p;

  size_t strides[3];
  {
    size_t s = n;
    for (int q = 0; q < P; q++) {
      s >>= plan->logR[q];
      strides[q] = s;
    }
  }
  for (int q = 0; q < P - 1; q++) {
    PassArgs a{};
    a.logR = plan->logR[q];
    a.T = NTT_TILE >> a.logR;
    a.S = (uint32_t)strides[q];
    a.n = n;
    dim3 grid(cdiv(n, NTT_TILE), batch);
    ZK_LAUNCH(ctx, st, "ntt_pass", k_ntt_pass_mid, grid, dim3(NTT_THREADS), 0, scr, q == 0 ? src : scr, a,
              plan->dir[d].twr[q].d, plan->dir[d].twp[q].d, q == 0 ? pre : nullptr);
  }
  PassArgs a{};
  a.logR = plan->logR[P - 1];
  a.n = n;
  if (P == 1) {
    a.T = 1;
    a.R0 = 1;
    a.S0 = 0;
    a.R1 = 1;
    a.S1 = 0;
  } else {
    a.T = NTT_TILE >> a.logR;
    a.R0 = 1u << plan->logR[0];
    a.S0 = (uint32_t)strides[0];
    a.R1 = P == 3 ? (1u << plan->logR[1]) : 1;
    a.S1 = P == 3 ? (uint32_t)strides[1] : 0;
  }
  const uint32_t tiles = P == 1 ? 1 : (uint32_t)(n / ((size_t)a.T << a.logR));
  dim3 grid(tiles, batch);
  ZK_LAUNCH(ctx, st, "ntt_pass", k_ntt_pass_last, grid, dim3(NTT_THREADS), 0, out, P == 1 ? src : scr, a,
            plan->dir[d].twr[P - 1].d, P == 1 ? pre : nullptr, post, scale, post ? 0 : scale_en);
  return ZK_OK;
}

int quotient_pointwise(zk_context* ctx, void* d_h, const void* d_a, const void* d_b, const void* d_c, size_t n,
                       const uint64_t zinv_mont[4], hipStream_t st) {
  // kc = 2^256 mod r as a raw integer.  With z_mont = z 2^256 (raw words),
  // zk = z 2^266 = fmul(z_mont, 2^271 raw).
  static const uint32_t K256[8] = {0x4ffffffbu, 0xac96341cu, 0x9f60cd29u, 0x36fc7695u,
                                   0x7879462eu, 0x666ea36fu, 0x9a07df2fu, 0x0e0a77c1u};  // 2^256 mod r
  static const uint32_t K271[8] = {0x2ffd5addu, 0x29ab3316u, 0xf4f5739fu, 0x3b9f942fu,
                                   0x3ca28ff2u, 0x84aad391u, 0xf9a8c5dfu, 0x1ed378c2u};  // 2^271 mod r
  fr kc = repack_in<FrP>(K256);
  uint32_t zw[8];
  memcpy(zw, zinv_mont, 32);
  fr zk = fmul(repack_in<FrP>(zw), repack_in<FrP>(K271));
  ZK_LAUNCH(ctx, st, "quotient_pointwise", k_quotient_pointwise, dim3(cdiv(n, 256)), dim3(256), 0, (uint4*)d_h,
            (const uint4*)d_a, (const uint4*)d_b, (const uint4*)d_c, n, kc, zk);
  return ZK_OK;
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

}  // extern "C"
