// TEST INFRASTRUCTURE ONLY -- CPU oracle for the Groth16 hot path.
// See zk_oracle.hpp for the scope.  Every function names the reference
// file:line whose algorithm it restates.
#include "zk_oracle.hpp"

#include <omp.h>
#include <stdio.h>
#include <stdlib.h>

#include <algorithm>
#include <chrono>

namespace orc {

constexpr uint64_t QParams::M[4];
constexpr uint64_t QParams::ONE[4];
constexpr uint64_t QParams::R2[4];
constexpr uint64_t RParams::M[4];
constexpr uint64_t RParams::ONE[4];
constexpr uint64_t RParams::R2[4];

static double now_ms() {
  return std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now().time_since_epoch()).count();
}

G1A g1_generator() {
  G1A g;
  g.x = Fq::from_uint(1);
  g.y = Fq::from_uint(2);
  g.inf = false;
  return g;
}

// EIP-197 generator, given by its standard-form coordinates; the reference
// stores the same values as raw Montgomery limbs (src/curve/g2.cuh:47-65).
G2A g2_generator() {
  static const uint64_t X0[4] = {0x46debd5cd992f6edULL, 0x674322d4f75edaddULL, 0x426a00665e5c4479ULL,
                                 0x1800deef121f1e76ULL};
  static const uint64_t X1[4] = {0x97e485b7aef312c2ULL, 0xf1aa493335a9e712ULL, 0x7260bfb731fb5d25ULL,
                                 0x198e9393920d483aULL};
  static const uint64_t Y0[4] = {0x4ce6cc0166fa7daaULL, 0xe3d1e7690c43d37bULL, 0x4aab71808dcb408fULL,
                                 0x12c85ea5db8c6debULL};
  static const uint64_t Y1[4] = {0x55acdadcd122975bULL, 0xbc4b313370b38ef3ULL, 0xec9e99ad690c3395ULL,
                                 0x090689d0585ff075ULL};
  G2A g;
  g.x = Fq2{Fq::from_std(X0), Fq::from_std(X1)};
  g.y = Fq2{Fq::from_std(Y0), Fq::from_std(Y1)};
  g.inf = false;
  return g;
}

template <class E>
void batch_to_affine(const std::vector<Jac<E>>& in, std::vector<Aff<E>>& out) {
  size_t n = in.size();
  out.resize(n);
  std::vector<E> pre(n);
  E acc = E::one();
  for (size_t i = 0; i < n; i++) {
    pre[i] = acc;
    if (!in[i].is_inf()) acc = acc * in[i].z;
  }
  E inv = acc.inv();
  for (size_t i = n; i-- > 0;) {
    if (in[i].is_inf()) {
      out[i].x = E::zero();
      out[i].y = E::zero();
      out[i].inf = true;
      continue;
    }
    E zi = inv * pre[i];
    inv = inv * in[i].z;
    E zi2 = zi.sqr();
    out[i].x = in[i].x * zi2;
    out[i].y = in[i].y * zi2 * zi;
    out[i].inf = false;
  }
}
template void batch_to_affine<Fq>(const std::vector<G1J>&, std::vector<G1A>&);
template void batch_to_affine<Fq2>(const std::vector<G2J>&, std::vector<G2A>&);

// ---------------------------------------------------------------- NTT
// omega_{2^28} in Montgomery form and its inverse (src/ntt/ntt.cu:53-62).
static const uint64_t OMEGA28[4] = {0x636E735580D13D9CULL, 0xA22BF3742445FFD6ULL, 0x56452AC01EB203D8ULL,
                                    0x1860EF942963F9E7ULL};
static const uint64_t OMEGA28_INV[4] = {0x89BCC016584BB683ULL, 0xE8D9887F0164A50CULL, 0x755E95CB795EDA3DULL,
                                        0x0F572B871323B130ULL};

Fr omega(int log_n) {  // ntt.cu:64-87
  Fr w = Fr::raw(OMEGA28);
  for (int i = 0; i < 28 - log_n; i++) w = w * w;
  return w;
}
Fr omega_inv(int log_n) {  // ntt.cu:89-111
  Fr w = Fr::raw(OMEGA28_INV);
  for (int i = 0; i < 28 - log_n; i++) w = w * w;
  return w;
}

// Radix-2 DIT after a bit-reversal permutation, stage twiddles
// w^(pos << (log_n-1-s)), iNTT scaled by ((r+1)/2)^log_n (ntt.cu:354-465).
void ntt_radix2(std::vector<Fr>& a, int log_n, bool inverse, int threads) {
  const size_t n = (size_t)1 << log_n;
  std::vector<Fr> b(n);
  for (size_t i = 0; i < n; i++) {
    size_t rev = 0, v = i;
    for (int k = 0; k < log_n; k++) {
      rev = (rev << 1) | (v & 1);
      v >>= 1;
    }
    b[rev] = a[i];
  }
  const Fr w = inverse ? omega_inv(log_n) : omega(log_n);
  std::vector<Fr> tw(n / 2 + 1);
  for (int s = 0; s < log_n; s++) {
    const size_t stride = (size_t)1 << s;
    Fr step = w;
    for (int i = 0; i < log_n - 1 - s; i++) step = step * step;
    Fr cur = Fr::one();
    for (size_t pos = 0; pos < stride; pos++) {
      tw[pos] = cur;
      cur = cur * step;
    }
#pragma omp parallel for num_threads(threads) schedule(static)
    for (long long idx = 0; idx < (long long)(n / 2); idx++) {
      size_t group = (size_t)idx / stride, pos = (size_t)idx % stride;
      size_t i0 = group * 2 * stride + pos, i1 = i0 + stride;
      Fr t = tw[pos] * b[i1];
      Fr x = b[i0];
      b[i0] = x + t;
      b[i1] = x - t;
    }
  }
  if (inverse) {
    static const uint64_t HALF[4] = {0xA1F0FAC9F8000001ULL, 0x9419F4243CDCB848ULL, 0xDC2822DB40C0AC2EULL,
                                     0x183227397098D014ULL};  // (r+1)/2, ntt.cu:441-448
    Fr half = Fr::from_std(HALF);
    Fr scale = Fr::one();
    for (int i = 0; i < log_n; i++) scale = scale * half;
#pragma omp parallel for num_threads(threads) schedule(static)
    for (long long i = 0; i < (long long)n; i++) b[i] = b[i] * scale;
  }
  a.swap(b);
}

// out[i] = sum_j in[j] * w^(i*j)   (tests/test_ntt.cu:19-37)
void dft_naive(const std::vector<Fr>& in, std::vector<Fr>& out, const Fr& w) {
  size_t n = in.size();
  out.assign(n, Fr::zero());
  Fr wi = Fr::one();
  for (size_t i = 0; i < n; i++) {
    Fr s = Fr::zero(), wij = Fr::one();
    for (size_t j = 0; j < n; j++) {
      s = s + in[j] * wij;
      wij = wij * wi;
    }
    out[i] = s;
    wi = wi * w;
  }
}

// ---------------------------------------------------------------- MSM
MsmConfig MsmConfig::for_size(int n, bool g2) {  // msm.cuh:46-63, msm.cu:529-533
  MsmConfig c;
  if (n <= (1 << 10)) c.c = 10;
  else if (n <= (1 << 14)) c.c = 12;
  else if (n <= (1 << 18)) c.c = 14;
  else if (n <= (1 << 22)) c.c = 15;
  else c.c = 16;
  if (g2 && c.c > 12) c.c = 12;
  c.windows = (253 + c.c) / c.c;
  c.buckets = (1 << c.c) - 1;
  return c;
}

// Unsigned c-bit window digit of a standard-form scalar (msm.cu:128-143).
static inline uint64_t window_bits(const uint64_t* s, int w, int c) {
  const uint64_t mask = ((uint64_t)1 << c) - 1;
  int off = w * c, limb = off / 64, sh = off % 64;
  if (limb >= 4) return 0;
  if (sh + c <= 64) return (s[limb] >> sh) & mask;
  if (limb + 1 < 4) return ((s[limb] >> sh) | (s[limb + 1] << (64 - sh))) & mask;
  return (s[limb] >> sh) & mask;
}

template <class E, class J = Jac<E>>
static J msm_pippenger(const Aff<E>* pts, const Fr* sc, int n, bool g2, int threads) {
  if (n == 0) return J::identity();
  // CPU fallback for small n (msm.cu:330-339, 537-544)
  if (n <= (g2 ? 128 : 256)) {
    J r = J::identity();
    for (int i = 0; i < n; i++) r = r.add(J::from_affine(pts[i]).mul(sc[i]));
    return r;
  }
  MsmConfig cfg = MsmConfig::for_size(n, g2);
  std::vector<uint64_t> s((size_t)n * 4);
  for (int i = 0; i < n; i++) sc[i].to_std(&s[(size_t)i * 4]);
  std::vector<J> wres(cfg.windows);
  // Bucket accumulation (msm.cu:104-154) and serial weighted reduction
  // (msm.cu:284-307), one window per OpenMP thread.
#pragma omp parallel for num_threads(threads) schedule(dynamic, 1)
  for (int w = 0; w < cfg.windows; w++) {
    std::vector<J> buckets(cfg.buckets, J::identity());
    for (int i = 0; i < n; i++) {
      if (pts[i].inf) continue;
      uint64_t b = window_bits(&s[(size_t)i * 4], w, cfg.c);
      if (b == 0) continue;
      buckets[b - 1] = buckets[b - 1].add_affine(pts[i]);
    }
    J run = J::identity(), sum = J::identity();
    for (int b = cfg.buckets - 1; b >= 0; b--) {
      if (!buckets[b].is_inf()) run = run.add(buckets[b]);
      sum = sum.add(run);
    }
    wres[w] = sum;
  }
  // Host window combination (msm.cu:423-430)
  J r = J::identity();
  for (int w = cfg.windows - 1; w >= 0; w--) {
    for (int i = 0; i < cfg.c; i++) r = r.dbl();
    r = r.add(wres[w]);
  }
  return r;
}

G1J msm_g1(const G1A* pts, const Fr* sc, int n, int threads) { return msm_pippenger<Fq>(pts, sc, n, false, threads); }
G2J msm_g2(const G2A* pts, const Fr* sc, int n, int threads) { return msm_pippenger<Fq2>(pts, sc, n, true, threads); }
G2Ref msm_g2_affine_ref(const G2A* pts, const Fr* sc, int n, int threads) {
  return msm_pippenger<Fq2, G2Ref>(pts, sc, n, true, threads);
}

G1J msm_g1_naive(const G1A* pts, const Fr* sc, int n) {
  G1J r = G1J::identity();
  for (int i = 0; i < n; i++) r = r.add(G1J::from_affine(pts[i]).mul(sc[i]));
  return r;
}
G2J msm_g2_naive(const G2A* pts, const Fr* sc, int n) {
  G2J r = G2J::identity();
  for (int i = 0; i < n; i++) r = r.add(G2J::from_affine(pts[i]).mul(sc[i]));
  return r;
}

// ---------------------------------------------------------------- fixed base
// Scalar multiples of a fixed point through 8-bit window tables; the group
// element is the same as double-and-add, so the affine output is identical.
template <class E>
struct FixedBase {
  std::vector<Aff<E>> tab;  // 32 x 256
  explicit FixedBase(const Aff<E>& g) {
    std::vector<Jac<E>> j(32 * 256);
    Jac<E> base = Jac<E>::from_affine(g);
    for (int k = 0; k < 32; k++) {
      j[k * 256] = Jac<E>::identity();
      for (int d = 1; d < 256; d++) j[k * 256 + d] = j[k * 256 + d - 1].add(base);
      for (int i = 0; i < 8; i++) base = base.dbl();
    }
    batch_to_affine(j, tab);
  }
  Jac<E> mul_std(const uint64_t* s) const {
    Jac<E> acc = Jac<E>::identity();
    for (int k = 0; k < 32; k++) {
      unsigned d = (unsigned)((s[k >> 3] >> (8 * (k & 7))) & 0xff);
      if (d) acc = acc.add_affine(tab[k * 256 + d]);
    }
    return acc;
  }
  void batch(const Fr* k, size_t n, Aff<E>* out, int threads) const {
    const size_t chunk = 4096;
#pragma omp parallel for num_threads(threads) schedule(dynamic, 1)
    for (long long c0 = 0; c0 < (long long)n; c0 += chunk) {
      size_t c1 = std::min(n, (size_t)c0 + chunk);
      std::vector<Jac<E>> j(c1 - c0);
      for (size_t i = c0; i < c1; i++) {
        uint64_t s[4];
        k[i].to_std(s);
        j[i - c0] = mul_std(s);
      }
      std::vector<Aff<E>> a;
      batch_to_affine(j, a);
      for (size_t i = c0; i < c1; i++) out[i] = a[i - c0];
    }
  }
};

// ---------------------------------------------------------------- R1CS
bool R1CS::verify_witness(const std::vector<Fr>& w) const {  // circuit.cuh:93-124
  if ((int)w.size() != num_variables) return false;
  std::vector<Fr> a(num_constraints, Fr::zero()), b(num_constraints, Fr::zero()), c(num_constraints, Fr::zero());
  for (auto& e : A) a[e.row] = a[e.row] + e.value * w[e.col];
  for (auto& e : B) b[e.row] = b[e.row] + e.value * w[e.col];
  for (auto& e : C) c[e.row] = c[e.row] + e.value * w[e.col];
  for (int i = 0; i < num_constraints; i++)
    if (!(a[i] * b[i] == c[i])) return false;
  return true;
}

int qap_log_n(int nc) {  // groth16.cu:225-242
  int log_n = 0, n = 1;
  while (n < nc) {
    n <<= 1;
    log_n++;
  }
  if (n < 4) log_n = 2;
  return log_n;
}

static Fr inv_fr(const Fr& x) { return x.inv(); }

// groth16.cu:263-390
std::vector<Fr> compute_h(const R1CS& c, const std::vector<Fr>& w, int threads) {
  const int log_n = qap_log_n(c.num_constraints);
  const int n = 1 << log_n;
  const int m = c.num_variables;
  const int use = std::min(m, (int)w.size());
  std::vector<Fr> A(n, Fr::zero()), B(n, Fr::zero()), C(n, Fr::zero());
  for (auto& e : c.A)
    if (e.row < n && e.col < use) A[e.row] = A[e.row] + w[e.col] * e.value;
  for (auto& e : c.B)
    if (e.row < n && e.col < use) B[e.row] = B[e.row] + w[e.col] * e.value;
  for (auto& e : c.C)
    if (e.row < n && e.col < use) C[e.row] = C[e.row] + w[e.col] * e.value;
  ntt_radix2(A, log_n, true, threads);
  ntt_radix2(B, log_n, true, threads);
  ntt_radix2(C, log_n, true, threads);
  // coset shift 5 unless 5^n == 1, then 7 (groth16.cu:329-342)
  Fr g = Fr::from_uint(5), z = g;
  for (int i = 0; i < log_n; i++) z = z * z;
  z = z - Fr::one();
  if (z.is_zero()) {
    g = Fr::from_uint(7);
    z = g;
    for (int i = 0; i < log_n; i++) z = z * z;
    z = z - Fr::one();
  }
  Fr gp = Fr::one();
  for (int i = 0; i < n; i++) {
    A[i] = A[i] * gp;
    B[i] = B[i] * gp;
    C[i] = C[i] * gp;
    gp = gp * g;
  }
  ntt_radix2(A, log_n, false, threads);
  ntt_radix2(B, log_n, false, threads);
  ntt_radix2(C, log_n, false, threads);
  Fr zi = inv_fr(z);
  std::vector<Fr> H(n);
  for (int j = 0; j < n; j++) H[j] = (A[j] * B[j] - C[j]) * zi;
  ntt_radix2(H, log_n, true, threads);
  Fr gi = inv_fr(g), gip = Fr::one();
  for (int i = 0; i < n; i++) {
    H[i] = H[i] * gip;
    gip = gip * gi;
  }
  return H;
}

// Lagrange basis at tau and the QAP column evaluations (groth16.cu:97-189).
static void qap_at_tau(const R1CS& c, int log_n, const Fr& tau, std::vector<Fr>& At, std::vector<Fr>& Bt,
                       std::vector<Fr>& Ct, Fr& vanish) {
  const int n = 1 << log_n, m = c.num_variables;
  At.assign(m, Fr::zero());
  Bt.assign(m, Fr::zero());
  Ct.assign(m, Fr::zero());
  Fr w = omega(log_n);
  Fr tn = tau;
  for (int i = 0; i < log_n; i++) tn = tn * tn;
  vanish = tn - Fr::one();
  static const uint64_t HALF[4] = {0xA1F0FAC9F8000001ULL, 0x9419F4243CDCB848ULL, 0xDC2822DB40C0AC2EULL,
                                   0x183227397098D014ULL};
  Fr half = Fr::from_std(HALF), ninv = Fr::one();
  for (int i = 0; i < log_n; i++) ninv = ninv * half;
  std::vector<Fr> L(n), den(n);
  Fr wj = Fr::one();
  for (int j = 0; j < n; j++) {
    L[j] = vanish * wj * ninv;
    den[j] = tau - wj;
    wj = wj * w;
  }
  std::vector<Fr> pre(n);
  pre[0] = den[0];
  for (int i = 1; i < n; i++) pre[i] = pre[i - 1] * den[i];
  Fr ti = inv_fr(pre[n - 1]);
  std::vector<Fr> di(n);
  for (int i = n - 1; i > 0; i--) {
    di[i] = pre[i - 1] * ti;
    ti = ti * den[i];
  }
  di[0] = ti;
  for (int j = 0; j < n; j++) L[j] = L[j] * di[j];
  for (auto& e : c.A)
    if (e.row < n && e.col < m) At[e.col] = At[e.col] + e.value * L[e.row];
  for (auto& e : c.B)
    if (e.row < n && e.col < m) Bt[e.col] = Bt[e.col] + e.value * L[e.row];
  for (auto& e : c.C)
    if (e.row < n && e.col < m) Ct[e.col] = Ct[e.col] + e.value * L[e.row];
}

static Fr random_nonzero(std::mt19937_64& rng) {  // groth16.cu:48-58
  Fr v = Fr::from_uint(rng());
  while (v.is_zero()) v = Fr::from_uint(rng());
  return v;
}

// groth16.cu:446-642 (deterministic seed path)
void setup(const R1CS& c, uint64_t seed, ProvingKey& pk, VerifyingKey& vk, int threads) {
  const int log_n = qap_log_n(c.num_constraints), n = 1 << log_n, m = c.num_variables;
  std::mt19937_64 rng(seed);
  Fr tau = random_nonzero(rng), alpha = random_nonzero(rng), beta = random_nonzero(rng);
  Fr gamma = random_nonzero(rng), delta = random_nonzero(rng);
  G1A g1 = g1_generator();
  G2A g2 = g2_generator();
  FixedBase<Fq> fb1(g1);
  FixedBase<Fq2> fb2(g2);
  auto m1 = [&](const Fr& k) {
    uint64_t s[4];
    k.to_std(s);
    return fb1.mul_std(s).to_affine();
  };
  auto m2 = [&](const Fr& k) {
    uint64_t s[4];
    k.to_std(s);
    return fb2.mul_std(s).to_affine();
  };
  pk.alpha_g1 = m1(alpha);
  pk.beta_g1 = m1(beta);
  pk.beta_g2 = m2(beta);
  pk.gamma_g2 = m2(gamma);
  pk.delta_g1 = m1(delta);
  pk.delta_g2 = m2(delta);
  vk.alpha_g1 = pk.alpha_g1;
  vk.beta_g2 = pk.beta_g2;
  vk.gamma_g2 = pk.gamma_g2;
  vk.delta_g2 = pk.delta_g2;
  pk.tau_g1.clear();
  pk.tau_g2 = {g2, m2(tau)};
  std::vector<Fr> At, Bt, Ct;
  Fr vanish;
  qap_at_tau(c, log_n, tau, At, Bt, Ct, vanish);
  pk.A_query.resize(m);
  pk.B_g1_query.resize(m);
  pk.B_g2_query.resize(m);
  fb1.batch(At.data(), m, pk.A_query.data(), threads);
  fb1.batch(Bt.data(), m, pk.B_g1_query.data(), threads);
  fb2.batch(Bt.data(), m, pk.B_g2_query.data(), threads);
  const int npub = c.num_public;
  int l = m - npub - 1;
  if (l < 0) l = 0;
  Fr dinv = inv_fr(delta), ginv = inv_fr(gamma);
  std::vector<Fr> ls(l);
  for (int i = 0; i < l; i++) {
    int v = i + 1 + npub;
    ls[i] = (beta * At[v] + alpha * Bt[v] + Ct[v]) * dinv;
  }
  pk.L_query.resize(l);
  fb1.batch(ls.data(), l, pk.L_query.data(), threads);
  std::vector<Fr> hs(n);
  Fr tp = vanish * dinv;
  for (int i = 0; i < n; i++) {
    hs[i] = tp;
    tp = tp * tau;
  }
  pk.H_query.resize(n);
  fb1.batch(hs.data(), n, pk.H_query.data(), threads);
  vk.ic.resize(npub + 1);
  for (int i = 0; i <= npub; i++) {
    Fr s = Fr::zero();
    if (i < m) s = (beta * At[i] + alpha * Bt[i] + Ct[i]) * ginv;
    vk.ic[i] = m1(s);
  }
  vk.num_public = npub;
  pk.num_constraints = n;
  pk.num_variables = m;
  pk.num_public = npub;
}

// groth16.cu:655-920 (group-element path, deterministic seed)
Proof prove(const ProvingKey& pk, const R1CS& c, const std::vector<Fr>& w, uint64_t seed, int threads,
            double* ms, bool g2_affine_ref) {
  Proof pf;
  const int m = (int)w.size();
  if (m == 0 || m != c.num_variables) return pf;
  if (c.num_public != pk.num_public) return pf;
  if (1 + pk.num_public > m) return pf;
  if (!c.verify_witness(w)) return pf;
  double t0 = now_ms();
  std::vector<Fr> h = compute_h(c, w, threads);
  double t1 = now_ms();
  std::mt19937_64 rng(seed);
  Fr r = random_nonzero(rng), s = random_nonzero(rng);
  int na = std::min(m, (int)pk.A_query.size());
  G1J A = G1J::from_affine(pk.alpha_g1).add(na > 0 ? msm_g1(pk.A_query.data(), w.data(), na, threads)
                                                   : G1J::identity());
  A = A.add(G1J::from_affine(pk.delta_g1).mul(r));
  pf.A = A.to_affine();
  double t2 = now_ms();
  int nb = std::min(m, (int)pk.B_g2_query.size());
  if (g2_affine_ref) {  // groth16.cu:790-798 on the reference's G2 arithmetic
    G2Ref B = G2Ref::from_affine(pk.beta_g2)
                  .add(nb > 0 ? msm_g2_affine_ref(pk.B_g2_query.data(), w.data(), nb, threads) : G2Ref::identity());
    B = B.add(G2Ref::from_affine(pk.delta_g2).mul(s));
    pf.B = B.to_affine();
  } else {
    G2J B = G2J::from_affine(pk.beta_g2).add(nb > 0 ? msm_g2(pk.B_g2_query.data(), w.data(), nb, threads)
                                                    : G2J::identity());
    B = B.add(G2J::from_affine(pk.delta_g2).mul(s));
    pf.B = B.to_affine();
  }
  double t3 = now_ms();
  G1J C = G1J::identity();
  int npriv = std::min((int)pk.L_query.size(), m - 1 - pk.num_public);
  if (npriv > 0) C = C.add(msm_g1(pk.L_query.data(), w.data() + 1 + pk.num_public, npriv, threads));
  int nh = std::min((int)h.size(), (int)pk.H_query.size());
  if (nh > 0) C = C.add(msm_g1(pk.H_query.data(), h.data(), nh, threads));
  C = C.add(G1J::from_affine(pf.A).mul(s));
  int nb1 = std::min(m, (int)pk.B_g1_query.size());
  if (nb1 > 0) {
    G1J B1 = G1J::from_affine(pk.beta_g1).add(msm_g1(pk.B_g1_query.data(), w.data(), nb1, threads));
    C = C.add(B1.mul(r));
  }
  pf.C = C.to_affine();
  double t4 = now_ms();
  if (ms) {
    ms[0] = t1 - t0;  // compute_h
    ms[1] = t2 - t1;  // A
    ms[2] = t3 - t2;  // B (G2)
    ms[3] = t4 - t3;  // C
  }
  pf.valid = true;
  return pf;
}

// ---------------------------------------------------------------- file formats
static void put_fq(std::vector<uint8_t>& b, const Fq& x) {
  uint64_t s[4];
  x.to_std(s);
  const uint8_t* p = (const uint8_t*)s;
  b.insert(b.end(), p, p + 32);
}

void Proof::serialize(uint8_t out[256]) const {  // groth16.cu:1058-1074
  std::vector<uint8_t> b;
  put_fq(b, A.x);
  put_fq(b, A.y);
  put_fq(b, B.x.c0);
  put_fq(b, B.x.c1);
  put_fq(b, B.y.c0);
  put_fq(b, B.y.c1);
  put_fq(b, C.x);
  put_fq(b, C.y);
  memcpy(out, b.data(), 256);
}

bool ProvingKey::save(const char* path) const {  // groth16.cu:1104-1188
  std::vector<uint8_t> b;
  auto u32 = [&](uint32_t v) { b.insert(b.end(), (uint8_t*)&v, (uint8_t*)&v + 4); };
  auto g1 = [&](const G1A& p) {
    b.push_back(p.inf ? 1 : 0);
    put_fq(b, p.x);
    put_fq(b, p.y);
  };
  auto g2 = [&](const G2A& p) {
    b.push_back(p.inf ? 1 : 0);
    put_fq(b, p.x.c0);
    put_fq(b, p.x.c1);
    put_fq(b, p.y.c0);
    put_fq(b, p.y.c1);
  };
  const char magic[8] = {'Z', 'K', 'M', 'L', 'P', 'K', '3', 0};
  b.insert(b.end(), magic, magic + 8);
  u32(3);
  u32((uint32_t)num_constraints);
  u32((uint32_t)num_variables);
  u32((uint32_t)num_public);
  g1(alpha_g1);
  g1(beta_g1);
  g1(delta_g1);
  g2(beta_g2);
  g2(gamma_g2);
  g2(delta_g2);
  auto v1 = [&](const std::vector<G1A>& v) {
    u32((uint32_t)v.size());
    for (auto& p : v) g1(p);
  };
  auto v2 = [&](const std::vector<G2A>& v) {
    u32((uint32_t)v.size());
    for (auto& p : v) g2(p);
  };
  v1(tau_g1);
  v2(tau_g2);
  v1(A_query);
  v1(B_g1_query);
  v2(B_g2_query);
  v1(L_query);
  v1(H_query);
  FILE* f = fopen(path, "wb");
  if (!f) return false;
  bool ok = fwrite(b.data(), 1, b.size(), f) == b.size();
  fclose(f);
  return ok;
}

struct Reader {
  std::vector<uint8_t> d;
  size_t off = 0;
  bool ok = true;
  bool open(const char* path) {
    FILE* f = fopen(path, "rb");
    if (!f) return false;
    fseek(f, 0, SEEK_END);
    long sz = ftell(f);
    fseek(f, 0, SEEK_SET);
    d.resize(sz);
    ok = fread(d.data(), 1, sz, f) == (size_t)sz;
    fclose(f);
    return ok;
  }
  void raw(void* p, size_t n) {
    if (!ok || off + n > d.size()) {
      ok = false;
      return;
    }
    memcpy(p, d.data() + off, n);
    off += n;
  }
  int32_t i32() {
    int32_t v = 0;
    raw(&v, 4);
    return v;
  }
  Fq fq() {
    uint64_t s[4] = {0, 0, 0, 0};
    raw(s, 32);
    return Fq::from_std(s);
  }
  G1A g1(bool flag) {
    uint8_t inf = 0;
    if (flag) raw(&inf, 1);
    G1A p;
    p.x = fq();
    p.y = fq();
    p.inf = false;
    if (inf) {
      p.x = Fq::zero();
      p.y = Fq::zero();
      p.inf = true;
    }
    return p;
  }
  G2A g2(bool flag) {
    uint8_t inf = 0;
    if (flag) raw(&inf, 1);
    G2A p;
    p.x.c0 = fq();
    p.x.c1 = fq();
    p.y.c0 = fq();
    p.y.c1 = fq();
    p.inf = false;
    if (inf) {
      p.x = Fq2::zero();
      p.y = Fq2::zero();
      p.inf = true;
    }
    return p;
  }
};

bool ProvingKey::load(const char* path) {  // groth16.cu:1190-1314
  Reader r;
  if (!r.open(path)) return false;
  char magic[8];
  r.raw(magic, 8);
  if (!r.ok || memcmp(magic, "ZKMLPK3", 7) != 0) return false;
  uint32_t ver = 0;
  r.raw(&ver, 4);
  if (!r.ok || ver != 3) return false;
  num_constraints = r.i32();
  num_variables = r.i32();
  num_public = r.i32();
  if (!r.ok || num_constraints < 0 || num_variables <= 0 || num_public < 0) return false;
  alpha_g1 = r.g1(true);
  beta_g1 = r.g1(true);
  delta_g1 = r.g1(true);
  beta_g2 = r.g2(true);
  gamma_g2 = r.g2(true);
  delta_g2 = r.g2(true);
  auto v1 = [&](std::vector<G1A>& v) {
    int32_t n = r.i32();
    if (!r.ok || n < 0 || n > (1 << 28)) {
      r.ok = false;
      return;
    }
    v.resize(n);
    for (int i = 0; i < n; i++) v[i] = r.g1(true);
  };
  auto v2 = [&](std::vector<G2A>& v) {
    int32_t n = r.i32();
    if (!r.ok || n < 0 || n > (1 << 28)) {
      r.ok = false;
      return;
    }
    v.resize(n);
    for (int i = 0; i < n; i++) v[i] = r.g2(true);
  };
  v1(tau_g1);
  v2(tau_g2);
  v1(A_query);
  v1(B_g1_query);
  v2(B_g2_query);
  v1(L_query);
  v1(H_query);
  if (!r.ok) return false;
  if ((int)A_query.size() < num_variables || (int)B_g1_query.size() < num_variables ||
      (int)B_g2_query.size() < num_variables)
    return false;
  return true;
}

bool VerifyingKey::save(const char* path) const {  // verifier.cu:103-148
  std::vector<uint8_t> b;
  int32_t np = num_public;
  b.insert(b.end(), (uint8_t*)&np, (uint8_t*)&np + 4);
  put_fq(b, alpha_g1.x);
  put_fq(b, alpha_g1.y);
  for (const G2A* q : {&beta_g2, &gamma_g2, &delta_g2}) {
    put_fq(b, q->x.c0);
    put_fq(b, q->x.c1);
    put_fq(b, q->y.c0);
    put_fq(b, q->y.c1);
  }
  int32_t ni = (int32_t)ic.size();
  b.insert(b.end(), (uint8_t*)&ni, (uint8_t*)&ni + 4);
  for (auto& p : ic) {
    put_fq(b, p.x);
    put_fq(b, p.y);
  }
  FILE* f = fopen(path, "wb");
  if (!f) return false;
  bool ok = fwrite(b.data(), 1, b.size(), f) == b.size();
  fclose(f);
  return ok;
}

bool VerifyingKey::load(const char* path) {  // verifier.cu:150-195
  Reader r;
  if (!r.open(path)) return false;
  num_public = r.i32();
  alpha_g1 = r.g1(false);
  beta_g2 = r.g2(false);
  gamma_g2 = r.g2(false);
  delta_g2 = r.g2(false);
  int32_t ni = r.i32();
  if (!r.ok || ni < 0) return false;
  ic.resize(ni);
  for (int i = 0; i < ni; i++) ic[i] = r.g1(false);
  return r.ok;
}

}  // namespace orc

// ======================================================================
// C API for the Python test harness (ctypes).  Buffers use the reference's
// in-memory layout: field elements are 4 x u64 little-endian Montgomery
// (R = 2^256) unless a name says _std; G1 affine = x,y (8 u64), G2 affine =
// x.c0,x.c1,y.c0,y.c1 (16 u64); the point at infinity is all zeros.
// ======================================================================
using namespace orc;

static void put_g1(const G1A& p, uint64_t* o) {
  if (p.inf) {
    memset(o, 0, 64);
    return;
  }
  memcpy(o, p.x.v, 32);
  memcpy(o + 4, p.y.v, 32);
}
static G1A get_g1(const uint64_t* o) {
  G1A p;
  p.x = Fq::raw(o);
  p.y = Fq::raw(o + 4);
  p.inf = p.x.is_zero() && p.y.is_zero();
  return p;
}
static void put_g2(const G2A& p, uint64_t* o) {
  if (p.inf) {
    memset(o, 0, 128);
    return;
  }
  memcpy(o, p.x.c0.v, 32);
  memcpy(o + 4, p.x.c1.v, 32);
  memcpy(o + 8, p.y.c0.v, 32);
  memcpy(o + 12, p.y.c1.v, 32);
}
static G2A get_g2(const uint64_t* o) {
  G2A p;
  p.x.c0 = Fq::raw(o);
  p.x.c1 = Fq::raw(o + 4);
  p.y.c0 = Fq::raw(o + 8);
  p.y.c1 = Fq::raw(o + 12);
  p.inf = p.x.is_zero() && p.y.is_zero();
  return p;
}

extern "C" {

int orc_abi_version() { return 1; }

void orc_fr_mul(const uint64_t* a, const uint64_t* b, uint64_t* o) { Fr::mont(o, a, b); }
void orc_fq_mul(const uint64_t* a, const uint64_t* b, uint64_t* o) { Fq::mont(o, a, b); }
void orc_fr_add(const uint64_t* a, const uint64_t* b, uint64_t* o) {
  Fr r = Fr::raw(a) + Fr::raw(b);
  memcpy(o, r.v, 32);
}
void orc_fr_sub(const uint64_t* a, const uint64_t* b, uint64_t* o) {
  Fr r = Fr::raw(a) - Fr::raw(b);
  memcpy(o, r.v, 32);
}
void orc_fq_add(const uint64_t* a, const uint64_t* b, uint64_t* o) {
  Fq r = Fq::raw(a) + Fq::raw(b);
  memcpy(o, r.v, 32);
}
void orc_fq_sub(const uint64_t* a, const uint64_t* b, uint64_t* o) {
  Fq r = Fq::raw(a) - Fq::raw(b);
  memcpy(o, r.v, 32);
}
void orc_fr_inv(const uint64_t* a, uint64_t* o) {
  Fr r = Fr::raw(a).inv();
  memcpy(o, r.v, 32);
}
void orc_fq_inv(const uint64_t* a, uint64_t* o) {
  Fq r = Fq::raw(a).inv();
  memcpy(o, r.v, 32);
}
void orc_fr_from_std(const uint64_t* s, uint64_t* o) {
  Fr r = Fr::from_std(s);
  memcpy(o, r.v, 32);
}
void orc_fr_to_std(const uint64_t* a, uint64_t* o) { Fr::raw(a).to_std(o); }
void orc_fq_from_std(const uint64_t* s, uint64_t* o) {
  Fq r = Fq::from_std(s);
  memcpy(o, r.v, 32);
}
void orc_fq_to_std(const uint64_t* a, uint64_t* o) { Fq::raw(a).to_std(o); }
void orc_fr_from_u64_array(const uint64_t* v, size_t n, uint64_t* o) {
  for (size_t i = 0; i < n; i++) {
    Fr r = Fr::from_uint(v[i]);
    memcpy(o + 4 * i, r.v, 32);
  }
}
void orc_fr_batch_from_std(const uint64_t* s, size_t n, uint64_t* o) {
  for (size_t i = 0; i < n; i++) {
    Fr r = Fr::from_std(s + 4 * i);
    memcpy(o + 4 * i, r.v, 32);
  }
}

void orc_omega(int log_n, int inverse, uint64_t* o) {
  Fr w = inverse ? omega_inv(log_n) : omega(log_n);
  memcpy(o, w.v, 32);
}

void orc_g1_generator(uint64_t* o) { put_g1(g1_generator(), o); }
void orc_g2_generator(uint64_t* o) { put_g2(g2_generator(), o); }

// k*G by double-and-add (the reference's scalar_mul path)
void orc_g1_mul(const uint64_t* pt, const uint64_t* k_mont, uint64_t* o) {
  put_g1(G1J::from_affine(get_g1(pt)).mul(Fr::raw(k_mont)).to_affine(), o);
}
void orc_g2_mul(const uint64_t* pt, const uint64_t* k_mont, uint64_t* o) {
  put_g2(G2J::from_affine(get_g2(pt)).mul(Fr::raw(k_mont)).to_affine(), o);
}
void orc_g1_add(const uint64_t* a, const uint64_t* b, uint64_t* o) {
  put_g1(G1J::from_affine(get_g1(a)).add(G1J::from_affine(get_g1(b))).to_affine(), o);
}
void orc_g2_add(const uint64_t* a, const uint64_t* b, uint64_t* o) {
  put_g2(G2J::from_affine(get_g2(a)).add(G2J::from_affine(get_g2(b))).to_affine(), o);
}
int orc_g1_on_curve(const uint64_t* pt) {
  G1A p = get_g1(pt);
  if (p.inf) return 1;
  return p.y.sqr() == p.x.sqr() * p.x + Fq::from_uint(3);
}

// P_i = k_i * G (k_i Montgomery Fr) via fixed-base tables.
void orc_g1_gen_batch(const uint64_t* k_mont, size_t n, uint64_t* o, int threads) {
  static FixedBase<Fq>* fb = nullptr;
#pragma omp critical
  if (!fb) fb = new FixedBase<Fq>(g1_generator());
  std::vector<G1A> out(n);
  fb->batch((const Fr*)k_mont, n, out.data(), threads);
  for (size_t i = 0; i < n; i++) put_g1(out[i], o + 8 * i);
}
void orc_g2_gen_batch(const uint64_t* k_mont, size_t n, uint64_t* o, int threads) {
  static FixedBase<Fq2>* fb = nullptr;
#pragma omp critical
  if (!fb) fb = new FixedBase<Fq2>(g2_generator());
  std::vector<G2A> out(n);
  fb->batch((const Fr*)k_mont, n, out.data(), threads);
  for (size_t i = 0; i < n; i++) put_g2(out[i], o + 16 * i);
}

// mode 0: reference Pippenger (with its n<=256 / n<=128 CPU fallback); 1: naive;
// 2 (G2 only): reference Pippenger on the reference's affine-inversion G2Ref
void orc_msm_g1(const uint64_t* pts, const uint64_t* sc, size_t n, int mode, int threads, uint64_t* o) {
  std::vector<G1A> p(n);
  for (size_t i = 0; i < n; i++) p[i] = get_g1(pts + 8 * i);
  G1J r = mode == 1 ? msm_g1_naive(p.data(), (const Fr*)sc, (int)n) : msm_g1(p.data(), (const Fr*)sc, (int)n, threads);
  put_g1(r.to_affine(), o);
}
void orc_msm_g2(const uint64_t* pts, const uint64_t* sc, size_t n, int mode, int threads, uint64_t* o) {
  std::vector<G2A> p(n);
  for (size_t i = 0; i < n; i++) p[i] = get_g2(pts + 16 * i);
  if (mode == 2) {
    put_g2(msm_g2_affine_ref(p.data(), (const Fr*)sc, (int)n, threads).to_affine(), o);
    return;
  }
  G2J r = mode == 1 ? msm_g2_naive(p.data(), (const Fr*)sc, (int)n) : msm_g2(p.data(), (const Fr*)sc, (int)n, threads);
  put_g2(r.to_affine(), o);
}

void orc_ntt(uint64_t* data, int log_n, int inverse, int threads) {
  size_t n = (size_t)1 << log_n;
  std::vector<Fr> a(n);
  memcpy(a.data(), data, n * 32);
  ntt_radix2(a, log_n, inverse != 0, threads);
  memcpy(data, a.data(), n * 32);
}
// sum_i a_i b_i mod r for standard-form words (the scalar of a closed-form
// MSM over points k_i G with scalars s_i), written in standard form.
void orc_fr_dot_std(const uint64_t* a, const uint64_t* b, size_t n, uint64_t* out) {
  Fr acc = Fr::zero();
  for (size_t i = 0; i < n; i++) acc = acc + Fr::from_std(a + 4 * i) * Fr::from_std(b + 4 * i);
  acc.to_std(out);
}

// coeff[i] *= g^i (g^-i with inverse): the coset loops of compute_h
// (groth16.cu:352-358 and 377-383) for a small plain integer g.
void orc_coset_scale(uint64_t* data, int log_n, uint64_t g, int inverse) {
  const size_t n = (size_t)1 << log_n;
  Fr gi = Fr::from_uint(g);
  if (inverse) gi = gi.inv();
  Fr gp = Fr::one();
  for (size_t i = 0; i < n; i++) {
    Fr x = Fr::raw(data + 4 * i) * gp;
    memcpy(data + 4 * i, x.v, 32);
    gp = gp * gi;
  }
}

void orc_dft_naive(const uint64_t* in, uint64_t* out, int log_n, int inverse) {
  size_t n = (size_t)1 << log_n;
  std::vector<Fr> a(n), b;
  memcpy(a.data(), in, n * 32);
  dft_naive(a, b, inverse ? omega_inv(log_n) : omega(log_n));
  memcpy(out, b.data(), n * 32);
}

// ---- R1CS handle
void* orc_r1cs_new(int nc, int nv, int npub, int npriv) {
  R1CS* c = new R1CS();
  c->num_constraints = nc;
  c->num_variables = nv;
  c->num_public = npub;
  c->num_private = npriv;
  return c;
}
void orc_r1cs_free(void* h) { delete (R1CS*)h; }
void orc_r1cs_add(void* h, int which, const int32_t* rows, const int32_t* cols, const uint64_t* vals, size_t cnt) {
  R1CS* c = (R1CS*)h;
  std::vector<Entry>& v = which == 0 ? c->A : (which == 1 ? c->B : c->C);
  for (size_t i = 0; i < cnt; i++) v.push_back(Entry{rows[i], cols[i], Fr::raw(vals + 4 * i)});
}
int orc_r1cs_verify(void* h, const uint64_t* w, size_t m) {
  std::vector<Fr> wv(m);
  memcpy(wv.data(), w, m * 32);
  return ((R1CS*)h)->verify_witness(wv) ? 1 : 0;
}
int orc_qap_log_n(int nc) { return qap_log_n(nc); }
int orc_compute_h(void* h, const uint64_t* w, size_t m, uint64_t* out, int threads) {
  std::vector<Fr> wv(m);
  memcpy(wv.data(), w, m * 32);
  std::vector<Fr> hv = compute_h(*(R1CS*)h, wv, threads);
  memcpy(out, hv.data(), hv.size() * 32);
  return (int)hv.size();
}
int orc_setup(void* h, uint64_t seed, const char* pk_path, const char* vk_path, int threads) {
  ProvingKey pk;
  VerifyingKey vk;
  setup(*(R1CS*)h, seed, pk, vk, threads);
  if (!pk.save(pk_path)) return -1;
  if (!vk.save(vk_path)) return -2;
  return 0;
}
// Returns 0 and fills 256 bytes on success; ms[0..3] = h, A, B, C phases.
// g2_affine_ref: the B term on the reference's affine-inversion G2 (same bytes).
int orc_prove_g2mode(const char* pk_path, void* h, const uint64_t* w, size_t m, uint64_t seed, int threads,
                     uint8_t* out, double* ms, int g2_affine_ref) {
  ProvingKey pk;
  if (!pk.load(pk_path)) return -1;
  std::vector<Fr> wv(m);
  memcpy(wv.data(), w, m * 32);
  Proof pf = prove(pk, *(R1CS*)h, wv, seed, threads, ms, g2_affine_ref != 0);
  if (!pf.valid) return -2;
  pf.serialize(out);
  return 0;
}
int orc_prove(const char* pk_path, void* h, const uint64_t* w, size_t m, uint64_t seed, int threads, uint8_t* out,
              double* ms) {
  ProvingKey pk;
  if (!pk.load(pk_path)) return -1;
  std::vector<Fr> wv(m);
  memcpy(wv.data(), w, m * 32);
  Proof pf = prove(pk, *(R1CS*)h, wv, seed, threads, ms);
  if (!pf.valid) return -2;
  pf.serialize(out);
  return 0;
}
// Load a ZKMLPK3 file and emit its vectors in the interchange layout, for
// loader-parity tests.  sizes[0..6] = tau_g1, tau_g2, A, B1, B2, L, H;
// hdr[0..2] = n, m, npub.  Buffers may be null to query sizes.
int orc_pk_read(const char* path, int32_t* hdr, int32_t* sizes, uint64_t* fixed6, uint64_t* A, uint64_t* B1,
                uint64_t* B2, uint64_t* L, uint64_t* H) {
  ProvingKey pk;
  if (!pk.load(path)) return -1;
  hdr[0] = pk.num_constraints;
  hdr[1] = pk.num_variables;
  hdr[2] = pk.num_public;
  sizes[0] = (int32_t)pk.tau_g1.size();
  sizes[1] = (int32_t)pk.tau_g2.size();
  sizes[2] = (int32_t)pk.A_query.size();
  sizes[3] = (int32_t)pk.B_g1_query.size();
  sizes[4] = (int32_t)pk.B_g2_query.size();
  sizes[5] = (int32_t)pk.L_query.size();
  sizes[6] = (int32_t)pk.H_query.size();
  if (fixed6) {  // alpha1, beta1, delta1 (3 x 8), beta2, gamma2, delta2 (3 x 16)
    put_g1(pk.alpha_g1, fixed6);
    put_g1(pk.beta_g1, fixed6 + 8);
    put_g1(pk.delta_g1, fixed6 + 16);
    put_g2(pk.beta_g2, fixed6 + 24);
    put_g2(pk.gamma_g2, fixed6 + 40);
    put_g2(pk.delta_g2, fixed6 + 56);
  }
  if (A)
    for (size_t i = 0; i < pk.A_query.size(); i++) put_g1(pk.A_query[i], A + 8 * i);
  if (B1)
    for (size_t i = 0; i < pk.B_g1_query.size(); i++) put_g1(pk.B_g1_query[i], B1 + 8 * i);
  if (B2)
    for (size_t i = 0; i < pk.B_g2_query.size(); i++) put_g2(pk.B_g2_query[i], B2 + 16 * i);
  if (L)
    for (size_t i = 0; i < pk.L_query.size(); i++) put_g1(pk.L_query[i], L + 8 * i);
  if (H)
    for (size_t i = 0; i < pk.H_query.size(); i++) put_g1(pk.H_query[i], H + 8 * i);
  return 0;
}

int orc_threads_max() { return omp_get_max_threads(); }

}  // extern "C"
