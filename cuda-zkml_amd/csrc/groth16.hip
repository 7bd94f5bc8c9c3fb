// Groth16 prover core: R1CS on the device, quotient polynomial h(x), proving
// key loading, trusted setup and prove, behind the C ABI.
//
// Reference: src/prover/groth16.cu (compute_h :263-390, setup :446-642,
// prove :655-920, ZKMLPK3 save/load :1104-1314), src/prover/circuit.cuh
// (R1CS, verify_witness :93-124), src/verifier/verifier.cu (VK layout).
#include <stdio.h>
#include <string.h>

#include <algorithm>
#include <atomic>
#include <chrono>
#include <condition_variable>
#include <functional>
#include <mutex>
#include <random>
#include <thread>
#include <vector>

#include "curve.hpp"
#include "host_bn254.hpp"
#include "zk_internal.hpp"

using namespace zk;

struct zk_r1cs {
  int nc = 0, nv = 0, npub = 0, log_n = 0;
  size_t n = 0;
  // CSR per matrix (A, B, C), rows < n; values are the reference's Montgomery
  // words multiplied by 32 so that fmul(w, v') = w v in Montgomery form.
  uint32_t* col[3] = {nullptr, nullptr, nullptr};
  uint4* val[3] = {nullptr, nullptr, nullptr};
  size_t nnz[3] = {0, 0, 0};
  // rows cut into segments of at most SPMV_SEG nonzeros: segment s covers
  // nonzeros [seg[s].x, seg[s].y); row r owns segments [segptr[r], segptr[r+1])
  uint32_t* segptr[3] = {nullptr, nullptr, nullptr};
  uint2* seg[3] = {nullptr, nullptr, nullptr};
  size_t nseg[3] = {0, 0, 0};
  // host COO copies for setup (QAP evaluation at tau)
  std::vector<zk_sparse_entry> coo[3];
};

struct zk_pk {
  int n = 0, m = 0, npub = 0;
  // fixed points, Montgomery words, x = y = 0 at infinity
  uint64_t alpha1[8], beta1[8], delta1[8];
  uint64_t beta2[16], gamma2[16], delta2[16];
  size_t nA = 0, nB1 = 0, nB2 = 0, nL = 0, nH = 0, ntau1 = 0, ntau2 = 0;
  void *A = nullptr, *B1 = nullptr, *B2 = nullptr, *L = nullptr, *H = nullptr;  // device point records
  // window tables of the queries (null: the MSM runs over the records)
  void *tA = nullptr, *tB1 = nullptr, *tB2 = nullptr, *tL = nullptr, *tH = nullptr;
  zk::MsmTab tab_w, tab_b2, tab_h;  // shapes: A, B1 and L (one shared sort), B2, H
};

namespace {

// ------------------------------------------------------------------ kernels
__device__ __forceinline__ fr ld_fr(const uint4* __restrict__ p, size_t i) {
  uint4 a = p[2 * i], b = p[2 * i + 1];
  uint32_t w[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
  return repack_in<FrP>(w);
}

__device__ __forceinline__ void st_fr(uint4* __restrict__ p, size_t i, const fr& x) {
  uint32_t w[8];
  repack_out(x, w);
  p[2 * i] = make_uint4(w[0], w[1], w[2], w[3]);
  p[2 * i + 1] = make_uint4(w[4], w[5], w[6], w[7]);
}

constexpr uint32_t SPMV_SEG = 8;  // nonzeros per segment

struct Csr3 {
  const uint32_t* segptr[3];
  const uint2* seg[3];
  const uint32_t* col[3];
  const uint4* val[3];
  size_t nseg[3];
  size_t part_off[3];  // first partial of each matrix
};

// A.w, B.w, C.w in evaluation form (groth16.cu:275-294) in two steps so that
// no thread walks a long row: one thread per (segment, matrix) forms the
// segment's partial sum sum_e w[col_e] * v_e ...
__global__ void k_spmv_seg(uint4* __restrict__ part, const uint4* __restrict__ w, Csr3 m) {
  quotient_priority();
  const size_t s = blockIdx.x * (size_t)blockDim.x + threadIdx.x;
  const int mat = blockIdx.y;
  if (s >= m.nseg[mat]) return;
  const uint2 r = m.seg[mat][s];
  fr acc = fe_zero<FrP>();
  for (uint32_t k = r.x; k < r.y; k++) acc = fadd(acc, fmul(ld_fr(w, m.col[mat][k]), ld_fr(m.val[mat], k)));
  st_fr(part, m.part_off[mat] + s, acc);
}

// ... then one thread per (row, matrix) adds its segments' partials:
// out[mat * n + row].
__global__ void k_spmv_rows(uint4* __restrict__ out, const uint4* __restrict__ part, Csr3 m, size_t n) {
  quotient_priority();
  const size_t row = blockIdx.x * (size_t)blockDim.x + threadIdx.x;
  const int mat = blockIdx.y;
  if (row >= n) return;
  const uint32_t b = m.segptr[mat][row], e = m.segptr[mat][row + 1];
  fr acc = fe_zero<FrP>();
  for (uint32_t k = b; k < e; k++) acc = fadd(acc, ld_fr(part, m.part_off[mat] + k));
  st_fr(out, (size_t)mat * n + row, acc);
}

// Row check (A.w)(B.w) = C.w for rows < nc (circuit.cuh:93-124).  With raw
// Montgomery words fmul(a, b) = ab 2^251 and fmul(c, 2^256) = c 2^251.
__global__ void k_check_rows(const uint4* __restrict__ abc, size_t n, size_t nc, uint32_t* __restrict__ bad) {
  quotient_priority();
  const size_t row = blockIdx.x * (size_t)blockDim.x + threadIdx.x;
  if (row >= nc) return;
  const uint32_t K256[8] = {0x4ffffffbu, 0xac96341cu, 0x9f60cd29u, 0x36fc7695u,
                            0x7879462eu, 0x666ea36fu, 0x9a07df2fu, 0x0e0a77c1u};
  fr lhs = fmul(ld_fr(abc, row), ld_fr(abc, n + row));
  fr rhs = fmul(ld_fr(abc, 2 * n + row), repack_in<FrP>(K256));
  if (!feq(lhs, rhs)) atomicAdd(bad, 1u);
}

// Montgomery words (R = 2^256) -> standard form, in place.  fmul(x 2^256, 32)
// in the internal radix 2^261 gives x.
template <class P>
__global__ void k_mont_to_std(uint4* __restrict__ p, size_t count) {
  const size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x;
  if (i >= count) return;
  uint4 a = p[2 * i], b = p[2 * i + 1];
  uint32_t w[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
  fe<P> k32 = fe_zero<P>();
  k32.l[0] = 32;
  repack_out(fmul(repack_in<P>(w), k32), w);
  p[2 * i] = make_uint4(w[0], w[1], w[2], w[3]);
  p[2 * i + 1] = make_uint4(w[4], w[5], w[6], w[7]);
}

// ------------------------------------------------------------------ host helpers
using zkh::Fq;
using zkh::Fq2;
using zkh::Fr;
using zkh::G1;
using zkh::G2;

struct DevMem {
  zk_context* ctx;
  std::vector<void*> ptrs;
  explicit DevMem(zk_context* c) : ctx(c) {}
  ~DevMem() {
    for (void* p : ptrs) (void)hipFree(p);
  }
  int alloc(void** p, size_t bytes) {
    if (hipMalloc(p, bytes ? bytes : 1) != hipSuccess) return ctx->fail(ZK_ERR_OOM, "device allocation failed");
    ptrs.push_back(*p);
    return ZK_OK;
  }
};

G1 g1_from_words(const uint64_t* w) {
  bool inf = true;
  for (int i = 0; i < 8; i++) inf = inf && w[i] == 0;
  if (inf) return G1::inf();
  return G1::affine(Fq::raw(w), Fq::raw(w + 4));
}
G2 g2_from_words(const uint64_t* w) {
  bool inf = true;
  for (int i = 0; i < 16; i++) inf = inf && w[i] == 0;
  if (inf) return G2::inf();
  return G2::affine(Fq2{Fq::raw(w), Fq::raw(w + 4)}, Fq2{Fq::raw(w + 8), Fq::raw(w + 12)});
}
// Jacobian words x, y, z (an MSM's jac_out result; z = 0 at infinity)
G1 g1_from_jac_words(const uint64_t* w) {
  const G1 p{Fq::raw(w), Fq::raw(w + 4), Fq::raw(w + 8)};
  return p.is_inf() ? G1::inf() : p;
}
G2 g2_from_jac_words(const uint64_t* w) {
  const G2 p{Fq2{Fq::raw(w), Fq::raw(w + 4)}, Fq2{Fq::raw(w + 8), Fq::raw(w + 12)},
             Fq2{Fq::raw(w + 16), Fq::raw(w + 20)}};
  return p.is_inf() ? G2::inf() : p;
}

// Affine words of the three proof points with one field inversion: the
// Jacobian z of A and C and the norm z0^2 + z1^2 of B's z (1 / z = conj(z) /
// norm in Fq2) are inverted together (Montgomery's trick); a point at
// infinity enters as 1 and is written as zeros.
void proof_to_words(const G1& A, const G2& B, const G1& C, uint64_t* aw, uint64_t* bw, uint64_t* cw) {
  const Fq one = Fq::one();
  const Fq za = A.is_inf() ? one : A.z, zc = C.is_inf() ? one : C.z;
  const Fq nb = B.is_inf() ? one : B.z.c0.sqr() + B.z.c1.sqr();
  const Fq ac = za * zc;
  const Fq inv = (ac * nb).inv();
  const Fq ia = inv * zc * nb, ic = inv * za * nb, inb = inv * ac;
  auto g1w = [](const G1& p, const Fq& zi, uint64_t* w) {
    memset(w, 0, 64);
    if (p.is_inf()) return;
    const Fq zi2 = zi.sqr();
    const Fq x = p.x * zi2, y = p.y * (zi2 * zi);
    memcpy(w, x.v, 32);
    memcpy(w + 4, y.v, 32);
  };
  g1w(A, ia, aw);
  g1w(C, ic, cw);
  memset(bw, 0, 128);
  if (!B.is_inf()) {
    const Fq2 zi{B.z.c0 * inb, -(B.z.c1 * inb)};
    const Fq2 zi2 = zi.sqr();
    const Fq2 x = B.x * zi2, y = B.y * (zi2 * zi);
    memcpy(bw, x.c0.v, 32);
    memcpy(bw + 4, x.c1.v, 32);
    memcpy(bw + 8, y.c0.v, 32);
    memcpy(bw + 12, y.c1.v, 32);
  }
}

// Fr::from_uint(rng()) until nonzero (groth16.cu:48-58)
Fr random_nonzero(std::mt19937_64& rng) {
  Fr v = Fr::from_u64(rng());
  while (v.is_zero()) v = Fr::from_u64(rng());
  return v;
}

int log2_domain(int nc) {  // QAP::from_r1cs, groth16.cu:225-242
  int log_n = 0, n = 1;
  while (n < nc) {
    n <<= 1;
    log_n++;
  }
  if (n < 4) log_n = 2;
  return log_n;
}

// Coset shift: 5 unless 5^n = 1, then 7 (groth16.cu:329-342).  Returns g and
// (g^n - 1)^-1 in Montgomery words.
uint64_t coset_shift(int log_n, Fr& zinv) {
  for (uint64_t g : {5ull, 7ull}) {
    Fr z = Fr::from_u64(g);
    for (int i = 0; i < log_n; i++) z = z.sqr();
    z = z - Fr::one();
    if (!z.is_zero()) {
      zinv = z.inv();
      return g;
    }
  }
  zinv = Fr::zero();
  return 0;
}

int quotient_run(zk_context* ctx, const zk_r1cs* c, const void* d_w, void* d_h, void* d_abc, hipStream_t st,
                 bool check, uint32_t* d_bad) {
  const size_t n = c->n;
  Csr3 m;
  size_t nparts = 0, segmax = 1;
  for (int k = 0; k < 3; k++) {
    m.segptr[k] = c->segptr[k];
    m.seg[k] = c->seg[k];
    m.col[k] = c->col[k];
    m.val[k] = c->val[k];
    m.nseg[k] = c->nseg[k];
    m.part_off[k] = nparts;
    nparts += c->nseg[k];
    segmax = std::max(segmax, c->nseg[k]);
  }
  ZK_TRY(ctx->ensure(ctx->scratch_d, std::max<size_t>(nparts, 1) * 32));
  uint4* part = (uint4*)ctx->scratch_d.p;
  ZK_LAUNCH(ctx, st, "quotient_spmv", k_spmv_seg, dim3(cdiv(segmax, 256), 3), dim3(256), 0, part, (const uint4*)d_w,
            m);
  ZK_LAUNCH(ctx, st, "quotient_spmv", k_spmv_rows, dim3(cdiv(n, 256), 3), dim3(256), 0, (uint4*)d_abc,
            (const uint4*)part, m, n);
  if (check) {
    ZK_HIP(ctx, hipMemsetAsync(d_bad, 0, 4, st));
    ZK_LAUNCH(ctx, st, "witness_check", k_check_rows, dim3(cdiv((size_t)c->nc, 256)), dim3(256), 0,
              (const uint4*)d_abc, n, (size_t)c->nc, d_bad);
  }
  Fr zinv;
  const uint64_t g = coset_shift(c->log_n, zinv);
  if (!g) return ctx->fail(ZK_ERR_INVALID, "no valid coset shift");
  // 3 iNTT -> coefficients; 3 coset NTT -> evaluations on g*H
  // (groth16.cu:321-363); (A B - C) / Z and the coset iNTT h_i = iNTT(H)_i g^-i
  // (groth16.cu:366-383), the pointwise step inside the last transform
  uint4* abc = (uint4*)d_abc;
  return quotient_ntts(ctx, d_h, abc, abc + 6 * n, c->log_n, g, zinv.v, st);
}

// ------------------------------------------------------------------ ZKMLPK3
struct FileBuf {
  std::vector<uint8_t> d;
  size_t off = 0;
  bool ok = true;
  bool read(const char* path) {
    FILE* f = fopen(path, "rb");
    if (!f) return false;
    fseek(f, 0, SEEK_END);
    long sz = ftell(f);
    fseek(f, 0, SEEK_SET);
    if (sz < 0) {
      fclose(f);
      return false;
    }
    d.resize((size_t)sz);
    ok = fread(d.data(), 1, d.size(), f) == d.size();
    fclose(f);
    return ok;
  }
  bool take(void* p, size_t n) {
    if (!ok || off + n > d.size()) return ok = false;
    memcpy(p, d.data() + off, n);
    off += n;
    return true;
  }
  int32_t i32() {
    int32_t v = 0;
    take(&v, 4);
    return v;
  }
};

// One record: u8 infinity + `coords` standard-form 32-byte coordinates.
void parse_point(FileBuf& f, int coords, uint64_t* std_out, uint8_t* flag) {
  uint8_t inf = 0;
  f.take(&inf, 1);
  f.take(std_out, 32 * coords);
  *flag = inf;
}

void fixed_g1(const uint64_t* s, uint8_t inf, uint64_t* w) {
  memset(w, 0, 64);
  if (inf) return;
  Fq x = Fq::from_std(s), y = Fq::from_std(s + 4);
  memcpy(w, x.v, 32);
  memcpy(w + 4, y.v, 32);
}
void fixed_g2(const uint64_t* s, uint8_t inf, uint64_t* w) {
  memset(w, 0, 128);
  if (inf) return;
  for (int k = 0; k < 4; k++) {
    Fq v = Fq::from_std(s + 4 * k);
    memcpy(w + 4 * k, v.v, 32);
  }
}

int upload_query(zk_context* ctx, FileBuf& f, bool g2, size_t count, void** d_recs) {
  const int coords = g2 ? 4 : 2;
  std::vector<uint64_t> std_words(count * coords * 4);
  std::vector<uint8_t> flags(count);
  for (size_t i = 0; i < count; i++) parse_point(f, coords, &std_words[i * coords * 4], &flags[i]);
  if (!f.ok) return ctx->fail(ZK_ERR_IO, "proving key truncated");
  void *d_std = nullptr, *d_flags = nullptr;
  if (hipMalloc(d_recs, std::max<size_t>(count, 1) * rec_bytes(g2)) != hipSuccess)
    return ctx->fail(ZK_ERR_OOM, "proving key allocation failed");
  if (count == 0) return ZK_OK;
  DevMem tmp(ctx);
  ZK_TRY(tmp.alloc(&d_std, std_words.size() * 8));
  ZK_TRY(tmp.alloc(&d_flags, count));
  ZK_HIP(ctx, hipMemcpyAsync(d_std, std_words.data(), std_words.size() * 8, hipMemcpyHostToDevice, ctx->stream));
  ZK_HIP(ctx, hipMemcpyAsync(d_flags, flags.data(), count, hipMemcpyHostToDevice, ctx->stream));
  ZK_TRY(recs_from_std(ctx, g2, *d_recs, d_std, d_flags, count, ctx->stream));
  ZK_HIP(ctx, hipStreamSynchronize(ctx->stream));
  return ZK_OK;
}

void skip_query(FileBuf& f, bool g2, size_t count) {
  const size_t rec = g2 ? 129 : 65;
  if (f.off + rec * count > f.d.size()) f.ok = false;
  else f.off += rec * count;
}

// ------------------------------------------------------------------ file writers
struct Bytes {
  std::vector<uint8_t> b;
  void u32(uint32_t v) { b.insert(b.end(), (uint8_t*)&v, (uint8_t*)&v + 4); }
  void raw(const void* p, size_t n) { b.insert(b.end(), (const uint8_t*)p, (const uint8_t*)p + n); }
  bool write(const char* path) const {
    FILE* f = fopen(path, "wb");
    if (!f) return false;
    bool ok = fwrite(b.data(), 1, b.size(), f) == b.size();
    return fclose(f) == 0 && ok;
  }
};

void put_std(Bytes& o, const Fq& v) {
  uint64_t s[4];
  v.to_std(s);
  o.raw(s, 32);
}
void put_g1_rec(Bytes& o, const G1& p) {
  Fq x, y;
  uint8_t inf = p.to_affine(x, y) ? 0 : 1;
  o.raw(&inf, 1);
  put_std(o, x);
  put_std(o, y);
}
void put_g2_rec(Bytes& o, const G2& p) {
  Fq2 x, y;
  uint8_t inf = p.to_affine(x, y) ? 0 : 1;
  o.raw(&inf, 1);
  put_std(o, x.c0);
  put_std(o, x.c1);
  put_std(o, y.c0);
  put_std(o, y.c1);
}

// Points generated on the device (standard-form words after k_mont_to_std)
// appended as ZKMLPK3 records.
void put_std_points(Bytes& o, const std::vector<uint64_t>& w, size_t count, int coords) {
  for (size_t i = 0; i < count; i++) {
    const uint64_t* p = &w[i * coords * 4];
    bool inf = true;
    for (int k = 0; k < coords * 4; k++) inf = inf && p[k] == 0;
    uint8_t f = inf ? 1 : 0;
    o.raw(&f, 1);
    o.raw(p, 32 * coords);
  }
}

// k_i * G on the device for a host vector of Fr scalars; returns
// standard-form coordinates (zeros at infinity).
int gen_points_std(zk_context* ctx, const std::vector<Fr>& k, bool g2, std::vector<uint64_t>& out) {
  const size_t n = k.size();
  const int words = g2 ? 16 : 8;
  out.assign(n * words, 0);
  if (n == 0) return ZK_OK;
  DevMem tmp(ctx);
  void *d_k = nullptr, *d_p = nullptr;
  ZK_TRY(tmp.alloc(&d_k, n * 32));
  ZK_TRY(tmp.alloc(&d_p, n * words * 8));
  ZK_HIP(ctx, hipMemcpyAsync(d_k, k.data(), n * 32, hipMemcpyHostToDevice, ctx->stream));
  if (g2) ZK_TRY(g2_generator_mul(ctx, d_k, n, d_p, ctx->stream));
  else ZK_TRY(g1_generator_mul(ctx, d_k, n, d_p, ctx->stream));
  const size_t elems = n * words / 4;
  ZK_LAUNCH(ctx, ctx->stream, "pk_convert", k_mont_to_std<FqP>, dim3(cdiv(elems, 256)), dim3(256), 0,
            (uint4*)d_p, elems);
  ZK_HIP(ctx, hipMemcpyAsync(out.data(), d_p, n * words * 8, hipMemcpyDeviceToHost, ctx->stream));
  ZK_HIP(ctx, hipStreamSynchronize(ctx->stream));
  // the point at infinity comes out as x = y = 0 in either form
  return ZK_OK;
}

}  // namespace

// ======================================================================
extern "C" {

static int zk_r1cs_create_impl(zk_context* ctx, int num_constraints, int num_variables, int num_public,
                               const zk_sparse_entry* A, size_t nA, const zk_sparse_entry* B, size_t nB,
                               const zk_sparse_entry* C, size_t nC, zk_r1cs** out) {
  if (!ctx || !out) return ZK_ERR_INVALID;
  *out = nullptr;
  if (num_constraints < 0 || num_variables <= 0 || num_public < 0 || num_public + 1 > num_variables)
    return ctx->fail(ZK_ERR_INVALID, "r1cs: bad sizes");
  if ((nA && !A) || (nB && !B) || (nC && !C)) return ctx->fail(ZK_ERR_INVALID, "r1cs: null matrix");
  const int log_n = log2_domain(num_constraints);
  if (log_n > 24) return ctx->fail(ZK_ERR_SIZE, "r1cs: domain above 2^24");
  zk_r1cs* c = new zk_r1cs();
  c->nc = num_constraints;
  c->nv = num_variables;
  c->npub = num_public;
  c->log_n = log_n;
  c->n = (size_t)1 << log_n;
  const zk_sparse_entry* mats[3] = {A, B, C};
  const size_t cnts[3] = {nA, nB, nC};
  int st = ZK_OK;
  for (int k = 0; k < 3 && st == ZK_OK; k++) {
    c->coo[k].assign(mats[k], mats[k] + cnts[k]);
    // CSR over rows < n; entries outside [0, n) x [0, m) are dropped as in
    // compute_h (groth16.cu:282-293)
    std::vector<uint32_t> rowptr(c->n + 1, 0);
    for (size_t i = 0; i < cnts[k]; i++) {
      const zk_sparse_entry& e = mats[k][i];
      if (e.row >= 0 && (size_t)e.row < c->n && e.col >= 0 && e.col < num_variables) rowptr[e.row + 1]++;
    }
    for (size_t r = 0; r < c->n; r++) rowptr[r + 1] += rowptr[r];
    const size_t nnz = rowptr[c->n];
    std::vector<uint32_t> fill(rowptr.begin(), rowptr.end() - 1), col(nnz);
    std::vector<uint64_t> val(nnz * 4);
    for (size_t i = 0; i < cnts[k]; i++) {
      const zk_sparse_entry& e = mats[k][i];
      if (!(e.row >= 0 && (size_t)e.row < c->n && e.col >= 0 && e.col < num_variables)) continue;
      const uint32_t p = fill[e.row]++;
      col[p] = (uint32_t)e.col;
      Fr v = Fr::raw(e.value);
      for (int d = 0; d < 5; d++) v = v.dbl();  // x 32
      memcpy(&val[(size_t)p * 4], v.v, 32);
    }
    c->nnz[k] = nnz;
    // segments of at most SPMV_SEG nonzeros per row
    std::vector<uint32_t> segptr(c->n + 1, 0);
    std::vector<uint2> seg;
    for (size_t r = 0; r < c->n; r++) {
      segptr[r] = (uint32_t)seg.size();
      for (uint32_t b = rowptr[r]; b < rowptr[r + 1]; b += SPMV_SEG)
        seg.push_back(make_uint2(b, std::min<uint32_t>(b + SPMV_SEG, rowptr[r + 1])));
    }
    segptr[c->n] = (uint32_t)seg.size();
    c->nseg[k] = seg.size();
    if (hipMalloc(&c->segptr[k], segptr.size() * 4) != hipSuccess ||
        hipMalloc(&c->seg[k], std::max<size_t>(seg.size(), 1) * sizeof(uint2)) != hipSuccess ||
        hipMemcpy(c->segptr[k], segptr.data(), segptr.size() * 4, hipMemcpyHostToDevice) != hipSuccess ||
        (!seg.empty() && hipMemcpy(c->seg[k], seg.data(), seg.size() * sizeof(uint2), hipMemcpyHostToDevice) !=
                             hipSuccess)) {
      st = ctx->fail(ZK_ERR_OOM, "r1cs allocation failed");
      break;
    }
    if (hipMalloc(&c->col[k], std::max<size_t>(nnz, 1) * 4) != hipSuccess ||
        hipMalloc(&c->val[k], std::max<size_t>(nnz, 1) * 32) != hipSuccess) {
      st = ctx->fail(ZK_ERR_OOM, "r1cs allocation failed");
      break;
    }
    if ((nnz && hipMemcpy(c->col[k], col.data(), nnz * 4, hipMemcpyHostToDevice) != hipSuccess) ||
        (nnz && hipMemcpy(c->val[k], val.data(), nnz * 32, hipMemcpyHostToDevice) != hipSuccess))
      st = ctx->fail(ZK_ERR_HIP, "r1cs upload failed");
  }
  if (st != ZK_OK) {
    zk_r1cs_destroy(c);
    return st;
  }
  *out = c;
  return ZK_OK;
}

int zk_r1cs_create(zk_context* ctx, int num_constraints, int num_variables, int num_public,
                   const zk_sparse_entry* A, size_t nA, const zk_sparse_entry* B, size_t nB,
                   const zk_sparse_entry* C, size_t nC, zk_r1cs** out) {
  return zk::guard(ctx, [&] {
    return zk_r1cs_create_impl(ctx, num_constraints, num_variables, num_public, A, nA, B, nB, C, nC, out);
  });
}

void zk_r1cs_destroy(zk_r1cs* c) {
  if (!c) return;
  for (int k = 0; k < 3; k++) {
    if (c->col[k]) (void)hipFree(c->col[k]);
    if (c->val[k]) (void)hipFree(c->val[k]);
    if (c->segptr[k]) (void)hipFree(c->segptr[k]);
    if (c->seg[k]) (void)hipFree(c->seg[k]);
  }
  delete c;
}

int zk_r1cs_domain(const zk_r1cs* c, int* log_n) {
  if (!c || !log_n) return ZK_ERR_INVALID;
  *log_n = c->log_n;
  return ZK_OK;
}

static int zk_quotient_h_impl(zk_context* ctx, const zk_r1cs* c, const void* d_witness, size_t m, void* d_h,
                              void* stream) {
  if (!ctx || !c || !d_witness || !d_h) return ZK_ERR_INVALID;
  if (m != (size_t)c->nv) return ctx->fail(ZK_ERR_MISMATCH, "quotient: witness length != num_variables");
  ZK_TRY(ctx->ensure(ctx->scratch_b, c->n * 32 * 6));  // A | B | C and the transforms' work space
  return quotient_run(ctx, c, d_witness, d_h, ctx->scratch_b.p, ctx->s(stream), false, nullptr);
}

int zk_quotient_h(zk_context* ctx, const zk_r1cs* c, const void* d_witness, size_t m, void* d_h, void* stream) {
  return zk::guard(ctx, [&] { return zk_quotient_h_impl(ctx, c, d_witness, m, d_h, stream); });
}

// Window tables of the proving-key queries, built at load for MSMs of
// 2^ZK_PK_TAB_MIN_LOG .. 2^ZK_PK_TAB_MAX_LOG scalars.  The digit windows of a
// table MSM share one bucket space, so wider windows cost no reduction per
// window: 16 windows of 16 bits (or 20 of 13), against 24-26 windows of 10-11
// bits in the plain MSMs at 2^16 points, reduced in sub-windows of 2^SUB
// buckets.  A table holds W copies of its query.  Measured on the 2^16 proof
// (config 4): 1.63 -> 1.45 ms with W = 16 for the witness G1 sets (A, B1, L
// share one sort) and W = 20 for B2 and H (a 16-bit single window sorts
// slower, and H's sort runs beside the other MSMs' accumulations); 2^13
// (config 1) was 5% slower with tables (W = 20 or 26), so they start at 2^14.
#ifndef ZK_PK_TAB_MIN_LOG
#define ZK_PK_TAB_MIN_LOG 14
#endif
#ifndef ZK_PK_TAB_MAX_LOG
#define ZK_PK_TAB_MAX_LOG 23
#endif
#ifndef ZK_PK_TAB_W_HUGE
#define ZK_PK_TAB_W_HUGE 13
#endif
#ifndef ZK_PK_TAB_SUB
#define ZK_PK_TAB_SUB 10
#endif
#ifndef ZK_PK_TAB_W_LARGE
#define ZK_PK_TAB_W_LARGE 16
#endif
#ifndef ZK_PK_TAB_W_LARGE_B2
#define ZK_PK_TAB_W_LARGE_B2 20
#endif
#ifndef ZK_PK_TAB_W_LARGE_H
#define ZK_PK_TAB_W_LARGE_H 20
#endif

// H's sub-windows: 2^8 buckets, level 1 one bucket per thread (H sorts and
// reduces after the quotient, on the 2^16 proof's critical path: its reduction
// 4 -> 16 workgroups, H 0.70 -> 0.66 ms)
#ifndef ZK_PK_TAB_SUB_H
#define ZK_PK_TAB_SUB_H 8
#endif
// B2's sub-windows: 2^9 buckets (the G2 job ends the 2^16 proof; its
// reduction chains are Fq2 additions, one level shallower this way: config 4
// 1.32-1.36 -> 1.30 ms; 2^8 and 2^7 1.30-1.31 ms)
#ifndef ZK_PK_TAB_SUB_B2
#define ZK_PK_TAB_SUB_B2 9
#endif
// Table shape for MSMs of n scalars (W = 0: no table); wlarge: windows from
// 2^15 scalars on; sub: log2 of the sub-window size up to 2^18 scalars.
static MsmTab table_shape(size_t n, int wlarge, int sub = ZK_PK_TAB_SUB) {
  MsmTab t;
  if (n < ((size_t)1 << ZK_PK_TAB_MIN_LOG) || n > ((size_t)1 << ZK_PK_TAB_MAX_LOG)) return t;
  const bool huge = n > ((size_t)1 << 18);
  t.W = huge ? ZK_PK_TAB_W_HUGE : n >= ((size_t)1 << 15) ? wlarge : 20;
  if ((size_t)t.W * n > MSM_MAX_N) return MsmTab{};  // positions of all windows beyond the sort's range
  const int c = (254 + t.W - 1) / t.W;  // widest window
  // above 2^18 scalars: 2^15-bucket sub-windows (the plain MSMs' reduction
  // shape at 2^20 .. 2^22 points)
  t.log_sub = std::min(huge ? 15 : sub, c - 1);
  return t;
}

static int pk_table(zk_context* ctx, bool g2, const void* recs, size_t count, const MsmTab& t, void** out) {
  *out = nullptr;
  if (count == 0) return ZK_OK;
  if (dev_malloc(out, msm_table_bytes(g2, count, t)) != hipSuccess) {
    *out = nullptr;
    return ctx->fail(ZK_ERR_OOM, "proving key: window table allocation failed");
  }
  return msm_table_build(ctx, g2, recs, count, t, *out, ctx->stream);
}

// Frees a key's window tables: its MSMs then run over the query records.
static void pk_drop_tables(zk_pk* pk) {
  for (void** t : {&pk->tA, &pk->tB1, &pk->tB2, &pk->tL, &pk->tH}) {
    if (*t) (void)hipFree(*t);
    *t = nullptr;
  }
}

static int pk_tables_build(zk_context* ctx, zk_pk* pk) {
  pk->tab_w = table_shape((size_t)pk->m, ZK_PK_TAB_W_LARGE);
  pk->tab_b2 = table_shape((size_t)pk->m, ZK_PK_TAB_W_LARGE_B2, ZK_PK_TAB_SUB_B2);
  pk->tab_h = table_shape((size_t)pk->n, ZK_PK_TAB_W_LARGE_H, ZK_PK_TAB_SUB_H);
  if (pk->tab_w.W) {
    ZK_TRY(pk_table(ctx, false, pk->A, pk->nA, pk->tab_w, &pk->tA));
    ZK_TRY(pk_table(ctx, false, pk->B1, pk->nB1, pk->tab_w, &pk->tB1));
    ZK_TRY(pk_table(ctx, false, pk->L, pk->nL, pk->tab_w, &pk->tL));
  }
  if (pk->tab_b2.W) ZK_TRY(pk_table(ctx, true, pk->B2, pk->nB2, pk->tab_b2, &pk->tB2));
  if (pk->tab_h.W) ZK_TRY(pk_table(ctx, false, pk->H, pk->nH, pk->tab_h, &pk->tH));
  return ZK_OK;
}

// The tables only speed the proof up: when device memory for them (or for
// their temporary) runs out, the key loads without any (the three witness
// G1 sets use them all or none) and proofs take the plain MSMs, same bytes.
static int pk_tables(zk_context* ctx, zk_pk* pk) {
  const int rc = pk_tables_build(ctx, pk);
  if (rc != ZK_ERR_OOM) return rc;
  pk_drop_tables(pk);
  (void)hipGetLastError();  // the failed allocation's error is not this call's
  std::lock_guard<std::mutex> lk(ctx->mu);
  ctx->last_error.clear();
  return ZK_OK;
}

static int zk_pk_load_impl(zk_context* ctx, const char* path, zk_pk** out) {
  if (!ctx || !path || !out) return ZK_ERR_INVALID;
  *out = nullptr;
  FileBuf f;
  if (!f.read(path)) return ctx->fail(ZK_ERR_IO, "cannot read proving key", path);
  char magic[8] = {0};
  f.take(magic, 8);
  if (!f.ok || memcmp(magic, "ZKMLPK3", 7) != 0) return ctx->fail(ZK_ERR_IO, "not a ZKMLPK3 proving key", path);
  uint32_t ver = 0;
  f.take(&ver, 4);
  if (!f.ok || ver != 3) return ctx->fail(ZK_ERR_IO, "unsupported proving-key version");
  zk_pk* pk = new zk_pk();
  pk->n = f.i32();
  pk->m = f.i32();
  pk->npub = f.i32();
  if (!f.ok || pk->n < 0 || pk->m <= 0 || pk->npub < 0) {
    delete pk;
    return ctx->fail(ZK_ERR_IO, "invalid proving-key metadata");
  }
  uint64_t s[16];
  uint8_t inf;
  parse_point(f, 2, s, &inf);
  fixed_g1(s, inf, pk->alpha1);
  parse_point(f, 2, s, &inf);
  fixed_g1(s, inf, pk->beta1);
  parse_point(f, 2, s, &inf);
  fixed_g1(s, inf, pk->delta1);
  parse_point(f, 4, s, &inf);
  fixed_g2(s, inf, pk->beta2);
  parse_point(f, 4, s, &inf);
  fixed_g2(s, inf, pk->gamma2);
  parse_point(f, 4, s, &inf);
  fixed_g2(s, inf, pk->delta2);
  int st = ZK_OK;
  auto count = [&](size_t& dst) {
    int32_t k = f.i32();
    if (!f.ok || k < 0 || k > (1 << 28)) {
      f.ok = false;
      return false;
    }
    dst = (size_t)k;
    return true;
  };
  // tau powers (not used by prove), then A, B1, B2, L, H
  if (count(pk->ntau1)) skip_query(f, false, pk->ntau1);
  if (f.ok && count(pk->ntau2)) skip_query(f, true, pk->ntau2);
  if (f.ok && count(pk->nA)) st = upload_query(ctx, f, false, pk->nA, &pk->A);
  if (st == ZK_OK && f.ok && count(pk->nB1)) st = upload_query(ctx, f, false, pk->nB1, &pk->B1);
  if (st == ZK_OK && f.ok && count(pk->nB2)) st = upload_query(ctx, f, true, pk->nB2, &pk->B2);
  if (st == ZK_OK && f.ok && count(pk->nL)) st = upload_query(ctx, f, false, pk->nL, &pk->L);
  if (st == ZK_OK && f.ok && count(pk->nH)) st = upload_query(ctx, f, false, pk->nH, &pk->H);
  if (st == ZK_OK && !f.ok) st = ctx->fail(ZK_ERR_IO, "proving key truncated or malformed");
  if (st == ZK_OK && ((int)pk->nA < pk->m || (int)pk->nB1 < pk->m || (int)pk->nB2 < pk->m))
    st = ctx->fail(ZK_ERR_IO, "incomplete proving key (A/B queries shorter than num_variables)");
  if (st == ZK_OK) st = pk_tables(ctx, pk);
  if (st != ZK_OK) {
    zk_pk_destroy(pk);
    return st;
  }
  *out = pk;
  return ZK_OK;
}

int zk_pk_load(zk_context* ctx, const char* path, zk_pk** out) {
  return zk::guard(ctx, [&] { return zk_pk_load_impl(ctx, path, out); });
}

void zk_pk_destroy(zk_pk* pk) {
  if (!pk) return;
  pk_drop_tables(pk);
  for (void* p : {pk->A, pk->B1, pk->B2, pk->L, pk->H})
    if (p) (void)hipFree(p);
  delete pk;
}

int zk_pk_info(const zk_pk* pk, int* n, int* m, int* npub) {
  if (!pk) return ZK_ERR_INVALID;
  if (n) *n = pk->n;
  if (m) *m = pk->m;
  if (npub) *npub = pk->npub;
  return ZK_OK;
}

// Host-to-device copy of a large host buffer (the witness) on st through
// pinned staging: UP_SLOTS slots of UP_CHUNK bytes, each chunk copied into
// its slot by UP_THREADS host threads (one stripe each) while the DMA engine
// moves the previous chunks.  A copy from pageable memory is staged by the
// calling thread alone (28 GB/s on the box for 128 MB, against 45-49 GB/s
// staged this way).  Returns once every chunk is enqueued on st.
constexpr size_t UP_CHUNK = 8u << 20;
constexpr int UP_SLOTS = 4;
constexpr int UP_THREADS = 4;
static int upload_staged(zk_context* ctx, void* d_dst, const void* h_src, size_t bytes, hipStream_t st) {
  if (bytes < 2 * UP_CHUNK) {
    ZK_HIP(ctx, hipMemcpyAsync(d_dst, h_src, bytes, hipMemcpyHostToDevice, st));
    return ZK_OK;
  }
  if (!ctx->h_stage) {
    for (auto& e : ctx->stage_ev)
      if (!e) ZK_HIP(ctx, hipEventCreateWithFlags(&e, hipEventDisableTiming));
    ZK_HIP(ctx, hipHostMalloc((void**)&ctx->h_stage, UP_CHUNK * UP_SLOTS, hipHostMallocDefault));
  }
  // the slots' last transfers (from an earlier upload) are done before reuse
  for (hipEvent_t e : ctx->stage_ev) ZK_HIP(ctx, hipEventSynchronize(e));
  const size_t K = (bytes + UP_CHUNK - 1) / UP_CHUNK;
  std::vector<std::atomic<int>> copied(K);
  for (auto& c : copied) c.store(0);
  std::atomic<long> writable{UP_SLOTS - 1};  // highest chunk whose slot may be filled
  std::atomic<bool> stop{false};
  const uint8_t* src = (const uint8_t*)h_src;
  auto worker = [&](int t) {
    for (size_t k = 0; k < K; k++) {
      while (writable.load(std::memory_order_acquire) < (long)k) {
        if (stop.load(std::memory_order_acquire)) return;
        std::this_thread::yield();
      }
      const size_t len = std::min(UP_CHUNK, bytes - k * UP_CHUNK);
      const size_t a = len * t / UP_THREADS, b = len * (t + 1) / UP_THREADS;
      memcpy(ctx->h_stage + (k % UP_SLOTS) * UP_CHUNK + a, src + k * UP_CHUNK + a, b - a);
      copied[k].fetch_add(1, std::memory_order_release);
    }
  };
  int rc = ZK_OK;
  {
    std::vector<std::thread> th;
    ThreadJoiner joiner{th};
    struct Stop {  // workers never wait on a chunk the loop below will not release
      std::atomic<bool>& s;
      ~Stop() { s.store(true, std::memory_order_release); }
    } stop_on_exit{stop};
    for (int t = 0; t < UP_THREADS; t++) th.emplace_back(worker, t);
    for (size_t k = 0; k < K && rc == ZK_OK; k++) {
      while (copied[k].load(std::memory_order_acquire) < UP_THREADS) std::this_thread::yield();
      const int s = (int)(k % UP_SLOTS);
      const size_t len = std::min(UP_CHUNK, bytes - k * UP_CHUNK);
      if (hipMemcpyAsync((uint8_t*)d_dst + k * UP_CHUNK, ctx->h_stage + s * UP_CHUNK, len, hipMemcpyHostToDevice,
                         st) != hipSuccess ||
          hipEventRecord(ctx->stage_ev[s], st) != hipSuccess) {
        rc = ctx->fail(ZK_ERR_HIP, "prove: witness upload");
        break;
      }
      // chunk k + 1 reuses the slot of chunk k + 1 - UP_SLOTS
      if (k + 1 < K && k + 1 >= (size_t)UP_SLOTS) {
        if (hipEventSynchronize(ctx->stage_ev[(k + 1) % UP_SLOTS]) != hipSuccess) {
          rc = ctx->fail(ZK_ERR_HIP, "prove: witness upload wait");
          break;
        }
        writable.store((long)k + 1, std::memory_order_release);
      }
    }
  }
  return rc;
}

static int zk_prove_impl(zk_context* ctx, const zk_pk* pk, const zk_r1cs* c, const void* h_witness, size_t m,
                         int num_public, uint64_t blind_seed, int check_witness, uint8_t proof_out[256],
                         double* timings) {
  if (!ctx || !pk || !c || !proof_out || (m && !h_witness)) return ZK_ERR_INVALID;
  // events: 0 start, 1 witness resident, 2 quotient done, 3 + 2j / 4 + 2j
  // start / end of MSM job j
  constexpr int NEV = 3 + 2 * ZK_JOBS;
// From a 2^21 domain on, the three-set G1 job holds its accumulation until
// the quotient is done: the quotient's transforms then get the CU slots
// they wait for beside the accumulations (2^22 proof 45.9 -> 45.0 ms).  At
// 2^16 every such gate lost (1.42 ms -> 1.53 ms gating the G1 job, 1.70 ms
// gating B2, 1.69 ms both; measured again with the current kernels: 1.27 ->
// 1.33 ms gating G1, 1.37 ms gating B2, 1.44 ms both), and so did holding the
// G1 accumulation until the G2 accumulation kernel had finished (1.33 -> 1.52
// ms; 2^20 9.09 -> 9.17 ms).
constexpr size_t GATE_G1_MIN_N = (size_t)1 << 21;
  hipEvent_t ev[NEV];
  for (auto& e : ev) ZK_HIP(ctx, hipEventCreate(&e));
  struct EvGuard {
    hipEvent_t* e;
    ~EvGuard() {
      for (int i = 0; i < NEV; i++) (void)hipEventDestroy(e[i]);
    }
  } guard{ev};
  hipStream_t st = ctx->stream;
  // preconditions (groth16.cu:665-697)
  if (m == 0) return ctx->fail(ZK_ERR_MISMATCH, "empty witness");
  if ((int)m != c->nv) return ctx->fail(ZK_ERR_MISMATCH, "witness size != circuit variables");
  if (num_public != pk->npub) return ctx->fail(ZK_ERR_MISMATCH, "witness public count != proving key");
  if ((size_t)(1 + pk->npub) > m) return ctx->fail(ZK_ERR_MISMATCH, "public inputs exceed witness");
  const size_t n = c->n;
  ZK_TRY(ctx->ensure(ctx->scratch_b, n * 32 * 6));  // A | B | C and the transforms' work space
  ZK_TRY(ctx->ensure(ctx->scratch_c, n * 32 + m * 32 + 64));
  // Streams: the context stream (witness upload, quotient, then the H MSM),
  // one for the G2 MSM and one for the G1 MSMs over the witness (A, B1 and
  // L as one multi-set MSM).  A process gets 4 hardware queues; streams
  // beyond that share a queue and their kernels then run strictly in order.
  constexpr int JOB_STREAMS = 2, S_G2 = 0, S_G1 = 1;
  for (int j = 0; j < JOB_STREAMS; j++)
    if (!ctx->job_stream[j]) ZK_HIP(ctx, hipStreamCreateWithFlags(&ctx->job_stream[j], hipStreamNonBlocking));
  for (int j = 0; j < ZK_JOBS; j++)
    if (!ctx->job_ws[j]) ctx->job_ws[j] = msm_workspace_new();
  // The quotient gate: jobs set here hold their accumulation until the
  // quotient is done, so that its transforms find CU slots.
  MsmGate quotient_done;
  quotient_done.ev = ev[2];
  struct GateUnset {  // after the jobs are joined: the gate lives on this stack
    zk_context* ctx;
    ~GateUnset() {
      for (int j = 0; j < ZK_JOBS; j++) msm_workspace_gate(ctx->job_ws[j], nullptr);
    }
  } gate_unset{ctx};
  struct GateRelease {  // before the jobs are joined, on every way out: no waiter is left waiting
    MsmGate& g;
    ~GateRelease() {
      int pending = 0;
      g.state.compare_exchange_strong(pending, 2);
    }
  };
  // idle workers spin while the proof runs (its jobs and per-set
  // combinations then start within a microsecond)
  WorkerPool::Hot hot_workers(ctx->pool);
  uint8_t* base = (uint8_t*)ctx->scratch_c.p;
  void* d_h = base;
  void* d_w = base + n * 32;
  uint32_t* d_bad = (uint32_t*)(base + n * 32 + m * 32);
  const auto t_start = std::chrono::steady_clock::now();
  ZK_HIP(ctx, hipEventRecord(ev[0], st));
  ZK_TRY(upload_staged(ctx, d_w, h_witness, m * 32, st));
  ZK_HIP(ctx, hipEventRecord(ev[1], st));
  // blinding factors (groth16.cu:708-718)
  std::mt19937_64 rng(blind_seed);
  Fr r = random_nonzero(rng);
  Fr s = random_nonzero(rng);
  // B2 and H come back as Jacobian words: they are only added to other
  // points before proof_to_words' one inversion
  uint64_t a_msm[8], b2_msm[24], l_msm[8], h_msm[12], b1_msm[8];
  memset(l_msm, 0, sizeof(l_msm));
  const size_t na = std::min(m, pk->nA);
  const size_t nb2 = std::min(m, pk->nB2);
  const long npriv_l = std::min<long>((long)pk->nL, (long)m - 1 - pk->npub);
  const size_t nh = std::min(n, pk->nH);
  const size_t nb1 = std::min(m, pk->nB1);
  // The five MSMs are independent (groth16.cu:776-827).  A, B1 and L multiply
  // slices of the witness, so they run as one three-set MSM sharing the digit
  // sort and the latency-bound combine and reduction; B2 (G2) runs beside it;
  // H follows the quotient on the context stream.  Each is driven from its
  // own host thread (the MSM reads bucket statistics back mid-way).
  // Job slots (timings): 0 A, 1 B2, 2 L, 3 H, 4 B1; A, L and B1 share one run.
  constexpr int JOB_G1 = 0, JOB_B2 = 1, JOB_H = 3;
  int rc_g1 = ZK_OK, rc_b2 = ZK_OK, rc_h = ZK_OK;
  // Assembly (groth16.cu:769-840): A = alpha1 + A_msm + r delta1,
  // B = beta2 + B2_msm + s delta2, C = L + H + s A + r (beta1 + B1_msm), the
  // last term only when B1 is not empty.  Split by what each part waits for:
  // pre_a = alpha1 + r delta1, pre_b = beta2 + s delta2 and
  // pre_c = s pre_a + r beta1 need no MSM and are computed on a host thread
  // while the GPU works; g1_tail = s A_msm + L + r B1_msm as soon as the G1
  // job returns; what is left after the last MSM is three additions and the
  // affine conversions.
  G1 pre_a = G1::inf(), pre_c = G1::inf(), g1_tail = G1::inf();
  G2 pre_b = G2::inf();
  int rc_pre = ZK_OK;
  auto precompute = [&] {
    pre_a = g1_from_words(pk->alpha1).add(g1_from_words(pk->delta1).mul(r));
    pre_b = g2_from_words(pk->beta2).add(g2_from_words(pk->delta2).mul(s));
    pre_c = pre_a.mul(s);
    if (nb1 > 0) pre_c = pre_c.add(g1_from_words(pk->beta1).mul(r));
  };
  auto record = [&](int slot, hipStream_t s, int& rc) {
    if (hipEventRecord(ev[slot], s) != hipSuccess && rc == ZK_OK) rc = ctx->fail(ZK_ERR_HIP, "prove: event record");
  };
  // Each job makes its own stream wait for the resident witness, on its own
  // thread: the call took ~17 us on the GPU hosts, and two of them on this
  // thread delayed the quotient by that much.
  auto wait_witness = [&](hipStream_t js, int& rc) {
    if (hipStreamWaitEvent(js, ev[1], 0) != hipSuccess && rc == ZK_OK) rc = ctx->fail(ZK_ERR_HIP, "prove: stream wait");
  };
  auto run_b2 = [&] {
    hipStream_t js = ctx->job_stream[S_G2];
    wait_witness(js, rc_b2);
    record(3 + 2 * JOB_B2, js, rc_b2);
    if (rc_b2 == ZK_OK && nb2 && pk->tB2)
      rc_b2 = msm_recs_tab(ctx, ctx->job_ws[JOB_B2], true, pk->tB2, pk->nB2, pk->tab_b2, d_w, nb2, b2_msm, js,
                           /*beside=*/true, /*jac_out=*/true);
    else if (rc_b2 == ZK_OK && nb2)
      rc_b2 = msm_recs_ws(ctx, ctx->job_ws[JOB_B2], true, pk->B2, d_w, nb2, b2_msm, js, /*beside=*/true,
                          /*jac_out=*/true);
    record(4 + 2 * JOB_B2, js, rc_b2);
  };
  auto run_g1 = [&] {
    hipStream_t js = ctx->job_stream[S_G1];
    wait_witness(js, rc_g1);
    record(3 + 2 * JOB_G1, js, rc_g1);
    const void* recs[3];
    size_t lo[3], cnt[3], rows[3];
    uint64_t* outs[3];
    int ns = 0;
    // the three sets run over their window tables when the key has them
    const bool tab = pk->tA != nullptr;
    auto add = [&](const void* r, const void* t, size_t nrows, size_t l, size_t k, uint64_t* o) {
      if (k == 0) return;  // empty set: the result stays the identity
      recs[ns] = tab ? t : r;
      rows[ns] = nrows;
      lo[ns] = l;
      cnt[ns] = k;
      outs[ns++] = o;
    };
    memset(a_msm, 0, sizeof(a_msm));
    memset(b1_msm, 0, sizeof(b1_msm));
    add(pk->A, pk->tA, pk->nA, 0, na, a_msm);
    add(pk->B1, pk->tB1, pk->nB1, 0, nb1, b1_msm);
    add(pk->L, pk->tL, pk->nL, 1 + (size_t)pk->npub, npriv_l > 0 ? (size_t)npriv_l : 0, l_msm);
    if (rc_g1 == ZK_OK && ns)
      rc_g1 = msm_g1_sets_ws(ctx, ctx->job_ws[JOB_G1], ns, recs, lo, cnt, d_w, m, outs, js, /*beside=*/true,
                             tab ? &pk->tab_w : nullptr, tab ? rows : nullptr);
    record(4 + 2 * JOB_G1, js, rc_g1);
    if (rc_g1 == ZK_OK) {
      const G1 sa_rb = nb1 > 0 ? G1::mul2(g1_from_words(a_msm), s, g1_from_words(b1_msm), r)
                               : g1_from_words(a_msm).mul(s);
      g1_tail = sa_rb.add(g1_from_words(l_msm));
    }
  };
  // Each job reports a C++ exception (a failed host allocation) as a status;
  // the joiner waits for the threads on every way out of this function.
  auto job = [&](const std::function<void()>& fn, int& rc) {
    return [&fn, &rc] {
      try {
        fn();
      } catch (...) {
        rc = ZK_ERR_OOM;
      }
    };
  };
  const std::function<void()> f_b2(run_b2), f_g1(run_g1), f_pre(precompute);
  if (n >= GATE_G1_MIN_N) msm_workspace_gate(ctx->job_ws[JOB_G1], &quotient_done);
  // The jobs run on the context's worker threads.  TaskJoiner finishes them
  // on every way out of this function (after GateRelease has opened the
  // gate: destructors run in reverse order).
  struct TaskJoiner {
    std::vector<WorkerPool::TaskRef> v;
    void join() {
      for (const WorkerPool::TaskRef& t : v) WorkerPool::finish(t);
    }
    ~TaskJoiner() { join(); }
  } joiner;
  GateRelease gate_release{quotient_done};
  const std::function<void()> jobs[3] = {job(f_b2, rc_b2), job(f_g1, rc_g1), job(f_pre, rc_pre)};
  // A job that no worker can take runs on this thread once the quotient is
  // enqueued and its gate is set: the gated G1 job waits for that gate, so
  // running it here first would wait forever.
  std::vector<const std::function<void()>*> inline_jobs;
  for (const std::function<void()>& fn : jobs) {
    WorkerPool::TaskRef t;
    try {
      t = ctx->pool.submit(fn, debug_thread_start_refused());
    } catch (...) {
      t = nullptr;
    }
    if (t) joiner.v.push_back(t);
    else inline_jobs.push_back(&fn);
  }
  int qrc = quotient_run(ctx, c, d_w, d_h, ctx->scratch_b.p, st, check_witness != 0, d_bad);
  // the check's count goes to pinned memory: the copy does not block this
  // thread, which goes on to enqueue H right behind the quotient
  if (qrc == ZK_OK && check_witness) {
    if (!ctx->h_flag && hipHostMalloc((void**)&ctx->h_flag, 4, hipHostMallocDefault) != hipSuccess)
      qrc = ctx->fail(ZK_ERR_OOM, "prove: pinned flag");
    if (qrc == ZK_OK && hipMemcpyAsync(ctx->h_flag, d_bad, 4, hipMemcpyDeviceToHost, st) != hipSuccess)
      qrc = ctx->fail(ZK_ERR_HIP, "prove: witness check read-back");
  }
  if (qrc == ZK_OK && hipEventRecord(ev[2], st) != hipSuccess) qrc = ctx->fail(ZK_ERR_HIP, "prove: event record");
  quotient_done.state.store(qrc == ZK_OK ? 1 : 2);
  for (const std::function<void()>* fn : inline_jobs) (*fn)();
  if (qrc == ZK_OK) {  // H after the quotient, same stream
    record(3 + 2 * JOB_H, st, rc_h);
    if (rc_h == ZK_OK && nh && pk->tH)
      rc_h = msm_recs_tab(ctx, ctx->job_ws[JOB_H], false, pk->tH, pk->nH, pk->tab_h, d_h, nh, h_msm, st,
                          /*beside=*/true, /*jac_out=*/true);
    else if (rc_h == ZK_OK && nh)
      rc_h = msm_recs_ws(ctx, ctx->job_ws[JOB_H], false, pk->H, d_h, nh, h_msm, st, /*beside=*/true,
                         /*jac_out=*/true);
    else if (!nh) memset(h_msm, 0, sizeof(h_msm));
    record(4 + 2 * JOB_H, st, rc_h);
  }
  joiner.join();
  ZK_TRY(qrc);
  ZK_TRY(rc_pre);
  if (check_witness) {
    ZK_HIP(ctx, hipStreamSynchronize(st));
    if (*ctx->h_flag) return ctx->fail(ZK_ERR_WITNESS, "witness does not satisfy the R1CS");
  }
  ZK_TRY(rc_b2);
  ZK_TRY(rc_g1);
  ZK_TRY(rc_h);
  // the rest of the assembly; an empty A, L, H or B1 set left its result at
  // the identity (all-zero words)
  const G1 A = pre_a.add(g1_from_words(a_msm));
  const G2 B = pre_b.add(nb2 > 0 ? g2_from_jac_words(b2_msm) : G2::inf());
  const G1 Cj = g1_tail.add(g1_from_jac_words(h_msm)).add(pre_c);
  uint64_t Aw[8], Bw[16], Cw[8];
  proof_to_words(A, B, Cj, Aw, Bw, Cw);
  // 256-byte serialization in standard form (groth16.cu:1058-1074)
  uint8_t* o = proof_out;
  auto put = [&](const uint64_t* mont) {
    uint64_t sdt[4];
    Fq::raw(mont).to_std(sdt);
    memcpy(o, sdt, 32);
    o += 32;
  };
  put(Aw);
  put(Aw + 4);
  put(Bw);
  put(Bw + 4);
  put(Bw + 8);
  put(Bw + 12);
  put(Cw);
  put(Cw + 4);
  // Every MSM job synchronized its stream before its host step; the context
  // stream still runs the quotient when H had nothing to do.
  if (hipStreamQuery(st) != hipSuccess) ZK_HIP(ctx, hipStreamSynchronize(st));
  if (timings) {
    // total by the host clock (no event round trip after the assembly); the
    // GPU phases from the events, all complete by now
    timings[0] = std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - t_start).count();
    auto elapsed = [](hipEvent_t a, hipEvent_t b) {
      float t = 0;
      if (hipEventElapsedTime(&t, a, b) != hipSuccess) {
        (void)hipEventSynchronize(b);
        if (hipEventElapsedTime(&t, a, b) != hipSuccess) t = 0;
      }
      return (double)t;
    };
    timings[1] = elapsed(ev[0], ev[2]);  // witness upload + quotient (+ check)
    // each MSM from its start to its result on the host (they overlap); A,
    // L and B1 are one run and report its time
    const int slot_of[ZK_JOBS] = {0, 1, 0, 3, 0};  // A, B (G2), L, H, B1
    double last = 0;
    for (int j = 0; j < ZK_JOBS; j++) {
      const int e = slot_of[j];
      timings[2 + j] = elapsed(ev[3 + 2 * e], ev[4 + 2 * e]);
      last = std::max(last, elapsed(ev[0], ev[4 + 2 * e]));
    }
    timings[7] = std::max(0.0, timings[0] - last);  // host assembly after the last MSM
  }
  return ZK_OK;
}

int zk_prove(zk_context* ctx, const zk_pk* pk, const zk_r1cs* c, const void* h_witness, size_t m, int num_public,
             uint64_t blind_seed, int check_witness, uint8_t proof_out[256], double* timings) {
  return zk::guard(ctx, [&] {
    return zk_prove_impl(ctx, pk, c, h_witness, m, num_public, blind_seed, check_witness, proof_out, timings);
  });
}

static int zk_setup_impl(zk_context* ctx, const zk_r1cs* c, uint64_t toxic_seed, const char* pk_path,
                         const char* vk_path) {
  if (!ctx || !c || !pk_path || !vk_path) return ZK_ERR_INVALID;
  const int log_n = c->log_n;
  const size_t n = c->n, m = c->nv;
  const int npub = c->npub;
  // toxic waste (groth16.cu:456-472)
  std::mt19937_64 rng(toxic_seed);
  Fr tau = random_nonzero(rng), alpha = random_nonzero(rng), beta = random_nonzero(rng);
  Fr gamma = random_nonzero(rng), delta = random_nonzero(rng);
  // Lagrange basis at tau and QAP columns (groth16.cu:97-189)
  static const uint64_t W28[4] = {0x636E735580D13D9CULL, 0xA22BF3742445FFD6ULL, 0x56452AC01EB203D8ULL,
                                  0x1860EF942963F9E7ULL};
  Fr w = Fr::raw(W28);
  for (int i = 0; i < 28 - log_n; i++) w = w.sqr();
  Fr tn = tau;
  for (int i = 0; i < log_n; i++) tn = tn.sqr();
  const Fr vanish = tn - Fr::one();
  Fr two_inv = Fr::from_u64(2).inv(), ninv = Fr::one();
  for (int i = 0; i < log_n; i++) ninv = ninv * two_inv;
  std::vector<Fr> Lt(n), den(n), pre(n);
  Fr wj = Fr::one();
  for (size_t j = 0; j < n; j++) {
    Lt[j] = vanish * wj * ninv;
    den[j] = tau - wj;
    wj = wj * w;
  }
  pre[0] = den[0];
  for (size_t i = 1; i < n; i++) pre[i] = pre[i - 1] * den[i];
  Fr ti = pre[n - 1].inv();
  for (size_t i = n - 1; i > 0; i--) {
    Fr di = pre[i - 1] * ti;
    ti = ti * den[i];
    Lt[i] = Lt[i] * di;
  }
  Lt[0] = Lt[0] * ti;
  std::vector<Fr> At(m, Fr::zero()), Bt(m, Fr::zero()), Ct(m, Fr::zero());
  std::vector<Fr>* cols[3] = {&At, &Bt, &Ct};
  for (int k = 0; k < 3; k++)
    for (const zk_sparse_entry& e : c->coo[k])
      if (e.row >= 0 && (size_t)e.row < n && e.col >= 0 && (size_t)e.col < m)
        (*cols[k])[e.col] = (*cols[k])[e.col] + Fr::raw(e.value) * Lt[e.row];
  Lt.clear();
  den.clear();
  pre.clear();
  // query scalars (groth16.cu:540-606)
  const Fr dinv = delta.inv(), ginv = gamma.inv();
  long l = (long)m - npub - 1;
  if (l < 0) l = 0;
  std::vector<Fr> ls((size_t)l);
  for (long i = 0; i < l; i++) {
    const size_t v = (size_t)i + 1 + npub;
    ls[i] = (beta * At[v] + alpha * Bt[v] + Ct[v]) * dinv;
  }
  std::vector<Fr> hs(n);
  Fr tp = vanish * dinv;
  for (size_t i = 0; i < n; i++) {
    hs[i] = tp;
    tp = tp * tau;
  }
  std::vector<Fr> ic(npub + 1);
  for (int i = 0; i <= npub; i++)
    ic[i] = (size_t)i < m ? (beta * At[i] + alpha * Bt[i] + Ct[i]) * ginv : Fr::zero();
  // group elements: fixed points on the host, queries on the device
  const G1 g1 = G1::affine(Fq::from_u64(1), Fq::from_u64(2));
  std::vector<uint64_t> gen2_std;
  ZK_TRY(gen_points_std(ctx, std::vector<Fr>{Fr::one()}, true, gen2_std));
  const G2 g2 = G2::affine(Fq2{Fq::from_std(&gen2_std[0]), Fq::from_std(&gen2_std[4])},
                           Fq2{Fq::from_std(&gen2_std[8]), Fq::from_std(&gen2_std[12])});
  std::vector<uint64_t> qa, qb1, qb2, ql, qh, qic;
  ZK_TRY(gen_points_std(ctx, At, false, qa));
  ZK_TRY(gen_points_std(ctx, Bt, false, qb1));
  ZK_TRY(gen_points_std(ctx, Bt, true, qb2));
  ZK_TRY(gen_points_std(ctx, ls, false, ql));
  ZK_TRY(gen_points_std(ctx, hs, false, qh));
  ZK_TRY(gen_points_std(ctx, ic, false, qic));
  // ZKMLPK3 (groth16.cu:1104-1188)
  Bytes pkb;
  const char magic[8] = {'Z', 'K', 'M', 'L', 'P', 'K', '3', 0};
  pkb.raw(magic, 8);
  pkb.u32(3);
  pkb.u32((uint32_t)n);
  pkb.u32((uint32_t)m);
  pkb.u32((uint32_t)npub);
  const G1 alpha1 = g1.mul(alpha), beta1 = g1.mul(beta), delta1 = g1.mul(delta);
  const G2 beta2 = g2.mul(beta), gamma2 = g2.mul(gamma), delta2 = g2.mul(delta);
  put_g1_rec(pkb, alpha1);
  put_g1_rec(pkb, beta1);
  put_g1_rec(pkb, delta1);
  put_g2_rec(pkb, beta2);
  put_g2_rec(pkb, gamma2);
  put_g2_rec(pkb, delta2);
  pkb.u32(0);  // tau powers in G1: empty
  pkb.u32(2);  // tau powers in G2: [G2, tau G2]
  put_g2_rec(pkb, g2);
  put_g2_rec(pkb, g2.mul(tau));
  pkb.u32((uint32_t)m);
  put_std_points(pkb, qa, m, 2);
  pkb.u32((uint32_t)m);
  put_std_points(pkb, qb1, m, 2);
  pkb.u32((uint32_t)m);
  put_std_points(pkb, qb2, m, 4);
  pkb.u32((uint32_t)l);
  put_std_points(pkb, ql, (size_t)l, 2);
  pkb.u32((uint32_t)n);
  put_std_points(pkb, qh, n, 2);
  if (!pkb.write(pk_path)) return ctx->fail(ZK_ERR_IO, "cannot write proving key", pk_path);
  // verification key (verifier.cu:103-148): no infinity flags
  Bytes vkb;
  vkb.u32((uint32_t)npub);
  auto put_aff_g1 = [&](const G1& p) {
    Fq x, y;
    p.to_affine(x, y);
    put_std(vkb, x);
    put_std(vkb, y);
  };
  auto put_aff_g2 = [&](const G2& p) {
    Fq2 x, y;
    p.to_affine(x, y);
    put_std(vkb, x.c0);
    put_std(vkb, x.c1);
    put_std(vkb, y.c0);
    put_std(vkb, y.c1);
  };
  put_aff_g1(alpha1);
  put_aff_g2(beta2);
  put_aff_g2(gamma2);
  put_aff_g2(delta2);
  vkb.u32((uint32_t)(npub + 1));
  for (int i = 0; i <= npub; i++) vkb.raw(&qic[(size_t)i * 8], 64);
  if (!vkb.write(vk_path)) return ctx->fail(ZK_ERR_IO, "cannot write verification key", vk_path);
  return ZK_OK;
}

int zk_setup(zk_context* ctx, const zk_r1cs* c, uint64_t toxic_seed, const char* pk_path, const char* vk_path) {
  return zk::guard(ctx, [&] { return zk_setup_impl(ctx, c, toxic_seed, pk_path, vk_path); });
}

}  // extern "C"
