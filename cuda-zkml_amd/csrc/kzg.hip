// KZG polynomial commitment over G1 for gfx950 (reference KZGCommitment,
// src/prover/groth16.cuh:188-207, groth16.cu:393-438):
//   commit(f)  = sum_i f_i [tau^i]_1                      (one G1 MSM)
//   open(f, z) = sum_i q_i [tau^i]_1,  q = (f - f(z)) / (x - z)
// with f given by its d coefficients (ascending) and q by synthetic division
//   q_{d-2} = f_{d-1},  q_i = f_{i+1} + z q_{i+1},
// i.e. q_i = sum_{j >= i} f_{j+1} z^(j-i): a suffix Horner scan, which the
// reference runs as a serial host loop.  Here it runs on the GPU as a blocked
// scan: every thread folds a chunk of KZG_L values from the top (local
// values and the chunk total), the chunk totals are scanned the same way
// with multiplier z^L (recursively, until one chunk is left), and a last pass
// adds z^(e-i) * q_e (q_e = scanned total of the next chunk) to every local
// value.  The map is linear, so it runs on the reference's Montgomery words
// directly (repack only) with z prepared in the internal radix.
#include <string.h>

#include "zk_internal.hpp"

namespace zk {

constexpr int KZG_L = 32;
constexpr int KZG_THREADS = 256;

struct ZPow {
  fr p[KZG_L + 1];  // p[k] = y^k in the internal radix, k = 0..L
};

__device__ __forceinline__ fr kzg_load(const uint4* __restrict__ p, size_t i) {
  uint4 a = p[2 * i], b = p[2 * i + 1];
  uint32_t w[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
  return repack_in<FrP>(w);
}

__device__ __forceinline__ void kzg_store(uint4* __restrict__ p, size_t i, const fr& x) {
  uint32_t w[8];
  repack_out(x, w);
  p[2 * i] = make_uint4(w[0], w[1], w[2], w[3]);
  p[2 * i + 1] = make_uint4(w[4], w[5], w[6], w[7]);
}

// Chunk c = [c L, min(n, (c + 1) L)): x_i <- sum_{i <= j < e} x_j y^(j-i) in
// place; tot[c] = the value at the chunk start.
__global__ __launch_bounds__(KZG_THREADS) void k_kzg_fold(uint4* __restrict__ x, size_t n, ZPow y,
                                                          uint4* __restrict__ tot) {
  const size_t c = blockIdx.x * (size_t)blockDim.x + threadIdx.x;
  const size_t s = c * KZG_L;
  if (s >= n) return;
  const size_t e = s + KZG_L < n ? s + KZG_L : n;
  fr acc = fe_zero<FrP>();
  for (size_t j = e; j-- > s;) {
    acc = fadd(kzg_load(x, j), fmul(acc, y.p[1]));
    kzg_store(x, j, acc);
  }
  kzg_store(tot, c, acc);
}

// x_i += y^(e-i) * tot[c + 1] for i in chunk c (tot holds the scanned chunk
// starts; the last chunk has no carry).
__global__ __launch_bounds__(KZG_THREADS) void k_kzg_carry(uint4* __restrict__ x, size_t n, ZPow y,
                                                           const uint4* __restrict__ tot) {
  const size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x;
  if (i >= n) return;
  const size_t c = i / KZG_L, e = (c + 1) * KZG_L;
  if (e >= n) return;
  const fr carry = kzg_load(tot, c + 1);
  kzg_store(x, i, fadd(kzg_load(x, i), fmul(carry, y.p[e - i])));
}

static ZPow zpow_table(const fr& y) {
  ZPow t;
  t.p[0] = fe_one<FrP>();
  for (int k = 1; k <= KZG_L; k++) t.p[k] = fmul(t.p[k - 1], y);
  return t;
}

// In-place suffix Horner scan of n raw Montgomery elements with multiplier y
// (internal radix); tot: scratch of at least n / (L - 1) + 8 elements.
static int suffix_horner(zk_context* ctx, uint4* x, size_t n, const fr& y, uint4* tot, hipStream_t st) {
  if (n == 0) return ZK_OK;
  const ZPow yp = zpow_table(y);
  const size_t m = (n + KZG_L - 1) / KZG_L;
  ZK_LAUNCH(ctx, st, "kzg_division", k_kzg_fold, dim3(cdiv(m, KZG_THREADS)), dim3(KZG_THREADS), 0, x, n, yp, tot);
  if (m == 1) return ZK_OK;  // one chunk: the fold is the whole scan
  ZK_TRY(suffix_horner(ctx, tot, m, yp.p[KZG_L], tot + 2 * m, st));
  ZK_LAUNCH(ctx, st, "kzg_division", k_kzg_carry, dim3(cdiv(n, KZG_THREADS)), dim3(KZG_THREADS), 0, x, n, yp, tot);
  return ZK_OK;
}

static size_t tot_capacity(size_t n) {
  size_t t = 0;
  while (n > 1) {
    n = (n + KZG_L - 1) / KZG_L;
    t += n;
  }
  return t + 1;
}

static fr fr_internal(const uint64_t mont[4]) {
  uint32_t w[8];
  memcpy(w, mont, 32);
  return from_mont256<FrP>(w);
}

}  // namespace zk

extern "C" {

static int zk_kzg_commit_impl(zk_context* ctx, const void* d_srs_g1, const void* d_coeffs, size_t degree,
                              void* h_commitment, void* stream) {
  if (!ctx || !h_commitment || (degree && (!d_srs_g1 || !d_coeffs))) return ZK_ERR_INVALID;
  return zk::msm_g1_run(ctx, d_srs_g1, d_coeffs, degree, (uint64_t*)h_commitment, ctx->s(stream));
}

int zk_kzg_commit(zk_context* ctx, const void* d_srs_g1, const void* d_coeffs, size_t degree, void* h_commitment,
                  void* stream) {
  return zk::guard(ctx, [&] { return zk_kzg_commit_impl(ctx, d_srs_g1, d_coeffs, degree, h_commitment, stream); });
}

static int zk_kzg_open_impl(zk_context* ctx, const void* d_srs_g1, const void* d_coeffs, size_t degree,
                            const uint64_t z[4], void* h_proof, uint64_t f_z[4], void* stream) {
  using namespace zk;
  if (!ctx || !h_proof || !z || (degree && (!d_srs_g1 || !d_coeffs))) return ZK_ERR_INVALID;
  if (degree > MSM_MAX_N + 1) return ctx->fail(ZK_ERR_SIZE, "kzg: degree above the MSM limit");
  hipStream_t st = ctx->s(stream);
  const uint64_t* zm = z;
  if (degree <= 1) {  // constant polynomial: the proof is the identity (groth16.cu:414-416)
    memset(h_proof, 0, 64);
    if (f_z) {
      memset(f_z, 0, 32);
      if (degree == 1) ZK_HIP(ctx, hipMemcpyAsync(f_z, d_coeffs, 32, hipMemcpyDeviceToHost, st));
      ZK_HIP(ctx, hipStreamSynchronize(st));
    }
    return ZK_OK;
  }
  const size_t nq = degree - 1;
  ZK_TRY(ctx->ensure(ctx->scratch_b, nq * 32));
  ZK_TRY(ctx->ensure(ctx->scratch_c, tot_capacity(nq) * 32 + 64));
  uint4* q = (uint4*)ctx->scratch_b.p;
  // q starts as f_1 .. f_{d-1}
  ZK_HIP(ctx, hipMemcpyAsync(q, (const uint8_t*)d_coeffs + 32, nq * 32, hipMemcpyDeviceToDevice, st));
  ZK_TRY(suffix_horner(ctx, q, nq, fr_internal(zm), (uint4*)ctx->scratch_c.p, st));
  if (f_z) {  // f(z) = f_0 + z q_0 (host, reference words)
    uint64_t w[8];
    ZK_HIP(ctx, hipMemcpyAsync(w, d_coeffs, 32, hipMemcpyDeviceToHost, st));
    ZK_HIP(ctx, hipMemcpyAsync(w + 4, q, 32, hipMemcpyDeviceToHost, st));
    ZK_HIP(ctx, hipStreamSynchronize(st));
    fr f0, q0;
    {
      uint32_t a[8], b[8];
      memcpy(a, w, 32);
      memcpy(b, w + 4, 32);
      f0 = repack_in<FrP>(a);
      q0 = repack_in<FrP>(b);
    }
    uint32_t out[8];
    repack_out(fadd(f0, fmul(q0, fr_internal(zm))), out);
    memcpy(f_z, out, 32);
  }
  return msm_g1_run(ctx, d_srs_g1, q, nq, (uint64_t*)h_proof, st);
}

int zk_kzg_open(zk_context* ctx, const void* d_srs_g1, const void* d_coeffs, size_t degree, const uint64_t z[4],
                void* h_proof, uint64_t f_z[4], void* stream) {
  return zk::guard(ctx, [&] { return zk_kzg_open_impl(ctx, d_srs_g1, d_coeffs, degree, z, h_proof, f_z, stream); });
}

}  // extern "C"
