// Fixed-base scalar multiplication k_i * G for the group generators: used by
// trusted setup (every proving-key query is a multiple of G1 or G2, reference
// src/prover/groth16.cu:519-606) and to build seeded synthetic MSM inputs
// P_i = k_i * G1.  Each thread adds one precomputed multiple per 8-bit window
// of k (32 mixed XYZZ additions) and converts its results to affine with one
// field inversion shared by PER points (Montgomery's trick).
#include <string.h>

#include <vector>

#include "curve.hpp"
#include "host_bn254.hpp"
#include "zk_internal.hpp"

namespace zk {

__device__ __forceinline__ void put_ext(uint32_t* o, const fq& a) { to_mont256(a, o); }
__device__ __forceinline__ void put_ext(uint32_t* o, const fq2& a) {
  to_mont256(a.c0, o);
  to_mont256(a.c1, o + 8);
}

template <class F>
__device__ __forceinline__ void load_tab(const uint32_t* __restrict__ tab, int idx, F& x, F& y);
template <>
__device__ __forceinline__ void load_tab<fq>(const uint32_t* __restrict__ tab, int idx, fq& x, fq& y) {
  const uint32_t* p = tab + (size_t)idx * 18;
#pragma unroll
  for (int i = 0; i < NL; i++) {
    x.l[i] = p[i];
    y.l[i] = p[NL + i];
  }
}
template <>
__device__ __forceinline__ void load_tab<fq2>(const uint32_t* __restrict__ tab, int idx, fq2& x, fq2& y) {
  const uint32_t* p = tab + (size_t)idx * 36;
#pragma unroll
  for (int i = 0; i < NL; i++) {
    x.c0.l[i] = p[i];
    x.c1.l[i] = p[NL + i];
    y.c0.l[i] = p[2 * NL + i];
    y.c1.l[i] = p[3 * NL + i];
  }
}

template <class F, int PG_PER>
__global__ __launch_bounds__(128) void k_fixed_base(uint32_t* __restrict__ out, const uint4* __restrict__ scalars,
                                                    size_t n, const uint32_t* __restrict__ tab) {
  const size_t base = (blockIdx.x * (size_t)blockDim.x + threadIdx.x) * PG_PER;
  if (base >= n) return;
  constexpr int EW = sizeof(F) / 36 * 8;  // external words per coordinate
  xyzz<F> acc[PG_PER];
  for (int j = 0; j < PG_PER; j++) {
    xyzz_set_inf(acc[j]);
    const size_t i = base + j;
    if (i >= n) continue;
    uint4 a = scalars[2 * i], b = scalars[2 * i + 1];
    uint32_t sm[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
    fr k32 = fe_zero<FrP>();
    k32.l[0] = 32;
    uint32_t s[8];
    repack_out(fmul(repack_in<FrP>(sm), k32), s);  // standard form
    for (int w = 0; w < 32; w++) {
      const uint32_t d = (s[w >> 2] >> (8 * (w & 3))) & 0xffu;
      if (!d) continue;
      F x, y;
      load_tab<F>(tab, w * 256 + (int)d, x, y);
      xyzz_madd(acc[j], x, y);
    }
  }
  F x[PG_PER], y[PG_PER];
  bool inf[PG_PER];
  xyzz_to_affine_batch<F, PG_PER>(acc, x, y, inf);
  for (int j = 0; j < PG_PER; j++) {
    const size_t i = base + j;
    uint32_t o[2 * EW];
    if (inf[j]) {
      for (int k = 0; k < 2 * EW; k++) o[k] = 0;
    } else {
      put_ext(o, x[j]);
      put_ext(o + EW, y[j]);
    }
    if (i < n)
      for (int k = 0; k < 2 * EW; k++) out[i * 2 * EW + k] = o[k];
  }
}

// ------------------------------------------------------------------ tables
template <class E>
static std::vector<zkh::Jac<E>> window_multiples(const zkh::Jac<E>& g) {
  std::vector<zkh::Jac<E>> t(32 * 256);
  zkh::Jac<E> base = g;
  for (int k = 0; k < 32; k++) {
    t[k * 256] = zkh::Jac<E>::inf();
    for (int d = 1; d < 256; d++) t[k * 256 + d] = t[k * 256 + d - 1].add(base);
    for (int i = 0; i < 8; i++) base = base.dbl();
  }
  return t;
}

static void fq_to_internal(const zkh::Fq& a, uint32_t* o) {
  uint32_t w[8];
  memcpy(w, a.v, 32);
  fq x = from_mont256<FqP>(w);
  fq c = fcanon(x);
  memcpy(o, c.l, NL * 4);
}

static zkh::G1 g1_gen() { return zkh::G1::affine(zkh::Fq::from_u64(1), zkh::Fq::from_u64(2)); }

static zkh::G2 g2_gen() {
  static const uint64_t X0[4] = {0x46debd5cd992f6edULL, 0x674322d4f75edaddULL, 0x426a00665e5c4479ULL,
                                 0x1800deef121f1e76ULL};
  static const uint64_t X1[4] = {0x97e485b7aef312c2ULL, 0xf1aa493335a9e712ULL, 0x7260bfb731fb5d25ULL,
                                 0x198e9393920d483aULL};
  static const uint64_t Y0[4] = {0x4ce6cc0166fa7daaULL, 0xe3d1e7690c43d37bULL, 0x4aab71808dcb408fULL,
                                 0x12c85ea5db8c6debULL};
  static const uint64_t Y1[4] = {0x55acdadcd122975bULL, 0xbc4b313370b38ef3ULL, 0xec9e99ad690c3395ULL,
                                 0x090689d0585ff075ULL};
  zkh::Fq2 x{zkh::Fq::from_std(X0), zkh::Fq::from_std(X1)}, y{zkh::Fq::from_std(Y0), zkh::Fq::from_std(Y1)};
  return zkh::G2::affine(x, y);
}

static int build_table_g1(zk_context* ctx) {
  if (ctx->g1_table) return ZK_OK;
  auto t = window_multiples(g1_gen());
  std::vector<uint32_t> host(32 * 256 * 18, 0);
  for (int i = 0; i < 32 * 256; i++) {
    zkh::Fq x, y;
    if (!t[i].to_affine(x, y)) continue;
    fq_to_internal(x, &host[(size_t)i * 18]);
    fq_to_internal(y, &host[(size_t)i * 18 + NL]);
  }
  ZK_HIP(ctx, hipMalloc(&ctx->g1_table, host.size() * 4));
  ZK_HIP(ctx, hipMemcpy(ctx->g1_table, host.data(), host.size() * 4, hipMemcpyHostToDevice));
  return ZK_OK;
}

static int build_table_g2(zk_context* ctx) {
  if (ctx->g2_table) return ZK_OK;
  auto t = window_multiples(g2_gen());
  std::vector<uint32_t> host(32 * 256 * 36, 0);
  for (int i = 0; i < 32 * 256; i++) {
    zkh::Fq2 x, y;
    if (!t[i].to_affine(x, y)) continue;
    uint32_t* o = &host[(size_t)i * 36];
    fq_to_internal(x.c0, o);
    fq_to_internal(x.c1, o + NL);
    fq_to_internal(y.c0, o + 2 * NL);
    fq_to_internal(y.c1, o + 3 * NL);
  }
  ZK_HIP(ctx, hipMalloc(&ctx->g2_table, host.size() * 4));
  ZK_HIP(ctx, hipMemcpy(ctx->g2_table, host.data(), host.size() * 4, hipMemcpyHostToDevice));
  return ZK_OK;
}

int g1_generator_mul(zk_context* ctx, const void* d_scalars, size_t n, void* d_out, hipStream_t st) {
  if (n == 0) return ZK_OK;
  if (!d_scalars || !d_out) return ctx->fail(ZK_ERR_INVALID, "generator_mul: null buffer");
  ZK_TRY(build_table_g1(ctx));
  constexpr int PER = 4;  // points per thread sharing one inversion
  const size_t threads = (n + PER - 1) / PER;
  ZK_LAUNCH(ctx, st, "fixed_base_g1", (k_fixed_base<fq, PER>), dim3(cdiv(threads, 128)), dim3(128), 0, (uint32_t*)d_out,
            (const uint4*)d_scalars, n, (const uint32_t*)ctx->g1_table);
  return ZK_OK;
}

int g2_generator_mul(zk_context* ctx, const void* d_scalars, size_t n, void* d_out, hipStream_t st) {
  if (n == 0) return ZK_OK;
  if (!d_scalars || !d_out) return ctx->fail(ZK_ERR_INVALID, "generator_mul: null buffer");
  ZK_TRY(build_table_g2(ctx));
  constexpr int PER = 1;
  const size_t threads = (n + PER - 1) / PER;
  ZK_LAUNCH(ctx, st, "fixed_base_g2", (k_fixed_base<fq2, PER>), dim3(cdiv(threads, 128)), dim3(128), 0, (uint32_t*)d_out,
            (const uint4*)d_scalars, n, (const uint32_t*)ctx->g2_table);
  return ZK_OK;
}

}  // namespace zk

extern "C" {

static int zk_g1_generator_mul_impl(zk_context* ctx, const void* d_scalars, size_t n, void* d_out, void* stream) {
  if (!ctx) return ZK_ERR_INVALID;
  return zk::g1_generator_mul(ctx, d_scalars, n, d_out, ctx->s(stream));
}

int zk_g1_generator_mul(zk_context* ctx, const void* d_scalars, size_t n, void* d_out, void* stream) {
  return zk::guard(ctx, [&] { return zk_g1_generator_mul_impl(ctx, d_scalars, n, d_out, stream); });
}

static int zk_g2_generator_mul_impl(zk_context* ctx, const void* d_scalars, size_t n, void* d_out, void* stream) {
  if (!ctx) return ZK_ERR_INVALID;
  return zk::g2_generator_mul(ctx, d_scalars, n, d_out, ctx->s(stream));
}

int zk_g2_generator_mul(zk_context* ctx, const void* d_scalars, size_t n, void* d_out, void* stream) {
  return zk::guard(ctx, [&] { return zk_g2_generator_mul_impl(ctx, d_scalars, n, d_out, stream); });
}

}  // extern "C"
