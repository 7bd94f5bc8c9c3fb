// Internal declarations shared by the HIP translation units of libzkml_gpu.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdio.h>

#include <atomic>
#include <map>
#include <memory>
#include <mutex>
#include <string>
#include <thread>
#include <vector>

#include "../../include/zkml_gpu.h"
#include "field.hpp"
#include "worker_pool.hpp"

namespace zk {

// Status carrier: functions return int status codes; ZK_TRY propagates.
#define ZK_TRY(expr)               \
  do {                             \
    int _st = (expr);              \
    if (_st != ZK_OK) return _st;  \
  } while (0)

// HIP error -> status with message on the context.
#define ZK_HIP(ctx, expr)                                                            \
  do {                                                                               \
    hipError_t _e = (expr);                                                          \
    if (_e != hipSuccess) return (ctx)->fail(ZK_ERR_HIP, #expr, hipGetErrorString(_e)); \
  } while (0)

struct DevBuf {
  void* p = nullptr;
  size_t bytes = 0;
};

// hipMalloc for the library's own device memory (workspaces, NTT plan and
// coset tables).  Fails without allocating while a test has armed
// zk_debug_fail_device_alloc.
hipError_t dev_malloc(void** p, size_t bytes);
// True when a test armed zk_debug_fail_thread_start and a refusal is left
// (consumes it): the caller then behaves as if std::thread had thrown.
bool debug_thread_start_refused();

struct NttPlan;
struct MsmWorkspace;

struct KernelStat {
  uint64_t launches = 0;
  double total_ms = 0;
};

struct PendingTiming {
  std::string name;
  hipEvent_t a, b;
};

// One kernel's timing bracket (events recorded on the launch stream).
struct TimingToken {
  const char* name = nullptr;
  hipEvent_t a = nullptr, b = nullptr;
};

// Concurrent MSM jobs of one proof: a stream and a workspace each.
constexpr int ZK_JOBS = 5;

}  // namespace zk

struct zk_context {
  int device = 0;
  hipStream_t stream = nullptr;
  std::string last_error;
  // NTT plans keyed by log_n; coset tables keyed by (log_n, g, inverse).
  std::map<int, zk::NttPlan*> ntt_plans;
  std::map<uint64_t, void*> coset_tables;
  zk::MsmWorkspace* msm_ws = nullptr;
  zk::MsmWorkspace* msm_ws_g2 = nullptr;
  zk::DevBuf scratch_a, scratch_b, scratch_c, scratch_d;
  // fixed-base tables for the generators (device), built on first use
  void* g1_table = nullptr;
  void* g2_table = nullptr;
  // streams and workspaces of the concurrent MSMs inside zk_prove
  hipStream_t job_stream[zk::ZK_JOBS] = {};
  zk::MsmWorkspace* job_ws[zk::ZK_JOBS] = {};
  uint32_t* h_flag = nullptr;  // pinned word: the proof's witness-check count
  // pinned staging slots of large host-to-device uploads (zk_prove's witness)
  uint8_t* h_stage = nullptr;
  hipEvent_t stage_ev[4] = {};
  // profiling
  bool profiling = false;
  std::string profile_only;  // when set, only kernels of this name are timed
  std::map<std::string, zk::KernelStat> stats;
  std::vector<zk::PendingTiming> pending;
  std::string stat_names;
  // guards last_error and pending: zk_prove runs MSMs from several threads
  std::mutex mu;
  // host workers of zk_prove's MSM jobs and the three-set MSM's per-set
  // window combination (started on first use, joined by zk_destroy)
  zk::WorkerPool pool{5};

  int fail(int code, const char* what, const char* detail = "") {
    std::lock_guard<std::mutex> lk(mu);
    last_error = std::string(what) + (detail && *detail ? std::string(": ") + detail : std::string());
    return code;
  }
  hipStream_t s(void* st) { return st ? (hipStream_t)st : stream; }
  int ensure(zk::DevBuf& b, size_t bytes);
  // Kernel timing brackets; no-ops unless profiling is enabled.
  zk::TimingToken tic(const char* name, hipStream_t st);
  void toc(zk::TimingToken& t, hipStream_t st);
  void collect();
};

namespace zk {

// Joins every thread of `v` on join() and when it goes out of scope, so no
// path out of a function leaves a joinable std::thread behind.
struct ThreadJoiner {
  std::vector<std::thread>& v;
  void join() {
    for (auto& t : v)
      if (t.joinable()) t.join();
  }
  ~ThreadJoiner() { join(); }
};

// Body of a C entry point: a C++ exception (a failed host allocation, mostly)
// becomes a status instead of crossing the C ABI.
template <class Fn>
int guard(zk_context* ctx, Fn&& fn) noexcept {
  int code = ZK_ERR_INVALID;
  const char* what = "internal error";
  try {
    return fn();
  } catch (const std::bad_alloc&) {
    code = ZK_ERR_OOM;
    what = "host allocation failed";
  } catch (...) {
  }
  if (ctx) {
    try {
      return ctx->fail(code, what);
    } catch (...) {
    }
  }
  return code;
}

// Issue priority of the quotient's kernels (sparse products, NTTs, pointwise
// step).  In a proof they run beside the G2 MSM's accumulation and the H MSM
// waits for them: their waves outrank the MSM waves sharing a SIMD.
__device__ __forceinline__ void quotient_priority() { __builtin_amdgcn_s_setprio(3); }

// Launch helper with error capture.
// The error state is cleared first: a handled failure earlier in the thread
// (an allocation that ran out of memory and was answered with a fallback or
// a status) must not read as this launch's failure.
#define ZK_LAUNCH(ctx, st, name, kernel, grid, block, shmem, ...)                            \
  do {                                                                                     \
    (void)hipGetLastError();                                                               \
    zk::TimingToken _tk = (ctx)->tic(name, st);                                            \
    hipLaunchKernelGGL(kernel, grid, block, shmem, st, __VA_ARGS__);                       \
    hipError_t _e = hipGetLastError();                                                     \
    if (_e != hipSuccess) return (ctx)->fail(ZK_ERR_HIP, name, hipGetErrorString(_e));    \
    (ctx)->toc(_tk, st);                                                                   \
  } while (0)

inline uint32_t cdiv(size_t a, size_t b) { return (uint32_t)((a + b - 1) / b); }

// ---- NTT (ntt.hip)
int ntt_run(zk_context* ctx, void* d_out, const void* d_in, int log_n, int inverse, int batch, uint64_t coset_g,
            hipStream_t st);
// Device address of the no-allocation NTT's fixed scratch on `device`
// (looked up once per device, with that device current).
int ntt_scratch_init(int device);
int ntt_run_noalloc(zk_context* ctx, void* d_out, const void* d_in, int log_n, int inverse, int batch,
                    hipStream_t st);
// The quotient's transforms (ntt.hip): abc = A | B | C evaluations on the
// domain (3n elements, destroyed), work: 3n elements; h receives the
// coefficients of (A B - C) / (x^n - 1) through the coset g H.
int quotient_ntts(zk_context* ctx, void* d_h, void* d_abc, void* d_work, int log_n, uint64_t g,
                  const uint64_t zinv_mont[4], hipStream_t st);
// Pointwise H step: h = (a*b - c) * zinv over n elements (ntt.hip)
int quotient_pointwise(zk_context* ctx, void* d_h, const void* d_a, const void* d_b, const void* d_c, size_t n,
                       const uint64_t zinv_mont[4], hipStream_t st);

// ---- MSM (msm.hip); results are canonical affine in the zk_g*_affine layout
constexpr size_t MSM_MAX_N = (size_t)1 << 26;  // largest MSM; keeps W * n_pad below 2^32
int msm_g1_run(zk_context* ctx, const void* d_points, const void* d_scalars, size_t n, uint64_t out_affine[8],
               hipStream_t st);
int msm_g2_run(zk_context* ctx, const void* d_points, const void* d_scalars, size_t n, uint64_t out_affine[16],
               hipStream_t st);
// MSM over prepared point records (proving-key queries stay in this form)
int msm_points_to_recs(zk_context* ctx, bool g2, const void* d_points, size_t n, void* d_recs, hipStream_t st);
int msm_g1_recs(zk_context* ctx, const void* d_recs, const void* d_scalars, size_t n, uint64_t out_affine[8],
                hipStream_t st);
int msm_g2_recs(zk_context* ctx, const void* d_recs, const void* d_scalars, size_t n, uint64_t out_affine[16],
                hipStream_t st);
int recs_from_std(zk_context* ctx, bool g2, void* d_recs, const void* d_std, const void* d_flags, size_t n,
                  hipStream_t st);
size_t rec_bytes(bool g2);
MsmWorkspace* msm_workspace_new();
void msm_workspace_free(MsmWorkspace* ws);
// Holds an MSM's accumulation until another stream's work is done (MSMs of
// one proof on different streams and host threads): the signalling thread
// records `ev` and then sets state 1, or sets 2 when it records nothing; the
// MSM waits on the host for a nonzero state and, for 1, makes its stream
// wait for `ev` before the accumulation.
struct MsmGate {
  std::atomic<int> state{0};
  hipEvent_t ev = nullptr;
};
// Gate of a workspace's next MSMs (null: none).
void msm_workspace_gate(MsmWorkspace* ws, MsmGate* wait_before_accumulate);
// MSM over records with an explicit workspace (one per concurrent caller).
// beside: the MSM shares the GPU with other kernels (a proof); the
// latency-bound combine and reduction then choose their lane layouts for a
// shared GPU.  out gets affine words x, y (8 words G1, 16 G2), or with
// jac_out Jacobian words x, y, z (12 / 24 words); all zeros at infinity.
int msm_recs_ws(zk_context* ctx, MsmWorkspace* ws, bool g2, const void* d_recs, const void* d_scalars, size_t n,
                uint64_t* out, hipStream_t st, bool beside = false, bool jac_out = false);
// Window tables of fixed bases (proving-key queries): for W digit windows
// (the widths of the MSM's window split of 254 bits) row w holds 2^(bits of
// the windows below w) P_j for every point; an MSM over a table has one
// bucket space for all windows, reduced in sub-windows of 2^log_sub buckets.
struct MsmTab {
  int W = 0;
  int log_sub = 0;
};
size_t msm_table_bytes(bool g2, size_t count, const MsmTab& t);
// Fills d_table (msm_table_bytes) from count point records on st; uses
// count * W * (point size) bytes of temporary device memory.
int msm_table_build(zk_context* ctx, bool g2, const void* d_recs, size_t count, const MsmTab& t, void* d_table,
                    hipStream_t st);
// G1 MSMs of up to 3 point sets over one scalar vector of n entries, sharing
// the digit sort and every latency-bound step: set k multiplies recs[k][j] by
// scalar lo[k] + j for j < count[k]; outs[k] gets its affine result.  With
// `tab`, recs[k] are window tables of rows[k] >= count[k] points per window.
int msm_g1_sets_ws(zk_context* ctx, MsmWorkspace* ws, int nsets, const void* const* recs, const size_t* lo,
                   const size_t* count, const void* d_scalars, size_t n, uint64_t* const* outs, hipStream_t st,
                   bool beside = false, const MsmTab* tab = nullptr, const size_t* rows = nullptr);
// msm_recs_ws over a window table of `rows` points per window (n <= rows).
int msm_recs_tab(zk_context* ctx, MsmWorkspace* ws, bool g2, const void* d_table, size_t rows, const MsmTab& tab,
                 const void* d_scalars, size_t n, uint64_t* out, hipStream_t st, bool beside = false,
                 bool jac_out = false);

// ---- fixed base (pointgen.hip)
int g1_generator_mul(zk_context* ctx, const void* d_scalars, size_t n, void* d_out, hipStream_t st);
int g2_generator_mul(zk_context* ctx, const void* d_scalars, size_t n, void* d_out, hipStream_t st);

void ntt_plans_free(zk_context* ctx);

}  // namespace zk
