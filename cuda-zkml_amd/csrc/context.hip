// Context, device memory and kernel-timing entry points of the C ABI.
#include <string.h>

#include <atomic>

#include "zk_internal.hpp"

using namespace zk;

namespace zk {
// Allocations left until the injected failure (0: none armed).
static std::atomic<int> g_fail_at{0};

hipError_t dev_malloc(void** p, size_t bytes) {
  int n = g_fail_at.load();
  while (n > 0) {
    if (g_fail_at.compare_exchange_weak(n, n - 1)) {
      if (n == 1) {
        *p = nullptr;
        return hipErrorOutOfMemory;
      }
      break;
    }
  }
  return hipMalloc(p, bytes);
}
}  // namespace zk

namespace zk {
// Host-thread starts left to refuse (0: none armed).
static std::atomic<int> g_fail_threads{0};

bool debug_thread_start_refused() {
  int n = g_fail_threads.load();
  while (n > 0)
    if (g_fail_threads.compare_exchange_weak(n, n - 1)) return true;
  return false;
}
}  // namespace zk

int zk_debug_fail_thread_start(int count) {
  if (count < 0) return ZK_ERR_INVALID;
  g_fail_threads.store(count);
  return ZK_OK;
}

int zk_debug_fail_device_alloc(int nth) {
  if (nth < 0) return ZK_ERR_INVALID;
  g_fail_at.store(nth);
  return ZK_OK;
}

int zk_context::ensure(DevBuf& b, size_t bytes) {
  if (b.bytes >= bytes) return ZK_OK;
  if (b.p) {
    (void)hipFree(b.p);
    b.p = nullptr;
    b.bytes = 0;
  }
  if (bytes == 0) return ZK_OK;
  if (dev_malloc(&b.p, bytes) != hipSuccess) {
    b.p = nullptr;
    return fail(ZK_ERR_OOM, "device allocation failed");
  }
  b.bytes = bytes;
  return ZK_OK;
}

zk::TimingToken zk_context::tic(const char* name, hipStream_t st) {
  zk::TimingToken t;
  if (!profiling || (!profile_only.empty() && profile_only != name)) return t;
  t.name = name;
  (void)hipEventCreate(&t.a);
  (void)hipEventCreate(&t.b);
  (void)hipEventRecord(t.a, st);
  return t;
}

void zk_context::toc(zk::TimingToken& t, hipStream_t st) {
  if (!t.name) return;
  (void)hipEventRecord(t.b, st);
  std::lock_guard<std::mutex> lk(mu);
  pending.push_back(zk::PendingTiming{t.name, t.a, t.b});
}

void zk_context::collect() {
  std::lock_guard<std::mutex> lk(mu);
  for (auto& t : pending) {
    (void)hipEventSynchronize(t.b);
    float ms = 0;
    (void)hipEventElapsedTime(&ms, t.a, t.b);
    KernelStat& k = stats[t.name];
    k.launches++;
    k.total_ms += ms;
    (void)hipEventDestroy(t.a);
    (void)hipEventDestroy(t.b);
  }
  pending.clear();
}

extern "C" {

int zk_create(int device, zk_context** out) {
  if (!out) return ZK_ERR_INVALID;
  *out = nullptr;
  int count = 0;
  if (hipGetDeviceCount(&count) != hipSuccess || count <= 0) return ZK_ERR_HIP;
  if (device < 0 || device >= count) return ZK_ERR_INVALID;
  if (hipSetDevice(device) != hipSuccess) return ZK_ERR_HIP;
  // device address of the no-allocation NTT's fixed scratch, once per
  // device with the device current; a failed lookup is recorded and only
  // zk_ntt_noalloc reports it
  (void)ntt_scratch_init(device);
  zk_context* ctx = new zk_context();
  ctx->device = device;
  if (hipStreamCreateWithFlags(&ctx->stream, hipStreamNonBlocking) != hipSuccess) {
    delete ctx;
    return ZK_ERR_HIP;
  }
  *out = ctx;
  return ZK_OK;
}

void zk_destroy(zk_context* ctx) {
  if (!ctx) return;
  (void)hipSetDevice(ctx->device);
  (void)hipStreamSynchronize(ctx->stream);
  ctx->collect();
  ntt_plans_free(ctx);
  if (ctx->msm_ws) msm_workspace_free(ctx->msm_ws);
  if (ctx->msm_ws_g2) msm_workspace_free(ctx->msm_ws_g2);
  for (int j = 0; j < ZK_JOBS; j++) {
    if (ctx->job_ws[j]) msm_workspace_free(ctx->job_ws[j]);
    if (ctx->job_stream[j]) (void)hipStreamDestroy(ctx->job_stream[j]);
  }
  for (DevBuf* b : {&ctx->scratch_a, &ctx->scratch_b, &ctx->scratch_c, &ctx->scratch_d})
    if (b->p) (void)hipFree(b->p);
  if (ctx->h_flag) (void)hipHostFree(ctx->h_flag);
  if (ctx->h_stage) (void)hipHostFree(ctx->h_stage);
  for (hipEvent_t e : ctx->stage_ev)
    if (e) (void)hipEventDestroy(e);
  if (ctx->g1_table) (void)hipFree(ctx->g1_table);
  if (ctx->g2_table) (void)hipFree(ctx->g2_table);
  (void)hipStreamDestroy(ctx->stream);
  delete ctx;
}

const char* zk_status_string(int status) {
  switch (status) {
    case ZK_OK: return "ok";
    case ZK_ERR_INVALID: return "invalid argument";
    case ZK_ERR_SIZE: return "size out of supported range";
    case ZK_ERR_OOM: return "out of memory";
    case ZK_ERR_HIP: return "HIP runtime error";
    case ZK_ERR_IO: return "file missing, truncated or malformed";
    case ZK_ERR_WITNESS: return "witness does not satisfy the constraint system";
    case ZK_ERR_MISMATCH: return "sizes of witness, key and circuit disagree";
    default: return "unknown status";
  }
}

const char* zk_last_error(const zk_context* ctx) { return ctx ? ctx->last_error.c_str() : "no context"; }

int zk_synchronize(zk_context* ctx) {
  if (!ctx) return ZK_ERR_INVALID;
  ZK_HIP(ctx, hipStreamSynchronize(ctx->stream));
  return ZK_OK;
}

void* zk_get_stream(zk_context* ctx) { return ctx ? (void*)ctx->stream : nullptr; }

int zk_dev_alloc(zk_context* ctx, size_t bytes, void** d_ptr) {
  if (!ctx || !d_ptr) return ZK_ERR_INVALID;
  *d_ptr = nullptr;
  if (bytes == 0) bytes = 1;
  if (hipMalloc(d_ptr, bytes) != hipSuccess) {
    *d_ptr = nullptr;
    return ctx->fail(ZK_ERR_OOM, "hipMalloc failed");
  }
  return ZK_OK;
}

int zk_dev_free(zk_context* ctx, void* d_ptr) {
  if (!ctx) return ZK_ERR_INVALID;
  if (d_ptr) ZK_HIP(ctx, hipFree(d_ptr));
  return ZK_OK;
}

int zk_memcpy_h2d(zk_context* ctx, void* d_dst, const void* h_src, size_t bytes) {
  if (!ctx || (!d_dst && bytes) || (!h_src && bytes)) return ZK_ERR_INVALID;
  if (!bytes) return ZK_OK;
  ZK_HIP(ctx, hipMemcpyAsync(d_dst, h_src, bytes, hipMemcpyHostToDevice, ctx->stream));
  ZK_HIP(ctx, hipStreamSynchronize(ctx->stream));
  return ZK_OK;
}

int zk_memcpy_d2h(zk_context* ctx, void* h_dst, const void* d_src, size_t bytes) {
  if (!ctx || (!d_src && bytes) || (!h_dst && bytes)) return ZK_ERR_INVALID;
  if (!bytes) return ZK_OK;
  ZK_HIP(ctx, hipMemcpyAsync(h_dst, d_src, bytes, hipMemcpyDeviceToHost, ctx->stream));
  ZK_HIP(ctx, hipStreamSynchronize(ctx->stream));
  return ZK_OK;
}

int zk_memcpy_d2d(zk_context* ctx, void* d_dst, const void* d_src, size_t bytes) {
  if (!ctx || (!d_src && bytes) || (!d_dst && bytes)) return ZK_ERR_INVALID;
  if (!bytes) return ZK_OK;
  ZK_HIP(ctx, hipMemcpyAsync(d_dst, d_src, bytes, hipMemcpyDeviceToDevice, ctx->stream));
  ZK_HIP(ctx, hipStreamSynchronize(ctx->stream));
  return ZK_OK;
}

int zk_set_profiling(zk_context* ctx, int enable) {
  if (!ctx) return ZK_ERR_INVALID;
  ctx->collect();
  ctx->profiling = enable != 0;
  return ZK_OK;
}

int zk_set_profiling_only(zk_context* ctx, const char* kernel) {
  if (!ctx) return ZK_ERR_INVALID;
  ctx->collect();
  ctx->profile_only = kernel ? kernel : "";
  return ZK_OK;
}

int zk_kernel_stats(zk_context* ctx, const char* kernel, uint64_t* launches, double* total_ms) {
  if (!ctx || !kernel) return ZK_ERR_INVALID;
  ctx->collect();
  auto it = ctx->stats.find(kernel);
  if (launches) *launches = it == ctx->stats.end() ? 0 : it->second.launches;
  if (total_ms) *total_ms = it == ctx->stats.end() ? 0 : it->second.total_ms;
  return ZK_OK;
}

int zk_reset_kernel_stats(zk_context* ctx) {
  if (!ctx) return ZK_ERR_INVALID;
  ctx->collect();
  ctx->stats.clear();
  return ZK_OK;
}

const char* zk_kernel_stats_names(zk_context* ctx) {
  if (!ctx) return "";
  ctx->collect();
  ctx->stat_names.clear();
  for (auto& kv : ctx->stats) {
    if (!ctx->stat_names.empty()) ctx->stat_names += ",";
    ctx->stat_names += kv.first;
  }
  return ctx->stat_names.c_str();
}

}  // extern "C"
