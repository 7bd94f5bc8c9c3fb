// Radix sort of the MSM (window, bucket) keys with their point indices.
// rocPRIM onesweep with 8-bit digits, 1024 x 8 tiles and match-based ranking:
// 10% faster than rocPRIM's default configuration for 21-bit keys on gfx950
// (16.8 M pairs: 0.39 ms against 0.435 ms).
#include <cstring>
#include <rocprim/rocprim.hpp>

#include "zk_internal.hpp"

namespace zk {

using SortCfg = rocprim::radix_sort_config<
    rocprim::default_config, rocprim::default_config,
    rocprim::radix_sort_onesweep_config<rocprim::kernel_config<1024, 8>, rocprim::kernel_config<1024, 8>, 8,
                                        rocprim::block_radix_rank_algorithm::match>>;

int sort_pairs_u32(zk_context* ctx, DevBuf& tmp, const uint32_t* kin, uint32_t* kout, const uint32_t* vin,
                   uint32_t* vout, size_t n, unsigned end_bit, hipStream_t st) {
  size_t bytes = 0;
  ZK_HIP(ctx, rocprim::radix_sort_pairs<SortCfg>(nullptr, bytes, kin, kout, vin, vout, n, 0u, end_bit, st));
  ZK_TRY(ctx->ensure(tmp, bytes));
  ctx->tic("msm_sort", st);
  ZK_HIP(ctx, rocprim::radix_sort_pairs<SortCfg>(tmp.p, bytes, kin, kout, vin, vout, n, 0u, end_bit, st));
  ctx->toc(st);
  return ZK_OK;
}

}  // namespace zk
