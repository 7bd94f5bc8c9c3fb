// Entry points not yet implemented in this build step.
#include "zk_internal.hpp"
extern "C" {
#define NI(ctx) ((ctx) ? (ctx)->fail(ZK_ERR_INVALID, "not implemented") : ZK_ERR_INVALID)
int zk_r1cs_create(zk_context* ctx, int, int, int, const zk_sparse_entry*, size_t, const zk_sparse_entry*, size_t,
                   const zk_sparse_entry*, size_t, zk_r1cs**) { return NI(ctx); }
void zk_r1cs_destroy(zk_r1cs*) {}
int zk_r1cs_domain(const zk_r1cs*, int*) { return ZK_ERR_INVALID; }
int zk_quotient_h(zk_context* ctx, const zk_r1cs*, const void*, size_t, void*, void*) { return NI(ctx); }
int zk_pk_load(zk_context* ctx, const char*, zk_pk**) { return NI(ctx); }
void zk_pk_destroy(zk_pk*) {}
int zk_pk_info(const zk_pk*, int*, int*, int*) { return ZK_ERR_INVALID; }
int zk_setup(zk_context* ctx, const zk_r1cs*, uint64_t, const char*, const char*) { return NI(ctx); }
int zk_prove(zk_context* ctx, const zk_pk*, const zk_r1cs*, const void*, size_t, int, uint64_t, int, uint8_t*,
             double*) { return NI(ctx); }
}
