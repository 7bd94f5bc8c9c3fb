/* zkml_gpu.h -- C ABI of the MI355X (gfx950) Groth16 prover core.
 *
 * Drop-in boundary for the data-parallel hot path of gdtsitlauri/cuda-zkml's
 * prover.  Every entry point names the reference interface it replaces
 * (paths relative to the reference root).  Plain pointers and sizes only.
 *
 * Data layouts are the reference's in-memory layouts:
 *   zk_fr, zk_fq      32 bytes: 4 x uint64 little endian, Montgomery form with
 *                     R = 2^256 (src/field/fp.cuh:28-31, 322-324).
 *   zk_g1_affine      64 bytes: x, y (zk_fq).  x = y = 0 encodes the point at
 *                     infinity (no finite curve point has x = y = 0).
 *   zk_g2_affine      128 bytes: x.c0, x.c1, y.c0, y.c1.
 *   reference structs G1Affine (72 bytes: x, y, bool infinity at byte 64) and
 *                     G2Affine (136 bytes, bool at byte 128) are accepted by the
 *                     *_host entry points (src/curve/g1.cuh:29-33, g2.cuh:25-29).
 *   zk_sparse_entry   40 bytes {int32 row; int32 col; zk_fr value}
 *                     (src/prover/circuit.cuh:32-36).
 *
 * Errors: every function returns ZK_OK (0) or a positive zk_status; the
 * reference instead exits the process on a device error (src/common.cuh:11-19).
 * zk_last_error() gives a message for the last failure on a context.
 *
 * Streams: `stream` arguments are hipStream_t values; NULL selects the
 * context's own stream.  Calls that return a host value synchronize.
 * A context is not re-entrant: one host thread per context at a time.
 * The NTT calls (zk_ntt, zk_coset_ntt, zk_quotient_h) of one context share
 * its pass-to-pass scratch buffer whatever stream they are given: two such
 * calls on different streams must not overlap (order the second stream after
 * the first with an event, or synchronize between them).  Twiddle and coset
 * tables are complete before a call returns, so they are safe on any stream.
 */
#ifndef ZKML_GPU_H
#define ZKML_GPU_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct zk_context zk_context;
typedef struct zk_r1cs zk_r1cs;
typedef struct zk_pk zk_pk;

enum zk_status {
  ZK_OK = 0,
  ZK_ERR_INVALID = 1,   /* bad argument */
  ZK_ERR_SIZE = 2,      /* size outside the supported range */
  ZK_ERR_OOM = 3,       /* device or host allocation failed */
  ZK_ERR_HIP = 4,       /* HIP runtime error */
  ZK_ERR_IO = 5,        /* file missing, truncated or malformed */
  ZK_ERR_WITNESS = 6,   /* witness does not satisfy the R1CS */
  ZK_ERR_MISMATCH = 7   /* witness / key / circuit sizes disagree */
};

typedef struct zk_sparse_entry {
  int32_t row;
  int32_t col;
  uint64_t value[4];
} zk_sparse_entry;

/* ---- context and device memory ---------------------------------------- */
int zk_create(int device, zk_context** out);
void zk_destroy(zk_context* ctx);
const char* zk_status_string(int status);
const char* zk_last_error(const zk_context* ctx);
int zk_synchronize(zk_context* ctx);
void* zk_get_stream(zk_context* ctx);
int zk_dev_alloc(zk_context* ctx, size_t bytes, void** d_ptr);
int zk_dev_free(zk_context* ctx, void* d_ptr);
int zk_memcpy_h2d(zk_context* ctx, void* d_dst, const void* h_src, size_t bytes);
int zk_memcpy_d2h(zk_context* ctx, void* h_dst, const void* d_src, size_t bytes);
int zk_memcpy_d2d(zk_context* ctx, void* d_dst, const void* d_src, size_t bytes);
/* Test hook, no counterpart in the reference: the nth device allocation
 * from now that the library makes for its own workspaces and NTT tables
 * (1 = the next one) fails with ZK_ERR_OOM, once; 0 disarms.  For tests of
 * the error paths only; affects every context of the process. */
int zk_debug_fail_device_alloc(int nth);
/* Test hook, no counterpart in the reference: the next `count` MSM jobs that
 * zk_prove would hand to the context's host worker threads are refused as if
 * no worker could be started, so the jobs run on the calling thread instead;
 * 0 disarms.  For tests of that fallback only; affects every context of the
 * process. */
int zk_debug_fail_thread_start(int count);

/* Per-kernel timing with HIP events recorded on the stream each kernel is
 * launched on (off by default).  Names: see zk_kernel_stats_names(). */
int zk_set_profiling(zk_context* ctx, int enable);
/* Time only the kernels of this name (NULL or "": all).  Each timed launch
 * adds two event records to its stream, so a throughput run times just the
 * kernel it reports. */
int zk_set_profiling_only(zk_context* ctx, const char* kernel);
int zk_kernel_stats(zk_context* ctx, const char* kernel, uint64_t* launches, double* total_ms);
int zk_reset_kernel_stats(zk_context* ctx);
const char* zk_kernel_stats_names(zk_context* ctx);

/* ---- NTT over Fr -------------------------------------------------------
 * Replaces bn254::ntt_gpu(Fr* d_out, const Fr* d_in, int log_n, bool inverse)
 * (src/ntt/ntt.cuh:49, src/ntt/ntt.cu:354-465) and ntt_gpu_inplace (:467).
 * out[j] = sum_i in[i] * w^(i*j), w = 5^((r-1)/2^28)^(2^(28-log_n)); the
 * inverse uses w^-1 and scales by n^-1.  Natural order in and out; d_out may
 * equal d_in.  1 <= log_n <= 24 (NTT_MAX_LOG, src/common.cuh:78); the reference
 * returns silently above that, this returns ZK_ERR_SIZE.  `batch` transforms
 * of n elements each are laid out back to back. */
int zk_ntt(zk_context* ctx, void* d_out, const void* d_in, int log_n, int inverse, int batch, void* stream);

/* No counterpart in the reference: zk_ntt for callers that cannot allocate
 * device memory (code under HIP graph capture, tight serving loops, harnesses
 * that forbid hipMalloc).  Same transform, layouts and stream argument as
 * zk_ntt, with 1 <= log_n <= 16 and batch * 2^log_n <= 2^18 elements; larger
 * sizes return ZK_ERR_SIZE.  Allocates nothing: its twiddle tables and
 * pass-to-pass buffer live in a fixed device array of the library (17 MB per
 * GPU, held from library load to process end) that every call on a GPU
 * shares.  Each log_n has its own table slot, filled by the first call of
 * that size; a call on a stream under graph capture records that fill into
 * the graph, so replays do not depend on the calls made between capture and
 * replay.  Calls that overlap on one GPU race on the pass-to-pass buffer:
 * order them on one stream or synchronize between them. */
int zk_ntt_noalloc(zk_context* ctx, void* d_out, const void* d_in, int log_n, int inverse, int batch, void* stream);

/* Coset NTT as used by Groth16Prover::compute_h (src/prover/groth16.cu:350-383):
 * forward: out = NTT(in[i] * g^i); inverse: out[i] = iNTT(in)[i] * g^-i.
 * g is a small plain integer (the prover uses 5; the coset tests also use 7). */
int zk_coset_ntt(zk_context* ctx, void* d_out, const void* d_in, int log_n, uint64_t g, int inverse, int batch,
                 void* stream);

/* ---- MSM ----------------------------------------------------------------
 * Replaces bn254::msm_g1 / msm_g2 (src/msm/msm.cuh:67-68, msm.cu:320-598):
 * result = sum_i scalars[i] * points[i].  Device-resident inputs (points in
 * zk_g1_affine / zk_g2_affine layout, scalars zk_fr), result written to host
 * memory as an affine point in the same layout (the reference returns a
 * Jacobian point whose callers convert it to affine).  n == 0 gives infinity;
 * n above 2^26 returns ZK_ERR_SIZE. */
int zk_msm_g1(zk_context* ctx, const void* d_points, const void* d_scalars, size_t n, void* h_result,
              void* stream);
int zk_msm_g2(zk_context* ctx, const void* d_points, const void* d_scalars, size_t n, void* h_result,
              void* stream);

/* MSMs over one base set, its conversion done once.  No counterpart in the
 * reference (bn254::msm_g1 / msm_g2 read affine points on every call); for
 * callers that run many MSMs over the same points.  zk_msm_prepare_points
 * writes the n points (zk_g1_affine, or zk_g2_affine when g2 != 0) as the
 * MSM's point records into d_recs, zk_msm_record_bytes(g2) bytes per point;
 * d_recs must not overlap d_points (ZK_ERR_INVALID).  zk_msm_g1_prepared /
 * zk_msm_g2_prepared then give the same result as zk_msm_g1 / zk_msm_g2 over
 * those points, without the per-call conversion; the records stay valid
 * while d_recs is unchanged. */
size_t zk_msm_record_bytes(int g2);
int zk_msm_prepare_points(zk_context* ctx, const void* d_points, size_t n, int g2, void* d_recs, void* stream);
int zk_msm_g1_prepared(zk_context* ctx, const void* d_recs, const void* d_scalars, size_t n, void* h_result,
                       void* stream);
int zk_msm_g2_prepared(zk_context* ctx, const void* d_recs, const void* d_scalars, size_t n, void* h_result,
                       void* stream);

/* Window configuration the MSM uses for n points (replaces
 * bn254::MSMConfig::for_size, src/msm/msm.cuh:40-64): window bits c (the
 * widest window) and the number of signed-digit windows.  CPU only. */
int zk_msm_config(size_t n, int g2, int* window_bits, int* windows);

/* KZG commitment over G1 (replaces KZGCommitment::commit / ::open,
 * src/prover/groth16.cuh:197-207, groth16.cu:393-438).  d_srs_g1: device
 * zk_g1_affine [tau^i]_1, i < degree; d_coeffs: device Fr (Montgomery), f_i
 * ascending, `degree` coefficients.  zk_kzg_commit writes sum f_i [tau^i]_1
 * (affine, as zk_msm_g1).  zk_kzg_open writes the opening proof
 * sum q_i [tau^i]_1 with q = (f - f(z)) / (x - z) (synthetic division on the
 * GPU; degree <= 1 gives infinity, as the reference) and, when f_z is not
 * NULL, f(z) (Montgomery Fr).  z: Montgomery Fr.  The verifier equation is
 * e(C - f(z) G1, G2) = e(proof, [tau]_2 - z G2). */
int zk_kzg_commit(zk_context* ctx, const void* d_srs_g1, const void* d_coeffs, size_t degree, void* h_commitment,
                  void* stream);
int zk_kzg_open(zk_context* ctx, const void* d_srs_g1, const void* d_coeffs, size_t degree, const uint64_t z[4],
                void* h_proof, uint64_t f_z[4], void* stream);

/* Host-pointer drop-ins with the reference's exact signature semantics:
 * h_points are reference G1Affine / G2Affine structs (72 / 136 bytes),
 * h_scalars are Fr, h_result receives a reference G1Jacobian / G2Jacobian
 * (96 / 192 bytes: x, y, z Montgomery; z = 1, or z = 0 for infinity). */
int zk_msm_g1_host(zk_context* ctx, const void* h_points, const void* h_scalars, int n, void* h_result_jacobian);
int zk_msm_g2_host(zk_context* ctx, const void* h_points, const void* h_scalars, int n, void* h_result_jacobian);

/* ---- fixed-base generation (setup and synthetic inputs) -----------------
 * d_out[i] = k[i] * G for the group generator G (G1 (1,2), G2 EIP-197:
 * src/curve/g1.cuh:40, g2.cuh:47-65); k in zk_fr layout (Montgomery). */
int zk_g1_generator_mul(zk_context* ctx, const void* d_scalars, size_t n, void* d_out, void* stream);
int zk_g2_generator_mul(zk_context* ctx, const void* d_scalars, size_t n, void* d_out, void* stream);

/* ---- R1CS and the quotient polynomial -----------------------------------
 * zk_r1cs_create uploads the reference's COO matrices (R1CS::A/B/C,
 * src/prover/circuit.cuh:39-50) once and keeps them on the device in CSR form.
 * zk_quotient_h replaces Groth16Prover::compute_h (groth16.cu:263-390):
 * h = (A.w * B.w - C.w) / (x^n - 1) via 3 iNTT, 3 coset NTT (shift 5, or 7
 * when 5^n = 1), a pointwise step and a coset iNTT, all resident on the
 * device.  d_h receives n = 2^ceil(log2(max(num_constraints, 4))) elements. */
int zk_r1cs_create(zk_context* ctx, int num_constraints, int num_variables, int num_public,
                   const zk_sparse_entry* A, size_t nA, const zk_sparse_entry* B, size_t nB,
                   const zk_sparse_entry* C, size_t nC, zk_r1cs** out);
void zk_r1cs_destroy(zk_r1cs* r1cs);
int zk_r1cs_domain(const zk_r1cs* r1cs, int* log_n);
int zk_quotient_h(zk_context* ctx, const zk_r1cs* r1cs, const void* d_witness, size_t m, void* d_h, void* stream);

/* ---- proving key, setup and prove ---------------------------------------
 * zk_pk_load replaces ProvingKey::load_streaming (groth16.cu:1190-1314): reads
 * a ZKMLPK3 file with the same checks and keeps all queries on the device.
 * For 2^14 .. 2^23 variables it also builds window tables of the queries (W
 * shifted copies of each, W = 13 to 20) that zk_prove's MSMs run on: device
 * memory grows by that factor (about 20 GB at 2^22) and the load takes longer
 * (1.5 s instead of 0.8 s at 2^22); proofs are the same bytes.
 * zk_setup replaces Groth16Prover::setup (groth16.cu:446-642) for a given
 * toxic-waste seed (the reference's deterministic seed is 0xDEADBEEF42) and
 * writes a ZKMLPK3 proving key and a verification key (verifier.cu:103-148).
 * zk_prove replaces Groth16Prover::prove (groth16.cu:655-920): r and s are the
 * first two nonzero Fr::from_uint(std::mt19937_64(blind_seed)()) draws (the
 * reference's deterministic seed is 0xCAFEBABE); the 256-byte proof is
 * A.x, A.y, B.x.c0, B.x.c1, B.y.c0, B.y.c1, C.x, C.y in standard form
 * (Groth16Proof::serialize, groth16.cu:1058-1074).  check_witness mirrors the
 * ZKML_SKIP_WITNESS_CHECK switch (groth16.cu:687-695).  The five MSMs run
 * concurrently on streams of the context (one host thread each).
 * timings_ms (optional, 8 doubles): total (host clock, from the witness
 * upload to the serialized proof), witness upload + quotient, then each
 * MSM's own duration (GPU events; they overlap): A, B(G2), L, H, B1, and the
 * host assembly after the last MSM. */
int zk_pk_load(zk_context* ctx, const char* path, zk_pk** out);
void zk_pk_destroy(zk_pk* pk);
int zk_pk_info(const zk_pk* pk, int* num_constraints, int* num_variables, int* num_public);
int zk_setup(zk_context* ctx, const zk_r1cs* r1cs, uint64_t toxic_seed, const char* pk_path, const char* vk_path);
int zk_prove(zk_context* ctx, const zk_pk* pk, const zk_r1cs* r1cs, const void* h_witness, size_t m,
             int num_public, uint64_t blind_seed, int check_witness, uint8_t proof_out[256], double* timings_ms);

/* ---- R1CS / witness files and the synthetic R1CS (host code) ------------
 * iden3 binary formats (circom / snarkjs): .r1cs version 1, .wtns version 2.
 * zk_iden3_r1cs_write replaces export_r1cs_iden3 and zk_wtns_write replaces
 * export_wtns_iden3 (src/prover/r1cs_export.cuh:41-92): same bytes for the
 * same R1CS (public wires as nPubOut, nPubIn = 0, identity label map).
 * Matrix values and witnesses are the reference's Montgomery Fr words; files
 * hold standard form.  Reading: zk_iden3_r1cs_info gives the sizes (public =
 * nPubOut + nPubIn), then zk_iden3_r1cs_read fills caller arrays of those
 * sizes; zk_wtns_info / zk_wtns_read likewise.
 * zk_synthetic_r1cs builds a large random R1CS (the shape of the 2^22-row
 * benchmark statement) from a seed: w[0] = 1, num_public + num_inputs uniform variables, then per row A and
 * B with 1-3 terms over earlier variables (uniform coefficients) and C = one
 * fresh variable set to (A.w)(B.w), so the witness satisfies every row.
 * Capacities: A, B 3 * num_constraints entries, C num_constraints, w_mont
 * 1 + num_public + num_inputs + num_constraints elements. */
int zk_iden3_r1cs_info(const char* path, int* num_constraints, int* num_variables, int* num_public,
                       int* num_private, size_t* nA, size_t* nB, size_t* nC);
int zk_iden3_r1cs_read(const char* path, zk_sparse_entry* A, zk_sparse_entry* B, zk_sparse_entry* C);
int zk_iden3_r1cs_write(const char* path, int num_constraints, int num_variables, int num_public, int num_private,
                        const zk_sparse_entry* A, size_t nA, const zk_sparse_entry* B, size_t nB,
                        const zk_sparse_entry* C, size_t nC);
int zk_wtns_info(const char* path, size_t* m);
int zk_wtns_read(const char* path, void* w_mont, size_t m);
int zk_wtns_write(const char* path, const void* w_mont, size_t m);
int zk_synthetic_r1cs(int num_constraints, int num_public, int num_inputs, uint64_t seed, zk_sparse_entry* A,
                      size_t* nA, zk_sparse_entry* B, size_t* nB, zk_sparse_entry* C, size_t* nC, void* w_mont);

/* ---- pairing and verification (host code, no device needed) -------------
 * zk_pairing replaces bn254::pairing (src/curve/pairing.cuh:198-282): the
 * reduced optimal ate pairing e(P, Q).  P: 64 bytes x, y; Q: 128 bytes x.c0,
 * x.c1, y.c0, y.c1; both standard form little endian, all-zero = infinity.
 * out: the Fp12 value as 12 x 32 bytes standard form in the reference's order
 * (c0.c0.c0, c0.c0.c1, c0.c1.c0, ..., c1.c2.c1).
 * zk_verify replaces Groth16Verifier::verify (groth16.cu:967-1022): vk_bytes
 * is a verification-key file image (verifier.cu:103-148), proof256 a proof
 * file image, publics npub x 32-byte standard-form scalars.  *valid = 1 when
 * e(-A, B) e(alpha, beta) e(vk_x, gamma) e(C, delta) == 1; a public-input
 * count other than the key's rejects (valid = 0, status ZK_OK), as in the
 * reference.  A and C must be on the curve and B on the twist and in the
 * order-r subgroup (the reference does not check; it would reject such
 * points only by chance).
 * zk_verify_files replaces zkml-verify's loading (src/cli/verify.cu): the
 * public-input file is .bin (i32 count + 32-byte scalars) or .json (decimal
 * list). */
int zk_pairing(const void* p_std, const void* q_std, void* out_std);
int zk_verify(const void* vk_bytes, size_t vk_len, const void* proof256, const void* publics_std, int npub,
              int* valid);
int zk_verify_files(const char* vk_path, const char* proof_path, const char* publics_path, int* valid);

/* ---- Poseidon (host code) -------------------------------------------------
 * BN254 Fr, t = 3, x^5, R_F = 8, R_P = 57: the circomlib instance of the
 * reference (src/prover/gadgets.cuh:323-427, poseidon_constants.cuh).  Values
 * cross as 4 x u64 standard form (inputs >= r are reduced mod r).
 * zk_poseidon_permute replaces poseidon_permute_native (state: 3 elements, in
 * place); zk_poseidon_hash2 replaces poseidon_hash2_native (= circomlib
 * Poseidon([a, b])); zk_poseidon_commit replaces poseidon_commit_native (rate-2
 * sponge, capacity (n << 64) | domain, output state[1]; domains "MODEL" =
 * 0x4d4f44454c and "INPUT" = 0x494e505554).  zk_poseidon_constants writes the
 * 195 round constants and the 3 x 3 MDS matrix (row major), either may be
 * NULL. */
int zk_poseidon_permute(uint64_t state[12]);
int zk_poseidon_hash2(const uint64_t a[4], const uint64_t b[4], uint64_t out[4]);
int zk_poseidon_commit(const uint64_t* values, size_t n, uint64_t domain, uint64_t out[4]);
int zk_poseidon_constants(uint64_t* round_constants, uint64_t* mds);

/* ---- statement producer (host code) ---------------------------------------
 * zk_statement_v2_build replaces build_statement_v2
 * (src/prover/statement_v2.cuh:82-253) with the TracedBuilder gadgets
 * (gadgets.cuh:128-457): one R1CS + witness for `batch` samples of a quantized
 * model, term for term the reference's (same variables, rows and term order).
 * Layers mirror NNModel::Layer (src/nn/inference.cuh:95-147); type values are
 * the reference's LayerType (src/nn/layers.cuh:36-43).  Model values and
 * inputs are signed integers (v -> v mod r; |v| >= 2^62 -> 0, as the
 * reference's Fp -> int64 conversion).  LINEAR: weights out_size x in_size row
 * major, bias out_size.  CONV2D: CHW, weights [out_c][in_c][kh][kw], bias
 * out_c; in_size / out_size are derived from the conv fields.  RELU_EXACT:
 * relu_bits in [1, 252], relu_shift in [0, 62].  RELU_APPROX: y = scale (c0 +
 * c1 x + c2 x^2 + c3 x^3).  SOFTMAX_APPROX only as the last layer (outside the
 * statement); SELF_ATTENTION is rejected.  inputs: batch x n_in.
 * Options mirror StatementV2Options (statement_v2.cuh:31-42); an all-zero
 * struct (or NULL) is the reference's default, compare_bits 0 meaning 48.
 * Field values are 4 x u64 standard form; input_blinding holds batch of them.
 * Errors: ZK_ERR_INVALID with the reference's message in err (err_cap bytes).
 * Results: zk_statement_info (sizes), zk_statement_r1cs (COO, Montgomery
 * values, caller arrays of nA / nB / nC entries), zk_statement_witness
 * (num_variables Montgomery Fr), zk_statement_layout (public-input layout,
 * ZK_LAYOUT_* indices; -1 for absent groups), zk_statement_scores (batch x
 * n_out final scores), zk_statement_check (R1CS::verify_witness,
 * src/prover/circuit.cuh:92-124: ZK_OK or ZK_ERR_WITNESS),
 * zk_statement_write (iden3 .r1cs / .wtns; either path may be NULL) and
 * zk_statement_meta_json (statement_v2_meta_json, statement_v2.cuh:255-287;
 * *len = length without the terminator, ZK_ERR_SIZE if cap is too small). */
enum zk_layer_type {
  ZK_LAYER_LINEAR = 0,
  ZK_LAYER_RELU_APPROX = 1,
  ZK_LAYER_SOFTMAX_APPROX = 2,
  ZK_LAYER_SELF_ATTENTION = 3,
  ZK_LAYER_RELU_EXACT = 4,
  ZK_LAYER_CONV2D = 5
};

typedef struct zk_layer {
  int32_t type;
  int32_t in_size, out_size;
  int32_t conv_in_c, conv_in_h, conv_in_w, conv_out_c, conv_kh, conv_kw, conv_stride, conv_pad;
  int32_t relu_bits, relu_shift;
  int64_t relu_c[4];
  int64_t relu_scale;
  const int64_t* weights;
  const int64_t* bias;
} zk_layer;

typedef struct zk_statement_options {
  uint64_t model_tag[4];
  int32_t has_context;
  uint64_t context[4];
  int32_t private_input;
  const uint64_t* input_blinding;
  int32_t private_model;
  int32_t private_outputs;
  int32_t route;
  int64_t route_threshold;
  int32_t compare_bits;
} zk_statement_options;

enum zk_statement_layout_index {
  ZK_LAYOUT_BATCH = 0,
  ZK_LAYOUT_N_IN,
  ZK_LAYOUT_N_OUT,
  ZK_LAYOUT_OUTPUTS_START,
  ZK_LAYOUT_MODEL_TAG,
  ZK_LAYOUT_CONTEXT,
  ZK_LAYOUT_MODEL_COMMITMENT,
  ZK_LAYOUT_INPUTS_START,
  ZK_LAYOUT_INPUT_SLOT,
  ZK_LAYOUT_ROUTE_START,
  ZK_LAYOUT_NUM_PUBLIC,
  ZK_STATEMENT_LAYOUT_WORDS
};

typedef struct zk_statement zk_statement;
int zk_statement_v2_build(const zk_layer* layers, int num_layers, const int64_t* inputs, int batch, int n_in,
                          const zk_statement_options* options, zk_statement** out, char* err, size_t err_cap);
void zk_statement_destroy(zk_statement* st);
int zk_statement_info(const zk_statement* st, int* num_constraints, int* num_variables, int* num_public,
                      int* num_private, size_t* nA, size_t* nB, size_t* nC);
int zk_statement_layout(const zk_statement* st, int32_t layout[ZK_STATEMENT_LAYOUT_WORDS]);
int zk_statement_r1cs(const zk_statement* st, zk_sparse_entry* A, zk_sparse_entry* B, zk_sparse_entry* C);
int zk_statement_witness(const zk_statement* st, void* w_mont);
int zk_statement_scores(const zk_statement* st, int64_t* scores);
int zk_statement_check(const zk_statement* st);
int zk_statement_write(const zk_statement* st, const char* r1cs_path, const char* wtns_path);
int zk_statement_meta_json(const zk_statement* st, uint64_t model_tag64, char* buf, size_t cap, size_t* len);

#ifdef __cplusplus
}
#endif
#endif /* ZKML_GPU_H */
