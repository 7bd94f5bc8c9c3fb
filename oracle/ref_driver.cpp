// TEST INFRASTRUCTURE ONLY -- thin C wrapper over the reference's own host
// code, compiled in place from /root/reference/src with the reference's own
// no-CUDA shim (tests/host/shim/cuda_runtime.h), into oracle/_ref/.  Nothing
// here is copied from the reference: it includes the reference headers and
// calls them.  Used by tests as a second, independent checker:
//   * the reference verifier (pairing check, src/curve/pairing.cuh:278-282,
//     with vk_x assembled as in src/prover/groth16.cu:967-1003) on artefact
//     files read by the reference's loaders (src/verifier/verifier.cu),
//   * the reference field and curve arithmetic (fp.cuh, fp2.cuh, g1.cuh,
//     g2.cuh -- G2 through its affine-inversion formulas).
#include <cstdint>
#include <cstring>
#include <random>
#include <string>
#include <vector>

#include "curve/pairing.cuh"
#include "prover/circuit.cuh"
#include "prover/r1cs_export.cuh"
#include "prover/statement_v2.cuh"
#include "verifier/verifier.cuh"

using namespace bn254;

static G1Affine in_g1(const uint64_t* o) {
  Fp x(o[0], o[1], o[2], o[3]), y(o[4], o[5], o[6], o[7]);
  if (x.is_zero() && y.is_zero()) return G1Affine();
  return G1Affine(x, y);
}
static void out_g1(const G1Affine& p, uint64_t* o) {
  if (p.infinity) {
    memset(o, 0, 64);
    return;
  }
  memcpy(o, p.x.val, 32);
  memcpy(o + 4, p.y.val, 32);
}
static G2Affine in_g2(const uint64_t* o) {
  Fp2 x(Fp(o[0], o[1], o[2], o[3]), Fp(o[4], o[5], o[6], o[7]));
  Fp2 y(Fp(o[8], o[9], o[10], o[11]), Fp(o[12], o[13], o[14], o[15]));
  if (x.is_zero() && y.is_zero()) return G2Affine();
  return G2Affine(x, y);
}
static void out_g2(const G2Affine& p, uint64_t* o) {
  if (p.infinity) {
    memset(o, 0, 128);
    return;
  }
  memcpy(o, p.x.c0.val, 32);
  memcpy(o + 4, p.x.c1.val, 32);
  memcpy(o + 8, p.y.c0.val, 32);
  memcpy(o + 12, p.y.c1.val, 32);
}

extern "C" {

int ref_abi_version() { return 1; }

void ref_fr_mul(const uint64_t* a, const uint64_t* b, uint64_t* o) { Fr::mont_mul_fr(o, a, b); }
void ref_fq_mul(const uint64_t* a, const uint64_t* b, uint64_t* o) { host_montgomery_mul(o, a, b); }
void ref_fr_inv(const uint64_t* a, uint64_t* o) {
  Fr r = Fr(a[0], a[1], a[2], a[3]).inv();
  memcpy(o, r.val, 32);
}
void ref_fq_from_std(const uint64_t* s, uint64_t* o) {
  Fp r = Fp::from_standard(s[0], s[1], s[2], s[3]);
  memcpy(o, r.val, 32);
}

void ref_g1_generator(uint64_t* o) { out_g1(G1Affine::generator(), o); }
void ref_g2_generator(uint64_t* o) { out_g2(G2Affine::generator(), o); }

void ref_g1_mul(const uint64_t* pt, const uint64_t* k, uint64_t* o) {
  Fr s(k[0], k[1], k[2], k[3]);
  out_g1(G1Jacobian::from_affine(in_g1(pt)).scalar_mul(s).to_affine(), o);
}
void ref_g2_mul(const uint64_t* pt, const uint64_t* k, uint64_t* o) {
  Fr s(k[0], k[1], k[2], k[3]);
  out_g2(G2Jacobian::from_affine(in_g2(pt)).scalar_mul(s).to_affine(), o);
}
void ref_g1_add(const uint64_t* a, const uint64_t* b, uint64_t* o) {
  out_g1((G1Jacobian::from_affine(in_g1(a)) + G1Jacobian::from_affine(in_g1(b))).to_affine(), o);
}
void ref_g2_add(const uint64_t* a, const uint64_t* b, uint64_t* o) {
  out_g2((G2Jacobian::from_affine(in_g2(a)) + G2Jacobian::from_affine(in_g2(b))).to_affine(), o);
}

// Sum of s_i * P_i by per-point double-and-add: the path the reference's
// msm_g1 takes for n <= 256 (src/msm/msm.cu:330-339, tests/test_msm.cu:20-28).
void ref_msm_g1_small(const uint64_t* pts, const uint64_t* sc, size_t n, uint64_t* o) {
  G1Jacobian acc = G1Jacobian::identity();
  for (size_t i = 0; i < n; i++) {
    Fr s(sc[4 * i], sc[4 * i + 1], sc[4 * i + 2], sc[4 * i + 3]);
    acc = acc + G1Jacobian::from_affine(in_g1(pts + 8 * i)).scalar_mul(s);
  }
  out_g1(acc.to_affine(), o);
}
void ref_msm_g2_small(const uint64_t* pts, const uint64_t* sc, size_t n, uint64_t* o) {
  G2Jacobian acc = G2Jacobian::identity();
  for (size_t i = 0; i < n; i++) {
    Fr s(sc[4 * i], sc[4 * i + 1], sc[4 * i + 2], sc[4 * i + 3]);
    acc = acc + G2Jacobian::from_affine(in_g2(pts + 16 * i)).scalar_mul(s);
  }
  out_g2(acc.to_affine(), o);
}

// Reduced optimal ate pairing with the reference's code (src/curve/pairing.cuh:
// 252-255).  p, q: Montgomery words as above; o: the Fp12 result as six Fp2
// (c0.c0, c0.c1, c0.c2, c1.c0, c1.c1, c1.c2), each c0 then c1, Montgomery words.
void ref_pairing(const uint64_t* p, const uint64_t* q, uint64_t* o) {
  Fp12 f = pairing(in_g1(p), in_g2(q));
  const Fp2* c[6] = {&f.c0.c0, &f.c0.c1, &f.c0.c2, &f.c1.c0, &f.c1.c1, &f.c1.c2};
  for (int i = 0; i < 6; i++) {
    memcpy(o + 8 * i, c[i]->c0.val, 32);
    memcpy(o + 8 * i + 4, c[i]->c1.val, 32);
  }
}

// Groth16 verification of artefact files with the reference's loaders and
// pairing.  Returns 1 valid, 0 invalid, -1 on a load error.
int ref_verify_files(const char* vk_path, const char* proof_path, const char* pub_path) {
  zkml::VerificationKey vk = zkml::load_vk(vk_path);
  if (vk.ic.empty()) return -1;
  zkml::Groth16Proof proof = zkml::load_proof(proof_path);
  if (!proof.valid) return -1;
  std::vector<Fr> pub = zkml::load_public_inputs(pub_path);
  if ((int)pub.size() != vk.num_public) return 0;
  G1Jacobian vk_x = G1Jacobian::from_affine(vk.ic[0]);
  for (int i = 0; i < (int)pub.size(); i++)
    if (i + 1 < (int)vk.ic.size()) vk_x = vk_x + G1Jacobian::from_affine(vk.ic[i + 1]).scalar_mul(pub[i]);
  G1Affine negA(proof.A.x, -proof.A.y);
  G1Affine P[4] = {negA, vk.alpha_g1, vk_x.to_affine(), proof.C};
  G2Affine Q[4] = {proof.B, vk.beta_g2, vk.gamma_g2, vk.delta_g2};
  return verify_pairing_product(P, Q, 4) ? 1 : 0;
}

// R1CS satisfaction with the reference's own checker (src/prover/circuit.cuh:93-124).
int ref_verify_witness(int nc, int nv, const int32_t* rows, const int32_t* cols, const uint64_t* vals,
                       const size_t* counts, const uint64_t* w) {
  zkml::R1CS c;
  c.num_constraints = nc;
  c.num_variables = nv;
  size_t off = 0;
  for (int which = 0; which < 3; which++) {
    std::vector<zkml::SparseEntry>& v = which == 0 ? c.A : (which == 1 ? c.B : c.C);
    for (size_t i = 0; i < counts[which]; i++, off++)
      v.push_back({rows[off], cols[off], Fr(vals[4 * off], vals[4 * off + 1], vals[4 * off + 2], vals[4 * off + 3])});
  }
  std::vector<Fr> wv(nv);
  for (int i = 0; i < nv; i++) wv[i] = Fr(w[4 * i], w[4 * i + 1], w[4 * i + 2], w[4 * i + 3]);
  return c.verify_witness(wv) ? 1 : 0;
}

// ------------------------------------------------------------------ statements
// BASELINE config 4's 62.7 k-constraint statement: the reference's tiny CNN
// (tests/host/test_statement_v2.cpp:28-43) as statement variant B (:129-137):
// private model (Poseidon commitment), private inputs, private outputs and
// in-circuit routing, batch of two.  Writes iden3 .r1cs/.wtns with the
// reference's exporters; info = {constraints, variables, public}.
static zkml::NNModel tiny_cnn_model() {
  using namespace zkml;
  NNModel m;
  Conv2DParams c;
  c.in_c = 1; c.in_h = 6; c.in_w = 6; c.out_c = 2; c.kh = 3; c.kw = 3; c.stride = 1; c.pad = 1;
  m.layers.push_back(NNModel::make_conv2d_layer(c));
  m.layers.push_back(NNModel::make_relu_exact_layer(c.out_size(), 24, 2));
  m.layers.push_back(NNModel::make_linear_layer(c.out_size(), 4));
  m.layers.push_back(NNModel::make_softmax_layer(4));
  auto& conv = m.layers[0];
  for (size_t i = 0; i < conv.weights.size(); i++) conv.weights[i] = i64_to_fp((int64_t)((i * 5) % 7) - 3);
  conv.bias[0] = i64_to_fp(4);
  conv.bias[1] = i64_to_fp(-2);
  auto& lin = m.layers[2];
  for (size_t i = 0; i < lin.weights.size(); i++) lin.weights[i] = i64_to_fp((int64_t)((i * 3) % 9) - 4);
  for (size_t i = 0; i < lin.bias.size(); i++) lin.bias[i] = i64_to_fp((int64_t)i - 1);
  return m;
}

static int emit_statement(const zkml::StatementV2& st, const char* r1cs_path, const char* wtns_path, int* info) {
  if (!st.r1cs.verify_witness(st.witness.values)) return -2;
  if (!zkml::export_r1cs_iden3(st.r1cs, r1cs_path) || !zkml::export_wtns_iden3(st.witness.values, wtns_path))
    return -3;
  info[0] = st.r1cs.num_constraints;
  info[1] = st.r1cs.num_variables;
  info[2] = st.layout.num_public;
  return 0;
}

int ref_statement_tiny_cnn_b(const char* r1cs_path, const char* wtns_path, int* info) {
  using namespace zkml;
  NNModel m = tiny_cnn_model();
  std::vector<std::vector<Fp>> batch(2, std::vector<Fp>(36));
  for (int i = 0; i < 36; i++) {
    batch[0][(size_t)i] = i64_to_fp((i * 7) % 13 - 4);
    batch[1][(size_t)i] = i64_to_fp((i * 11) % 17 - 8);
  }
  StatementV2Options bo;
  bo.model_tag = Fr::from_uint(0xC0FFEE);
  bo.private_input = true;
  bo.input_blinding = {Fr::from_uint(0x5EED1), Fr::from_uint(0x5EED2)};
  bo.private_model = true;
  bo.private_outputs = true;
  bo.route = true;
  bo.route_threshold = 5;
  StatementV2 sb;
  std::string err;
  if (!build_statement_v2(m, batch, bo, sb, err)) return -1;
  return emit_statement(sb, r1cs_path, wtns_path, info);
}

// seeded quantized MLP n_in -> hidden -> n_out with int8
// weights U[-127, 127], int32 biases, uint8 inputs U[0, 16] and RELU_EXACT
// (bits, shift) between the layers; public model, inputs and outputs
// (statement v2 defaults), `batch` samples.
int ref_statement_mlp(uint64_t seed, int batch, int n_in, int hidden, int n_out, int bits, int shift,
                      const char* r1cs_path, const char* wtns_path, int* info) {
  using namespace zkml;
  std::mt19937_64 rng(seed);
  NNModel m;
  m.layers.push_back(NNModel::make_linear_layer(n_in, hidden));
  m.layers.push_back(NNModel::make_relu_exact_layer(hidden, bits, shift));
  m.layers.push_back(NNModel::make_linear_layer(hidden, n_out));
  m.layers.push_back(NNModel::make_softmax_layer(n_out));
  for (size_t li : {(size_t)0, (size_t)2}) {
    for (auto& w : m.layers[li].weights) w = i64_to_fp((int64_t)(rng() % 255) - 127);
    for (auto& b : m.layers[li].bias) b = i64_to_fp((int64_t)(int32_t)(uint32_t)rng());
  }
  std::vector<std::vector<Fp>> xs((size_t)batch, std::vector<Fp>((size_t)n_in));
  for (auto& x : xs)
    for (auto& v : x) v = i64_to_fp((int64_t)(rng() % 17));
  StatementV2Options opt;
  StatementV2 st;
  std::string err;
  if (!build_statement_v2(m, xs, opt, st, err)) return -1;
  return emit_statement(st, r1cs_path, wtns_path, info);
}

// The reference's Poseidon table (src/prover/poseidon_constants.cuh), standard
// form: 195 round constants, then the 3 x 3 MDS matrix row major.
void ref_poseidon_constants(uint64_t* rc, uint64_t* mds) {
  using namespace zkml::poseidon_bn254;
  for (int i = 0; i < (RF + RP) * T; i++) memcpy(rc + 4 * i, ROUND_CONSTANTS[i], 32);
  for (int i = 0; i < 3; i++)
    for (int j = 0; j < 3; j++) memcpy(mds + 4 * (3 * i + j), MDS[i][j], 32);
}

// Any statement v2 through the reference builder, for parity sweeps.
// layer_ints: n_layers x 13 {type, in_size, out_size, conv in_c, in_h, in_w,
// out_c, kh, kw, stride, pad, relu bits, relu shift}; relu_params: n_layers x 5
// {c0, c1, c2, c3, scale} (RELU_APPROX); weights / biases: per layer (LINEAR,
// CONV2D).  opt_words: model_tag[4], context[4] standard form; opt_flags:
// {has_context, private_input, private_model, private_outputs, route,
// compare_bits}; blinding: batch x 4 standard form.  Writes the iden3 files
// and the metadata JSON (or the error message) into text; info = {constraints,
// variables, public, witness satisfies}.  Returns 0, or -1 when the builder
// rejects the statement.
int ref_statement_generic(int n_layers, const int32_t* layer_ints, const int64_t* relu_params,
                          const int64_t* const* weights, const int64_t* const* biases, const int64_t* inputs,
                          int batch, int n_in, const uint64_t* opt_words, const int32_t* opt_flags,
                          int64_t route_threshold, const uint64_t* blinding, uint64_t tag64, const char* r1cs_path,
                          const char* wtns_path, int* info, char* text, size_t text_cap) {
  using namespace zkml;
  NNModel m;
  for (int i = 0; i < n_layers; i++) {
    const int32_t* L = layer_ints + 13 * i;
    const int64_t* rp = relu_params + 5 * i;
    NNModel::Layer layer;
    switch ((LayerType)L[0]) {
      case LayerType::LINEAR: layer = NNModel::make_linear_layer(L[1], L[2]); break;
      case LayerType::CONV2D: {
        Conv2DParams c;
        c.in_c = L[3]; c.in_h = L[4]; c.in_w = L[5]; c.out_c = L[6];
        c.kh = L[7]; c.kw = L[8]; c.stride = L[9]; c.pad = L[10];
        layer = NNModel::make_conv2d_layer(c);
        break;
      }
      case LayerType::RELU_EXACT: layer = NNModel::make_relu_exact_layer(L[1], L[11], L[12]); break;
      case LayerType::RELU_APPROX:
        layer = NNModel::make_relu_layer(L[1]);
        layer.relu_params.c0 = i64_to_fp(rp[0]);
        layer.relu_params.c1 = i64_to_fp(rp[1]);
        layer.relu_params.c2 = i64_to_fp(rp[2]);
        layer.relu_params.c3 = i64_to_fp(rp[3]);
        layer.relu_params.scale = i64_to_fp(rp[4]);
        break;
      case LayerType::SOFTMAX_APPROX: layer = NNModel::make_softmax_layer(L[1]); break;
      default: layer.type = (LayerType)L[0]; layer.in_size = L[1]; layer.out_size = L[2]; break;
    }
    for (size_t k = 0; k < layer.weights.size(); k++) layer.weights[k] = i64_to_fp(weights[i][k]);
    for (size_t k = 0; k < layer.bias.size(); k++) layer.bias[k] = i64_to_fp(biases[i][k]);
    m.layers.push_back(layer);
  }
  std::vector<std::vector<Fp>> xs((size_t)batch, std::vector<Fp>((size_t)n_in));
  for (int b = 0; b < batch; b++)
    for (int i = 0; i < n_in; i++) xs[(size_t)b][(size_t)i] = i64_to_fp(inputs[(size_t)b * n_in + i]);
  StatementV2Options o;
  o.model_tag = fr_from_limbs(opt_words);
  o.has_context = opt_flags[0] != 0;
  o.context = fr_from_limbs(opt_words + 4);
  o.private_input = opt_flags[1] != 0;
  if (o.private_input && blinding)
    for (int b = 0; b < batch; b++) o.input_blinding.push_back(fr_from_limbs(blinding + 4 * b));
  o.private_model = opt_flags[2] != 0;
  o.private_outputs = opt_flags[3] != 0;
  o.route = opt_flags[4] != 0;
  o.route_threshold = route_threshold;
  o.compare_bits = opt_flags[5];
  StatementV2 st;
  std::string err;
  auto put_text = [&](const std::string& s) {
    if (text && text_cap) {
      size_t k = s.size() < text_cap - 1 ? s.size() : text_cap - 1;
      memcpy(text, s.data(), k);
      text[k] = 0;
    }
  };
  if (!build_statement_v2(m, xs, o, st, err)) {
    put_text(err);
    return -1;
  }
  info[0] = st.r1cs.num_constraints;
  info[1] = st.r1cs.num_variables;
  info[2] = st.layout.num_public;
  info[3] = st.r1cs.verify_witness(st.witness.values) ? 1 : 0;
  if (!export_r1cs_iden3(st.r1cs, r1cs_path) || !export_wtns_iden3(st.witness.values, wtns_path)) return -3;
  put_text(statement_v2_meta_json(st, o, tag64));
  return 0;
}

// iden3 exports with the reference's writers (src/prover/r1cs_export.cuh:41-92).
int ref_export_r1cs(int nc, int nv, int npub, int npriv, const int32_t* rows, const int32_t* cols,
                    const uint64_t* vals, const size_t* counts, const char* path) {
  zkml::R1CS c;
  c.num_constraints = nc;
  c.num_variables = nv;
  c.num_public_inputs = npub;
  c.num_private_inputs = npriv;
  size_t off = 0;
  for (int which = 0; which < 3; which++) {
    std::vector<zkml::SparseEntry>& v = which == 0 ? c.A : (which == 1 ? c.B : c.C);
    for (size_t i = 0; i < counts[which]; i++, off++)
      v.push_back({rows[off], cols[off], Fr(vals[4 * off], vals[4 * off + 1], vals[4 * off + 2], vals[4 * off + 3])});
  }
  return zkml::export_r1cs_iden3(c, path) ? 1 : 0;
}

int ref_export_wtns(const uint64_t* w, int m, const char* path) {
  std::vector<Fr> wv(m);
  for (int i = 0; i < m; i++) wv[i] = Fr(w[4 * i], w[4 * i + 1], w[4 * i + 2], w[4 * i + 3]);
  return zkml::export_wtns_iden3(wv, path) ? 1 : 0;
}

}  // extern "C"
