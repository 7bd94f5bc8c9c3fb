// TEST INFRASTRUCTURE ONLY -- never linked into the product.
//
// The reference's zkml-prove front end (src/cli/prove.cu), compiled in place
// from the reference sources with the reference's own host shim
// (tests/host/shim), its main() renamed.  Exposes the front end's own
// statement-v2 preparation so the product's zkml-prove can be checked
// against it: architecture sidecar parsing, the int32 model loader, the
// float32 .bin/.npy input loader, --integer-input conversion, the quantized
// model tag (compute_quantized_model_tag64) and the hex parser of --context /
// --input-blinding, feeding build_statement_v2 and the iden3 exporters.
//
// The GPU prover, setup and inference that the rest of prove.cu calls are
// not compiled here: load this library with RTLD_LAZY; none of the entry
// points below reaches those symbols.
#define main ref_prove_main
#include "cli/prove.cu"
#undef main

#include <cstring>

extern "C" {

// Statement of `zkml-prove --statement-v2 --integer-model --integer-input`
// (prove.cu:1034-1205): returns 0 and writes the iden3 files and the metadata
// JSON; info = {constraints, variables, public, witness satisfies};
// tag = the quantized model tag.  Negative return: the step that failed
// (-1 architecture, -2 model, -3 inputs, -4 blinding / context, -5 builder,
// -6 export).  inputs_csv: one or more sample files separated by commas.
int ref_cli_statement_v2(const char* arch_path, const char* model_path, const char* inputs_csv,
                         const char* context_hex, int private_input, const char* blinding_csv, int private_model,
                         int private_outputs, int route, long long route_threshold, const char* r1cs_path,
                         const char* wtns_path, char* meta, size_t meta_cap, int* info, uint64_t* tag) {
  zkml::NNModel model;
  if (!load_model_from_architecture(arch_path, model)) return -1;
  std::vector<int32_t> params;
  if (!load_int32_binary(model_path, params) || !model.load_integer_weights(params.data(), (int)params.size()))
    return -2;
  auto split = [](const std::string& text) {
    std::vector<std::string> parts;
    std::string cur;
    for (char c : text) {
      if (c == ',') {
        if (!cur.empty()) parts.push_back(cur);
        cur.clear();
      } else {
        cur.push_back(c);
      }
    }
    if (!cur.empty()) parts.push_back(cur);
    return parts;
  };
  std::vector<std::vector<bn254::Fp>> batch;
  int input_size = -1;
  for (const auto& f : split(inputs_csv)) {
    std::vector<float> raw;
    if (!load_input_float32_auto(f, raw)) return -3;
    if (input_size < 0) input_size = (int)raw.size();
    if ((int)raw.size() != input_size) return -3;
    std::vector<bn254::Fp> q(raw.size());
    for (size_t i = 0; i < raw.size(); i++) {
      double r = std::llround((double)raw[i]);
      if (std::fabs((double)raw[i] - r) > 1e-5 || r < (double)INT32_MIN || r > (double)INT32_MAX) return -3;
      q[i] = zkml::int_to_fp((int32_t)r);
    }
    batch.push_back(q);
  }
  zkml::StatementV2Options opt;
  if (context_hex) {
    opt.has_context = true;
    if (!zkml::fr_from_hex(context_hex, &opt.context)) return -4;
  }
  opt.private_input = private_input != 0;
  if (opt.private_input && blinding_csv)
    for (const auto& h : split(blinding_csv)) {
      bn254::Fr r;
      if (!zkml::fr_from_hex(h, &r)) return -4;
      opt.input_blinding.push_back(r);
    }
  opt.private_model = private_model != 0;
  opt.private_outputs = private_outputs != 0;
  opt.route = route != 0;
  opt.route_threshold = route_threshold;
  const uint64_t tag64 = compute_quantized_model_tag64(model);
  opt.model_tag = bn254::Fr::from_uint(tag64);
  *tag = tag64;
  zkml::StatementV2 st;
  std::string err;
  if (!zkml::build_statement_v2(model, batch, opt, st, err)) {
    if (meta && meta_cap) snprintf(meta, meta_cap, "%s", err.c_str());
    return -5;
  }
  info[0] = st.r1cs.num_constraints;
  info[1] = st.r1cs.num_variables;
  info[2] = st.layout.num_public;
  info[3] = st.r1cs.verify_witness(st.witness.values) ? 1 : 0;
  if (!zkml::export_r1cs_iden3(st.r1cs, r1cs_path) || !zkml::export_wtns_iden3(st.witness.values, wtns_path))
    return -6;
  const std::string js = zkml::statement_v2_meta_json(st, opt, tag64);
  if (meta && meta_cap) snprintf(meta, meta_cap, "%s", js.c_str());
  return 0;
}

}  // extern "C"
