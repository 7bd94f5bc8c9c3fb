// zkml-prove: Groth16 proving on one MI355X.
//
// Counterpart of the reference's zkml-prove (src/cli/prove.cu:782-1365).
// Statements come from one of:
//   --statement-v2 with an exact integer model (--model FILE.int32.bin
//     --integer-model, --arch FILE.arch.json or FILE.int32.bin.arch.json) and
//     integer samples (--input / --batch-inputs, float32 .bin or .npy,
//     --integer-input), built by the product's statement producer with the
//     reference's v2 options (--context, --private-input, --input-blinding,
//     --private-model, --private-outputs, --route-threshold) and the
//     quantized-model tag;
//   iden3 .r1cs/.wtns files (what --export-r1cs/--export-wtns write);
//   the synthetic config-5 R1CS.
// Keys: --pk-load an existing ZKMLPK3 key, or the GPU setup (--pk-save keeps
// the key; without either the key lives in a temporary file).  Prints
// "Proving time: %.2f ms", checks the proof against the verification key and
// exits 0 only if it verifies, as the reference does.  Output defaults are the
// reference's: proof.bin, vk.bin, public_inputs.bin.
// Seeds follow the reference's contract: the setup's toxic waste comes from a
// fresh random 64-bit seed unless ZKML_DETERMINISTIC_SETUP=1 selects
// 0xDEADBEEF42 (groth16.cu:455-462); --toxic-seed overrides both.
// ZKML_DETERMINISTIC_PROVE=1 selects the blinding seed 0xCAFEBABE and
// ZKML_SKIP_WITNESS_CHECK=1 skips the R1CS check (groth16.cu:687-718).
#include <stdlib.h>
#include <unistd.h>

#include <algorithm>
#include <chrono>
#include <random>
#include <string>
#include <vector>

#include "../csrc/host_bn254.hpp"
#include "cli_common.hpp"
#include "model_files.hpp"

static void usage() {
  printf("zkml-prove (MI355X build)\n");
  printf("Usage:\n");
  printf("  zkml-prove --statement-v2 --model M.int32.bin --integer-model [--arch M.arch.json]\n");
  printf("             (--input X.npy | --batch-inputs X0.npy,X1.npy) --integer-input [v2 options] [options]\n");
  printf("  zkml-prove (--r1cs FILE --wtns FILE | --synthetic N) [options]\n");
  printf("\nStatement v2 (reference build_statement_v2):\n");
  printf("  --model FILE              exact little-endian int32 parameters (with --integer-model)\n");
  printf("  --arch FILE               architecture sidecar (default MODEL.arch.json)\n");
  printf("  --input FILE              sample, float32 .bin or .npy holding exact integers (--integer-input)\n");
  printf("  --batch-inputs A,B,...    several samples in one statement\n");
  printf("  --context HEX             public context bound by ctx * ctx = ctx_sq\n");
  printf("  --private-input           commit to each sample with Poseidon (needs --input-blinding)\n");
  printf("  --input-blinding H0,H1    one hex blinding value per sample\n");
  printf("  --private-model           weights private under a Poseidon commitment\n");
  printf("  --private-outputs         scores private (needs --route-threshold)\n");
  printf("  --route-threshold T       in-circuit top-1 / top-2 routing flag [top1 - top2 >= T]\n");
  printf("  --statement-meta FILE     statement metadata JSON\n");
  printf("Other statements:\n");
  printf("  --r1cs FILE --wtns FILE   iden3 R1CS (v1) and witness (v2)\n");
  printf("  --synthetic N             random R1CS with N constraints (1-3 term rows, C a fresh variable)\n");
  printf("  --synthetic-public P      public inputs of the synthetic R1CS (default 4)\n");
  printf("  --synthetic-inputs K      free private inputs of the synthetic R1CS (default 16)\n");
  printf("  --synthetic-seed S        generator seed (default 42)\n");
  printf("Keys:\n");
  printf("  --pk-load FILE            ZKMLPK3 proving key; --vk names its verification key\n");
  printf("  --pk-save FILE            run the setup (GPU) and keep the proving key (default: temporary)\n");
  printf("  --toxic-seed S            setup toxic-waste seed (default: random; 0xDEADBEEF42 with\n");
  printf("                            ZKML_DETERMINISTIC_SETUP=1)\n");
  printf("Outputs:\n");
  printf("  --output FILE             256-byte proof (default proof.bin)\n");
  printf("  --vk FILE                 verification key (default vk.bin)\n");
  printf("  --public-inputs FILE      public inputs, .bin (i32 count + 32-byte scalars) or .json\n");
  printf("                            (default public_inputs.bin)\n");
  printf("  --export-r1cs FILE        write the statement as iden3 .r1cs\n");
  printf("  --export-wtns FILE        write the witness as iden3 .wtns\n");
  printf("Options:\n");
  printf("  --seed S                  blinding seed (default random)\n");
  printf("  --repeat K                prove K times and report the median (default 1)\n");
  printf("  --device D                GPU ordinal (default 0)\n");
  printf("  --help\n");
}

static bool env_is_1(const char* name) {
  const char* v = getenv(name);
  return v && !strcmp(v, "1");
}

// A fresh 64-bit seed: the OS entropy source mixed with the clock, as the
// reference's random_seed64 (groth16.cu:39-46) does for its setup.
static uint64_t fresh_seed64() {
  std::random_device rd;
  const uint64_t hi = ((uint64_t)rd() << 32) ^ (uint64_t)rd();
  const uint64_t t = (uint64_t)std::chrono::high_resolution_clock::now().time_since_epoch().count();
  return hi ^ t ^ 0x9E3779B97F4A7C15ULL;
}

static bool parse_u64(const char* s, uint64_t& v) {
  char* end = nullptr;
  v = strtoull(s, &end, 0);
  return end && *end == 0;
}

static std::string decimal(const uint64_t w[4]) {
  uint64_t x[4] = {w[0], w[1], w[2], w[3]};
  std::string s;
  for (;;) {
    unsigned __int128 rem = 0;
    bool nz = false;
    for (int k = 3; k >= 0; k--) {
      unsigned __int128 cur = (rem << 64) | x[k];
      x[k] = (uint64_t)(cur / 10);
      rem = cur % 10;
      nz |= x[k] != 0;
    }
    s.push_back((char)('0' + (int)rem));
    if (!nz) break;
  }
  std::reverse(s.begin(), s.end());
  return s;
}

static bool write_publics(const char* path, const std::vector<uint64_t>& std_words, int npub) {
  FILE* f = fopen(path, "wb");
  if (!f) return false;
  const std::string p(path);
  bool ok = true;
  if (p.size() >= 5 && p.substr(p.size() - 5) == ".json") {
    fprintf(f, "[");
    for (int i = 0; i < npub; i++) fprintf(f, "%s%s", i ? ", " : "", decimal(&std_words[4 * (size_t)i]).c_str());
    fprintf(f, "]\n");
  } else {
    const int32_t n = npub;
    ok = fwrite(&n, 4, 1, f) == 1 && (npub == 0 || fwrite(std_words.data(), 32, (size_t)npub, f) == (size_t)npub);
  }
  return fclose(f) == 0 && ok;
}

#define CHECK(expr, what)                                                                            \
  do {                                                                                               \
    int _st = (expr);                                                                                \
    if (_st != ZK_OK) {                                                                              \
      fprintf(stderr, "Error: %s failed: %s (%s)\n", what, cli::status_text(_st), ctx ? zk_last_error(ctx) : ""); \
      return 1;                                                                                      \
    }                                                                                                \
  } while (0)

int main(int argc, char** argv) {
  const char *r1cs = nullptr, *wtns = nullptr, *pk_load = nullptr, *pk_save = nullptr;
  const char *vk = "vk.bin", *out = "proof.bin", *pub_out = "public_inputs.bin";
  const char *exp_r1cs = nullptr, *exp_wtns = nullptr;
  long synthetic = -1, syn_pub = 4, syn_inputs = 16, repeat = 1, device = 0;
  uint64_t syn_seed = 42, toxic = 0, seed = 0;
  bool have_seed = false, have_toxic = false;
  // statement v2
  bool v2 = false, integer_model = false, integer_input = false, route = false;
  const char *model_path = nullptr, *arch_path = nullptr, *input_path = nullptr, *meta_path = nullptr;
  std::string batch_list, blinding_list;
  zk_statement_options v2opt;
  memset(&v2opt, 0, sizeof(v2opt));
  if (argc < 2) {
    usage();
    return 1;
  }
  for (int i = 1; i < argc; i++) {
    const std::string a = argv[i];
    const char* v = nullptr;
    auto val = [&]() { return (v = cli::arg_value(argc, argv, i)) != nullptr; };
    uint64_t u = 0;
    if (a == "--help") {
      usage();
      return 0;
    } else if (a == "--r1cs") {
      if (!val()) return 1;
      r1cs = v;
    } else if (a == "--wtns") {
      if (!val()) return 1;
      wtns = v;
    } else if (a == "--pk-load") {
      if (!val()) return 1;
      pk_load = v;
    } else if (a == "--pk-save") {
      if (!val()) return 1;
      pk_save = v;
    } else if (a == "--vk") {
      if (!val()) return 1;
      vk = v;
    } else if (a == "--output") {
      if (!val()) return 1;
      out = v;
    } else if (a == "--public-inputs") {
      if (!val()) return 1;
      pub_out = v;
    } else if (a == "--export-r1cs") {
      if (!val()) return 1;
      exp_r1cs = v;
    } else if (a == "--export-wtns") {
      if (!val()) return 1;
      exp_wtns = v;
    } else if (a == "--statement-v2") {
      v2 = true;
    } else if (a == "--integer-model") {
      integer_model = true;
    } else if (a == "--integer-input") {
      integer_input = true;
    } else if (a == "--private-input") {
      v2opt.private_input = 1;
    } else if (a == "--private-model") {
      v2opt.private_model = 1;
    } else if (a == "--private-outputs") {
      v2opt.private_outputs = 1;
    } else if (a == "--model" || a == "--arch" || a == "--input" || a == "--statement-meta") {
      if (!val()) return 1;
      (a == "--model" ? model_path : a == "--arch" ? arch_path : a == "--input" ? input_path : meta_path) = v;
    } else if (a == "--batch-inputs" || a == "--input-blinding") {
      if (!val()) return 1;
      (a == "--batch-inputs" ? batch_list : blinding_list) = v;
    } else if (a == "--context") {
      if (!val()) return 1;
      v2opt.has_context = 1;
      if (!cli::fr_hex(v, v2opt.context)) {
        fprintf(stderr, "--context expects a hex value\n");
        return 1;
      }
    } else if (a == "--route-threshold") {
      if (!val()) return 1;
      route = true;
      v2opt.route = 1;
      v2opt.route_threshold = atoll(v);
    } else if (a == "--synthetic" || a == "--synthetic-public" || a == "--synthetic-inputs" || a == "--repeat" ||
               a == "--device" || a == "--synthetic-seed" || a == "--toxic-seed" || a == "--seed") {
      if (!val() || !parse_u64(v, u)) {
        fprintf(stderr, "Error: %s needs a number\n", a.c_str());
        return 1;
      }
      if (a == "--synthetic") synthetic = (long)u;
      else if (a == "--synthetic-public") syn_pub = (long)u;
      else if (a == "--synthetic-inputs") syn_inputs = (long)u;
      else if (a == "--repeat") repeat = std::max<long>(1, (long)u);
      else if (a == "--device") device = (long)u;
      else if (a == "--synthetic-seed") syn_seed = u;
      else if (a == "--toxic-seed") {
        toxic = u;
        have_toxic = true;
      }
      else {
        seed = u;
        have_seed = true;
      }
    } else {
      fprintf(stderr, "Error: unknown option %s\n", a.c_str());
      usage();
      return 1;
    }
  }
  if (!v2 && (v2opt.has_context || v2opt.private_input || v2opt.private_model || route || !batch_list.empty())) {
    fprintf(stderr, "--context/--private-*/--route-threshold/--batch-inputs require --statement-v2\n");
    return 1;
  }
  const bool from_files = r1cs && wtns;
  if ((int)from_files + (int)(synthetic >= 0) + (int)v2 != 1 || (pk_load && pk_save)) {
    fprintf(stderr, "Error: give one statement (--statement-v2, --r1cs + --wtns, or --synthetic) and at most one "
                    "of --pk-load / --pk-save\n");
    return 1;
  }
  zk_context* ctx = nullptr;
  // ---- statement
  int nc = 0, nv = 0, npub = 0, npriv = 0;
  std::vector<zk_sparse_entry> A, B, C;
  std::vector<uint64_t> w;
  zk_statement* stmt = nullptr;
  uint64_t tag64 = 0;
  cli::Timer tload;
  if (v2) {
    std::vector<std::string> files = batch_list.empty() ? std::vector<std::string>() : cli::split_csv(batch_list);
    if (!input_path && !files.empty()) input_path = files[0].c_str();
    if (!model_path || !input_path) {
      fprintf(stderr, "Error: --model and --input are required\n");
      usage();
      return 1;
    }
    if (files.empty()) files.push_back(input_path);
    if (!integer_model || !integer_input) {
      fprintf(stderr, "Error: this build proves exact integer models only: pass --integer-model (int32 "
                      "parameters) and --integer-input (integer-valued samples)\n");
      return 1;
    }
    std::string arch = arch_path ? arch_path : "";
    if (arch.empty() || !fopen(arch.c_str(), "rb")) {
      arch = std::string(model_path) + ".arch.json";
      FILE* probe = fopen(arch.c_str(), "rb");
      if (!probe) {
        fprintf(stderr, "[Model] No architecture for %s. Pass --arch MODEL.arch.json\n", model_path);
        return 1;
      }
      fclose(probe);
    }
    std::vector<cli::LayerSpec> specs;
    std::string err;
    if (!cli::load_arch(arch.c_str(), specs, err)) {
      fprintf(stderr, "[Model] %s\n", err.c_str());
      fprintf(stderr, "Failed to load model architecture\n");
      return 1;
    }
    std::vector<int32_t> params;
    if (!cli::load_raw(model_path, params)) {
      fprintf(stderr, "Cannot load int32 model file: %s\n", model_path);
      return 1;
    }
    cli::Model model;
    if (!cli::build_model(specs, params, model, err)) {
      fprintf(stderr, "[NN] Error: %s\nFailed to load model weights\n", err.c_str());
      return 1;
    }
    const int n_in = specs[0].in_size;
    std::vector<int64_t> xs;
    for (const auto& fpath : files) {
      std::vector<float> raw;
      std::vector<int64_t> q;
      if (!cli::load_input(fpath.c_str(), raw) || (int)raw.size() != n_in || !cli::integer_samples(raw, q)) {
        fprintf(stderr, "Cannot load batch input %s (size must be %d, exact int32 values)\n", fpath.c_str(), n_in);
        return 1;
      }
      xs.insert(xs.end(), q.begin(), q.end());
    }
    std::vector<uint64_t> blind;
    if (v2opt.private_input) {
      for (const auto& hx : cli::split_csv(blinding_list)) {
        uint64_t b[4];
        if (!cli::fr_hex(hx, b)) {
          fprintf(stderr, "bad --input-blinding value\n");
          return 1;
        }
        blind.insert(blind.end(), b, b + 4);
      }
      if (blind.size() != 4 * files.size()) {
        fprintf(stderr, "Failed to build PCANI v2 statement: private_input needs one blinding value per sample\n");
        return 1;
      }
      v2opt.input_blinding = blind.data();
    }
    tag64 = cli::model_tag64(model);
    v2opt.model_tag[0] = tag64;
    printf("[PCANI v2] samples=%zu context=%s input=%s model=%s route=%s\n", files.size(),
           v2opt.has_context ? "bound" : "none", v2opt.private_input ? "committed" : "public",
           v2opt.private_model ? "committed" : "fixed", v2opt.route ? "in-circuit" : "off");
    char msg[256];
    const int st = zk_statement_v2_build(model.layers.data(), (int)model.layers.size(), xs.data(), (int)files.size(),
                                         n_in, &v2opt, &stmt, msg, sizeof(msg));
    if (st != ZK_OK) {
      fprintf(stderr, "Failed to build PCANI v2 statement: %s\n", msg);
      return 1;
    }
    size_t na = 0, nb = 0, ncc = 0;
    CHECK(zk_statement_info(stmt, &nc, &nv, &npub, &npriv, &na, &nb, &ncc), "statement sizes");
    A.resize(na);
    B.resize(nb);
    C.resize(ncc);
    w.resize(4 * (size_t)nv);
    CHECK(zk_statement_r1cs(stmt, A.data(), B.data(), C.data()), "statement R1CS");
    CHECK(zk_statement_witness(stmt, w.data()), "statement witness");
    printf("[PCANI v2] Quantized model tag: 0x%016llx\n", (unsigned long long)tag64);
    printf("[PCANI v2] R1CS: %d constraints, %d variables, %d public\n", nc, nv, npub);
    if (zk_statement_check(stmt) != ZK_OK) {
      fprintf(stderr, "Witness does not satisfy circuit constraints.\n");
      return 1;
    }
  } else if (from_files) {
    size_t na = 0, nb = 0, ncc = 0, m = 0;
    CHECK(zk_iden3_r1cs_info(r1cs, &nc, &nv, &npub, &npriv, &na, &nb, &ncc), "reading the .r1cs header");
    A.resize(na);
    B.resize(nb);
    C.resize(ncc);
    CHECK(zk_iden3_r1cs_read(r1cs, A.data(), B.data(), C.data()), "reading the .r1cs");
    CHECK(zk_wtns_info(wtns, &m), "reading the .wtns header");
    w.resize(m * 4);
    CHECK(zk_wtns_read(wtns, w.data(), m), "reading the .wtns");
  } else {
    nc = (int)synthetic;
    npub = (int)syn_pub;
    npriv = (int)syn_inputs;
    nv = 1 + npub + npriv + nc;
    A.resize(3 * (size_t)nc);
    B.resize(3 * (size_t)nc);
    C.resize((size_t)nc);
    w.resize(4 * (size_t)nv);
    size_t na = 0, nb = 0, ncc = 0;
    CHECK(zk_synthetic_r1cs(nc, npub, npriv, syn_seed, A.data(), &na, B.data(), &nb, C.data(), &ncc, w.data()),
          "generating the synthetic R1CS");
    A.resize(na);
    B.resize(nb);
    C.resize(ncc);
  }
  printf("Statement: %d constraints, %d variables, %d public inputs (%.1f ms)\n", nc, nv, npub, tload.ms());
  if (exp_r1cs) CHECK(zk_iden3_r1cs_write(exp_r1cs, nc, nv, npub, npriv, A.data(), A.size(), B.data(), B.size(),
                                          C.data(), C.size()), "writing the .r1cs");
  if (exp_wtns) CHECK(zk_wtns_write(exp_wtns, w.data(), w.size() / 4), "writing the .wtns");
  // ---- device
  CHECK(zk_create((int)device, &ctx), "creating the device context");
  zk_r1cs* rc = nullptr;
  CHECK(zk_r1cs_create(ctx, nc, nv, npub, A.data(), A.size(), B.data(), B.size(), C.data(), C.size(), &rc),
        "uploading the R1CS");
  std::string key_path = pk_load ? pk_load : pk_save ? pk_save : "";
  bool temp_key = false;
  if (pk_load) {
    FILE* probe = fopen(vk, "rb");
    if (!probe) {
      fprintf(stderr, "When using --pk-load, a verification key file must already exist at %s\n", vk);
      return 1;
    }
    fclose(probe);
  } else {
    if (!pk_save) {  // setup without a kept key: a private temporary file
      const char* tmpdir = getenv("TMPDIR");
      std::string templ = std::string(tmpdir && *tmpdir ? tmpdir : "/tmp") + "/zkml-pk-XXXXXX";
      std::vector<char> buf(templ.begin(), templ.end());
      buf.push_back(0);
      const int fd = mkstemp(buf.data());
      if (fd < 0) {
        fprintf(stderr, "Error: cannot create a temporary proving-key file in %s\n", templ.c_str());
        return 1;
      }
      close(fd);
      key_path = buf.data();
      temp_key = true;
    }
    // The seed is the whole toxic waste, so a random one is never printed.
    const char* mode = "explicit";
    if (!have_toxic) {
      const bool det = env_is_1("ZKML_DETERMINISTIC_SETUP");
      toxic = det ? 0xDEADBEEF42ULL : fresh_seed64();
      mode = det ? "deterministic" : "randomized";
    }
    if (!strcmp(mode, "randomized")) printf("[Setup] RNG seed: (randomized, not shown)\n");
    else printf("[Setup] RNG seed: 0x%016llx (%s)\n", (unsigned long long)toxic, mode);
    cli::Timer ts;
    const int st = zk_setup(ctx, rc, toxic, key_path.c_str(), vk);
    if (st != ZK_OK && temp_key) unlink(key_path.c_str());
    CHECK(st, "setup");
    printf("Setup time: %.2f ms (proving key %s, verification key %s)\n", ts.ms(),
           temp_key ? "temporary" : key_path.c_str(), vk);
  }
  zk_pk* pk = nullptr;
  cli::Timer tk;
  const int pk_st = zk_pk_load(ctx, key_path.c_str(), &pk);
  if (temp_key) unlink(key_path.c_str());
  CHECK(pk_st, "loading the proving key");
  printf("Proving key loaded in %.2f ms\n", tk.ms());
  // ---- prove
  if (!have_seed) {
    if (env_is_1("ZKML_DETERMINISTIC_PROVE")) {
      seed = 0xCAFEBABEULL;
    } else {
      std::random_device rd;
      seed = ((uint64_t)rd() << 32) ^ rd();
    }
  }
  const char* skip = getenv("ZKML_SKIP_WITNESS_CHECK");
  const int check = !(skip && !strcmp(skip, "1"));
  uint8_t proof[256];
  std::vector<double> times;
  for (long k = 0; k < repeat; k++) {
    cli::Timer tp;
    CHECK(zk_prove(ctx, pk, rc, w.data(), w.size() / 4, npub, seed, check, proof, nullptr), "prove");
    times.push_back(tp.ms());
  }
  std::sort(times.begin(), times.end());
  printf("Proving time: %.2f ms\n", times[times.size() / 2]);
  FILE* f = fopen(out, "wb");
  if (!f || fwrite(proof, 1, 256, f) != 256 || fclose(f) != 0) {
    fprintf(stderr, "Error: cannot write %s\n", out);
    return 1;
  }
  // ---- public inputs w[1..npub] in standard form, verification
  std::vector<uint64_t> pub_std(4 * (size_t)npub);
  for (int i = 0; i < npub; i++) zkh::Fr::raw(&w[4 * (size_t)(1 + i)]).to_std(&pub_std[4 * (size_t)i]);
  if (pub_out && !write_publics(pub_out, pub_std, npub)) {
    fprintf(stderr, "Error: cannot write %s\n", pub_out);
    return 1;
  }
  std::vector<uint8_t> vkb;
  {
    FILE* g = fopen(vk, "rb");
    if (!g) {
      fprintf(stderr, "Error: cannot read %s\n", vk);
      return 1;
    }
    uint8_t buf[65536];
    size_t got;
    while ((got = fread(buf, 1, sizeof(buf), g)) > 0) vkb.insert(vkb.end(), buf, buf + got);
    fclose(g);
  }
  int valid = 0;
  CHECK(zk_verify(vkb.data(), vkb.size(), proof, pub_std.data(), npub, &valid), "verification");
  printf("Proof %s: %s\n", out, valid ? "VALID" : "INVALID");
  if (stmt) {
    if (meta_path) {
      size_t len = 0;
      CHECK(zk_statement_meta_json(stmt, tag64, nullptr, 0, &len), "statement metadata");
      std::vector<char> text(len + 1);
      CHECK(zk_statement_meta_json(stmt, tag64, text.data(), text.size(), &len), "statement metadata");
      FILE* g = fopen(meta_path, "wb");
      if (!g || fwrite(text.data(), 1, len, g) != len || fclose(g) != 0) {
        fprintf(stderr, "Error: cannot write %s\n", meta_path);
        return 1;
      }
      printf("[PCANI v2] Statement metadata: %s\n", meta_path);
    }
    printf("Statement mode: PCANI v2\n");
    zk_statement_destroy(stmt);
  }
  zk_pk_destroy(pk);
  zk_r1cs_destroy(rc);
  zk_destroy(ctx);
  return valid ? 0 : 1;
}
