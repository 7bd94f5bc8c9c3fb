// zkml-prove: Groth16 proving from an R1CS statement on one MI355X.
//
// Counterpart of the reference's zkml-prove (src/cli/prove.cu:782-1365) for
// statements given as R1CS + witness: iden3 .r1cs/.wtns files (what the
// reference's --export-r1cs/--export-wtns write) or the synthetic config-5
// R1CS.  Keys: --pk-load an existing ZKMLPK3 key, or --pk-save to run the GPU
// setup and write key and verification key.  Prints "Proving time: %.2f ms",
// checks the proof against the verification key and exits 0 only if it
// verifies, as the reference does.  ZKML_DETERMINISTIC_PROVE=1 selects the
// blinding seed 0xCAFEBABE and ZKML_SKIP_WITNESS_CHECK=1 skips the R1CS check
// (groth16.cu:687-718).
#include <stdlib.h>

#include <algorithm>
#include <random>
#include <string>
#include <vector>

#include "../csrc/host_bn254.hpp"
#include "cli_common.hpp"

static void usage() {
  printf("zkml-prove (MI355X build)\n");
  printf("Usage:\n");
  printf("  zkml-prove (--r1cs FILE --wtns FILE | --synthetic N) (--pk-load PK | --pk-save PK) --vk VK\n");
  printf("             --output PROOF [--public-inputs FILE(.bin|.json)] [options]\n");
  printf("\nStatement:\n");
  printf("  --r1cs FILE --wtns FILE   iden3 R1CS (v1) and witness (v2)\n");
  printf("  --synthetic N             random R1CS with N constraints (BASELINE config 5 shape)\n");
  printf("  --synthetic-public P      public inputs of the synthetic R1CS (default 4)\n");
  printf("  --synthetic-inputs K      free private inputs of the synthetic R1CS (default 16)\n");
  printf("  --synthetic-seed S        generator seed (default 42)\n");
  printf("Keys:\n");
  printf("  --pk-load FILE            ZKMLPK3 proving key; --vk names its verification key\n");
  printf("  --pk-save FILE            run the setup (GPU) and write the proving key and --vk\n");
  printf("  --toxic-seed S            setup toxic-waste seed (default 0xDEADBEEF42)\n");
  printf("Outputs:\n");
  printf("  --output FILE             256-byte proof\n");
  printf("  --public-inputs FILE      public inputs, .bin (i32 count + 32-byte scalars) or .json\n");
  printf("  --export-r1cs FILE        write the statement as iden3 .r1cs\n");
  printf("  --export-wtns FILE        write the witness as iden3 .wtns\n");
  printf("Options:\n");
  printf("  --seed S                  blinding seed (default random)\n");
  printf("  --repeat K                prove K times and report the median (default 1)\n");
  printf("  --device D                GPU ordinal (default 0)\n");
  printf("  --help\n");
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
  const char *r1cs = nullptr, *wtns = nullptr, *pk_load = nullptr, *pk_save = nullptr, *vk = nullptr;
  const char *out = nullptr, *pub_out = nullptr, *exp_r1cs = nullptr, *exp_wtns = nullptr;
  long synthetic = -1, syn_pub = 4, syn_inputs = 16, repeat = 1, device = 0;
  uint64_t syn_seed = 42, toxic = 0xDEADBEEF42ULL, seed = 0;
  bool have_seed = false;
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
      else if (a == "--toxic-seed") toxic = u;
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
  const bool from_files = r1cs && wtns;
  if (from_files == (synthetic >= 0) || (!pk_load == !pk_save) || !vk || !out) {
    fprintf(stderr, "Error: give one statement (--r1cs + --wtns, or --synthetic), one of --pk-load / --pk-save, "
                    "--vk and --output\n");
    return 1;
  }
  zk_context* ctx = nullptr;
  // ---- statement
  int nc = 0, nv = 0, npub = 0, npriv = 0;
  std::vector<zk_sparse_entry> A, B, C;
  std::vector<uint64_t> w;
  cli::Timer tload;
  if (from_files) {
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
  if (pk_save) {
    cli::Timer ts;
    CHECK(zk_setup(ctx, rc, toxic, pk_save, vk), "setup");
    printf("Setup time: %.2f ms (proving key %s, verification key %s)\n", ts.ms(), pk_save, vk);
  }
  zk_pk* pk = nullptr;
  cli::Timer tk;
  CHECK(zk_pk_load(ctx, pk_save ? pk_save : pk_load, &pk), "loading the proving key");
  printf("Proving key loaded in %.2f ms\n", tk.ms());
  // ---- prove
  if (!have_seed) {
    const char* det = getenv("ZKML_DETERMINISTIC_PROVE");
    if (det && !strcmp(det, "1")) {
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
  zk_pk_destroy(pk);
  zk_r1cs_destroy(rc);
  zk_destroy(ctx);
  return valid ? 0 : 1;
}
