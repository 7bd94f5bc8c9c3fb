// zkml-verify: Groth16 verification of artefact files (replaces the
// reference's src/cli/verify.cu: same flags, messages and exit codes --
// 0 when the proof verifies, 1 otherwise).
#include "cli_common.hpp"

static void print_usage() {
  printf("zkml-verify (MI355X build)\n");
  printf("Usage:\n");
  printf("  zkml-verify --vk VK_FILE --proof PROOF_FILE --public-inputs PI_FILE\n");
  printf("\nOptions:\n");
  printf("  --vk FILE            Path to verification key\n");
  printf("  --proof FILE         Path to proof (256 bytes)\n");
  printf("  --public-inputs FILE Path to public inputs (.bin or .json)\n");
  printf("  --help               Show this help\n");
}

int main(int argc, char** argv) {
  if (argc < 2) {
    print_usage();
    return 1;
  }
  const char *vk = nullptr, *proof = nullptr, *pub = nullptr;
  for (int i = 1; i < argc; i++) {
    if (!strcmp(argv[i], "--help")) {
      print_usage();
      return 0;
    } else if (!strcmp(argv[i], "--vk")) {
      if (!(vk = cli::arg_value(argc, argv, i))) return 1;
    } else if (!strcmp(argv[i], "--proof")) {
      if (!(proof = cli::arg_value(argc, argv, i))) return 1;
    } else if (!strcmp(argv[i], "--public-inputs")) {
      if (!(pub = cli::arg_value(argc, argv, i))) return 1;
    }
  }
  if (!vk || !proof || !pub) {
    fprintf(stderr, "Error: --vk, --proof, and --public-inputs are required\n");
    print_usage();
    return 1;
  }
  printf("Verifying proof %s with %s and %s...\n", proof, vk, pub);
  cli::Timer t;
  int valid = 0;
  const int st = zk_verify_files(vk, proof, pub, &valid);
  const double ms = t.ms();
  if (st != ZK_OK) {
    fprintf(stderr, "Error: cannot load the verification inputs (%s)\n", cli::status_text(st));
    return 1;
  }
  printf("\n=============================\n");
  printf(valid ? "   PROOF VALID\n" : "   PROOF INVALID\n");
  printf("=============================\n");
  printf("Verification time: %.2f ms\n", ms);
  return valid ? 0 : 1;
}
