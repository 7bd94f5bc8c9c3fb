// Groth16 verification and the pairing on the host, behind the C ABI.
//
// Replaces Groth16Verifier::verify (reference src/prover/groth16.cu:967-1022)
// and the zkml-verify loaders (src/verifier/verifier.cu:47-210,
// src/cli/verify.cu:33-75): VK, 256-byte proof and public-input files
// (.bin: i32 count + 32-byte standard-form scalars; .json: decimal list).
// Pure host code: no device is touched.
#include <stdint.h>
#include <stdio.h>
#include <string.h>

#include <string>
#include <vector>

#include "abi_guard.hpp"
#include "../../include/zkml_gpu.h"
#include "pairing_host.hpp"

using namespace zkh;

namespace {

bool read_file(const char* path, std::vector<uint8_t>& out) {
  FILE* f = fopen(path, "rb");
  if (!f) return false;
  out.clear();
  uint8_t buf[1 << 16];
  size_t got;
  while ((got = fread(buf, 1, sizeof(buf), f)) > 0) out.insert(out.end(), buf, buf + got);
  fclose(f);
  return true;
}

Fq fq_std(const uint8_t* p) {
  uint64_t w[4];
  memcpy(w, p, 32);
  return Fq::from_std(w);
}

// x = y = 0 encodes the point at infinity (no finite point has x = y = 0).
G1A g1_std(const uint8_t* p) {
  G1A a{fq_std(p), fq_std(p + 32), false};
  a.inf = a.x.is_zero() && a.y.is_zero();
  return a;
}
G2A g2_std(const uint8_t* p) {
  G2A a{Fq2{fq_std(p), fq_std(p + 32)}, Fq2{fq_std(p + 64), fq_std(p + 96)}, false};
  a.inf = a.x.is_zero() && a.y.is_zero();
  return a;
}

// VK layout of src/verifier/verifier.cu:103-148.
int parse_vk(const uint8_t* b, size_t len, VerifyingKey& vk) {
  if (len < 4 + 64 + 3 * 128 + 4) return ZK_ERR_IO;
  int32_t npub, nic;
  memcpy(&npub, b, 4);
  size_t o = 4;
  vk.alpha = g1_std(b + o);
  o += 64;
  vk.beta = g2_std(b + o);
  o += 128;
  vk.gamma = g2_std(b + o);
  o += 128;
  vk.delta = g2_std(b + o);
  o += 128;
  memcpy(&nic, b + o, 4);
  o += 4;
  if (npub < 0 || nic < 0 || (size_t)nic > (len - o) / 64 || o + 64 * (size_t)nic != len) return ZK_ERR_IO;
  vk.npub = npub;
  vk.ic.resize(nic);
  for (int i = 0; i < nic; i++) vk.ic[i] = g1_std(b + o + 64 * (size_t)i);
  return ZK_OK;
}

// Decimal tokens with an optional sign, negatives taken mod r (the reference's
// JSON reader, src/cli/verify.cu:33-75).
bool parse_public_json(const std::vector<uint8_t>& text, std::vector<std::vector<uint64_t>>& out) {
  std::string tok;
  const Fr ten = Fr::from_u64(10);
  auto flush = [&]() {
    if (tok.empty() || tok == "-" || tok == "+") {
      tok.clear();
      return;
    }
    const bool neg = tok[0] == '-';
    const size_t s = (tok[0] == '-' || tok[0] == '+') ? 1 : 0;
    Fr v = Fr::zero();
    for (size_t i = s; i < tok.size(); i++) v = v * ten + Fr::from_u64((uint64_t)(tok[i] - '0'));
    if (neg) v = -v;
    std::vector<uint64_t> w(4);
    v.to_std(w.data());
    out.push_back(w);
    tok.clear();
  };
  for (uint8_t ch : text) {
    const char c = (char)ch;
    if ((c >= '0' && c <= '9') || c == '-' || c == '+') {
      if ((c == '-' || c == '+') && !tok.empty()) flush();
      tok.push_back(c);
    } else {
      flush();
    }
  }
  flush();
  return !out.empty();
}

bool ends_with_json(const char* path) {
  const size_t n = strlen(path);
  if (n < 5) return false;
  std::string t(path + n - 5);
  for (char& c : t) c = (char)tolower((unsigned char)c);
  return t == ".json";
}

}  // namespace

extern "C" {

static int zk_pairing_impl(const void* p_std, const void* q_std, void* out_std) {
  if (!p_std || !q_std || !out_std) return ZK_ERR_INVALID;
  const Fq12 f = pairing(g1_std((const uint8_t*)p_std), g2_std((const uint8_t*)q_std));
  const Fq2* c[6] = {&f.c0.c0, &f.c0.c1, &f.c0.c2, &f.c1.c0, &f.c1.c1, &f.c1.c2};
  uint64_t* o = (uint64_t*)out_std;
  for (int i = 0; i < 6; i++) {
    c[i]->c0.to_std(o + 8 * i);
    c[i]->c1.to_std(o + 8 * i + 4);
  }
  return ZK_OK;
}

int zk_pairing(const void* p_std, const void* q_std, void* out_std) {
  return zkh::abi_guard([&] { return zk_pairing_impl(p_std, q_std, out_std); });
}

static int zk_verify_impl(const void* vk_bytes, size_t vk_len, const void* proof256, const void* publics_std, int npub,
                          int* valid) {
  if (!vk_bytes || !proof256 || !valid || npub < 0 || (npub > 0 && !publics_std)) return ZK_ERR_INVALID;
  *valid = 0;
  VerifyingKey vk;
  {
    const int st = parse_vk((const uint8_t*)vk_bytes, vk_len, vk);
    if (st != ZK_OK) return st;
  }
  const uint8_t* pr = (const uint8_t*)proof256;
  const G1A A = g1_std(pr), C = g1_std(pr + 192);
  const G2A B = g2_std(pr + 64);
  std::vector<std::vector<uint64_t>> pub((size_t)npub, std::vector<uint64_t>(4));
  for (int i = 0; i < npub; i++) memcpy(pub[i].data(), (const uint8_t*)publics_std + 32 * (size_t)i, 32);
  *valid = groth16_verify(vk, A, B, C, pub) ? 1 : 0;
  return ZK_OK;
}

int zk_verify(const void* vk_bytes, size_t vk_len, const void* proof256, const void* publics_std, int npub,
              int* valid) {
  return zkh::abi_guard([&] { return zk_verify_impl(vk_bytes, vk_len, proof256, publics_std, npub, valid); });
}

static int zk_verify_files_impl(const char* vk_path, const char* proof_path, const char* publics_path, int* valid) {
  if (!vk_path || !proof_path || !publics_path || !valid) return ZK_ERR_INVALID;
  *valid = 0;
  std::vector<uint8_t> vkb, prb, pubb;
  if (!read_file(vk_path, vkb) || !read_file(proof_path, prb) || !read_file(publics_path, pubb)) return ZK_ERR_IO;
  if (prb.size() != 256) return ZK_ERR_IO;  // groth16 proof files are exactly 256 bytes
  std::vector<std::vector<uint64_t>> pub;
  if (ends_with_json(publics_path)) {
    if (!parse_public_json(pubb, pub)) return ZK_ERR_IO;
  } else {
    int32_t n;
    if (pubb.size() < 4) return ZK_ERR_IO;
    memcpy(&n, pubb.data(), 4);
    if (n < 0 || pubb.size() < 4 + 32 * (size_t)n) return ZK_ERR_IO;
    for (int32_t i = 0; i < n; i++) {
      std::vector<uint64_t> w(4);
      memcpy(w.data(), pubb.data() + 4 + 32 * (size_t)i, 32);
      pub.push_back(w);
    }
  }
  std::vector<uint8_t> flat(pub.size() * 32);
  for (size_t i = 0; i < pub.size(); i++) memcpy(flat.data() + 32 * i, pub[i].data(), 32);
  return zk_verify(vkb.data(), vkb.size(), prb.data(), flat.data(), (int)pub.size(), valid);
}

int zk_verify_files(const char* vk_path, const char* proof_path, const char* publics_path, int* valid) {
  return zkh::abi_guard([&] { return zk_verify_files_impl(vk_path, proof_path, publics_path, valid); });
}

}  // extern "C"
