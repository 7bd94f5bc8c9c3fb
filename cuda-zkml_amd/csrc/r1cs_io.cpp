// R1CS and witness files in the iden3 binary formats (circom / snarkjs:
// .r1cs version 1, .wtns version 2) and the synthetic large R1CS of the
// benchmark's config 5.  Host code, no device involved.
//
// Export follows the reference's writer (src/prover/r1cs_export.cuh:41-92):
//  - header: n8 = 32, prime r, nWires = num_variables, nPubOut = num_public,
//    nPubIn = 0, nPrvIn = num_private, nLabels = num_variables, mConstraints;
//  - constraints: per row the A, B, C linear combinations, terms in the order
//    they appear in the COO arrays, coefficients in standard form;
//  - wire-to-label map: identity.
// The reader accepts any section order and nPubIn > 0 (public count =
// nPubOut + nPubIn, circom's public wires 1..nPubOut+nPubIn) and checks the
// prime.  Matrix values cross the C ABI in the reference's in-memory form
// (Montgomery, R = 2^256).
#include <stdint.h>
#include <stdio.h>
#include <string.h>

#include <random>
#include <vector>

#include "abi_guard.hpp"
#include "../../include/zkml_gpu.h"
#include "host_bn254.hpp"

using zkh::Fr;

namespace {

void put_u32(std::vector<uint8_t>& b, uint32_t v) {
  for (int i = 0; i < 4; i++) b.push_back((uint8_t)(v >> (8 * i)));
}
void put_u64(std::vector<uint8_t>& b, uint64_t v) {
  for (int i = 0; i < 8; i++) b.push_back((uint8_t)(v >> (8 * i)));
}
void put_std(std::vector<uint8_t>& b, const uint64_t mont[4]) {
  uint64_t s[4];
  Fr::raw(mont).to_std(s);
  for (int k = 0; k < 4; k++) put_u64(b, s[k]);
}
void put_prime(std::vector<uint8_t>& b) {
  for (int k = 0; k < 4; k++) put_u64(b, zkh::RMod::M[k]);
}
void put_section(std::vector<uint8_t>& out, uint32_t type, const std::vector<uint8_t>& body) {
  put_u32(out, type);
  put_u64(out, (uint64_t)body.size());
  out.insert(out.end(), body.begin(), body.end());
}
bool write_file(const char* path, const std::vector<uint8_t>& b) {
  FILE* f = fopen(path, "wb");
  if (!f) return false;
  const bool ok = fwrite(b.data(), 1, b.size(), f) == b.size();
  return fclose(f) == 0 && ok;
}
bool read_file(const char* path, std::vector<uint8_t>& out) {
  FILE* f = fopen(path, "rb");
  if (!f) return false;
  if (fseek(f, 0, SEEK_END) != 0) {
    fclose(f);
    return false;
  }
  const long sz = ftell(f);
  if (sz < 0 || fseek(f, 0, SEEK_SET) != 0) {
    fclose(f);
    return false;
  }
  out.resize((size_t)sz);
  const bool ok = fread(out.data(), 1, out.size(), f) == out.size();
  fclose(f);
  return ok;
}

struct Reader {
  const uint8_t* p;
  size_t n, o = 0;
  bool ok = true;
  bool need(size_t k) {
    if (!ok || o + k > n) ok = false;
    return ok;
  }
  uint32_t u32() {
    if (!need(4)) return 0;
    uint32_t v;
    memcpy(&v, p + o, 4);
    o += 4;
    return v;
  }
  uint64_t u64() {
    if (!need(8)) return 0;
    uint64_t v;
    memcpy(&v, p + o, 8);
    o += 8;
    return v;
  }
  const uint8_t* bytes(size_t k) {
    if (!need(k)) return nullptr;
    const uint8_t* r = p + o;
    o += k;
    return r;
  }
};

bool is_prime_r(const uint8_t* b) { return memcmp(b, zkh::RMod::M, 32) == 0; }

// standard-form bytes (< r) -> Montgomery words
bool std_to_mont(const uint8_t* b, uint64_t out[4]) {
  uint64_t s[4];
  memcpy(s, b, 32);
  for (int k = 3; k >= 0; k--) {  // must be canonical
    if (s[k] != zkh::RMod::M[k]) {
      if (s[k] > zkh::RMod::M[k]) return false;
      break;
    }
    if (k == 0) return false;  // equal to r
  }
  memcpy(out, Fr::from_std(s).v, 32);
  return true;
}

struct Sections {
  const uint8_t* sec[4] = {nullptr, nullptr, nullptr, nullptr};
  uint64_t len[4] = {0, 0, 0, 0};
};

int scan_sections(const std::vector<uint8_t>& f, const char magic[4], uint32_t version, Sections& s) {
  Reader r{f.data(), f.size()};
  const uint8_t* m = r.bytes(4);
  if (!m || memcmp(m, magic, 4) != 0) return ZK_ERR_IO;
  if (r.u32() != version) return ZK_ERR_IO;
  const uint32_t nsec = r.u32();
  for (uint32_t i = 0; i < nsec && r.ok; i++) {
    const uint32_t type = r.u32();
    const uint64_t len = r.u64();
    if (!r.ok || len > f.size() - r.o) return ZK_ERR_IO;
    if (type >= 1 && type <= 3) {
      s.sec[type] = f.data() + r.o;
      s.len[type] = len;
    }
    r.o += (size_t)len;
  }
  return r.ok ? ZK_OK : ZK_ERR_IO;
}

struct R1csHeader {
  uint32_t nwires, npubout, npubin, nprvin, m;
};

int r1cs_header(const Sections& s, R1csHeader& h) {
  if (!s.sec[1] || !s.sec[2]) return ZK_ERR_IO;
  Reader r{s.sec[1], (size_t)s.len[1]};
  if (r.u32() != 32) return ZK_ERR_IO;
  const uint8_t* pr = r.bytes(32);
  if (!pr || !is_prime_r(pr)) return ZK_ERR_IO;
  h.nwires = r.u32();
  h.npubout = r.u32();
  h.npubin = r.u32();
  h.nprvin = r.u32();
  (void)r.u64();  // nLabels
  h.m = r.u32();
  if (!r.ok || h.nwires == 0 || h.m > (1u << 30) || (uint64_t)h.npubout + h.npubin + 1 > h.nwires) return ZK_ERR_IO;
  return ZK_OK;
}

// Walk the constraint section; with A/B/C null only count the terms.
int r1cs_constraints(const Sections& s, const R1csHeader& h, zk_sparse_entry* out[3], size_t cnt[3]) {
  Reader r{s.sec[2], (size_t)s.len[2]};
  cnt[0] = cnt[1] = cnt[2] = 0;
  for (uint32_t row = 0; row < h.m; row++) {
    for (int k = 0; k < 3; k++) {
      const uint32_t terms = r.u32();
      if (!r.ok || (uint64_t)terms * 36 > s.len[2] - r.o) return ZK_ERR_IO;
      for (uint32_t t = 0; t < terms; t++) {
        const uint32_t wire = r.u32();
        const uint8_t* v = r.bytes(32);
        if (!r.ok || wire >= h.nwires) return ZK_ERR_IO;
        if (out[k]) {
          zk_sparse_entry& e = out[k][cnt[k]];
          e.row = (int32_t)row;
          e.col = (int32_t)wire;
          if (!std_to_mont(v, e.value)) return ZK_ERR_IO;
        }
        cnt[k]++;
      }
    }
  }
  return r.ok && r.o == s.len[2] ? ZK_OK : ZK_ERR_IO;
}

// uniform element of [0, r) in Montgomery form (rejection sampling on the low
// 254 bits of four draws)
void random_fr(std::mt19937_64& rng, uint64_t out[4]) {
  uint64_t s[4];
  for (;;) {
    for (int k = 0; k < 4; k++) s[k] = rng();
    s[3] &= (1ULL << 62) - 1;
    bool less = false;
    for (int k = 3; k >= 0; k--)
      if (s[k] != zkh::RMod::M[k]) {
        less = s[k] < zkh::RMod::M[k];
        break;
      }
    if (less) break;
  }
  memcpy(out, Fr::from_std(s).v, 32);
}

}  // namespace

extern "C" {

static int zk_iden3_r1cs_info_impl(const char* path, int* num_constraints, int* num_variables, int* num_public,
                                   int* num_private, size_t* nA, size_t* nB, size_t* nC) {
  if (!path || !num_constraints || !num_variables || !num_public || !num_private || !nA || !nB || !nC)
    return ZK_ERR_INVALID;
  std::vector<uint8_t> f;
  if (!read_file(path, f)) return ZK_ERR_IO;
  Sections s;
  R1csHeader h;
  int st = scan_sections(f, "r1cs", 1, s);
  if (st == ZK_OK) st = r1cs_header(s, h);
  if (st != ZK_OK) return st;
  zk_sparse_entry* none[3] = {nullptr, nullptr, nullptr};
  size_t cnt[3];
  if ((st = r1cs_constraints(s, h, none, cnt)) != ZK_OK) return st;
  *num_constraints = (int)h.m;
  *num_variables = (int)h.nwires;
  *num_public = (int)(h.npubout + h.npubin);
  *num_private = (int)h.nprvin;
  *nA = cnt[0];
  *nB = cnt[1];
  *nC = cnt[2];
  return ZK_OK;
}

int zk_iden3_r1cs_info(const char* path, int* num_constraints, int* num_variables, int* num_public,
                       int* num_private, size_t* nA, size_t* nB, size_t* nC) {
  return zkh::abi_guard([&] {
    return zk_iden3_r1cs_info_impl(path, num_constraints, num_variables, num_public, num_private, nA, nB, nC);
  });
}

static int zk_iden3_r1cs_read_impl(const char* path, zk_sparse_entry* A, zk_sparse_entry* B, zk_sparse_entry* C) {
  if (!path) return ZK_ERR_INVALID;
  std::vector<uint8_t> f;
  if (!read_file(path, f)) return ZK_ERR_IO;
  Sections s;
  R1csHeader h;
  int st = scan_sections(f, "r1cs", 1, s);
  if (st == ZK_OK) st = r1cs_header(s, h);
  if (st != ZK_OK) return st;
  zk_sparse_entry* none[3] = {nullptr, nullptr, nullptr};
  size_t cnt[3];
  if ((st = r1cs_constraints(s, h, none, cnt)) != ZK_OK) return st;
  if ((cnt[0] && !A) || (cnt[1] && !B) || (cnt[2] && !C)) return ZK_ERR_INVALID;
  zk_sparse_entry* out[3] = {A, B, C};
  return r1cs_constraints(s, h, out, cnt);
}

int zk_iden3_r1cs_read(const char* path, zk_sparse_entry* A, zk_sparse_entry* B, zk_sparse_entry* C) {
  return zkh::abi_guard([&] { return zk_iden3_r1cs_read_impl(path, A, B, C); });
}

static int zk_iden3_r1cs_write_impl(const char* path, int num_constraints, int num_variables, int num_public,
                                    int num_private, const zk_sparse_entry* A, size_t nA, const zk_sparse_entry* B,
                                    size_t nB, const zk_sparse_entry* C, size_t nC) {
  if (!path || num_constraints < 0 || num_variables <= 0 || num_public < 0 || num_private < 0 ||
      (nA && !A) || (nB && !B) || (nC && !C))
    return ZK_ERR_INVALID;
  const size_t m = (size_t)num_constraints;
  const zk_sparse_entry* mats[3] = {A, B, C};
  const size_t cnts[3] = {nA, nB, nC};
  // per-row term lists in COO order (rows outside [0, m) are not exported)
  std::vector<uint32_t> start[3];
  std::vector<const zk_sparse_entry*> terms[3];
  for (int k = 0; k < 3; k++) {
    start[k].assign(m + 1, 0);
    for (size_t i = 0; i < cnts[k]; i++)
      if (mats[k][i].row >= 0 && (size_t)mats[k][i].row < m) start[k][mats[k][i].row + 1]++;
    for (size_t r = 0; r < m; r++) start[k][r + 1] += start[k][r];
    terms[k].resize(start[k][m]);
    std::vector<uint32_t> fill(start[k].begin(), start[k].end() - 1);
    for (size_t i = 0; i < cnts[k]; i++)
      if (mats[k][i].row >= 0 && (size_t)mats[k][i].row < m) terms[k][fill[mats[k][i].row]++] = &mats[k][i];
  }
  std::vector<uint8_t> hdr, cons, map, out;
  put_u32(hdr, 32);
  put_prime(hdr);
  put_u32(hdr, (uint32_t)num_variables);
  put_u32(hdr, (uint32_t)num_public);
  put_u32(hdr, 0);
  put_u32(hdr, (uint32_t)num_private);
  put_u64(hdr, (uint64_t)num_variables);
  put_u32(hdr, (uint32_t)m);
  for (size_t r = 0; r < m; r++)
    for (int k = 0; k < 3; k++) {
      put_u32(cons, start[k][r + 1] - start[k][r]);
      for (uint32_t t = start[k][r]; t < start[k][r + 1]; t++) {
        put_u32(cons, (uint32_t)terms[k][t]->col);
        put_std(cons, terms[k][t]->value);
      }
    }
  for (int i = 0; i < num_variables; i++) put_u64(map, (uint64_t)i);
  out.insert(out.end(), {'r', '1', 'c', 's'});
  put_u32(out, 1);
  put_u32(out, 3);
  put_section(out, 1, hdr);
  put_section(out, 2, cons);
  put_section(out, 3, map);
  return write_file(path, out) ? ZK_OK : ZK_ERR_IO;
}

int zk_iden3_r1cs_write(const char* path, int num_constraints, int num_variables, int num_public, int num_private,
                        const zk_sparse_entry* A, size_t nA, const zk_sparse_entry* B, size_t nB,
                        const zk_sparse_entry* C, size_t nC) {
  return zkh::abi_guard([&] {
    return zk_iden3_r1cs_write_impl(path, num_constraints, num_variables, num_public, num_private, A, nA, B, nB, C, nC);
  });
}

static int zk_wtns_info_impl(const char* path, size_t* m) {
  if (!path || !m) return ZK_ERR_INVALID;
  std::vector<uint8_t> f;
  if (!read_file(path, f)) return ZK_ERR_IO;
  Sections s;
  int st = scan_sections(f, "wtns", 2, s);
  if (st != ZK_OK) return st;
  if (!s.sec[1] || !s.sec[2]) return ZK_ERR_IO;
  Reader r{s.sec[1], (size_t)s.len[1]};
  if (r.u32() != 32) return ZK_ERR_IO;
  const uint8_t* pr = r.bytes(32);
  const uint32_t n = r.u32();
  if (!r.ok || !is_prime_r(pr) || s.len[2] != (uint64_t)n * 32) return ZK_ERR_IO;
  *m = n;
  return ZK_OK;
}

int zk_wtns_info(const char* path, size_t* m) {
  return zkh::abi_guard([&] { return zk_wtns_info_impl(path, m); });
}

static int zk_wtns_read_impl(const char* path, void* w_mont, size_t m) {
  size_t n = 0;
  int st = zk_wtns_info(path, &n);
  if (st != ZK_OK) return st;
  if (n != m || (m && !w_mont)) return ZK_ERR_INVALID;
  std::vector<uint8_t> f;
  if (!read_file(path, f)) return ZK_ERR_IO;
  Sections s;
  if ((st = scan_sections(f, "wtns", 2, s)) != ZK_OK) return st;
  uint64_t* w = (uint64_t*)w_mont;
  for (size_t i = 0; i < m; i++)
    if (!std_to_mont(s.sec[2] + 32 * i, w + 4 * i)) return ZK_ERR_IO;
  return ZK_OK;
}

int zk_wtns_read(const char* path, void* w_mont, size_t m) {
  return zkh::abi_guard([&] { return zk_wtns_read_impl(path, w_mont, m); });
}

static int zk_wtns_write_impl(const char* path, const void* w_mont, size_t m) {
  if (!path || (m && !w_mont) || m > 0xffffffffu) return ZK_ERR_INVALID;
  const uint64_t* w = (const uint64_t*)w_mont;
  std::vector<uint8_t> hdr, vals, out;
  put_u32(hdr, 32);
  put_prime(hdr);
  put_u32(hdr, (uint32_t)m);
  for (size_t i = 0; i < m; i++) put_std(vals, w + 4 * i);
  out.insert(out.end(), {'w', 't', 'n', 's'});
  put_u32(out, 2);
  put_u32(out, 2);
  put_section(out, 1, hdr);
  put_section(out, 2, vals);
  return write_file(path, out) ? ZK_OK : ZK_ERR_IO;
}

int zk_wtns_write(const char* path, const void* w_mont, size_t m) {
  return zkh::abi_guard([&] { return zk_wtns_write_impl(path, w_mont, m); });
}

static int zk_synthetic_r1cs_impl(int num_constraints, int num_public, int num_inputs, uint64_t seed,
                                  zk_sparse_entry* A, size_t* nA, zk_sparse_entry* B, size_t* nB, zk_sparse_entry* C,
                                  size_t* nC, void* w_mont) {
  if (num_constraints < 0 || num_public < 0 || num_inputs < 0 || !nA || !nB || !nC || !w_mont ||
      (num_constraints > 0 && (!A || !B || !C)))
    return ZK_ERR_INVALID;
  const size_t nv = 1 + (size_t)num_public + (size_t)num_inputs + (size_t)num_constraints;
  if (nv > 0x7fffffffu) return ZK_ERR_SIZE;
  std::mt19937_64 rng(seed);
  Fr* w = (Fr*)w_mont;
  w[0] = Fr::one();
  size_t have = 1;
  for (int i = 0; i < num_public + num_inputs; i++) random_fr(rng, w[have++].v);
  size_t ka = 0, kb = 0, kc = 0;
  for (int row = 0; row < num_constraints; row++) {
    Fr lin[2];
    zk_sparse_entry* mats[2] = {A, B};
    size_t* cnt[2] = {&ka, &kb};
    for (int s = 0; s < 2; s++) {
      lin[s] = Fr::zero();
      const int terms = 1 + (int)(rng() % 3);
      for (int t = 0; t < terms; t++) {
        zk_sparse_entry& e = mats[s][(*cnt[s])++];
        e.row = row;
        e.col = (int32_t)(rng() % have);
        random_fr(rng, e.value);
        lin[s] = lin[s] + Fr::raw(e.value) * w[e.col];
      }
    }
    zk_sparse_entry& e = C[kc++];
    e.row = row;
    e.col = (int32_t)have;
    memcpy(e.value, Fr::one().v, 32);
    w[have++] = lin[0] * lin[1];
  }
  *nA = ka;
  *nB = kb;
  *nC = kc;
  return ZK_OK;
}

int zk_synthetic_r1cs(int num_constraints, int num_public, int num_inputs, uint64_t seed, zk_sparse_entry* A,
                      size_t* nA, zk_sparse_entry* B, size_t* nB, zk_sparse_entry* C, size_t* nC, void* w_mont) {
  return zkh::abi_guard([&] {
    return zk_synthetic_r1cs_impl(num_constraints, num_public, num_inputs, seed, A, nA, B, nB, C, nC, w_mont);
  });
}

}  // extern "C"
