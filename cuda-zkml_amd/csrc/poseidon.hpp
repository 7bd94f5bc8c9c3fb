// Poseidon over the BN254 scalar field: t = 3, S-box x^5, R_F = 8 full and
// R_P = 57 partial rounds -- the circomlib / Poseidon-reference instance that
// the reference's statement builder uses (src/prover/gadgets.cuh:323-393,
// constants in src/prover/poseidon_constants.cuh).
//
// The 195 round constants and the 3x3 MDS matrix are not tabulated here.
// They are regenerated once, on first use, with the Grain LFSR procedure of
// the Poseidon paper (Grassi, Khovratovich, Rechberger, Roy, Schofnegger,
// "Poseidon", USENIX Security 2021, Appendix F, and its
// generate_parameters_grain.sage), which is also how the reference produces
// its table (python/zkml/poseidon.py:36-88):
//   - an 80-bit LFSR seeded with field = 1 (2 bits), S-box = 0 (4), n = 254
//     (12), t = 3 (12), R_F (10), R_P (10) and thirty 1 bits, MSB first;
//     feedback b[62] ^ b[51] ^ b[38] ^ b[23] ^ b[13] ^ b[0]; 160 warm-up clocks;
//   - output by self-shrinking: clock pairs (b1, b2), emit b2 when b1 = 1;
//   - a field element is 254 emitted bits read MSB first; round constants
//     reject values >= r; the 2t = 6 MDS seeds x_0..2, y_0..2 that follow are
//     reduced mod r, and M[i][j] = (x_i + y_j)^-1 (Cauchy matrix).
// Host code.
#pragma once
#include <stdint.h>
#include <string.h>

#include <vector>

#include "host_bn254.hpp"

namespace zkh {

struct Poseidon {
  static constexpr int T = 3, RF = 8, RP = 57, ROUNDS = RF + RP, NRC = ROUNDS * T;
  static constexpr int FIELD_BITS = 254;
  // sponge domains of the statement commitments (src/prover/poseidon_constants.cuh:212-213)
  static constexpr uint64_t DOMAIN_MODEL = 0x4d4f44454cULL;  // "MODEL"
  static constexpr uint64_t DOMAIN_INPUT = 0x494e505554ULL;  // "INPUT"

  Fr rc[NRC];
  Fr mds[T][T];

  static const Poseidon& get() {
    static const Poseidon p;  // thread-safe one-time initialisation
    return p;
  }

  void permute(Fr s[T]) const {
    for (int r = 0; r < ROUNDS; r++) {
      for (int i = 0; i < T; i++) s[i] = s[i] + rc[r * T + i];
      if (full_round(r)) {
        for (int i = 0; i < T; i++) s[i] = sbox(s[i]);
      } else {
        s[0] = sbox(s[0]);
      }
      Fr n[T];
      for (int i = 0; i < T; i++) n[i] = mds[i][0] * s[0] + mds[i][1] * s[1] + mds[i][2] * s[2];
      for (int i = 0; i < T; i++) s[i] = n[i];
    }
  }
  static bool full_round(int r) { return r < RF / 2 || r >= RF / 2 + RP; }
  static Fr sbox(const Fr& x) {
    const Fr x2 = x * x, x4 = x2 * x2;
    return x4 * x;
  }

 private:
  struct Grain {
    uint8_t b[80];
    int head = 0;  // b[(head + i) % 80] is the i-th oldest bit
    Grain() {
      int k = 0;
      auto put = [&](uint32_t v, int bits) {
        for (int i = bits - 1; i >= 0; i--) b[k++] = (uint8_t)((v >> i) & 1);
      };
      put(1, 2);  // prime field
      put(0, 4);  // S-box x^alpha
      put(FIELD_BITS, 12);
      put(T, 12);
      put(RF, 10);
      put(RP, 10);
      while (k < 80) b[k++] = 1;
      for (int i = 0; i < 160; i++) clock();
    }
    uint8_t at(int i) const { return b[(head + i) % 80]; }
    uint8_t clock() {
      const uint8_t nb = at(62) ^ at(51) ^ at(38) ^ at(23) ^ at(13) ^ at(0);
      b[head] = nb;  // the oldest bit leaves, the new one enters at the end
      head = (head + 1) % 80;
      return nb;
    }
    uint8_t bit() {
      for (;;) {
        const uint8_t b1 = clock(), b2 = clock();
        if (b1) return b2;
      }
    }
    // n bits, MSB first, into a little-endian 4-limb integer
    void raw(uint64_t out[4], int n) {
      memset(out, 0, 32);
      for (int i = 0; i < n; i++) {
        const uint64_t carry2 = out[2] >> 63, carry1 = out[1] >> 63, carry0 = out[0] >> 63;
        out[3] = (out[3] << 1) | carry2;
        out[2] = (out[2] << 1) | carry1;
        out[1] = (out[1] << 1) | carry0;
        out[0] = (out[0] << 1) | bit();
      }
    }
  };

  static bool below_r(const uint64_t v[4]) {
    for (int i = 3; i >= 0; i--) {
      if (v[i] != RMod::M[i]) return v[i] < RMod::M[i];
    }
    return false;
  }

  Poseidon() {
    Grain g;
    uint64_t v[4];
    for (int i = 0; i < NRC; i++) {
      do g.raw(v, FIELD_BITS);
      while (!below_r(v));
      rc[i] = Fr::from_std(v);  // canonical input: from_std is exact
    }
    for (;;) {
      Fr xy[2 * T];
      for (int i = 0; i < 2 * T; i++) {
        g.raw(v, FIELD_BITS);
        xy[i] = Fr::from_std(v);  // reduces v < 2^254 mod r
      }
      bool ok = true;
      for (int i = 0; i < 2 * T && ok; i++)
        for (int j = i + 1; j < 2 * T && ok; j++) ok = !(xy[i] == xy[j]);
      for (int i = 0; i < T && ok; i++)
        for (int j = 0; j < T && ok; j++) ok = !(xy[i] + xy[T + j]).is_zero();
      if (!ok) continue;
      for (int i = 0; i < T; i++)
        for (int j = 0; j < T; j++) mds[i][j] = (xy[i] + xy[T + j]).inv();
      break;
    }
  }
};

// 2^k in the field
inline Fr fr_pow2(int k) {
  Fr x = Fr::one();
  for (int i = 0; i < k; i++) x = x + x;
  return x;
}

// circomlib Poseidon([a, b]) = permute(0, a, b)[0] (reference gadgets.cuh:360-364)
inline Fr poseidon_hash2(const Fr& a, const Fr& b) {
  Fr s[3] = {Fr::zero(), a, b};
  Poseidon::get().permute(s);
  return s[0];
}

// Rate-2 sponge commitment with capacity (len << 64) | domain, two values
// absorbed per permutation (zero padded), output s[1]
// (reference gadgets.cuh:416-427).
inline Fr poseidon_commit(const std::vector<Fr>& vals, uint64_t domain) {
  const Poseidon& P = Poseidon::get();
  Fr s[3] = {fr_pow2(64) * Fr::from_u64((uint64_t)vals.size()) + Fr::from_u64(domain), Fr::zero(), Fr::zero()};
  const size_t n = vals.empty() ? 2 : vals.size() + (vals.size() % 2);
  for (size_t i = 0; i < n; i += 2) {
    s[1] = s[1] + (i < vals.size() ? vals[i] : Fr::zero());
    s[2] = s[2] + (i + 1 < vals.size() ? vals[i + 1] : Fr::zero());
    P.permute(s);
  }
  return s[1];
}

}  // namespace zkh
