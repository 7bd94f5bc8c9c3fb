// Statement producer: one R1CS + witness for B samples of a quantized model,
// built in a single traced pass (every gadget adds its constraints and
// assigns its witness values together).  Replaces the reference's
// TracedBuilder gadgets (src/prover/gadgets.cuh:128-457) and
// build_statement_v2 / statement_v2_meta_json (src/prover/statement_v2.cuh:
// 82-287).  Host code, no device involved.
//
// The output must be the reference's R1CS term for term -- same variable
// numbering, same row order, same terms in the same order, zero coefficients
// included -- because the proving key, the public-input layout and the iden3
// files all depend on it.  So the allocation and emission order below follows
// the reference gadget by gadget:
//   - constrain(a, b, c) merges repeated variables of each combination
//     (first occurrence keeps its place) and drops zero terms;
//   - linear(lhs, out) is the row  compress(lhs) * 1 = out;
//   - the linear and convolution layers and the model-tag row emit their term
//     lists as built (bias term last, even when zero), uncompressed;
//   - Poseidon carries its state as linear combinations, spends three rows
//     per S-box (x^2, x^4, x^5) and materialises a state word as a fresh
//     variable when its combination grows beyond 8 terms.
// Integers v are the field elements v mod r; model and input values outside
// (-2^62, 2^62) become 0, as the reference's Fp -> int64 conversion does
// (src/nn/exact_layers.cuh:15-23, statement_v2.cuh:59-63).
#include <stdint.h>
#include <stdio.h>
#include <string.h>

#include <string>
#include <utility>
#include <vector>

#include "abi_guard.hpp"
#include "../../include/zkml_gpu.h"
#include "host_bn254.hpp"
#include "poseidon.hpp"

using zkh::Fr;
using zkh::Poseidon;

namespace {

typedef std::vector<std::pair<int, Fr>> LC;

Fr fr_u64(uint64_t v) { return Fr::from_u64(v); }

Fr fr_i64(int64_t v) {
  if (v >= 0) return fr_u64((uint64_t)v);
  return -fr_u64((uint64_t)(-(v + 1)) + 1u);
}

// Model / input value -> field element (zero outside (-2^62, 2^62)).
Fr fr_signed(int64_t v) {
  const int64_t lim = (int64_t)1 << 62;
  if (v >= lim || v <= -lim) return Fr::zero();
  return fr_i64(v);
}

// Signed view of a field element when |x| < 2^62.
bool fr_to_i64(const Fr& x, int64_t* out) {
  uint64_t s[4];
  x.to_std(s);
  if (!s[1] && !s[2] && !s[3] && s[0] < (1ULL << 62)) {
    *out = (int64_t)s[0];
    return true;
  }
  (-x).to_std(s);
  if (!s[1] && !s[2] && !s[3] && s[0] < (1ULL << 62)) {
    *out = -(int64_t)s[0];
    return true;
  }
  return false;
}

Fr fr_std4(const uint64_t v[4]) {
  // standard-form input, reduced mod r if >= r
  return Fr::from_std(v);
}

LC compress(const LC& lc) {
  LC merged;
  for (const auto& t : lc) {
    bool found = false;
    for (auto& m : merged)
      if (m.first == t.first) {
        m.second = m.second + t.second;
        found = true;
        break;
      }
    if (!found) merged.push_back(t);
  }
  LC out;
  for (const auto& t : merged)
    if (!t.second.is_zero()) out.push_back(t);
  return out;
}

// ------------------------------------------------------------ traced builder
struct Tracer {
  std::vector<Fr> w{Fr::one()};  // w[0] = 1
  int next_var = 1;
  int rows = 0;
  std::vector<zk_sparse_entry> A, B, C;

  int var(const Fr& v) {
    const int idx = next_var++;
    if ((int)w.size() <= idx) w.resize((size_t)idx + 1, Fr::zero());
    w[(size_t)idx] = v;
    return idx;
  }
  int var_unset() { return var(Fr::zero()); }
  void set(int idx, const Fr& v) {
    if ((int)w.size() <= idx) w.resize((size_t)idx + 1, Fr::zero());
    w[(size_t)idx] = v;
  }
  const Fr& val(int idx) const { return w[(size_t)idx]; }
  Fr eval(const LC& lc) const {
    Fr acc = Fr::zero();
    for (const auto& t : lc) acc = acc + t.second * w[(size_t)t.first];
    return acc;
  }

  static void put(std::vector<zk_sparse_entry>& m, int row, int col, const Fr& c) {
    zk_sparse_entry e;
    e.row = row;
    e.col = col;
    memcpy(e.value, c.v, 32);
    m.push_back(e);
  }
  // raw rows (terms as given)
  void row(const LC& a, const LC& b, const LC& c) {
    const int r = rows++;
    for (const auto& t : a) put(A, r, t.first, t.second);
    for (const auto& t : b) put(B, r, t.first, t.second);
    for (const auto& t : c) put(C, r, t.first, t.second);
  }
  void row_linear(const LC& a, const LC& c) { row(a, LC{{0, Fr::one()}}, c); }
  // canonical rows
  void constrain(const LC& a, const LC& b, const LC& c) { row(compress(a), compress(b), compress(c)); }
  void linear(const LC& lhs, int out) { row_linear(compress(lhs), LC{{out, Fr::one()}}); }
  void constrain_zero(const LC& lc) { constrain(lc, LC{{0, Fr::one()}}, LC{}); }
  void mul(int x, int y, int z) { row(LC{{x, Fr::one()}}, LC{{y, Fr::one()}}, LC{{z, Fr::one()}}); }
};

// ------------------------------------------------------------------ gadgets
// ctx * ctx = ctx_sq binds a public context value (gadgets.cuh:155-160)
int context_binding(Tracer& t, int ctx) {
  const int sq = t.var(t.val(ctx) * t.val(ctx));
  t.mul(ctx, ctx, sq);
  return sq;
}

// k boolean variables b_i (LSB first) with sum 2^i b_i = lc + offset
// (gadgets.cuh:165-186); sound for values in [0, 2^k).
std::vector<int> bits_of(Tracer& t, const LC& lc, const Fr& offset, int k) {
  uint64_t s[4];
  (t.eval(lc) + offset).to_std(s);
  std::vector<int> bits((size_t)k);
  LC sum;
  Fr pw = Fr::one();
  for (int i = 0; i < k; i++) {
    const uint64_t b = (s[i / 64] >> (i % 64)) & 1;
    const int bv = t.var(fr_u64(b));
    bits[(size_t)i] = bv;
    t.constrain(LC{{bv, Fr::one()}}, LC{{bv, Fr::one()}, {0, -Fr::one()}}, LC{});
    sum.push_back({bv, pw});
    pw = pw + pw;
  }
  LC diff = sum;
  for (const auto& term : lc) diff.push_back({term.first, -term.second});
  diff.push_back({0, -offset});
  t.constrain_zero(diff);
  return bits;
}

// x in [-2^(k-1), 2^(k-1))
std::vector<int> signed_range(Tracer& t, int x, int k) {
  return bits_of(t, LC{{x, Fr::one()}}, zkh::fr_pow2(k - 1), k);
}

// y = [z >= 0] * z via the top bit of z + 2^(k-1) (gadgets.cuh:195-201)
int relu_exact(Tracer& t, int z, int k) {
  const std::vector<int> bits = signed_range(t, z, k);
  const int s = bits[(size_t)k - 1];
  const int y = t.var(t.val(s) * t.val(z));
  t.mul(s, z, y);
  return y;
}

// q = floor(y / 2^shift), remainder in [0, 2^shift), q in [-2^(kq-1), 2^(kq-1))
// (gadgets.cuh:205-217)
int rescale(Tracer& t, int y, int shift, int kq) {
  if (shift <= 0) return y;
  int64_t yv = 0;
  fr_to_i64(t.val(y), &yv);
  const int64_t q = yv >> shift;  // arithmetic shift: floor
  const int64_t r = yv - (int64_t)((uint64_t)q << shift);
  const int qv = t.var(fr_i64(q));
  const int rv = t.var(fr_i64(r));
  bits_of(t, LC{{rv, Fr::one()}}, Fr::zero(), shift);
  signed_range(t, qv, kq);
  t.constrain_zero(LC{{qv, zkh::fr_pow2(shift)}, {rv, Fr::one()}, {y, -Fr::one()}});
  return qv;
}

// f = [x - y - thr >= 0] for differences in [-2^(k-1), 2^(k-1)) (gadgets.cuh:221-225)
int geq_flag(Tracer& t, int x, int y, int64_t thr, int k) {
  const LC d{{x, Fr::one()}, {y, -Fr::one()}, {0, -fr_i64(thr)}};
  return bits_of(t, d, zkh::fr_pow2(k - 1), k)[(size_t)k - 1];
}

// b + f * (a - b) as a fresh variable (statement_v2.cuh:68-80)
int select(Tracer& t, int f, const LC& a, const LC& b) {
  LC diff = a;
  for (const auto& term : b) diff.push_back({term.first, -term.second});
  const int pv = t.var(t.val(f) * t.eval(diff));
  t.constrain(LC{{f, Fr::one()}}, diff, LC{{pv, Fr::one()}});
  LC out = b;
  out.push_back({pv, Fr::one()});
  const int ov = t.var(t.eval(out));
  t.linear(out, ov);
  return ov;
}

struct ConvShape {
  int in_c, in_h, in_w, out_c, kh, kw, stride, pad;
  int out_h() const { return (in_h + 2 * pad - kh) / stride + 1; }
  int out_w() const { return (in_w + 2 * pad - kw) / stride + 1; }
  int in_size() const { return in_c * in_h * in_w; }
  int out_size() const { return out_c * out_h() * out_w(); }
  size_t weight_count() const { return (size_t)out_c * in_c * kh * kw; }
};

// Public weights as row coefficients; zero weights add no term
// (gadgets.cuh:230-251).
std::vector<int> fixed_linear(Tracer& t, const std::vector<int>& x, const std::vector<Fr>& wt,
                              const std::vector<Fr>& bias, int out, int in) {
  std::vector<int> y((size_t)out);
  for (int i = 0; i < out; i++) {
    Fr acc = bias[(size_t)i];
    LC terms;
    for (int j = 0; j < in; j++) {
      const Fr& wij = wt[(size_t)i * in + j];
      if (wij.is_zero()) continue;
      terms.push_back({x[(size_t)j], wij});
      acc = acc + wij * t.val(x[(size_t)j]);
    }
    terms.push_back({0, bias[(size_t)i]});
    y[(size_t)i] = t.var(acc);
    t.row_linear(terms, LC{{y[(size_t)i], Fr::one()}});
  }
  return y;
}

// Private weights: one product row per weight (gadgets.cuh:254-276).
std::vector<int> private_linear(Tracer& t, const std::vector<int>& x, const std::vector<int>& wv,
                                const std::vector<int>& bv, int out, int in) {
  std::vector<int> y((size_t)out);
  for (int i = 0; i < out; i++) {
    LC terms;
    Fr acc = t.val(bv[(size_t)i]);
    for (int j = 0; j < in; j++) {
      const int w = wv[(size_t)i * in + j];
      const Fr p = t.val(w) * t.val(x[(size_t)j]);
      const int pv = t.var(p);
      t.mul(w, x[(size_t)j], pv);
      terms.push_back({pv, Fr::one()});
      acc = acc + p;
    }
    terms.push_back({bv[(size_t)i], Fr::one()});
    y[(size_t)i] = t.var(acc);
    t.row_linear(terms, LC{{y[(size_t)i], Fr::one()}});
  }
  return y;
}

// CHW convolution, weights [oc][ic][ky][kx]; only in-bounds non-zero taps
// (gadgets.cuh:283-316).  Private weights: one product row per in-bounds tap
// (gadgets.cuh:319-349).
std::vector<int> conv2d(Tracer& t, const std::vector<int>& x, const ConvShape& s, const std::vector<Fr>* wt,
                        const std::vector<Fr>* bias, const std::vector<int>* wv, const std::vector<int>* bv) {
  const int oh = s.out_h(), ow = s.out_w();
  std::vector<int> y((size_t)s.out_size());
  for (int oc = 0; oc < s.out_c; oc++)
    for (int oy = 0; oy < oh; oy++)
      for (int ox = 0; ox < ow; ox++) {
        LC terms;
        Fr acc = wt ? (*bias)[(size_t)oc] : t.val((*bv)[(size_t)oc]);
        for (int ic = 0; ic < s.in_c; ic++)
          for (int ky = 0; ky < s.kh; ky++)
            for (int kx = 0; kx < s.kw; kx++) {
              const int iy = oy * s.stride + ky - s.pad, ix = ox * s.stride + kx - s.pad;
              if (iy < 0 || ix < 0 || iy >= s.in_h || ix >= s.in_w) continue;
              const size_t widx = (((size_t)oc * s.in_c + ic) * s.kh + ky) * s.kw + kx;
              const int xv = x[((size_t)ic * s.in_h + iy) * s.in_w + ix];
              if (wt) {
                const Fr& w = (*wt)[widx];
                if (w.is_zero()) continue;
                terms.push_back({xv, w});
                acc = acc + w * t.val(xv);
              } else {
                const int w = (*wv)[widx];
                const Fr p = t.val(w) * t.val(xv);
                const int pv = t.var(p);
                t.mul(w, xv, pv);
                terms.push_back({pv, Fr::one()});
                acc = acc + p;
              }
            }
        if (wt) terms.push_back({0, (*bias)[(size_t)oc]});
        else terms.push_back({(*bv)[(size_t)oc], Fr::one()});
        const size_t o = ((size_t)oc * oh + oy) * ow + ox;
        y[o] = t.var(acc);
        t.row_linear(terms, LC{{y[o], Fr::one()}});
      }
  return y;
}

// In-circuit Poseidon permutation over LC state words (gadgets.cuh:368-393).
void poseidon_permute(Tracer& t, LC st[3]) {
  const Poseidon& P = Poseidon::get();
  auto sbox = [&](const LC& x) -> LC {
    const Fr xv = t.eval(x);
    const int x2 = t.var(xv * xv);
    t.constrain(x, x, LC{{x2, Fr::one()}});
    const int x4 = t.var(t.val(x2) * t.val(x2));
    t.mul(x2, x2, x4);
    const int x5 = t.var(t.val(x4) * xv);
    t.constrain(LC{{x4, Fr::one()}}, x, LC{{x5, Fr::one()}});
    return LC{{x5, Fr::one()}};
  };
  for (int r = 0; r < Poseidon::ROUNDS; r++) {
    for (int i = 0; i < 3; i++) st[i].push_back({0, P.rc[r * 3 + i]});
    if (Poseidon::full_round(r)) {
      for (int i = 0; i < 3; i++) st[i] = sbox(st[i]);
    } else {
      st[0] = sbox(st[0]);
    }
    LC n[3];
    for (int i = 0; i < 3; i++)
      for (int j = 0; j < 3; j++)
        for (const auto& term : st[j]) n[i].push_back({term.first, P.mds[i][j] * term.second});
    for (int i = 0; i < 3; i++) st[i] = compress(n[i]);
    for (int i = 0; i < 3; i++)
      if (st[i].size() > 8) {
        const int m = t.var(t.eval(st[i]));
        t.linear(st[i], m);
        st[i] = LC{{m, Fr::one()}};
      }
  }
}

// Sponge commitment in the circuit; out_preset >= 0 receives the result
// (gadgets.cuh:429-446).
int poseidon_commit(Tracer& t, const std::vector<int>& vars, uint64_t domain, int out_preset) {
  LC st[3] = {LC{{0, zkh::fr_pow2(64) * fr_u64((uint64_t)vars.size()) + fr_u64(domain)}}, LC{}, LC{}};
  const size_t n = vars.empty() ? 2 : vars.size() + (vars.size() % 2);
  for (size_t i = 0; i < n; i += 2) {
    if (i < vars.size()) st[1].push_back({vars[i], Fr::one()});
    if (i + 1 < vars.size()) st[2].push_back({vars[i + 1], Fr::one()});
    poseidon_permute(t, st);
  }
  int out = out_preset;
  if (out < 0) out = t.var(t.eval(st[1]));
  else t.set(out, t.eval(st[1]));
  t.linear(st[1], out);
  return out;
}

std::string hex_std(const Fr& x) {
  uint64_t s[4];
  x.to_std(s);
  char buf[80];
  snprintf(buf, sizeof(buf), "0x%016llx%016llx%016llx%016llx", (unsigned long long)s[3], (unsigned long long)s[2],
           (unsigned long long)s[1], (unsigned long long)s[0]);
  return buf;
}

void set_err(char* err, size_t cap, const std::string& msg) {
  if (err && cap) {
    const size_t k = msg.size() < cap - 1 ? msg.size() : cap - 1;
    memcpy(err, msg.data(), k);
    err[k] = 0;
  }
}

}  // namespace

struct zk_statement {
  int nc = 0, nv = 0, npub = 0, npriv = 0;
  std::vector<zk_sparse_entry> A, B, C;
  std::vector<Fr> w;
  int32_t layout[ZK_STATEMENT_LAYOUT_WORDS];
  std::vector<int64_t> scores;  // batch x n_out
  // options echoed by the metadata
  bool has_context = false, private_input = false, private_model = false, private_outputs = false;
  Fr context;
  int64_t route_threshold = 0;
};

extern "C" {

static int zk_poseidon_permute_impl(uint64_t state[12]) {
  if (!state) return ZK_ERR_INVALID;
  Fr s[3];
  for (int i = 0; i < 3; i++) s[i] = fr_std4(state + 4 * i);
  Poseidon::get().permute(s);
  for (int i = 0; i < 3; i++) s[i].to_std(state + 4 * i);
  return ZK_OK;
}

int zk_poseidon_permute(uint64_t state[12]) {
  return zkh::abi_guard([&] { return zk_poseidon_permute_impl(state); });
}

static int zk_poseidon_hash2_impl(const uint64_t a[4], const uint64_t b[4], uint64_t out[4]) {
  if (!a || !b || !out) return ZK_ERR_INVALID;
  zkh::poseidon_hash2(fr_std4(a), fr_std4(b)).to_std(out);
  return ZK_OK;
}

int zk_poseidon_hash2(const uint64_t a[4], const uint64_t b[4], uint64_t out[4]) {
  return zkh::abi_guard([&] { return zk_poseidon_hash2_impl(a, b, out); });
}

static int zk_poseidon_commit_impl(const uint64_t* values, size_t n, uint64_t domain, uint64_t out[4]) {
  if ((n && !values) || !out) return ZK_ERR_INVALID;
  std::vector<Fr> v(n);
  for (size_t i = 0; i < n; i++) v[i] = fr_std4(values + 4 * i);
  zkh::poseidon_commit(v, domain).to_std(out);
  return ZK_OK;
}

int zk_poseidon_commit(const uint64_t* values, size_t n, uint64_t domain, uint64_t out[4]) {
  return zkh::abi_guard([&] { return zk_poseidon_commit_impl(values, n, domain, out); });
}

static int zk_poseidon_constants_impl(uint64_t* round_constants, uint64_t* mds) {
  const Poseidon& P = Poseidon::get();
  if (round_constants)
    for (int i = 0; i < Poseidon::NRC; i++) P.rc[i].to_std(round_constants + 4 * i);
  if (mds)
    for (int i = 0; i < 3; i++)
      for (int j = 0; j < 3; j++) P.mds[i][j].to_std(mds + 4 * (3 * i + j));
  return ZK_OK;
}

int zk_poseidon_constants(uint64_t* round_constants, uint64_t* mds) {
  return zkh::abi_guard([&] { return zk_poseidon_constants_impl(round_constants, mds); });
}

static int zk_statement_v2_build_impl(const zk_layer* layers, int num_layers, const int64_t* inputs, int batch,
                                      int n_in, const zk_statement_options* options, zk_statement** out, char* err,
                                      size_t err_cap) {
  if (!out || (num_layers > 0 && !layers) || num_layers < 0 || n_in < 0) {
    set_err(err, err_cap, "invalid argument");
    return ZK_ERR_INVALID;
  }
  *out = nullptr;
  auto fail = [&](const std::string& msg) {
    set_err(err, err_cap, msg);
    return ZK_ERR_INVALID;
  };
  zk_statement_options opt;
  memset(&opt, 0, sizeof(opt));
  if (options) opt = *options;
  const int K = opt.compare_bits > 0 ? opt.compare_bits : 48;
  const int Bn = batch;
  if (Bn <= 0) return fail("no input samples");
  if (n_in > 0 && !inputs) return fail("invalid argument");

  // layer shapes and the output size (last layer that is not SOFTMAX_APPROX)
  std::vector<ConvShape> conv((size_t)num_layers);
  std::vector<int> in_size((size_t)num_layers), out_size((size_t)num_layers);
  int last = -1;
  for (int i = 0; i < num_layers; i++) {
    const zk_layer& l = layers[i];
    in_size[(size_t)i] = l.in_size;
    out_size[(size_t)i] = l.out_size;
    switch (l.type) {
      case ZK_LAYER_LINEAR:
        if (l.in_size < 0 || l.out_size < 0 || ((size_t)l.in_size * l.out_size != 0 && !l.weights) ||
            (l.out_size && !l.bias))
          return fail("LINEAR layer " + std::to_string(i) + ": bad sizes or missing weights");
        break;
      case ZK_LAYER_CONV2D: {
        ConvShape s{l.conv_in_c, l.conv_in_h, l.conv_in_w, l.conv_out_c, l.conv_kh, l.conv_kw, l.conv_stride,
                    l.conv_pad};
        if (s.in_c <= 0 || s.in_h <= 0 || s.in_w <= 0 || s.out_c <= 0 || s.kh <= 0 || s.kw <= 0 || s.stride <= 0 ||
            s.pad < 0 || s.out_h() <= 0 || s.out_w() <= 0 || !l.weights || !l.bias)
          return fail("CONV2D layer " + std::to_string(i) + ": bad shape or missing weights");
        conv[(size_t)i] = s;
        in_size[(size_t)i] = s.in_size();
        out_size[(size_t)i] = s.out_size();
        break;
      }
      case ZK_LAYER_RELU_EXACT:
        if (l.relu_bits < 1 || l.relu_bits > 252 || l.relu_shift < 0 || l.relu_shift > 62)
          return fail("RELU_EXACT layer " + std::to_string(i) + ": bits in [1, 252] and shift in [0, 62]");
        break;
      case ZK_LAYER_RELU_APPROX:
        break;
      case ZK_LAYER_SELF_ATTENTION:
        return fail("SELF_ATTENTION is not supported by statement v2");
      case ZK_LAYER_SOFTMAX_APPROX:
        if (i != num_layers - 1) return fail("SOFTMAX_APPROX only allowed as the last layer");
        break;
      default:
        return fail("unknown layer type at layer " + std::to_string(i));
    }
    if (l.type != ZK_LAYER_SOFTMAX_APPROX) last = i;
  }
  int n_out = 0;
  for (int i = num_layers - 1; i >= 0; i--)
    if (layers[i].type != ZK_LAYER_SOFTMAX_APPROX) {
      n_out = out_size[(size_t)i];
      break;
    }
  if (n_out <= 0) return fail("cannot determine output size");
  if (opt.private_input && !opt.input_blinding) return fail("private_input needs one blinding value per sample");
  if (opt.private_outputs && !opt.route) return fail("private_outputs requires route");
  if (opt.route && n_out < 2) return fail("route needs at least two output classes");

  Tracer t;
  zk_statement* st = new zk_statement();
  int32_t* L = st->layout;
  for (int i = 0; i < ZK_STATEMENT_LAYOUT_WORDS; i++) L[i] = -1;
  L[ZK_LAYOUT_BATCH] = Bn;
  L[ZK_LAYOUT_N_IN] = n_in;
  L[ZK_LAYOUT_N_OUT] = n_out;
  const Fr model_tag = fr_std4(opt.model_tag);

  // ---- public variables first (statement_v2.cuh:113-140)
  int idx = 0;
  std::vector<int> out_pub;
  if (!opt.private_outputs) {
    L[ZK_LAYOUT_OUTPUTS_START] = idx;
    for (int i = 0; i < Bn * n_out; i++, idx++) out_pub.push_back(t.var_unset());
  }
  L[ZK_LAYOUT_MODEL_TAG] = idx++;
  const int tag_var = t.var(model_tag);
  int ctx_var = -1;
  if (opt.has_context) {
    L[ZK_LAYOUT_CONTEXT] = idx++;
    ctx_var = t.var(fr_std4(opt.context));
  }
  int cmodel_var = -1;
  if (opt.private_model) {
    L[ZK_LAYOUT_MODEL_COMMITMENT] = idx++;
    cmodel_var = t.var_unset();
  }
  L[ZK_LAYOUT_INPUTS_START] = idx;
  L[ZK_LAYOUT_INPUT_SLOT] = opt.private_input ? 1 : n_in;
  std::vector<std::vector<int>> in_vars((size_t)Bn);
  std::vector<int> cin_vars((size_t)Bn, -1);
  for (int b = 0; b < Bn; b++) {
    if (opt.private_input) {
      cin_vars[(size_t)b] = t.var_unset();
      idx++;
    } else {
      for (int i = 0; i < n_in; i++, idx++) in_vars[(size_t)b].push_back(t.var(fr_signed(inputs[(size_t)b * n_in + i])));
    }
  }
  std::vector<int> route_flag((size_t)Bn, -1), route_class((size_t)Bn, -1);
  if (opt.route) {
    L[ZK_LAYOUT_ROUTE_START] = idx;
    for (int b = 0; b < Bn; b++, idx += 2) {
      route_flag[(size_t)b] = t.var_unset();
      route_class[(size_t)b] = t.var_unset();
    }
  }
  L[ZK_LAYOUT_NUM_PUBLIC] = idx;

  // ---- statement bindings
  t.row_linear(LC{{0, model_tag}}, LC{{tag_var, Fr::one()}});
  if (opt.has_context) context_binding(t, ctx_var);

  // ---- model values
  std::vector<std::vector<Fr>> wfr((size_t)num_layers), bfr((size_t)num_layers);
  for (int li = 0; li < num_layers; li++) {
    const zk_layer& l = layers[li];
    if (l.type != ZK_LAYER_LINEAR && l.type != ZK_LAYER_CONV2D) continue;
    const size_t nw = l.type == ZK_LAYER_LINEAR ? (size_t)l.in_size * l.out_size : conv[(size_t)li].weight_count();
    const size_t nb = l.type == ZK_LAYER_LINEAR ? (size_t)l.out_size : (size_t)conv[(size_t)li].out_c;
    for (size_t i = 0; i < nw; i++) wfr[(size_t)li].push_back(fr_signed(l.weights[i]));
    for (size_t i = 0; i < nb; i++) bfr[(size_t)li].push_back(fr_signed(l.bias[i]));
  }
  std::vector<std::vector<int>> w_vars((size_t)num_layers), b_vars((size_t)num_layers);
  if (opt.private_model) {
    std::vector<int> all;
    for (int li = 0; li < num_layers; li++) {
      for (const Fr& v : wfr[(size_t)li]) {
        w_vars[(size_t)li].push_back(t.var(v));
        all.push_back(w_vars[(size_t)li].back());
      }
      for (const Fr& v : bfr[(size_t)li]) {
        b_vars[(size_t)li].push_back(t.var(v));
        all.push_back(b_vars[(size_t)li].back());
      }
    }
    poseidon_commit(t, all, Poseidon::DOMAIN_MODEL, cmodel_var);
  }

  // ---- private inputs under commitments
  if (opt.private_input) {
    for (int b = 0; b < Bn; b++) {
      for (int i = 0; i < n_in; i++) in_vars[(size_t)b].push_back(t.var(fr_signed(inputs[(size_t)b * n_in + i])));
      std::vector<int> cv = in_vars[(size_t)b];
      cv.push_back(t.var(fr_std4(opt.input_blinding + 4 * b)));
      poseidon_commit(t, cv, Poseidon::DOMAIN_INPUT, cin_vars[(size_t)b]);
    }
  }

  // ---- per-sample model evaluation
  st->scores.assign((size_t)Bn * n_out, 0);
  for (int b = 0; b < Bn; b++) {
    std::vector<int> cur = in_vars[(size_t)b];
    for (int li = 0; li <= last; li++) {
      const zk_layer& l = layers[li];
      if ((int)cur.size() != in_size[(size_t)li]) {
        delete st;
        return fail("layer size mismatch at layer " + std::to_string(li));
      }
      switch (l.type) {
        case ZK_LAYER_LINEAR:
          cur = opt.private_model
                    ? private_linear(t, cur, w_vars[(size_t)li], b_vars[(size_t)li], l.out_size, l.in_size)
                    : fixed_linear(t, cur, wfr[(size_t)li], bfr[(size_t)li], l.out_size, l.in_size);
          break;
        case ZK_LAYER_CONV2D:
          cur = opt.private_model
                    ? conv2d(t, cur, conv[(size_t)li], nullptr, nullptr, &w_vars[(size_t)li], &b_vars[(size_t)li])
                    : conv2d(t, cur, conv[(size_t)li], &wfr[(size_t)li], &bfr[(size_t)li], nullptr, nullptr);
          break;
        case ZK_LAYER_RELU_EXACT:
          for (auto& v : cur) v = rescale(t, relu_exact(t, v, l.relu_bits), l.relu_shift, l.relu_bits);
          break;
        case ZK_LAYER_RELU_APPROX: {
          // (statement_v2.cuh:212-225)
          const Fr sc = fr_signed(l.relu_scale);
          const Fr c0 = fr_signed(l.relu_c[0]), c1 = fr_signed(l.relu_c[1]);
          const Fr c2 = fr_signed(l.relu_c[2]), c3 = fr_signed(l.relu_c[3]);
          for (auto& v : cur) {
            const int x2 = t.var(t.val(v) * t.val(v));
            t.mul(v, v, x2);
            const int x3 = t.var(t.val(x2) * t.val(v));
            t.mul(x2, v, x3);
            const LC lc{{0, sc * c0}, {v, sc * c1}, {x2, sc * c2}, {x3, sc * c3}};
            const int y = t.var(t.eval(lc));
            t.linear(lc, y);
            v = y;
          }
          break;
        }
        default:
          break;
      }
    }
    if ((int)cur.size() != n_out) {
      delete st;
      return fail("final layer size mismatch");
    }
    for (int i = 0; i < n_out; i++) {
      int64_t s = 0;
      fr_to_i64(t.val(cur[(size_t)i]), &s);
      st->scores[(size_t)b * n_out + i] = s;
      if (!opt.private_outputs) {
        const int pv = out_pub[(size_t)b * n_out + i];
        t.set(pv, t.val(cur[(size_t)i]));
        t.constrain_zero(LC{{pv, Fr::one()}, {cur[(size_t)i], -Fr::one()}});
      }
    }

    // ---- top-1 / top-2 routing on the scores (statement_v2.cuh:243-266)
    if (opt.route) {
      const LC one{{0, Fr::one()}};
      auto v1 = [](int v) { return LC{{v, Fr::one()}}; };
      const int f = geq_flag(t, cur[1], cur[0], 1, K);
      int m1 = select(t, f, v1(cur[1]), v1(cur[0]));
      int m2 = select(t, f, v1(cur[0]), v1(cur[1]));
      int i1 = select(t, f, one, LC{});
      for (int j = 2; j < n_out; j++) {
        const int x = cur[(size_t)j];
        const int f1 = geq_flag(t, x, m1, 1, K);
        const int f2 = geq_flag(t, x, m2, 1, K);
        const int tt = select(t, f2, v1(x), v1(m2));
        const int nm2 = select(t, f1, v1(m1), v1(tt));
        const int nm1 = select(t, f1, v1(x), v1(m1));
        const int ni1 = select(t, f1, LC{{0, fr_u64((uint64_t)j)}}, v1(i1));
        m1 = nm1;
        m2 = nm2;
        i1 = ni1;
      }
      const int flag = geq_flag(t, m1, m2, opt.route_threshold, K);
      t.set(route_flag[(size_t)b], t.val(flag));
      t.constrain_zero(LC{{route_flag[(size_t)b], Fr::one()}, {flag, -Fr::one()}});
      t.set(route_class[(size_t)b], t.val(i1));
      t.constrain_zero(LC{{route_class[(size_t)b], Fr::one()}, {i1, -Fr::one()}});
    }
  }

  st->nc = t.rows;
  st->nv = t.next_var;
  st->npub = L[ZK_LAYOUT_NUM_PUBLIC];
  st->npriv = opt.private_input ? Bn * n_in : 0;
  t.w.resize((size_t)st->nv, Fr::zero());
  st->w.swap(t.w);
  st->A.swap(t.A);
  st->B.swap(t.B);
  st->C.swap(t.C);
  st->has_context = opt.has_context != 0;
  st->context = fr_std4(opt.context);
  st->private_input = opt.private_input != 0;
  st->private_model = opt.private_model != 0;
  st->private_outputs = opt.private_outputs != 0;
  st->route_threshold = opt.route_threshold;
  *out = st;
  set_err(err, err_cap, "");
  return ZK_OK;
}

int zk_statement_v2_build(const zk_layer* layers, int num_layers, const int64_t* inputs, int batch, int n_in,
                          const zk_statement_options* options, zk_statement** out, char* err, size_t err_cap) {
  return zkh::abi_guard([&] {
    return zk_statement_v2_build_impl(layers, num_layers, inputs, batch, n_in, options, out, err, err_cap);
  });
}

void zk_statement_destroy(zk_statement* st) { delete st; }

static int zk_statement_info_impl(const zk_statement* st, int* num_constraints, int* num_variables, int* num_public,
                                  int* num_private, size_t* nA, size_t* nB, size_t* nC) {
  if (!st) return ZK_ERR_INVALID;
  if (num_constraints) *num_constraints = st->nc;
  if (num_variables) *num_variables = st->nv;
  if (num_public) *num_public = st->npub;
  if (num_private) *num_private = st->npriv;
  if (nA) *nA = st->A.size();
  if (nB) *nB = st->B.size();
  if (nC) *nC = st->C.size();
  return ZK_OK;
}

int zk_statement_info(const zk_statement* st, int* num_constraints, int* num_variables, int* num_public,
                      int* num_private, size_t* nA, size_t* nB, size_t* nC) {
  return zkh::abi_guard([&] {
    return zk_statement_info_impl(st, num_constraints, num_variables, num_public, num_private, nA, nB, nC);
  });
}

static int zk_statement_layout_impl(const zk_statement* st, int32_t layout[ZK_STATEMENT_LAYOUT_WORDS]) {
  if (!st || !layout) return ZK_ERR_INVALID;
  memcpy(layout, st->layout, sizeof(st->layout));
  return ZK_OK;
}

int zk_statement_layout(const zk_statement* st, int32_t layout[ZK_STATEMENT_LAYOUT_WORDS]) {
  return zkh::abi_guard([&] { return zk_statement_layout_impl(st, layout); });
}

static int zk_statement_r1cs_impl(const zk_statement* st, zk_sparse_entry* A, zk_sparse_entry* B, zk_sparse_entry* C) {
  if (!st || (!st->A.empty() && !A) || (!st->B.empty() && !B) || (!st->C.empty() && !C)) return ZK_ERR_INVALID;
  if (!st->A.empty()) memcpy(A, st->A.data(), st->A.size() * sizeof(zk_sparse_entry));
  if (!st->B.empty()) memcpy(B, st->B.data(), st->B.size() * sizeof(zk_sparse_entry));
  if (!st->C.empty()) memcpy(C, st->C.data(), st->C.size() * sizeof(zk_sparse_entry));
  return ZK_OK;
}

int zk_statement_r1cs(const zk_statement* st, zk_sparse_entry* A, zk_sparse_entry* B, zk_sparse_entry* C) {
  return zkh::abi_guard([&] { return zk_statement_r1cs_impl(st, A, B, C); });
}

static int zk_statement_witness_impl(const zk_statement* st, void* w_mont) {
  if (!st || !w_mont) return ZK_ERR_INVALID;
  memcpy(w_mont, st->w.data(), st->w.size() * 32);
  return ZK_OK;
}

int zk_statement_witness(const zk_statement* st, void* w_mont) {
  return zkh::abi_guard([&] { return zk_statement_witness_impl(st, w_mont); });
}

static int zk_statement_scores_impl(const zk_statement* st, int64_t* scores) {
  if (!st || !scores) return ZK_ERR_INVALID;
  memcpy(scores, st->scores.data(), st->scores.size() * sizeof(int64_t));
  return ZK_OK;
}

int zk_statement_scores(const zk_statement* st, int64_t* scores) {
  return zkh::abi_guard([&] { return zk_statement_scores_impl(st, scores); });
}

// (A w) o (B w) = C w on the host (reference R1CS::verify_witness,
// src/prover/circuit.cuh:92-124)
static int zk_statement_check_impl(const zk_statement* st) {
  if (!st) return ZK_ERR_INVALID;
  std::vector<Fr> acc[3];
  const std::vector<zk_sparse_entry>* m[3] = {&st->A, &st->B, &st->C};
  for (int k = 0; k < 3; k++) {
    acc[k].assign((size_t)st->nc, Fr::zero());
    for (const auto& e : *m[k]) {
      if (e.row < 0 || e.row >= st->nc || e.col < 0 || e.col >= st->nv) return ZK_ERR_INVALID;
      acc[k][(size_t)e.row] = acc[k][(size_t)e.row] + Fr::raw(e.value) * st->w[(size_t)e.col];
    }
  }
  for (int r = 0; r < st->nc; r++)
    if (!(acc[0][(size_t)r] * acc[1][(size_t)r] == acc[2][(size_t)r])) return ZK_ERR_WITNESS;
  return ZK_OK;
}

int zk_statement_check(const zk_statement* st) {
  return zkh::abi_guard([&] { return zk_statement_check_impl(st); });
}

static int zk_statement_write_impl(const zk_statement* st, const char* r1cs_path, const char* wtns_path) {
  if (!st) return ZK_ERR_INVALID;
  if (r1cs_path) {
    const int rc = zk_iden3_r1cs_write(r1cs_path, st->nc, st->nv, st->npub, st->npriv, st->A.data(), st->A.size(),
                                       st->B.data(), st->B.size(), st->C.data(), st->C.size());
    if (rc) return rc;
  }
  if (wtns_path) return zk_wtns_write(wtns_path, st->w.data(), st->w.size());
  return ZK_OK;
}

int zk_statement_write(const zk_statement* st, const char* r1cs_path, const char* wtns_path) {
  return zkh::abi_guard([&] { return zk_statement_write_impl(st, r1cs_path, wtns_path); });
}

// statement_v2_meta_json (statement_v2.cuh:255-287), same keys and layout
static int zk_statement_meta_json_impl(const zk_statement* st, uint64_t model_tag64, char* buf, size_t cap,
                                       size_t* len) {
  if (!st) return ZK_ERR_INVALID;
  const int32_t* L = st->layout;
  char tag[32];
  snprintf(tag, sizeof(tag), "0x%016llx", (unsigned long long)model_tag64);
  std::string o = "{\n";
  auto kv = [&](const char* k, const std::string& v, bool quote, bool last = false) {
    o += std::string("  \"") + k + "\": " + (quote ? "\"" + v + "\"" : v) + (last ? "\n" : ",\n");
  };
  kv("statement_version", "2", false);
  kv("statement_mode", "pcani-v2", true);
  kv("model_binding", st->private_model ? "poseidon-commitment-private-weights" : "fixed-quantized-parameters-in-r1cs",
     true);
  kv("model_tag64", tag, true);
  kv("input_visibility", st->private_input ? "poseidon-commitment" : "public", true);
  kv("output_visibility", st->private_outputs ? "private" : "public", true);
  kv("batch", std::to_string(L[ZK_LAYOUT_BATCH]), false);
  kv("input_size", std::to_string(L[ZK_LAYOUT_N_IN]), false);
  kv("output_size", std::to_string(L[ZK_LAYOUT_N_OUT]), false);
  kv("outputs_start_index", std::to_string(L[ZK_LAYOUT_OUTPUTS_START]), false);
  kv("model_tag_public_index", std::to_string(L[ZK_LAYOUT_MODEL_TAG]), false);
  kv("context_public_index", std::to_string(L[ZK_LAYOUT_CONTEXT]), false);
  kv("context", st->has_context ? hex_std(st->context) : std::string(), true);
  kv("model_commitment_index", std::to_string(L[ZK_LAYOUT_MODEL_COMMITMENT]), false);
  kv("inputs_start_index", std::to_string(L[ZK_LAYOUT_INPUTS_START]), false);
  kv("input_slot_size", std::to_string(L[ZK_LAYOUT_INPUT_SLOT]), false);
  kv("route_start_index", std::to_string(L[ZK_LAYOUT_ROUTE_START]), false);
  kv("route_threshold", std::to_string(st->route_threshold), false);
  kv("num_public", std::to_string(L[ZK_LAYOUT_NUM_PUBLIC]), false);
  kv("r1cs_constraints", std::to_string(st->nc), false);
  kv("r1cs_variables", std::to_string(st->nv), false, true);
  o += "}\n";
  if (len) *len = o.size();
  if (buf && cap) {
    const size_t k = o.size() < cap - 1 ? o.size() : cap - 1;
    memcpy(buf, o.data(), k);
    buf[k] = 0;
    if (o.size() >= cap) return ZK_ERR_SIZE;
  }
  return ZK_OK;
}

int zk_statement_meta_json(const zk_statement* st, uint64_t model_tag64, char* buf, size_t cap, size_t* len) {
  return zkh::abi_guard([&] { return zk_statement_meta_json_impl(st, model_tag64, buf, cap, len); });
}

}  // extern "C"
