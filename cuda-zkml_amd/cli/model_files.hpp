// Model and input files of zkml-prove's statement-v2 path: the architecture
// sidecar (.arch.json), the exact int32 parameter file (--integer-model), the
// float32 .bin / .npy inputs (--integer-input), the quantized-model tag and
// the hex field values of --context / --input-blinding.  Formats and rules
// follow the reference's front end (src/cli/prove.cu:60-520,
// src/nn/inference.cuh:306-341, src/prover/gadgets.cuh:68-91).
#pragma once
#include <ctype.h>
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

#include <string>
#include <vector>

#include "../csrc/host_bn254.hpp"
#include "zkml_gpu.h"

namespace cli {

struct LayerSpec {
  int type = 0, in_size = 0, out_size = 0;
  int bits = 32, shift = 0;                                     // RELU_EXACT
  int in_c = 0, in_h = 0, in_w = 0, out_c = 0, k = 0, stride = 1, pad = 0;  // CONV2D
};

inline std::string read_text(const char* path, bool& ok) {
  std::string s;
  FILE* f = fopen(path, "rb");
  ok = f != nullptr;
  if (!f) return s;
  char buf[65536];
  size_t got;
  while ((got = fread(buf, 1, sizeof(buf), f)) > 0) s.append(buf, got);
  fclose(f);
  return s;
}

// "field": "text"  (first occurrence inside one layer object)
inline bool json_string(const std::string& obj, const char* field, std::string& out) {
  const std::string key = std::string("\"") + field + "\"";
  for (size_t p = obj.find(key); p != std::string::npos; p = obj.find(key, p + 1)) {
    size_t i = p + key.size();
    while (i < obj.size() && isspace((unsigned char)obj[i])) i++;
    if (i >= obj.size() || obj[i] != ':') continue;
    i++;
    while (i < obj.size() && isspace((unsigned char)obj[i])) i++;
    if (i >= obj.size() || obj[i] != '"') continue;
    const size_t e = obj.find('"', i + 1);
    if (e == std::string::npos || e == i + 1) continue;
    out = obj.substr(i + 1, e - i - 1);
    return true;
  }
  return false;
}

// "field": digits  (non-negative integers only, as the reference's parser)
inline bool json_uint(const std::string& obj, const char* field, int& out) {
  const std::string key = std::string("\"") + field + "\"";
  for (size_t p = obj.find(key); p != std::string::npos; p = obj.find(key, p + 1)) {
    size_t i = p + key.size();
    while (i < obj.size() && isspace((unsigned char)obj[i])) i++;
    if (i >= obj.size() || obj[i] != ':') continue;
    i++;
    while (i < obj.size() && isspace((unsigned char)obj[i])) i++;
    if (i >= obj.size() || !isdigit((unsigned char)obj[i])) continue;
    out = atoi(obj.c_str() + i);
    return true;
  }
  return false;
}

inline bool layer_type(std::string t, int& out) {
  for (auto& c : t) c = (char)tolower((unsigned char)c);
  if (t == "linear") out = ZK_LAYER_LINEAR;
  else if (t == "relu" || t == "relu_approx") out = ZK_LAYER_RELU_APPROX;
  else if (t == "softmax" || t == "softmax_approx") out = ZK_LAYER_SOFTMAX_APPROX;
  else if (t == "self_attention" || t == "attention" || t == "transformer_attention") out = ZK_LAYER_SELF_ATTENTION;
  else if (t == "relu_exact") out = ZK_LAYER_RELU_EXACT;
  else if (t == "conv2d" || t == "conv") out = ZK_LAYER_CONV2D;
  else return false;
  return true;
}

// Architecture sidecar: {"layers": [{"type": ..., "in_features": ...,
// "out_features": ..., ...}, ...]} (reference load_architecture_json,
// prove.cu:160-257).
inline bool load_arch(const char* path, std::vector<LayerSpec>& specs, std::string& err) {
  bool ok = false;
  const std::string text = read_text(path, ok);
  if (!ok) {
    err = std::string("cannot read ") + path;
    return false;
  }
  const size_t lp = text.find("\"layers\"");
  const size_t a0 = lp == std::string::npos ? lp : text.find('[', lp);
  if (a0 == std::string::npos) {
    err = "no layers array in the architecture sidecar";
    return false;
  }
  std::vector<std::string> objs;
  int depth = 0;
  size_t start = std::string::npos;
  for (size_t i = a0; i < text.size(); i++) {
    const char c = text[i];
    if (c == '{') {
      if (depth++ == 0) start = i;
    } else if (c == '}') {
      if (--depth == 0 && start != std::string::npos) {
        objs.push_back(text.substr(start, i - start + 1));
        start = std::string::npos;
      }
    } else if (c == ']' && depth == 0) {
      break;
    }
  }
  if (objs.empty()) {
    err = "no layers array in the architecture sidecar";
    return false;
  }
  specs.clear();
  for (const auto& o : objs) {
    LayerSpec s;
    std::string t;
    if (!json_string(o, "type", t) || !json_uint(o, "in_features", s.in_size) ||
        !json_uint(o, "out_features", s.out_size)) {
      err = "invalid layer object in the architecture sidecar";
      return false;
    }
    if (!layer_type(t, s.type)) {
      err = "unsupported layer type in the architecture: " + t;
      return false;
    }
    if (s.in_size <= 0 || s.out_size <= 0) {
      err = "invalid layer dimensions in the architecture sidecar";
      return false;
    }
    if (s.type == ZK_LAYER_RELU_EXACT) {
      json_uint(o, "bits", s.bits);
      json_uint(o, "shift", s.shift);
      if (s.bits < 2 || s.bits > 62 || s.shift < 0 || s.shift >= s.bits || s.in_size != s.out_size) {
        err = "relu_exact needs 2 <= bits <= 62, 0 <= shift < bits, in == out";
        return false;
      }
    } else if (s.type == ZK_LAYER_CONV2D) {
      const bool have = json_uint(o, "in_channels", s.in_c) && json_uint(o, "in_height", s.in_h) &&
                        json_uint(o, "in_width", s.in_w) && json_uint(o, "out_channels", s.out_c) &&
                        json_uint(o, "kernel_size", s.k);
      json_uint(o, "stride", s.stride);
      json_uint(o, "padding", s.pad);
      const int oh = s.stride > 0 ? (s.in_h + 2 * s.pad - s.k) / s.stride + 1 : 0;
      const int ow = s.stride > 0 ? (s.in_w + 2 * s.pad - s.k) / s.stride + 1 : 0;
      if (!have || s.k <= 0 || s.stride <= 0 || s.in_c * s.in_h * s.in_w != s.in_size ||
          s.out_c * oh * ow != s.out_size) {
        err = "conv2d needs in_channels/in_height/in_width/out_channels/kernel_size consistent with "
              "in_features/out_features";
        return false;
      }
    }
    specs.push_back(s);
  }
  for (size_t i = 0; i + 1 < specs.size(); i++)
    if (specs[i].type == ZK_LAYER_SOFTMAX_APPROX) {
      err = "only a final softmax layer is supported in architecture sidecars";
      return false;
    }
  return true;
}

template <class T>
inline bool load_raw(const char* path, std::vector<T>& out) {
  bool ok = false;
  const std::string s = read_text(path, ok);
  if (!ok || s.empty() || s.size() % sizeof(T)) return false;
  out.resize(s.size() / sizeof(T));
  memcpy(out.data(), s.data(), s.size());
  return true;
}

// float32 input: raw little-endian .bin, or .npy ('<f4' / '|f4', C order)
inline bool load_input(const char* path, std::vector<float>& out) {
  const std::string p(path);
  if (p.size() < 4 || p.substr(p.size() - 4) != ".npy") return load_raw(path, out);
  bool ok = false;
  const std::string s = read_text(path, ok);
  if (!ok || s.size() < 10 || memcmp(s.data(), "\x93NUMPY", 6) != 0) return false;
  const int major = (unsigned char)s[6];
  size_t hl = 0, off = 0;
  if (major == 1) {
    hl = (unsigned char)s[8] | ((size_t)(unsigned char)s[9] << 8);
    off = 10;
  } else if (major == 2 || major == 3) {
    if (s.size() < 12) return false;
    hl = (unsigned char)s[8] | ((size_t)(unsigned char)s[9] << 8) | ((size_t)(unsigned char)s[10] << 16) |
         ((size_t)(unsigned char)s[11] << 24);
    off = 12;
  } else {
    return false;
  }
  if (hl == 0 || off + hl > s.size()) return false;
  const std::string h = s.substr(off, hl);
  if (h.find("<f4") == std::string::npos && h.find("|f4") == std::string::npos) return false;
  if (h.find("fortran_order") != std::string::npos && h.find("True") != std::string::npos) return false;
  const size_t p0 = h.find('('), p1 = p0 == std::string::npos ? p0 : h.find(')', p0 + 1);
  if (p1 == std::string::npos || p1 <= p0 + 1) return false;
  size_t n = 1, dims = 0;
  std::string tok;
  for (size_t i = p0 + 1; i <= p1; i++) {
    const char c = h[i];
    if (c == ',' || c == ')') {
      if (!tok.empty()) {
        const long long d = atoll(tok.c_str());
        if (d <= 0) return false;
        n *= (size_t)d;
        dims++;
      }
      tok.clear();
    } else if (!isspace((unsigned char)c)) {
      tok.push_back(c);
    }
  }
  if (!dims || off + hl + 4 * n > s.size()) return false;
  out.resize(n);
  memcpy(out.data(), s.data() + off + hl, 4 * n);
  return true;
}

// exact int32 samples (reference --integer-input, prove.cu:1096-1110)
inline bool integer_samples(const std::vector<float>& in, std::vector<int64_t>& out) {
  out.resize(in.size());
  for (size_t i = 0; i < in.size(); i++) {
    const double r = (double)llround((double)in[i]);
    if (fabs((double)in[i] - r) > 1e-5 || r < (double)INT32_MIN || r > (double)INT32_MAX) return false;
    out[i] = (int64_t)r;
  }
  return true;
}

// Model layers over an int32 parameter file in load_integer_weights order:
// per LINEAR / CONV2D layer its weights then its biases (inference.cuh:306-341).
struct Model {
  std::vector<LayerSpec> specs;
  std::vector<std::vector<int64_t>> w, b;
  std::vector<zk_layer> layers;
};

inline bool build_model(const std::vector<LayerSpec>& specs, const std::vector<int32_t>& params, Model& m,
                        std::string& err) {
  m.specs = specs;
  m.w.assign(specs.size(), {});
  m.b.assign(specs.size(), {});
  m.layers.assign(specs.size(), zk_layer());
  size_t off = 0;
  for (size_t i = 0; i < specs.size(); i++) {
    const LayerSpec& s = specs[i];
    zk_layer& L = m.layers[i];
    memset(&L, 0, sizeof(L));
    L.type = s.type;
    L.in_size = s.in_size;
    // element-wise layers are built from in_features alone (NNModel::create_from_specs)
    L.out_size = (s.type == ZK_LAYER_RELU_APPROX || s.type == ZK_LAYER_SOFTMAX_APPROX) ? s.in_size : s.out_size;
    if (s.type == ZK_LAYER_SELF_ATTENTION) {
      err = "SELF_ATTENTION is not supported by statement v2";
      return false;
    }
    if (s.type == ZK_LAYER_RELU_EXACT) {
      L.relu_bits = s.bits;
      L.relu_shift = s.shift;
    } else if (s.type == ZK_LAYER_RELU_APPROX) {  // NNModel::make_relu_layer
      L.relu_c[0] = 64;
      L.relu_c[1] = 64;
      L.relu_c[2] = 1;
      L.relu_c[3] = 0;
      L.relu_scale = 1;
    } else if (s.type == ZK_LAYER_LINEAR || s.type == ZK_LAYER_CONV2D) {
      size_t nw, nb;
      if (s.type == ZK_LAYER_CONV2D) {
        L.conv_in_c = s.in_c;
        L.conv_in_h = s.in_h;
        L.conv_in_w = s.in_w;
        L.conv_out_c = s.out_c;
        L.conv_kh = L.conv_kw = s.k;
        L.conv_stride = s.stride;
        L.conv_pad = s.pad;
        nw = (size_t)s.out_c * s.in_c * s.k * s.k;
        nb = (size_t)s.out_c;
      } else {
        nw = (size_t)s.out_size * s.in_size;
        nb = (size_t)s.out_size;
      }
      if (off + nw + nb > params.size()) {
        err = "not enough integer weight data";
        return false;
      }
      m.w[i].assign(params.begin() + off, params.begin() + off + nw);
      m.b[i].assign(params.begin() + off + nw, params.begin() + off + nw + nb);
      off += nw + nb;
    }
  }
  if (off != params.size()) {
    err = "integer model payload has " + std::to_string(params.size() - off) + " trailing values";
    return false;
  }
  for (size_t i = 0; i < specs.size(); i++) {
    m.layers[i].weights = m.w[i].empty() ? nullptr : m.w[i].data();
    m.layers[i].bias = m.b[i].empty() ? nullptr : m.b[i].data();
  }
  return true;
}

inline uint64_t fnv1a(uint64_t h, const void* data, size_t n) {
  const unsigned char* p = (const unsigned char*)data;
  for (size_t i = 0; i < n; i++) {
    h ^= p[i];
    h *= 1099511628211ULL;
  }
  return h;
}

// Audit tag of the quantized model (reference compute_quantized_model_tag64,
// prove.cu:477-521): FNV-1a 64 over version 1 and, per layer, its type and
// sizes, then its parameters as base-field (Fq) standard-form words.
inline uint64_t model_tag64(const Model& m) {
  uint64_t h = 1469598103934665603ULL;
  const uint32_t version = 1;
  h = fnv1a(h, &version, 4);
  auto fq_words = [&](int64_t v) {
    zkh::Fq x = zkh::Fq::from_u64(v >= 0 ? (uint64_t)v : (uint64_t)(-v));
    if (v < 0) x = -x;
    uint64_t s[4];
    x.to_std(s);
    h = fnv1a(h, s, 32);
  };
  auto vec = [&](const std::vector<int64_t>& v) {
    const uint64_t n = v.size();
    h = fnv1a(h, &n, 8);
    for (int64_t x : v) fq_words(x);
  };
  for (size_t i = 0; i < m.specs.size(); i++) {
    const zk_layer& L = m.layers[i];
    const uint32_t type = (uint32_t)L.type;
    int32_t in_size = L.in_size, out_size = L.out_size;
    h = fnv1a(h, &type, 4);
    h = fnv1a(h, &in_size, 4);
    h = fnv1a(h, &out_size, 4);
    if (L.type == ZK_LAYER_LINEAR) {
      vec(m.w[i]);
      vec(m.b[i]);
    } else if (L.type == ZK_LAYER_CONV2D) {
      const int32_t dims[8] = {L.conv_in_c, L.conv_in_h, L.conv_in_w, L.conv_out_c,
                               L.conv_kh,   L.conv_kw,   L.conv_stride, L.conv_pad};
      h = fnv1a(h, dims, sizeof(dims));
      vec(m.w[i]);
      vec(m.b[i]);
    } else if (L.type == ZK_LAYER_RELU_EXACT) {
      h = fnv1a(h, &L.relu_bits, 4);
      h = fnv1a(h, &L.relu_shift, 4);
    } else if (L.type == ZK_LAYER_RELU_APPROX) {
      for (int k = 0; k < 4; k++) fq_words(L.relu_c[k]);
      fq_words(L.relu_scale);
    }
  }
  return h;
}

// Hex field value, optional 0x, at most 64 digits, low 253 bits kept
// (reference fr_from_hex, gadgets.cuh:68-91); out: standard-form words.
inline bool fr_hex(const std::string& text, uint64_t out[4]) {
  std::string h = text;
  if (h.size() >= 2 && h[0] == '0' && (h[1] == 'x' || h[1] == 'X')) h = h.substr(2);
  if (h.empty() || h.size() > 64) return false;
  uint64_t v[4] = {0, 0, 0, 0};
  for (char c : h) {
    int d;
    if (c >= '0' && c <= '9') d = c - '0';
    else if (c >= 'a' && c <= 'f') d = c - 'a' + 10;
    else if (c >= 'A' && c <= 'F') d = c - 'A' + 10;
    else return false;
    v[3] = (v[3] << 4) | (v[2] >> 60);
    v[2] = (v[2] << 4) | (v[1] >> 60);
    v[1] = (v[1] << 4) | (v[0] >> 60);
    v[0] = (v[0] << 4) | (uint64_t)d;
  }
  v[3] &= 0x1FFFFFFFFFFFFFFFULL;
  memcpy(out, v, 32);
  return true;
}

inline std::vector<std::string> split_csv(const std::string& text) {
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
}

}  // namespace cli
