// soc_oracle.cpp - CPU oracle (test infrastructure only; see soc_oracle.h).
//
// Each function restates one piece of the reference CPU runtime and names the file:line it follows. The
// arithmetic order is the reference's: this file must be built without FMA contraction (-ffp-contract=off) and
// without -ffast-math so that every `a += b * c` rounds twice, as the reference's scalar loops do.
#include "soc_oracle.h"

#include <algorithm>
#include <cmath>
#include <cstring>
#include <limits>
#include <map>
#include <string>
#include <vector>

#include <omp.h>

namespace {

int g_threads = 1;

inline float F16(uint16_t v) { return orc_f16_to_f32(v); }

}  // namespace

extern "C" {

int orc_set_threads(int n) {
  int prev = g_threads;
  g_threads = n < 1 ? 1 : n;
  return prev;
}

// Mac/cpu/src/dtype.cpp:76-106: exact binary16 -> binary32; subnormals normalised by a shift loop.
float orc_f16_to_f32(uint16_t value) {
  const uint32_t sign = static_cast<uint32_t>(value & 0x8000u) << 16;
  const uint32_t exponent = (value >> 10) & 0x1fu;
  uint32_t mantissa = value & 0x03ffu;
  uint32_t bits;
  if (exponent == 0) {
    if (mantissa == 0) {
      bits = sign;
    } else {
      int32_t e = -14;
      while ((mantissa & 0x0400u) == 0) {
        mantissa <<= 1;
        --e;
      }
      bits = sign | static_cast<uint32_t>(e + 127) << 23 | ((mantissa & 0x03ffu) << 13);
    }
  } else if (exponent == 0x1fu) {
    bits = sign | 0x7f800000u | (mantissa << 13);
  } else {
    bits = sign | ((exponent + 112u) << 23) | (mantissa << 13);
  }
  float out;
  std::memcpy(&out, &bits, sizeof(out));
  return out;
}

// Mac/cpu/src/dtype.cpp:115-156: binary32 -> binary16. Normal range rounds half up on the magnitude
// (+0x1000 then truncate), subnormals likewise after the shift; NaN keeps a quiet payload bit.
uint16_t orc_f32_to_f16(float value) {
  uint32_t bits;
  std::memcpy(&bits, &value, sizeof(bits));
  const uint32_t sign = (bits >> 16) & 0x8000u;
  int32_t exponent = static_cast<int32_t>((bits >> 23) & 0xffu) - 127 + 15;
  uint32_t mantissa = bits & 0x7fffffu;
  if (((bits >> 23) & 0xffu) == 0xffu) {
    if (mantissa == 0) return static_cast<uint16_t>(sign | 0x7c00u);
    return static_cast<uint16_t>(sign | 0x7c00u | (mantissa >> 13) | 1u);
  }
  if (exponent <= 0) {
    if (exponent < -10) return static_cast<uint16_t>(sign);
    mantissa |= 0x800000u;
    const uint32_t shifted = mantissa >> static_cast<uint32_t>(1 - exponent);
    return static_cast<uint16_t>(sign | ((shifted + 0x1000u) >> 13));
  }
  if (exponent >= 0x1f) return static_cast<uint16_t>(sign | 0x7c00u);
  const uint32_t rounded = mantissa + 0x1000u;
  if (rounded & 0x800000u) {
    mantissa = 0;
    ++exponent;
    if (exponent >= 0x1f) return static_cast<uint16_t>(sign | 0x7c00u);
  } else {
    mantissa = rounded;
  }
  return static_cast<uint16_t>(sign | (static_cast<uint32_t>(exponent) << 10) | (mantissa >> 13));
}

void orc_f16_to_f32_array(const uint16_t* in, float* out, int64_t n) {
  for (int64_t i = 0; i < n; ++i) out[i] = F16(in[i]);
}

// Mac/cpu/src/linear.cpp:145-157 (loop body at :75-78): value starts at 0.0f, in_index ascending.
void orc_linear_f16(const float* x, int64_t rows, int64_t in_dim, const uint16_t* w, int64_t out_dim, float* y) {
  for (int64_t r = 0; r < rows; ++r) {
    const float* xr = x + r * in_dim;
    float* yr = y + r * out_dim;
#pragma omp parallel for num_threads(g_threads) schedule(static)
    for (int64_t o = 0; o < out_dim; ++o) {
      const uint16_t* wr = w + o * in_dim;
      float value = 0.0f;
      for (int64_t i = 0; i < in_dim; ++i) value += xr[i] * F16(wr[i]);
      yr[o] = value;
    }
  }
}

void orc_linear_f32(const float* x, int64_t rows, int64_t in_dim, const float* w, int64_t out_dim, float* y) {
  for (int64_t r = 0; r < rows; ++r) {
    const float* xr = x + r * in_dim;
    float* yr = y + r * out_dim;
#pragma omp parallel for num_threads(g_threads) schedule(static)
    for (int64_t o = 0; o < out_dim; ++o) {
      const float* wr = w + o * in_dim;
      float value = 0.0f;
      for (int64_t i = 0; i < in_dim; ++i) value += xr[i] * wr[i];
      yr[o] = value;
    }
  }
}

}  // extern "C"

// Mac/cpu/src/rms_norm_module.cpp:56-66: mean of squares in fp32, scale = 1/sqrt(ms+eps), y = x*scale*w.
template <typename G>
static void rmsnorm_impl(const float* x, int64_t rows, int64_t n, G gain, float eps, float* y) {
  for (int64_t r = 0; r < rows; ++r) {
    const float* xr = x + r * n;
    float* yr = y + r * n;
    float ms = 0.0f;
    for (int64_t i = 0; i < n; ++i) ms += xr[i] * xr[i];
    ms /= static_cast<float>(n);
    const float scale = 1.0f / std::sqrt(ms + eps);
    for (int64_t i = 0; i < n; ++i) yr[i] = xr[i] * scale * gain(i);
  }
}

extern "C" {

void orc_rmsnorm_f16(const float* x, int64_t rows, int64_t n, const uint16_t* gain, float eps, float* y) {
  rmsnorm_impl(x, rows, n, [gain](int64_t i) { return F16(gain[i]); }, eps, y);
}

void orc_rmsnorm_f32(const float* x, int64_t rows, int64_t n, const float* gain, float eps, float* y) {
  rmsnorm_impl(x, rows, n, [gain](int64_t i) { return gain[i]; }, eps, y);
}

// Mac/cpu/src/rope.cpp:70-88: angle = (offset+pos) / theta^(2i/d) in double; cos/sin rounded to float;
// rotate-half pairs (i, i + d/2).
void orc_rope(float* x, int64_t seq, int64_t heads, int64_t head_dim, double theta, int64_t position_offset) {
  const int64_t half = head_dim / 2;
  for (int64_t p = 0; p < seq; ++p) {
    const double abs_pos = static_cast<double>(position_offset + p);
    for (int64_t h = 0; h < heads; ++h) {
      float* base = x + (p * heads + h) * head_dim;
      for (int64_t i = 0; i < half; ++i) {
        const double exponent = static_cast<double>(i * 2) / static_cast<double>(head_dim);
        const double angle = abs_pos / std::pow(theta, exponent);
        const float c = static_cast<float>(std::cos(angle));
        const float s = static_cast<float>(std::sin(angle));
        const float first = base[i];
        const float second = base[i + half];
        base[i] = first * c - second * s;
        base[i + half] = first * s + second * c;
      }
    }
  }
}

// Mac/cpu/src/grouped_query_attention.cpp:91-139.
int orc_gqa(const float* q, const float* k, const float* v, int64_t T, int64_t S, int64_t nq, int64_t nkv, int64_t d,
            int64_t prefix, int causal, float* out) {
  if (nq <= 0 || nkv <= 0 || d <= 0 || nq % nkv != 0 || prefix + T > S) return -1;
  const int64_t group = nq / nkv;
  const float scale = 1.0f / std::sqrt(static_cast<float>(d));
#pragma omp parallel num_threads(g_threads)
  {
    std::vector<float> scores(static_cast<size_t>(S) + 1), weights(static_cast<size_t>(S) + 1);
#pragma omp for collapse(2) schedule(static)
    for (int64_t t = 0; t < T; ++t) {
      for (int64_t h = 0; h < nq; ++h) {
        const int64_t visible = causal ? std::min(S, prefix + t + 1) : S;
        const int64_t g = h / group;
        const float* qv = q + (t * nq + h) * d;
        float max_score = -std::numeric_limits<float>::infinity();
        for (int64_t j = 0; j < visible; ++j) {
          const float* kv = k + (j * nkv + g) * d;
          float s = 0.0f;
          for (int64_t i = 0; i < d; ++i) s += qv[i] * kv[i];
          s *= scale;
          scores[j] = s;
          if (s > max_score) max_score = s;
        }
        float sum = 0.0f;
        for (int64_t j = 0; j < visible; ++j) {
          const float w = std::exp(scores[j] - max_score);
          weights[j] = w;
          sum += w;
        }
        float* o = out + (t * nq + h) * d;
        for (int64_t i = 0; i < d; ++i) o[i] = 0.0f;
        for (int64_t j = 0; j < visible; ++j) {
          const float nw = weights[j] / sum;
          const float* vv = v + (j * nkv + g) * d;
          for (int64_t i = 0; i < d; ++i) o[i] += nw * vv[i];
        }
      }
    }
  }
  return 0;
}

// Mac/cpu/src/sampler.cpp:26-61: partial_sort of the top-k by logit/temperature (strict >), then the best of the
// kept candidates. With top_k == 1 this is the first (lowest-index) maximum.
int orc_sample(const float* row, int64_t vocab, float temperature, int64_t top_k) {
  if (!(temperature > 0.0f) || top_k <= 0 || vocab <= 0) return -1;
  std::vector<int64_t> cand(static_cast<size_t>(vocab));
  for (int64_t i = 0; i < vocab; ++i) cand[i] = i;
  const int64_t k = std::min(top_k, vocab);
  std::partial_sort(cand.begin(), cand.begin() + k, cand.end(), [row, temperature](int64_t l, int64_t r) {
    return row[l] / temperature > row[r] / temperature;
  });
  int64_t best = cand[0];
  float best_score = row[best] / temperature;
  for (int64_t rank = 1; rank < k; ++rank) {
    const float s = row[cand[rank]] / temperature;
    if (s > best_score) {
      best_score = s;
      best = cand[rank];
    }
  }
  return static_cast<int>(best);
}

// Mac/gpu/src/runtime/sampler.cpp:44-66: top_k clamped to [1, vocab], a non-positive temperature taken as 1, the
// same std::partial_sort of candidate ids by logit / temperature; writes the k ids in that order and their raw
// logits, returns the first id.
int orc_sample_topk(const float* row, int64_t vocab, float temperature, int64_t top_k, int32_t* ids, float* vals) {
  if (vocab <= 0) return -1;
  const int64_t k = std::max<int64_t>(1, std::min<int64_t>(top_k, vocab));
  const float t = temperature <= 0.0f ? 1.0f : temperature;
  std::vector<int64_t> cand(static_cast<size_t>(vocab));
  for (int64_t i = 0; i < vocab; ++i) cand[i] = i;
  std::partial_sort(cand.begin(), cand.begin() + k, cand.end(),
                    [row, t](int64_t l, int64_t r) { return row[l] / t > row[r] / t; });
  for (int64_t r = 0; r < k; ++r) {
    ids[r] = static_cast<int32_t>(cand[r]);
    vals[r] = row[cand[r]];
  }
  return static_cast<int>(cand[0]);
}

// Group quantizer (the int8 per-column rule of Mac/cpu/header/matrix_ops.h:42-74 applied per group of 64 along K
// of each weight row, with the scale stored in fp16): amax = max |w| over the group; a zero group keeps scale 0 and
// codes 0; else s = fp16(amax / Q) (Q = 127 for 8 bits, 7 for 4 bits; a scale that rounds to 0 is stored as a zero
// group), code = clamp(round_half_away(w * (1 / s)), -Q, Q). Codes [N][K] int8, or int4 two per byte with the even k
// in the low nibble; scales [N][K/64] fp16.
int orc_quantize_group(const uint16_t* w, int64_t N, int64_t K, int bits, void* codes, uint16_t* scales) {
  if (!w || !codes || !scales || N <= 0 || K <= 0 || K % 64 != 0 || (bits != 8 && bits != 4)) return -1;
  for (int64_t i = 0; i < N * K; ++i)
    if ((w[i] & 0x7C00u) == 0x7C00u) return -1;  // inf / NaN: the rule has no scale for them
  const int Q = bits == 8 ? 127 : 7;
  const int64_t G = K / 64;
  for (int64_t n = 0; n < N; ++n)
    for (int64_t g = 0; g < G; ++g) {
      const uint16_t* src = w + n * K + g * 64;
      float amax = 0.0f;
      for (int i = 0; i < 64; ++i) amax = std::max(amax, std::fabs(F16(src[i])));
      uint16_t s16 = 0;
      float s = 0.0f;
      if (amax != 0.0f) {
        s16 = orc_f32_to_f16(amax / static_cast<float>(Q));
        s = F16(s16);
        if (s == 0.0f) s16 = 0;
      }
      scales[n * G + g] = s16;
      const float inv = s != 0.0f ? 1.0f / s : 0.0f;
      for (int i = 0; i < 64; ++i) {
        int q = 0;
        if (s != 0.0f) q = std::clamp(static_cast<int>(std::round(F16(src[i]) * inv)), -Q, Q);
        const int64_t k = g * 64 + i;
        if (bits == 8) {
          static_cast<int8_t*>(codes)[n * K + k] = static_cast<int8_t>(q);
        } else {
          uint8_t& byte = static_cast<uint8_t*>(codes)[(n * K + k) / 2];
          const uint8_t nib = static_cast<uint8_t>(q & 0xF);
          byte = (k % 2 == 0) ? static_cast<uint8_t>((byte & 0xF0) | nib) : static_cast<uint8_t>((byte & 0x0F) | (nib << 4));
        }
      }
    }
  return 0;
}

// Mac/cpu/src/qwen_mlp.cpp:65-74 with ApplySiLU (:20-35) and HadamardProduct (:37-54).
void orc_mlp_f16(const float* x, int64_t rows, int64_t hidden, int64_t inter, const uint16_t* gate,
                 const uint16_t* up, const uint16_t* down, float* y) {
  std::vector<float> g(static_cast<size_t>(rows * inter)), u(static_cast<size_t>(rows * inter));
  orc_linear_f16(x, rows, hidden, gate, inter, g.data());
  orc_linear_f16(x, rows, hidden, up, inter, u.data());
  for (int64_t i = 0; i < rows * inter; ++i) {
    const float value = g[i];
    const float act = value / (1.0f + std::exp(-value));
    g[i] = act * u[i];
  }
  orc_linear_f16(g.data(), rows, inter, down, hidden, y);
}

}  // extern "C"

// ------------------------------------------------------------------------------------------------------------
// Model
// ------------------------------------------------------------------------------------------------------------
struct orc_layer {
  const uint16_t* input_norm = nullptr;
  const uint16_t* q = nullptr;
  const uint16_t* k = nullptr;
  const uint16_t* v = nullptr;
  const uint16_t* o = nullptr;
  const uint16_t* q_norm = nullptr;
  const uint16_t* k_norm = nullptr;
  const uint16_t* post_norm = nullptr;
  const uint16_t* gate = nullptr;
  const uint16_t* up = nullptr;
  const uint16_t* down = nullptr;
  // fp32 projections (dequantized group-quantized weights), used instead of the fp16 ones when set
  const float* qf = nullptr;
  const float* kf = nullptr;
  const float* vf = nullptr;
  const float* of = nullptr;
  const float* gatef = nullptr;
  const float* upf = nullptr;
  const float* downf = nullptr;
};

struct orc_model {
  int64_t V, H, L, nq, nkv, d, I;
  double theta;
  float eps;
  bool tied;
  const uint16_t* embed = nullptr;
  const uint16_t* final_norm = nullptr;
  const uint16_t* lm_head = nullptr;
  std::vector<orc_layer> layers;
};

struct orc_cache {
  int64_t L, nkv, d, cap;
  int64_t length = 0;
  std::vector<float> key, value;  // [layer][kv_head][pos][d] (Mac/cpu/src/kv_cache.cpp:148-155, batch 1)
  size_t off(int64_t layer, int64_t head, int64_t pos) const {
    return static_cast<size_t>(((layer * nkv + head) * cap + pos) * d);
  }
};

extern "C" {

orc_model* orc_model_create(int64_t vocab, int64_t hidden, int64_t layers, int64_t nq, int64_t nkv, int64_t head_dim,
                            int64_t inter, double rope_theta, float eps, int tie) {
  if (vocab <= 0 || hidden <= 0 || layers < 0 || nq <= 0 || nkv <= 0 || head_dim <= 0 || head_dim % 2 != 0 ||
      inter <= 0 || nq % nkv != 0 || !(eps > 0.0f) || !(rope_theta > 0.0))
    return nullptr;
  orc_model* m = new orc_model();
  m->V = vocab;
  m->H = hidden;
  m->L = layers;
  m->nq = nq;
  m->nkv = nkv;
  m->d = head_dim;
  m->I = inter;
  m->theta = rope_theta;
  m->eps = eps;
  m->tied = tie != 0;
  m->layers.resize(static_cast<size_t>(layers));
  return m;
}

void orc_model_destroy(orc_model* m) { delete m; }

// Names and shapes follow Mac/cpu/src/qwen_model_loader.cpp:43-92.
int orc_model_set(orc_model* m, const char* name_c, const uint16_t* data, int64_t numel) {
  if (!m || !name_c || !data) return -1;
  const std::string name(name_c);
  const int64_t qd = m->nq * m->d, kvd = m->nkv * m->d;
  auto expect = [&](int64_t n) { return numel == n ? 0 : -2; };
  if (name == "model.embed_tokens.weight") {
    m->embed = data;
    return expect(m->V * m->H);
  }
  if (name == "model.norm.weight") {
    m->final_norm = data;
    return expect(m->H);
  }
  if (name == "lm_head.weight") {
    m->lm_head = data;
    return expect(m->V * m->H);
  }
  const std::string prefix = "model.layers.";
  if (name.compare(0, prefix.size(), prefix) != 0) return -3;
  size_t dot = name.find('.', prefix.size());
  if (dot == std::string::npos) return -3;
  const int64_t li = std::stoll(name.substr(prefix.size(), dot - prefix.size()));
  if (li < 0 || li >= m->L) return -3;
  const std::string suffix = name.substr(dot + 1);
  orc_layer& l = m->layers[static_cast<size_t>(li)];
  if (suffix == "input_layernorm.weight") { l.input_norm = data; return expect(m->H); }
  if (suffix == "post_attention_layernorm.weight") { l.post_norm = data; return expect(m->H); }
  if (suffix == "self_attn.q_proj.weight") { l.q = data; return expect(qd * m->H); }
  if (suffix == "self_attn.k_proj.weight") { l.k = data; return expect(kvd * m->H); }
  if (suffix == "self_attn.v_proj.weight") { l.v = data; return expect(kvd * m->H); }
  if (suffix == "self_attn.o_proj.weight") { l.o = data; return expect(m->H * qd); }
  if (suffix == "self_attn.q_norm.weight") { l.q_norm = data; return expect(m->d); }
  if (suffix == "self_attn.k_norm.weight") { l.k_norm = data; return expect(m->d); }
  if (suffix == "mlp.gate_proj.weight") { l.gate = data; return expect(m->I * m->H); }
  if (suffix == "mlp.up_proj.weight") { l.up = data; return expect(m->I * m->H); }
  if (suffix == "mlp.down_proj.weight") { l.down = data; return expect(m->H * m->I); }
  return -3;
}

// fp32 weights for a layer's projections (the reference Linear reads Float32 tensors as they are,
// Mac/cpu/src/dtype.cpp:165-176): for models whose projections were group-quantized and dequantized.
int orc_model_set_f32(orc_model* m, const char* name_c, const float* data, int64_t numel) {
  if (!m || !name_c || !data) return -1;
  const std::string name(name_c);
  const int64_t qd = m->nq * m->d, kvd = m->nkv * m->d;
  auto expect = [&](int64_t n) { return numel == n ? 0 : -2; };
  const std::string prefix = "model.layers.";
  if (name.compare(0, prefix.size(), prefix) != 0) return -3;
  size_t dot = name.find('.', prefix.size());
  if (dot == std::string::npos) return -3;
  const int64_t li = std::stoll(name.substr(prefix.size(), dot - prefix.size()));
  if (li < 0 || li >= m->L) return -3;
  const std::string suffix = name.substr(dot + 1);
  orc_layer& l = m->layers[static_cast<size_t>(li)];
  if (suffix == "self_attn.q_proj.weight") { l.qf = data; return expect(qd * m->H); }
  if (suffix == "self_attn.k_proj.weight") { l.kf = data; return expect(kvd * m->H); }
  if (suffix == "self_attn.v_proj.weight") { l.vf = data; return expect(kvd * m->H); }
  if (suffix == "self_attn.o_proj.weight") { l.of = data; return expect(m->H * qd); }
  if (suffix == "mlp.gate_proj.weight") { l.gatef = data; return expect(m->I * m->H); }
  if (suffix == "mlp.up_proj.weight") { l.upf = data; return expect(m->I * m->H); }
  if (suffix == "mlp.down_proj.weight") { l.downf = data; return expect(m->H * m->I); }
  return -3;
}

int orc_model_check(const orc_model* m) {
  if (!m || !m->embed || !m->final_norm) return -1;
  if (!m->tied && !m->lm_head) return -1;
  for (const orc_layer& l : m->layers) {
    if (!l.input_norm || !(l.q || l.qf) || !(l.k || l.kf) || !(l.v || l.vf) || !(l.o || l.of) || !l.q_norm ||
        !l.k_norm || !l.post_norm || !(l.gate || l.gatef) || !(l.up || l.upf) || !(l.down || l.downf))
      return -1;
  }
  return 0;
}

orc_cache* orc_cache_create(const orc_model* m, int64_t max_seq) {
  if (!m || max_seq <= 0) return nullptr;
  orc_cache* c = new orc_cache();
  c->L = m->L;
  c->nkv = m->nkv;
  c->d = m->d;
  c->cap = max_seq;
  const size_t n = static_cast<size_t>(m->L * m->nkv * max_seq * m->d);
  c->key.assign(n, 0.0f);
  c->value.assign(n, 0.0f);
  return c;
}

void orc_cache_destroy(orc_cache* c) { delete c; }
void orc_cache_clear(orc_cache* c) {
  if (c) c->length = 0;
}
int64_t orc_cache_length(const orc_cache* c) { return c ? c->length : -1; }

int orc_cache_write(orc_cache* c, int64_t layer, int64_t pos, const float* key, const float* value) {
  if (!c || layer < 0 || layer >= c->L || pos < 0 || pos >= c->cap) return -1;
  for (int64_t h = 0; h < c->nkv; ++h)
    for (int64_t i = 0; i < c->d; ++i) {
      c->key[c->off(layer, h, pos) + i] = key[h * c->d + i];
      c->value[c->off(layer, h, pos) + i] = value[h * c->d + i];
    }
  if (pos + 1 > c->length) c->length = pos + 1;
  return 0;
}

}  // extern "C"

namespace {

// A projection with fp16 weights, or fp32 ones when the layer has them.
void lin(const float* x, int64_t rows, int64_t in_dim, const uint16_t* w16, const float* w32, int64_t out_dim,
         float* y) {
  if (w32 != nullptr) orc_linear_f32(x, rows, in_dim, w32, out_dim, y);
  else orc_linear_f16(x, rows, in_dim, w16, out_dim, y);
}

// Mac/cpu/src/qwen_attention.cpp:103-140 (uncached) and :142-205 (cached). Returns o_proj output [T][H].
void attention_forward(const orc_model* m, int64_t li, const float* xn, int64_t T, int64_t pos, orc_cache* cache,
                       float* out) {
  const orc_layer& l = m->layers[static_cast<size_t>(li)];
  const int64_t qd = m->nq * m->d, kvd = m->nkv * m->d;
  std::vector<float> q(static_cast<size_t>(T * qd)), k(static_cast<size_t>(T * kvd)), v(static_cast<size_t>(T * kvd));
  lin(xn, T, m->H, l.q, l.qf, qd, q.data());
  lin(xn, T, m->H, l.k, l.kf, kvd, k.data());
  lin(xn, T, m->H, l.v, l.vf, kvd, v.data());
  // q_norm / k_norm over each head's d features (qwen_attention.cpp:168-169), then RoPE (:170-171).
  std::vector<float> qn(q.size()), kn(k.size());
  orc_rmsnorm_f16(q.data(), T * m->nq, m->d, l.q_norm, m->eps, qn.data());
  orc_rmsnorm_f16(k.data(), T * m->nkv, m->d, l.k_norm, m->eps, kn.data());
  orc_rope(qn.data(), T, m->nq, m->d, m->theta, pos);
  orc_rope(kn.data(), T, m->nkv, m->d, m->theta, pos);
  std::vector<float> attn(static_cast<size_t>(T * qd));
  if (cache == nullptr) {
    orc_gqa(qn.data(), kn.data(), v.data(), T, T, m->nq, m->nkv, m->d, 0, 1, attn.data());
  } else {
    // TensorKVCache::Write per token (kv_cache.cpp:50-78), then Read of the whole prefix (:80-110).
    for (int64_t t = 0; t < T; ++t) {
      const int64_t p = pos + t;
      for (int64_t h = 0; h < m->nkv; ++h)
        for (int64_t i = 0; i < m->d; ++i) {
          cache->key[cache->off(li, h, p) + i] = kn[(t * m->nkv + h) * m->d + i];
          cache->value[cache->off(li, h, p) + i] = v[(t * m->nkv + h) * m->d + i];
        }
      if (p + 1 > cache->length) cache->length = p + 1;
    }
    const int64_t S = pos + T;
    std::vector<float> ck(static_cast<size_t>(S * kvd)), cv(static_cast<size_t>(S * kvd));
    for (int64_t p = 0; p < S; ++p)
      for (int64_t h = 0; h < m->nkv; ++h)
        for (int64_t i = 0; i < m->d; ++i) {
          ck[(p * m->nkv + h) * m->d + i] = cache->key[cache->off(li, h, p) + i];
          cv[(p * m->nkv + h) * m->d + i] = cache->value[cache->off(li, h, p) + i];
        }
    orc_gqa(qn.data(), ck.data(), cv.data(), T, S, m->nq, m->nkv, m->d, pos, 1, attn.data());
  }
  lin(attn.data(), T, qd, l.o, l.of, m->H, out);
}

// Mac/cpu/src/qwen_block.cpp:63-73 (cached) / :51-61 (uncached): pre-norm residual block.
void block_forward(const orc_model* m, int64_t li, std::vector<float>& x, int64_t T, int64_t pos, orc_cache* cache) {
  const orc_layer& l = m->layers[static_cast<size_t>(li)];
  const size_t n = static_cast<size_t>(T * m->H);
  std::vector<float> xn(n), a(n), r(n), mo(n);
  orc_rmsnorm_f16(x.data(), T, m->H, l.input_norm, m->eps, xn.data());
  attention_forward(m, li, xn.data(), T, pos, cache, a.data());
  for (size_t i = 0; i < n; ++i) r[i] = x[i] + a[i];  // AddTensors (qwen_block.cpp:19-34)
  orc_rmsnorm_f16(r.data(), T, m->H, l.post_norm, m->eps, xn.data());
  if (l.gatef == nullptr && l.upf == nullptr && l.downf == nullptr) {
    orc_mlp_f16(xn.data(), T, m->H, m->I, l.gate, l.up, l.down, mo.data());
  } else {  // the same steps (qwen_mlp.cpp:65-74) with fp32 projections
    std::vector<float> g(static_cast<size_t>(T * m->I)), u(g.size());
    lin(xn.data(), T, m->H, l.gate, l.gatef, m->I, g.data());
    lin(xn.data(), T, m->H, l.up, l.upf, m->I, u.data());
    for (size_t i = 0; i < g.size(); ++i) {
      const float value = g[i];
      g[i] = value / (1.0f + std::exp(-value)) * u[i];
    }
    lin(g.data(), T, m->I, l.down, l.downf, m->H, mo.data());
  }
  for (size_t i = 0; i < n; ++i) x[i] = r[i] + mo[i];
}

// Mac/cpu/src/qwen_causal_lm.cpp:50-80: embedding -> blocks -> final norm. Returns normed hidden [T][H].
std::vector<float> hidden_forward(const orc_model* m, const int32_t* ids, int64_t T, int64_t pos, orc_cache* cache) {
  std::vector<float> x(static_cast<size_t>(T * m->H));
  // Embedding::Forward (embedding.cpp:51-77).
  for (int64_t t = 0; t < T; ++t) {
    const int64_t id = ids[t];
    for (int64_t i = 0; i < m->H; ++i) x[t * m->H + i] = F16(m->embed[id * m->H + i]);
  }
  for (int64_t li = 0; li < m->L; ++li) block_forward(m, li, x, T, pos, cache);
  std::vector<float> y(x.size());
  orc_rmsnorm_f16(x.data(), T, m->H, m->final_norm, m->eps, y.data());
  return y;
}

// Mac/cpu/src/qwen_causal_lm.cpp:82-116 (tied) or lm_head Linear (:68-70).
void logits_rows(const orc_model* m, const float* h, int64_t rows, float* logits) {
  const uint16_t* head = m->tied ? m->embed : m->lm_head;
  orc_linear_f16(h, rows, m->H, head, m->V, logits);
}

bool ids_valid(const orc_model* m, const int32_t* ids, int64_t T) {
  for (int64_t t = 0; t < T; ++t)
    if (ids[t] < 0 || ids[t] >= m->V) return false;  // embedding.cpp:66-68 throws on out-of-range ids
  return true;
}

}  // namespace

extern "C" {

int orc_forward_logits(const orc_model* m, const int32_t* ids, int64_t T, int64_t pos, float* logits,
                       float* hidden_out) {
  if (!m || orc_model_check(m) != 0 || T <= 0 || !ids_valid(m, ids, T)) return -1;
  std::vector<float> h = hidden_forward(m, ids, T, pos, nullptr);
  if (hidden_out) std::memcpy(hidden_out, h.data(), h.size() * sizeof(float));
  if (logits) logits_rows(m, h.data(), T, logits);
  return 0;
}

int orc_forward_logits_cached(const orc_model* m, orc_cache* c, const int32_t* ids, int64_t T, int64_t pos,
                              int64_t logit_rows, float* logits) {
  if (!m || !c || orc_model_check(m) != 0 || T <= 0 || !ids_valid(m, ids, T)) return -1;
  if (pos + T > c->cap || pos > c->length) return -2;  // kv_cache.cpp:53 / :84
  std::vector<float> h = hidden_forward(m, ids, T, pos, c);
  if (logits && logit_rows > 0) {
    const int64_t rows = std::min(logit_rows, T);
    logits_rows(m, h.data() + (T - rows) * m->H, rows, logits);
  }
  return 0;
}

// Mac/cpu/src/generation_session.cpp:46-79 and DecodeNextToken (:16-44). The prompt's uncached forward
// (:54) and cached forward (:56) produce bit-identical last-row logits (each row depends only on earlier rows and
// the cache stores exact fp32 copies), so the cached forward alone supplies the first token here.
int orc_generate(const orc_model* m, const int32_t* prompt, int64_t T, int64_t max_new, int eos, int64_t max_seq,
                 float temperature, int64_t top_k, int32_t* out, float* step_logits) {
  if (!m || orc_model_check(m) != 0 || T <= 0 || max_new < 0 || !ids_valid(m, prompt, T)) return -1;
  if (T + max_new > max_seq + 1) return -2;
  orc_cache* c = orc_cache_create(m, max_seq);
  std::vector<float> logits(static_cast<size_t>(m->V));
  int produced = 0;
  if (max_new > 0) {
    int rc = orc_forward_logits_cached(m, c, prompt, T, 0, 1, logits.data());
    if (rc != 0) {
      orc_cache_destroy(c);
      return rc;
    }
    int tok = orc_sample(logits.data(), m->V, temperature, top_k);
    if (step_logits) std::memcpy(step_logits, logits.data(), logits.size() * sizeof(float));
    out[produced++] = tok;
    int64_t len = T + 1;
    while (produced < max_new && !(eos >= 0 && tok == eos)) {
      const int32_t last = tok;
      rc = orc_forward_logits_cached(m, c, &last, 1, len - 1, 1, logits.data());
      if (rc != 0) {
        orc_cache_destroy(c);
        return rc;
      }
      tok = orc_sample(logits.data(), m->V, temperature, top_k);
      if (step_logits) std::memcpy(step_logits + produced * m->V, logits.data(), logits.size() * sizeof(float));
      out[produced++] = tok;
      ++len;
    }
  }
  orc_cache_destroy(c);
  return produced;
}

// ---- Group-quantized format (defined by this project, written down in the header). ----
static inline int32_t code_at(const void* codes, int bits, int64_t K, int64_t n, int64_t k) {
  if (bits == 8) return static_cast<const int8_t*>(codes)[n * K + k];
  const uint8_t byte = static_cast<const uint8_t*>(codes)[n * (K / 2) + k / 2];
  const int32_t nib = (k & 1) ? (byte >> 4) : (byte & 0xf);
  return nib >= 8 ? nib - 16 : nib;
}

int orc_dequant_group(const void* codes, int bits, const uint16_t* scales, int64_t group, int64_t N, int64_t K,
                      float* w) {
  if ((bits != 8 && bits != 4) || group <= 0 || K % group != 0 || (bits == 4 && K % 2 != 0)) return -1;
  const int64_t G = K / group;
  for (int64_t n = 0; n < N; ++n)
    for (int64_t k = 0; k < K; ++k)
      w[n * K + k] = static_cast<float>(code_at(codes, bits, K, n, k)) * F16(scales[n * G + k / group]);
  return 0;
}

int orc_qmm_group(const uint16_t* a, int64_t M, int64_t K, const void* codes, int bits, const uint16_t* scales,
                  int64_t group, int64_t N, float* y) {
  if ((bits != 8 && bits != 4) || group <= 0 || K % group != 0 || (bits == 4 && K % 2 != 0)) return -1;
  const int64_t G = K / group;
  std::vector<float> af(static_cast<size_t>(M * K));
  for (int64_t i = 0; i < M * K; ++i) af[i] = F16(a[i]);
  for (int64_t mi = 0; mi < M; ++mi) {
#pragma omp parallel for num_threads(g_threads) schedule(static)
    for (int64_t n = 0; n < N; ++n) {
      float value = 0.0f;
      for (int64_t k = 0; k < K; ++k) {
        const float w = static_cast<float>(code_at(codes, bits, K, n, k)) * F16(scales[n * G + k / group]);
        value += af[mi * K + k] * w;
      }
      y[mi * N + n] = value;
    }
  }
  return 0;
}

// Mac/cpu/header/matrix_ops.h:42-74: symmetric per-output-column int8, scale = max|w|/127, round half away.
void orc_quant_int8_percol(const float* rhs, int64_t K, int64_t N, int8_t* codes, float* scales) {
  for (int64_t n = 0; n < N; ++n) {
    float max_abs = 0.0f;
    for (int64_t k = 0; k < K; ++k) max_abs = std::max(max_abs, std::fabs(rhs[k * N + n]));
    scales[n] = 0.0f;
    for (int64_t k = 0; k < K; ++k) codes[n * K + k] = 0;
    if (max_abs == 0.0f) continue;
    const float scale = max_abs / 127.0f;
    const float inv = 1.0f / scale;
    scales[n] = scale;
    for (int64_t k = 0; k < K; ++k) {
      int qv = static_cast<int>(std::round(rhs[k * N + n] * inv));
      qv = std::min(127, std::max(-127, qv));
      codes[n * K + k] = static_cast<int8_t>(qv);
    }
  }
}

// Mac/cpu/header/matrix_ops.h:308-350: sum_k a*float(q), k ascending (the 4-way unroll keeps the order), then
// times the column scale; a zero scale gives 0.
void orc_matmul_quant_int8(const float* a, int64_t M, int64_t K, const int8_t* codes, const float* scales, int64_t N,
                           float* y) {
  for (int64_t mi = 0; mi < M; ++mi)
    for (int64_t n = 0; n < N; ++n) {
      if (scales[n] == 0.0f) {
        y[mi * N + n] = 0.0f;
        continue;
      }
      float sum = 0.0f;
      for (int64_t k = 0; k < K; ++k) sum += a[mi * K + k] * static_cast<float>(codes[n * K + k]);
      y[mi * N + n] = sum * scales[n];
    }
}

}  // extern "C"
