// ref_driver.cpp - a C entry layer over the reference CPU runtime's own classes.
//
// TEST INFRASTRUCTURE ONLY. oracle/Makefile compiles this file together with the reference's hot-path sources
// where they lie (/root/reference/Mac/cpu/src/*.cpp, headers under Mac/cpu/header) into oracle/_ref/libsocref.so.
// The fixture writer (tests/golden/make_golden.py) and the CPU baseline in bench.py call it; nothing in the
// product does. Nothing from the reference is copied here: this file only constructs the reference's objects from
// caller-owned buffers (Storage::External) and calls their public methods.
//
// The reference's GenerationSession (Mac/cpu/src/generation_session.cpp) cannot be linked: it holds a
// TokenizerRuntime whose JSON layer needs Apple libc++. ref_generate therefore drives the reference model,
// TensorKVCache and Sampler through the same steps as GenerationSession::Generate (:46-79) and
// DecodeNextToken (:16-44), including the uncached prompt forward for the first token.
#include <cstdint>
#include <cstring>
#include <map>
#include <memory>
#include <stdexcept>
#include <string>
#include <vector>

#include "header/dtype.h"
#include "header/embedding.h"
#include "header/grouped_query_attention.h"
#include "header/kv_cache.h"
#include "header/linear.h"
#include "header/matrix_ops.h"
#include "header/qwen_attention.h"
#include "header/qwen_block.h"
#include "header/qwen_causal_lm.h"
#include "header/qwen_mlp.h"
#include "header/rms_norm_module.h"
#include "header/rope.h"
#include "header/sampler.h"
#include "header/storage.h"
#include "header/tensor.h"

namespace {

Tensor F16View(const uint16_t* p, std::vector<std::size_t> shape) {
  std::size_t n = 1;
  for (std::size_t s : shape) n *= s;
  return Tensor(Storage::External(const_cast<uint16_t*>(p), n * 2), DType::Float16, std::move(shape));
}

Tensor F32View(const float* p, std::vector<std::size_t> shape) {
  std::size_t n = 1;
  for (std::size_t s : shape) n *= s;
  return Tensor(Storage::External(const_cast<float*>(p), n * 4), DType::Float32, std::move(shape));
}

Tensor I32Copy(const int32_t* p, std::size_t n) {
  return Tensor(Storage::FromOwnedCopy(p, n * sizeof(int32_t)), DType::Int32, {1, n});
}

thread_local std::string g_error;

}  // namespace

struct ref_model {
  std::unique_ptr<QwenCausalLM> lm;
  std::size_t V, H, L, nkv, d;
};

struct ref_cache {
  std::unique_ptr<TensorKVCache> cache;
};

extern "C" {

const char* ref_last_error() { return g_error.c_str(); }

float ref_f16_to_f32(uint16_t v) { return Float16ToFloat32(v); }
uint16_t ref_f32_to_f16(float v) { return Float32ToFloat16(v); }

// Array forms move raw bits (a float returned by value through a foreign-function layer may have its NaN
// payload quieted).
void ref_f16_to_f32_array(const uint16_t* in, float* out, int64_t n) {
  for (int64_t i = 0; i < n; ++i) out[i] = Float16ToFloat32(in[i]);
}
void ref_f32_to_f16_array(const float* in, uint16_t* out, int64_t n) {
  for (int64_t i = 0; i < n; ++i) out[i] = Float32ToFloat16(in[i]);
}

int ref_linear_f16(const float* x, int64_t rows, int64_t in, const uint16_t* w, int64_t out, float* y) {
  try {
    Linear lin(F16View(w, {(size_t)out, (size_t)in}));
    Tensor r = lin.Forward(F32View(x, {(size_t)rows, (size_t)in}));
    std::memcpy(y, r.data<float>(), (size_t)(rows * out) * 4);
    return 0;
  } catch (const std::exception& e) {
    g_error = e.what();
    return -1;
  }
}

int ref_rmsnorm_f16(const float* x, int64_t rows, int64_t n, const uint16_t* gain, float eps, float* y) {
  try {
    RMSNormModule norm(F16View(gain, {(size_t)n}), eps);
    Tensor r = norm.Forward(F32View(x, {(size_t)rows, (size_t)n}));
    std::memcpy(y, r.data<float>(), (size_t)(rows * n) * 4);
    return 0;
  } catch (const std::exception& e) {
    g_error = e.what();
    return -1;
  }
}

int ref_rope(float* x, int64_t seq, int64_t heads, int64_t d, double theta, int64_t off) {
  try {
    RoPE rope((size_t)d, theta);
    Tensor t = F32View(x, {(size_t)seq, (size_t)heads, (size_t)d});
    rope.ApplyInPlace(t, (size_t)off);
    return 0;
  } catch (const std::exception& e) {
    g_error = e.what();
    return -1;
  }
}

int ref_gqa(const float* q, const float* k, const float* v, int64_t T, int64_t S, int64_t nq, int64_t nkv, int64_t d,
            int64_t prefix, int causal, float* out) {
  try {
    GroupedQueryAttention attn((size_t)nq, (size_t)nkv, (size_t)d, causal != 0);
    Tensor r = attn.ForwardWithPrefix(F32View(q, {1, (size_t)T, (size_t)nq, (size_t)d}),
                                      F32View(k, {1, (size_t)S, (size_t)nkv, (size_t)d}),
                                      F32View(v, {1, (size_t)S, (size_t)nkv, (size_t)d}), (size_t)prefix);
    std::memcpy(out, r.data<float>(), (size_t)(T * nq * d) * 4);
    return 0;
  } catch (const std::exception& e) {
    g_error = e.what();
    return -1;
  }
}

int ref_sample(const float* row, int64_t vocab, float temperature, int64_t top_k) {
  try {
    Sampler s(SamplerConfig{temperature, (size_t)top_k});
    return s.SampleFromLogits(F32View(row, {1, 1, (size_t)vocab}), 0, 0);
  } catch (const std::exception& e) {
    g_error = e.what();
    return -1;
  }
}

// Builds the model exactly as Mac/cpu/src/qwen_model_loader.cpp:35-93 does, from borrowed fp16 tensors.
ref_model* ref_model_create(int64_t V, int64_t H, int64_t L, int64_t nq, int64_t nkv, int64_t d, int64_t I,
                            double theta, float eps, int tied, const char* const* names, const uint16_t* const* ptrs,
                            int count) {
  try {
    std::map<std::string, const uint16_t*> t;
    for (int i = 0; i < count; ++i) t[names[i]] = ptrs[i];
    auto get = [&](const std::string& n) {
      auto it = t.find(n);
      if (it == t.end()) throw std::runtime_error("missing tensor " + n);
      return it->second;
    };
    const size_t qd = (size_t)(nq * d), kvd = (size_t)(nkv * d);
    Embedding emb(F16View(get("model.embed_tokens.weight"), {(size_t)V, (size_t)H}));
    std::vector<QwenBlock> blocks;
    for (int64_t li = 0; li < L; ++li) {
      const std::string p = "model.layers." + std::to_string(li) + ".";
      RMSNormModule in_norm(F16View(get(p + "input_layernorm.weight"), {(size_t)H}), eps);
      QwenAttention attn(Linear(F16View(get(p + "self_attn.q_proj.weight"), {qd, (size_t)H})),
                         Linear(F16View(get(p + "self_attn.k_proj.weight"), {kvd, (size_t)H})),
                         Linear(F16View(get(p + "self_attn.v_proj.weight"), {kvd, (size_t)H})),
                         Linear(F16View(get(p + "self_attn.o_proj.weight"), {(size_t)H, qd})),
                         RMSNormModule(F16View(get(p + "self_attn.q_norm.weight"), {(size_t)d}), eps),
                         RMSNormModule(F16View(get(p + "self_attn.k_norm.weight"), {(size_t)d}), eps),
                         RoPE((size_t)d, theta), GroupedQueryAttention((size_t)nq, (size_t)nkv, (size_t)d, true));
      RMSNormModule post_norm(F16View(get(p + "post_attention_layernorm.weight"), {(size_t)H}), eps);
      QwenMLP mlp(Linear(F16View(get(p + "mlp.gate_proj.weight"), {(size_t)I, (size_t)H})),
                  Linear(F16View(get(p + "mlp.up_proj.weight"), {(size_t)I, (size_t)H})),
                  Linear(F16View(get(p + "mlp.down_proj.weight"), {(size_t)H, (size_t)I})));
      blocks.emplace_back(in_norm, attn, post_norm, mlp);
    }
    RMSNormModule final_norm(F16View(get("model.norm.weight"), {(size_t)H}), eps);
    ref_model* m = new ref_model();
    if (tied) {
      m->lm.reset(new QwenCausalLM(emb, std::move(blocks), final_norm));
    } else {
      m->lm.reset(new QwenCausalLM(emb, std::move(blocks), final_norm,
                                   Linear(F16View(get("lm_head.weight"), {(size_t)V, (size_t)H}))));
    }
    m->V = (size_t)V;
    m->H = (size_t)H;
    m->L = (size_t)L;
    m->nkv = (size_t)nkv;
    m->d = (size_t)d;
    return m;
  } catch (const std::exception& e) {
    g_error = e.what();
    return nullptr;
  }
}

void ref_model_destroy(ref_model* m) { delete m; }

ref_cache* ref_cache_create(ref_model* m, int64_t max_seq) {
  try {
    ref_cache* c = new ref_cache();
    c->cache.reset(new TensorKVCache(m->L, 1, m->nkv, m->d, (size_t)max_seq));
    return c;
  } catch (const std::exception& e) {
    g_error = e.what();
    return nullptr;
  }
}

void ref_cache_destroy(ref_cache* c) { delete c; }

int ref_cache_write(ref_cache* c, int64_t layer, int64_t pos, const float* key, const float* value, int64_t nkv,
                    int64_t d) {
  try {
    c->cache->Write((size_t)layer, 0, (size_t)pos, F32View(key, {(size_t)nkv, (size_t)d}),
                    F32View(value, {(size_t)nkv, (size_t)d}));
    return 0;
  } catch (const std::exception& e) {
    g_error = e.what();
    return -1;
  }
}

// logits [T][V] (all rows, as the reference computes them).
int ref_forward_logits(ref_model* m, const int32_t* ids, int64_t T, int64_t pos, float* logits) {
  try {
    Tensor r = m->lm->ForwardLogits(I32Copy(ids, (size_t)T), (size_t)pos);
    std::memcpy(logits, r.data<float>(), (size_t)T * m->V * 4);
    return 0;
  } catch (const std::exception& e) {
    g_error = e.what();
    return -1;
  }
}

int ref_forward_logits_cached(ref_model* m, ref_cache* c, const int32_t* ids, int64_t T, int64_t pos, float* logits) {
  try {
    Tensor r = m->lm->ForwardLogitsCached(I32Copy(ids, (size_t)T), *c->cache, (size_t)pos);
    if (logits) std::memcpy(logits, r.data<float>(), (size_t)T * m->V * 4);
    return 0;
  } catch (const std::exception& e) {
    g_error = e.what();
    return -1;
  }
}

// GenerationSession::Generate (generation_session.cpp:46-79) with GenerationSession::DecodeNextToken (:16-44).
// step_logits (nullable): [max_new][V]; row 0 = the uncached prompt forward's last row.
int ref_generate(ref_model* m, const int32_t* prompt, int64_t T, int64_t max_new, int eos, int64_t max_seq,
                 float temperature, int64_t top_k, int32_t* out, float* step_logits) {
  try {
    Sampler sampler(SamplerConfig{temperature, (size_t)top_k});
    TensorKVCache cache(m->L, 1, m->nkv, m->d, (size_t)max_seq);
    std::vector<int32_t> running(prompt, prompt + T);
    int produced = 0;
    if (max_new == 0) return 0;
    const Tensor prompt_tensor = I32Copy(prompt, (size_t)T);
    const Tensor logits = m->lm->ForwardLogits(prompt_tensor, 0);
    static_cast<void>(m->lm->ForwardLogitsCached(prompt_tensor, cache, 0));
    int tok = sampler.SampleFromLogits(logits, 0, (size_t)T - 1);
    if (step_logits) std::memcpy(step_logits, logits.data<float>() + (size_t)(T - 1) * m->V, m->V * 4);
    out[produced++] = tok;
    running.push_back(tok);
    if (eos >= 0 && tok == eos) return produced;
    while (produced < max_new) {
      const size_t required_prefix = running.size() - 1;
      if (cache.length(0) != required_prefix) {
        // DecodeNextToken re-prefills when the cache does not hold exactly the prefix (:27-38).
        cache.ClearSequence(0);
        if (required_prefix != 0)
          static_cast<void>(m->lm->ForwardLogitsCached(I32Copy(running.data(), required_prefix), cache, 0));
      }
      const int32_t last = running.back();
      const Tensor step = m->lm->ForwardLogitsCached(I32Copy(&last, 1), cache, required_prefix);
      tok = sampler.SampleFromLogits(step, 0, 0);
      if (step_logits) std::memcpy(step_logits + (size_t)produced * m->V, step.data<float>(), m->V * 4);
      out[produced++] = tok;
      running.push_back(tok);
      if (eos >= 0 && tok == eos) break;
    }
    return produced;
  } catch (const std::exception& e) {
    g_error = e.what();
    return -1;
  }
}

// Mac/cpu/header/matrix_ops.h:42-74 (QuantizeMatMulRhs8) and :308-350 (MatMulQuantized).
int ref_quant_matmul_int8(const float* a, int64_t M, int64_t K, const float* rhs, int64_t N, int8_t* codes,
                          float* scales, float* y) {
  try {
    matrix<float> b((int)K, (int)N);
    std::memcpy(b.raw_data(), rhs, (size_t)(K * N) * 4);
    QuantizedPackedMatMulRhs8 packed = QuantizeMatMulRhs8(b);
    std::memcpy(codes, packed.values.data(), (size_t)(K * N));
    std::memcpy(scales, packed.scales.data(), (size_t)N * 4);
    matrix<float> am((int)M, (int)K);
    std::memcpy(am.raw_data(), a, (size_t)(M * K) * 4);
    matrix<float> r = MatMulQuantized(am, packed);
    std::memcpy(y, r.raw_data(), (size_t)(M * N) * 4);
    return 0;
  } catch (const std::exception& e) {
    g_error = e.what();
    return -1;
  }
}

}  // extern "C"
