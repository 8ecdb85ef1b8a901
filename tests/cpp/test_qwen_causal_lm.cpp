// C++ host-interface test of the model-level API: the call shape of the reference's GPU generation test
// (Mac/gpu/test/runtime/test_generation_context.mm:17-140) -- float32 device tensors built with MakeFloatTensor, a
// QwenCausalLM constructed from QwenCausalLMWeights, weights() checked, then GenerationContext::Generate -- at head
// dim 128 (the only head size the kernels take), so the identity model is 128 wide: one-hot embedding rows e_0..e_3,
// zero projections, unit gains. The residual stream stays e_t, the final RMSNorm scales it to sqrt(128) e_t and the
// tied head gives logit sqrt(128) to the input token and 0 to the others: Generate([1, 2], 3) = [2, 2, 2].
// Then the model's four forwards (qwen_causal_lm.h:47-80) on that model, whose outputs are known in closed form, a
// weights-constructor error, and the op classes (Mac/gpu/include/op/*.h) against host arithmetic.
#include <cmath>
#include <cstdio>
#include <string>
#include <vector>

#include "soc/gpu/runtime.h"

using namespace soc::gpu;

static int fails = 0;
#define EXPECT(cond, msg)                      \
  do {                                         \
    if (!(cond)) {                             \
      std::fprintf(stderr, "FAIL: %s\n", msg); \
      ++fails;                                 \
    }                                          \
  } while (0)

namespace {

DeviceTensor MakeFloatTensor(const MetalContext& context, const std::vector<std::size_t>& shape,
                             const std::vector<float>& values, const std::string& label, std::string* error_message) {
  auto buffer = MetalBuffer::CreateShared(context, values.size() * sizeof(float), label, error_message);
  if (buffer == nullptr) return {};
  if (!values.empty() && !buffer->Write(values.data(), values.size() * sizeof(float), 0, error_message)) return {};
  return DeviceTensor(buffer, 0, TensorDesc::CreateContiguous(DataType::kFloat32, shape));
}

DeviceTensor MakeIntTensor(const MetalContext& context, const std::vector<int>& values, std::string* error_message) {
  auto buffer = MetalBuffer::CreateShared(context, values.size() * sizeof(int), "ids", error_message);
  if (buffer == nullptr) return {};
  if (!buffer->Write(values.data(), values.size() * sizeof(int), 0, error_message)) return {};
  return DeviceTensor(buffer, 0, TensorDesc::CreateContiguous(DataType::kInt32, {values.size()}));
}

std::vector<float> ReadFloats(const DeviceTensor& t, std::size_t n) {
  std::vector<float> v(n);
  std::string err;
  t.GetBuffer()->Read(v.data(), n * sizeof(float), t.GetByteOffset(), &err);
  return v;
}

constexpr std::size_t kD = 128;

QwenCausalLMWeights IdentityWeights(const MetalContext& context, std::string* error_message) {
  std::vector<float> embed(4 * kD, 0.0f);
  for (std::size_t i = 0; i < 4; ++i) embed[i * kD + i] = 1.0f;
  const std::vector<float> ones(kD, 1.0f);
  const std::vector<float> zeros(kD * kD, 0.0f);

  QwenAttentionWeights attention_weights;
  attention_weights.q_proj_weight = MakeFloatTensor(context, {kD, kD}, zeros, "q_proj", error_message);
  attention_weights.k_proj_weight = MakeFloatTensor(context, {kD, kD}, zeros, "k_proj", error_message);
  attention_weights.v_proj_weight = MakeFloatTensor(context, {kD, kD}, zeros, "v_proj", error_message);
  attention_weights.o_proj_weight = MakeFloatTensor(context, {kD, kD}, zeros, "o_proj", error_message);
  attention_weights.q_norm_weight = MakeFloatTensor(context, {kD}, ones, "q_norm", error_message);
  attention_weights.k_norm_weight = MakeFloatTensor(context, {kD}, ones, "k_norm", error_message);

  QwenMlpWeights mlp_weights;
  mlp_weights.gate_proj_weight = MakeFloatTensor(context, {kD, kD}, zeros, "gate_proj", error_message);
  mlp_weights.up_proj_weight = MakeFloatTensor(context, {kD, kD}, zeros, "up_proj", error_message);
  mlp_weights.down_proj_weight = MakeFloatTensor(context, {kD, kD}, zeros, "down_proj", error_message);

  QwenBlockWeights block_weights;
  block_weights.input_layernorm_weight = MakeFloatTensor(context, {kD}, ones, "input_ln", error_message);
  block_weights.attention = attention_weights;
  block_weights.post_attention_layernorm_weight = MakeFloatTensor(context, {kD}, ones, "post_attn_ln", error_message);
  block_weights.mlp = mlp_weights;

  QwenCausalLMWeights model_weights;
  model_weights.embed_tokens_weight = MakeFloatTensor(context, {4, kD}, embed, "embed", error_message);
  model_weights.blocks = {block_weights};
  model_weights.final_norm_weight = MakeFloatTensor(context, {kD}, ones, "final_norm", error_message);
  model_weights.lm_head_weight = model_weights.embed_tokens_weight;
  model_weights.tie_word_embeddings = true;
  return model_weights;
}

QwenCausalLMParams IdentityParams() {
  QwenCausalLMParams params;
  params.vocab_size = 4;
  params.hidden_size = kD;
  params.num_hidden_layers = 1;
  params.num_attention_heads = 1;
  params.num_key_value_heads = 1;
  params.head_dim = kD;
  params.intermediate_size = kD;
  params.max_position_embeddings = 8;
  params.rms_norm_eps = 1.0e-6f;
  return params;
}

}  // namespace

int main() {
  std::string error_message;
  auto context = MetalContext::CreateDefault("build/shaders/gpu.metallib", "shaders/gpu_kernels.metal", &error_message);
  if (context == nullptr) {
    std::fprintf(stderr, "failed to create the context: %s\n", error_message.c_str());
    return 2;
  }
  auto temporary_arena = BufferArena::CreateShared(*context, 1 << 20, "temp", &error_message);
  EXPECT(temporary_arena != nullptr, "temporary arena");

  // ---- test_generation_context.mm:96-140 ----
  QwenCausalLM model(IdentityWeights(*context, &error_message), IdentityParams());
  EXPECT(model.weights().embed_tokens_weight.IsValid() && model.weights().final_norm_weight.IsValid(),
         "failed to build identity model");
  EXPECT(model.IsValid(), "the weights constructor built no device model");
  EXPECT(model.num_layers() == 1 && model.weights().blocks.size() == 1, "layer count from the blocks");
  PipelineCache pipeline_cache(*context);
  {
    GenerationContext generation_context(model, Sampler({1.0f, 2}), CommandScheduler(), 8);
    const std::vector<int> prompt_token_ids = {1, 2};
    std::vector<int> generated_token_ids;
    EXPECT(generation_context.Generate(*context, &pipeline_cache, prompt_token_ids, 3, -1, temporary_arena.get(),
                                       &generated_token_ids, &error_message),
           error_message.c_str());
    EXPECT(generated_token_ids == std::vector<int>({2, 2, 2}), "unexpected generated token sequence");
    EXPECT(generation_context.prompt_token_ids() == prompt_token_ids, "prompt token ids were not preserved");
    EXPECT(generation_context.running_token_ids() == std::vector<int>({1, 2, 2, 2, 2}),
           "running token ids do not reflect decode progression");
    generation_context.Reset();
    EXPECT(generation_context.prompt_token_ids().empty() && generation_context.running_token_ids().empty(),
           "reset did not clear generation state");
  }

  // ---- the four forwards of the identity model: hidden row t = sqrt(128) e_{id_t} (final RMSNorm of e_t), logits
  //      row t = sqrt(128) at id_t and 0 elsewhere, whatever the position offset ----
  const std::vector<int> ids = {3, 0, 2, 1};
  const DeviceTensor tokens = MakeIntTensor(*context, ids, &error_message);
  const float r = std::sqrt(static_cast<float>(kD));
  auto hidden_ok = [&](const std::vector<float>& h) {
    for (std::size_t t = 0; t < ids.size(); ++t)
      for (std::size_t i = 0; i < kD; ++i)
        if (std::fabs(h[t * kD + i] - (static_cast<int>(i) == ids[t] ? r : 0.0f)) > 1e-3f) return false;
    return true;
  };
  auto logits_ok = [&](const std::vector<float>& l, std::size_t rows) {
    for (std::size_t t = 0; t < rows; ++t)
      for (std::size_t v = 0; v < 4; ++v) {
        const int id = ids[ids.size() - rows + t];
        if (std::fabs(l[t * 4 + v] - (static_cast<int>(v) == id ? r : 0.0f)) > 1e-3f) return false;
      }
    return true;
  };
  const DeviceTensor hidden = MakeFloatTensor(*context, {ids.size(), kD}, std::vector<float>(ids.size() * kD), "h",
                                              &error_message);
  const DeviceTensor logits = MakeFloatTensor(*context, {ids.size(), 4}, std::vector<float>(ids.size() * 4), "l",
                                              &error_message);
  context->ResetProfiling();
  EXPECT(model.ForwardHidden(*context, &pipeline_cache, tokens, hidden, temporary_arena.get(), 3, &error_message),
         error_message.c_str());
  EXPECT(hidden_ok(ReadFloats(hidden, ids.size() * kD)), "ForwardHidden rows");
  EXPECT(model.ForwardLogits(*context, &pipeline_cache, tokens, logits, temporary_arena.get(), 2, &error_message),
         error_message.c_str());
  EXPECT(logits_ok(ReadFloats(logits, ids.size() * 4), ids.size()), "ForwardLogits rows");
  auto cache = KVCache::CreateShared(*context, 1, 1, kD, 8, "kv", &error_message);
  EXPECT(cache != nullptr, error_message.c_str());
  EXPECT(model.ForwardHiddenCached(*context, &pipeline_cache, tokens, cache.get(), hidden, temporary_arena.get(), 0,
                                   &error_message),
         error_message.c_str());
  EXPECT(hidden_ok(ReadFloats(hidden, ids.size() * kD)), "ForwardHiddenCached rows");
  EXPECT(cache->GetSequenceLength() == ids.size(), "cached forward appends every row");
  const DeviceTensor one = MakeIntTensor(*context, {ids[0]}, &error_message);
  const DeviceTensor row = MakeFloatTensor(*context, {1, 4}, std::vector<float>(4), "row", &error_message);
  EXPECT(model.ForwardLogitsCached(*context, &pipeline_cache, one, cache.get(), row, temporary_arena.get(), ids.size(),
                                   &error_message),
         error_message.c_str());
  const std::vector<float> rl = ReadFloats(row, 4);
  EXPECT(std::fabs(rl[static_cast<std::size_t>(ids[0])] - r) < 1e-3f, "ForwardLogitsCached decode row");
  EXPECT(context->GetProfilingSnapshot().command_buffer_count == 4 && context->GetProfilingSnapshot().gpu_ms > 0.0,
         "every forward is profiled");
  // error paths (qwen_causal_lm.cpp:44-66, 139-151)
  error_message.clear();
  EXPECT(!model.ForwardHiddenCached(*context, &pipeline_cache, tokens, nullptr, hidden, temporary_arena.get(), 0,
                                    &error_message) &&
             error_message == "QwenCausalLM cached forward requires a KVCache",
         "cached forward without a cache");
  const DeviceTensor bad = MakeFloatTensor(*context, {ids.size(), kD + 1}, std::vector<float>(ids.size() * (kD + 1)),
                                           "bad", &error_message);
  EXPECT(!model.ForwardHidden(*context, &pipeline_cache, tokens, bad, temporary_arena.get(), 0, &error_message) &&
             error_message == "QwenCausalLM hidden output shape must be [token_count, hidden_size]",
         "hidden output shape");
  EXPECT(!model.ForwardLogitsCached(*context, &pipeline_cache, one, cache.get(), row, temporary_arena.get(), 0,
                                    &error_message),
         "position_offset must equal the cache length");

  // ---- a weight of the wrong shape leaves the model invalid, with the reason on every forward ----
  {
    QwenCausalLMWeights w = IdentityWeights(*context, &error_message);
    w.blocks[0].mlp.down_proj_weight =
        MakeFloatTensor(*context, {kD, kD / 2}, std::vector<float>(kD * kD / 2), "down", &error_message);
    QwenCausalLM broken(std::move(w), IdentityParams());
    EXPECT(!broken.IsValid(), "a misshapen weight must leave the model invalid");
    error_message.clear();
    EXPECT(!broken.ForwardHidden(*context, &pipeline_cache, tokens, hidden, temporary_arena.get(), 0, &error_message),
           "forward of an invalid model");
    EXPECT(error_message.find("model.layers.0.mlp.down_proj.weight has shape [128, 64]") != std::string::npos,
           error_message.c_str());
  }

  // ---- the op classes against host arithmetic ----
  {
    const std::size_t M = 3, K = 40, N = 5;
    std::vector<float> a(M * K), b(K * N), bias(N), res(M * N);
    for (std::size_t i = 0; i < a.size(); ++i) a[i] = static_cast<float>((i * 7) % 13) * 0.25f - 1.5f;
    for (std::size_t i = 0; i < b.size(); ++i) b[i] = static_cast<float>((i * 5) % 11) * 0.125f - 0.5f;
    for (std::size_t i = 0; i < N; ++i) bias[i] = 0.1f * static_cast<float>(i);
    for (std::size_t i = 0; i < res.size(); ++i) res[i] = -0.2f * static_cast<float>(i % 3);
    const DeviceTensor ta = MakeFloatTensor(*context, {M, K}, a, "a", &error_message);
    const DeviceTensor tb = MakeFloatTensor(*context, {K, N}, b, "b", &error_message);
    const DeviceTensor tbias = MakeFloatTensor(*context, {N}, bias, "bias", &error_message);
    const DeviceTensor tres = MakeFloatTensor(*context, {M, N}, res, "res", &error_message);
    const DeviceTensor out = MakeFloatTensor(*context, {M, N}, std::vector<float>(M * N), "out", &error_message);
    LinearParams lp;
    lp.matmul.use_bias = true;
    lp.activation = LinearActivation::kSiLU;
    lp.add_residual = true;
    EXPECT(LinearOp::Run(*context, &pipeline_cache, ta, tb, &tbias, &tres, out, lp, temporary_arena.get(),
                         &error_message),
           error_message.c_str());
    const std::vector<float> got = ReadFloats(out, M * N);
    bool ok = true;
    for (std::size_t i = 0; i < M; ++i)
      for (std::size_t j = 0; j < N; ++j) {
        double z = bias[j] + res[i * N + j];
        for (std::size_t k = 0; k < K; ++k) z += static_cast<double>(a[i * K + k]) * b[k * N + j];
        const double want = z / (1.0 + std::exp(-z));
        if (std::fabs(got[i * N + j] - want) > 1e-4) ok = false;
      }
    EXPECT(ok, "LinearOp with bias, residual and SiLU");
    MatMulParams mp;
    mp.use_bias = true;
    EXPECT(!MatMulOp::Run(*context, &pipeline_cache, ta, tb, nullptr, nullptr, out, mp, temporary_arena.get(),
                          &error_message) &&
               error_message == "MatMul params.use_bias must match whether a bias tensor is provided",
           "MatMul use_bias check");
    EXPECT(!MatMulOp::Run(*context, &pipeline_cache, ta, ta, nullptr, nullptr, out, MatMulParams{},
                          temporary_arena.get(), &error_message) &&
               error_message == "MatMul inner dimensions must match",
           "MatMul inner dimension check");
    EXPECT(!MatMulOp::Run(*context, nullptr, ta, tb, nullptr, nullptr, out, MatMulParams{}, temporary_arena.get(),
                          &error_message) &&
               error_message == "Pipeline cache must not be null",
           "MatMul pipeline cache check");

    const std::vector<float> x = {3.0f, -4.0f, 1.0f, 2.0f};
    const DeviceTensor tx = MakeFloatTensor(*context, {1, 4}, x, "x", &error_message);
    const DeviceTensor tw = MakeFloatTensor(*context, {4}, {1.0f, 2.0f, 0.5f, 1.0f}, "w", &error_message);
    const DeviceTensor ty = MakeFloatTensor(*context, {1, 4}, std::vector<float>(4), "y", &error_message);
    RmsNormParams rp;
    rp.epsilon = 1e-6f;
    EXPECT(RmsNormOp::Run(*context, &pipeline_cache, tx, tw, ty, rp, temporary_arena.get(), &error_message),
           error_message.c_str());
    const float s = 1.0f / std::sqrt((9.0f + 16.0f + 1.0f + 4.0f) / 4.0f + 1e-6f);
    const std::vector<float> yn = ReadFloats(ty, 4);
    EXPECT(std::fabs(yn[0] - 3.0f * s) < 1e-5f && std::fabs(yn[1] + 8.0f * s) < 1e-5f, "RmsNormOp");
    SoftmaxParams sp;
    EXPECT(SoftmaxOp::Run(*context, &pipeline_cache, tx, ty, sp, temporary_arena.get(), &error_message),
           error_message.c_str());
    const std::vector<float> ys = ReadFloats(ty, 4);
    double zsum = 0;
    for (float v : x) zsum += std::exp(v - 3.0);
    EXPECT(std::fabs(ys[0] - std::exp(0.0) / zsum) < 1e-6, "SoftmaxOp");
    ElementwiseMulParams ep;
    EXPECT(ElementwiseMulOp::Run(*context, &pipeline_cache, tx, tx, ty, ep, temporary_arena.get(), &error_message),
           error_message.c_str());
    EXPECT(ReadFloats(ty, 4)[1] == 16.0f, "ElementwiseMulOp");
    // rope at position 0 is the identity (test_nn_modules.cpp:213-216)
    const DeviceTensor rx = MakeFloatTensor(*context, {1, kD}, std::vector<float>(kD, 0.5f), "rx", &error_message);
    const DeviceTensor ry = MakeFloatTensor(*context, {1, kD}, std::vector<float>(kD), "ry", &error_message);
    RopeParams ropep;
    ropep.head_count = 1;
    ropep.head_dim = kD;
    EXPECT(RopeOp::Run(*context, &pipeline_cache, rx, ry, ropep, temporary_arena.get(), &error_message),
           error_message.c_str());
    EXPECT(ReadFloats(ry, kD) == std::vector<float>(kD, 0.5f), "RopeOp at position 0");
    ropep.head_count = 2;
    EXPECT(!RopeOp::Run(*context, &pipeline_cache, rx, ry, ropep, temporary_arena.get(), &error_message) &&
               error_message == "RoPE params do not match tensor shapes",
           "RopeOp shape check");
    // embedding from the model's own fp16 table view (QwenCausalLM::weights() of a loaded model would also do)
    const DeviceTensor eo = MakeFloatTensor(*context, {2, kD}, std::vector<float>(2 * kD), "eo", &error_message);
    const DeviceTensor eids = MakeIntTensor(*context, {2, 7}, &error_message);
    EXPECT(EmbeddingOp::Run(*context, &pipeline_cache, eids, model.weights().embed_tokens_weight, eo, EmbeddingParams{},
                            temporary_arena.get(), &error_message),
           error_message.c_str());
    const std::vector<float> er = ReadFloats(eo, 2 * kD);
    EXPECT(er[2] == 1.0f && er[kD] == 0.0f && er[kD + 7] == 0.0f, "EmbeddingOp (an out-of-range id gives zeros)");
  }

  // ---- weights() of a model from the loader: fp16 views of the library's storage ----
  {
    QwenCausalLM loaded;
    EXPECT(QwenModelLoader::SynthesizeModel(*context, IdentityParams(), 3, 0.02f, &loaded, &error_message),
           error_message.c_str());
    const QwenCausalLMWeights& w = loaded.weights();
    EXPECT(w.blocks.size() == 1 && w.embed_tokens_weight.IsValid() &&
               w.embed_tokens_weight.GetDesc().GetDataType() == DataType::kFloat16 &&
               w.blocks[0].mlp.down_proj_weight.GetDesc().GetShape() == std::vector<std::size_t>({kD, kD}) &&
               w.lm_head_weight.IsValid(),
           "weight views of a loaded model");
    QwenCausalLM copy(w, loaded.params());  // a model over those views: same logits
    const DeviceTensor l1 = MakeFloatTensor(*context, {1, 4}, std::vector<float>(4), "l1", &error_message);
    const DeviceTensor l2 = MakeFloatTensor(*context, {1, 4}, std::vector<float>(4), "l2", &error_message);
    EXPECT(loaded.ForwardLogits(*context, &pipeline_cache, tokens, l1, temporary_arena.get(), 0, &error_message),
           error_message.c_str());
    EXPECT(copy.ForwardLogits(*context, &pipeline_cache, tokens, l2, temporary_arena.get(), 0, &error_message),
           error_message.c_str());
    EXPECT(ReadFloats(l1, 4) == ReadFloats(l2, 4), "a model rebuilt from weights() computes the same logits");
  }

  if (fails == 0) std::printf("test_qwen_causal_lm passed\n");
  return fails == 0 ? 0 : 1;
}
