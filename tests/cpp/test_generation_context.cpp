// C++ host-interface test: the reference's identity-model generation test
// (Mac/gpu/test/runtime/test_generation_context.mm:35-149) driven through soc::gpu::GenerationContext on the GPU.
// head_dim is 128 here (the only head size the kernels take), so the identity model is 128 wide: one-hot embedding
// rows e_0..e_3, zero projections, unit gains. The residual stream stays e_t, the final RMSNorm scales it to
// sqrt(128) e_t, and the tied head gives the largest logit to the input token: Generate([1,2], 3) = [2,2,2].
#include <algorithm>
#include <cmath>
#include <cstdio>
#include <map>
#include <string>
#include <vector>

#include "soc/gpu/runtime.h"

using namespace soc::gpu;

static int fails = 0;
#define EXPECT(cond, msg)                           \
  do {                                              \
    if (!(cond)) {                                  \
      std::fprintf(stderr, "FAIL: %s\n", msg);      \
      ++fails;                                      \
    }                                               \
  } while (0)

int main() {
  std::string err;
  auto ctx = HipContext::CreateDefault(0, &err);
  if (!ctx) {
    std::fprintf(stderr, "no HIP context: %s\n", err.c_str());
    return 2;
  }
  QwenCausalLMParams p;
  p.vocab_size = 4;
  p.hidden_size = 128;
  p.num_hidden_layers = 1;
  p.num_attention_heads = 1;
  p.num_key_value_heads = 1;
  p.head_dim = 128;
  p.intermediate_size = 128;
  p.max_position_embeddings = 8;
  const uint16_t one = 0x3c00, zero = 0;
  std::vector<uint16_t> embed(4 * 128, zero), ones(128, one), zeros(128 * 128, zero);
  for (int i = 0; i < 4; ++i) embed[i * 128 + i] = one;
  std::map<std::string, QwenModelLoader::HostTensor> t;
  t["model.embed_tokens.weight"] = {embed.data(), 4 * 128};
  t["model.norm.weight"] = {ones.data(), 128};
  const std::string l = "model.layers.0.";
  for (const char* n : {"input_layernorm.weight", "post_attention_layernorm.weight", "self_attn.q_norm.weight",
                        "self_attn.k_norm.weight"})
    t[l + n] = {ones.data(), 128};
  for (const char* n : {"self_attn.q_proj.weight", "self_attn.k_proj.weight", "self_attn.v_proj.weight",
                        "self_attn.o_proj.weight", "mlp.gate_proj.weight", "mlp.up_proj.weight",
                        "mlp.down_proj.weight"})
    t[l + n] = {zeros.data(), 128 * 128};

  QwenCausalLM model;
  EXPECT(QwenModelLoader::LoadModel(*ctx, p, t, &model, &err), err.c_str());
  PipelineCache cache(*ctx);
  auto arena = BufferArena::CreateShared(*ctx, 1 << 20, "temp", &err);
  EXPECT(arena != nullptr, "arena");

  for (std::size_t top_k : {std::size_t{2}, std::size_t{1}}) {
    GenerationContext gen(model, Sampler({1.0f, top_k}), CommandScheduler(), 8);
    const std::vector<int> prompt = {1, 2};
    std::vector<int> out;
    EXPECT(gen.Generate(*ctx, &cache, prompt, 3, -1, arena.get(), &out, &err), err.c_str());
    EXPECT(out == std::vector<int>({2, 2, 2}), "unexpected generated token sequence");
    EXPECT(gen.prompt_token_ids() == prompt, "prompt token ids were not preserved");
    EXPECT(gen.running_token_ids() == std::vector<int>({1, 2, 2, 2, 2}), "running ids do not reflect decoding");

    // the top-k lists of a step (sampler.cpp:56-66): input token 2 gives logits sqrt(128) at id 2 and 0 elsewhere;
    // the expected order is the reference's std::partial_sort over that row
    {
      GenerationStepResult r;
      EXPECT(gen.DecodeNextToken(*ctx, &cache, 2, arena.get(), &r, &err), err.c_str());
      std::vector<float> row(4, 0.0f);
      row[2] = std::sqrt(128.0f);
      std::vector<int> cand = {0, 1, 2, 3};
      std::partial_sort(cand.begin(), cand.begin() + top_k, cand.end(),
                        [&row](int a, int b) { return row[a] / 1.0f > row[b] / 1.0f; });
      EXPECT(r.token_id == 2, "top-k token");
      EXPECT(r.top_token_ids.size() == top_k && r.top_logits.size() == top_k, "top-k list sizes");
      for (std::size_t j = 0; j < top_k && j < r.top_token_ids.size(); ++j) {
        EXPECT(r.top_token_ids[j] == cand[j], "top-k ids follow the reference's partial sort");
        EXPECT(std::fabs(r.top_logits[j] - row[cand[j]]) < 1e-3f, "top-k logits");
      }
      gen.Reset();
      EXPECT(gen.Generate(*ctx, &cache, prompt, 3, -1, arena.get(), &out, &err), err.c_str());
    }

    // error paths (generation_context.cpp:67-90): wrong tail token, null result
    GenerationStepResult r;
    err.clear();
    EXPECT(!gen.DecodeNextToken(*ctx, &cache, 3, arena.get(), &r, &err), "tail mismatch must fail");
    EXPECT(err.find("sequence tail") != std::string::npos, "tail mismatch message");
    EXPECT(!gen.DecodeNextToken(*ctx, &cache, 2, arena.get(), nullptr, &err), "null result must fail");
    // capacity: running has 5 of 8; three more decodes fit, the fourth exceeds max_sequence_length
    int last = 2;
    for (int i = 0; i < 3; ++i) {
      EXPECT(gen.DecodeNextToken(*ctx, &cache, last, arena.get(), &r, &err), err.c_str());
      last = r.token_id;
    }
    EXPECT(!gen.DecodeNextToken(*ctx, &cache, last, arena.get(), &r, &err), "capacity must be enforced");
    EXPECT(gen.running_token_ids().size() == 8, "state unchanged by a failed decode");

    gen.Reset();
    EXPECT(gen.prompt_token_ids().empty() && gen.running_token_ids().empty(), "reset did not clear state");
    GenerationStepResult r2;
    EXPECT(!gen.DecodeNextToken(*ctx, &cache, 2, arena.get(), &r2, &err), "decode before prefill must fail");
    EXPECT(!gen.Prefill(*ctx, &cache, {}, arena.get(), &err), "empty prefill must fail");
  }
  if (fails == 0) std::printf("test_generation_context passed\n");
  return fails == 0 ? 0 : 1;
}
