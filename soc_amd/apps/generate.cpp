// generate.cpp - greedy generation through the kept C++ host API (GenerationContext::Generate and DecodeNextToken,
// Mac/gpu/src/runtime/generation_context.cpp:17-172) on a Qwen3 model with seeded random weights, timed. It is the
// path a caller of the reference's GPU runtime uses: token ids uploaded into a device tensor, CommandScheduler ->
// QwenCausalLM::ForwardLogitsCached -> soc_forward, then Sampler::SampleFromLogits on the device logits row.
//
// Usage: soc_generate [--model qwen3-0.6b|qwen3-4b] [--seed S] [--sigma X] [--prompt-len N] [--prompt-seed P]
//                     [--new N] [--repeat R] [--decode-steps D] [--top-k K]
// The prompt is soc_synth_tokens(prompt_seed, "prompt", vocab, prompt_len), the weights soc_model_synthesize(seed,
// sigma) (norm gains 1.0). Prints one JSON line: the generated ids, the wall time of each Generate call (one untimed
// warm-up first), the wall time of one Prefill, and the median wall time of D DecodeNextToken calls continuing the
// sequence a Generate call leaves.
#include <algorithm>
#include <chrono>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <string>
#include <vector>

#include "soc/gpu/runtime.h"

using namespace soc::gpu;

namespace {

double now_ms() {
  return std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now().time_since_epoch()).count();
}

QwenCausalLMParams ModelParams(const std::string& name) {
  QwenCausalLMParams p;
  p.vocab_size = 151936;
  p.head_dim = 128;
  p.max_position_embeddings = 40960;
  p.rope_theta = 1000000.0f;
  p.rms_norm_eps = 1e-6f;
  p.tie_word_embeddings = true;
  if (name == "qwen3-4b") {
    p.hidden_size = 2560;
    p.num_hidden_layers = 36;
    p.num_attention_heads = 32;
    p.num_key_value_heads = 8;
    p.intermediate_size = 9728;
  } else {
    p.hidden_size = 1024;
    p.num_hidden_layers = 28;
    p.num_attention_heads = 16;
    p.num_key_value_heads = 8;
    p.intermediate_size = 3072;
  }
  return p;
}

}  // namespace

int main(int argc, char** argv) {
  std::string model_name = "qwen3-0.6b";
  uint64_t seed = 1, prompt_seed = 1;
  float sigma = 0.02f;
  int prompt_len = 32, max_new = 16, repeat = 5, decode_steps = 64;
  std::size_t top_k = 1;
  for (int i = 1; i + 1 < argc; i += 2) {
    const std::string k = argv[i];
    const char* v = argv[i + 1];
    if (k == "--model") model_name = v;
    else if (k == "--seed") seed = std::strtoull(v, nullptr, 10);
    else if (k == "--sigma") sigma = std::strtof(v, nullptr);
    else if (k == "--prompt-len") prompt_len = std::atoi(v);
    else if (k == "--prompt-seed") prompt_seed = std::strtoull(v, nullptr, 10);
    else if (k == "--new") max_new = std::atoi(v);
    else if (k == "--repeat") repeat = std::atoi(v);
    else if (k == "--decode-steps") decode_steps = std::atoi(v);
    else if (k == "--top-k") top_k = static_cast<std::size_t>(std::atoi(v));
    else {
      std::fprintf(stderr, "unknown option %s\n", k.c_str());
      return 2;
    }
  }
  std::string err;
  auto context = HipContext::CreateDefault(0, &err);
  if (context == nullptr) {
    std::fprintf(stderr, "no HIP context: %s\n", err.c_str());
    return 1;
  }
  const QwenCausalLMParams params = ModelParams(model_name);
  QwenCausalLM model;
  if (!QwenModelLoader::SynthesizeModel(*context, params, seed, sigma, &model, &err)) {
    std::fprintf(stderr, "model: %s\n", err.c_str());
    return 1;
  }
  std::vector<int32_t> ids(static_cast<std::size_t>(prompt_len));
  if (soc_synth_tokens(prompt_seed, "prompt", static_cast<int32_t>(params.vocab_size), prompt_len, ids.data()) !=
      SOC_OK) {
    std::fprintf(stderr, "prompt: %s\n", soc_last_error());
    return 1;
  }
  const std::vector<int> prompt(ids.begin(), ids.end());
  PipelineCache cache(*context);
  auto arena = BufferArena::CreateShared(*context, 1 << 20, "temp", &err);
  const std::size_t max_seq = static_cast<std::size_t>(prompt_len + max_new + decode_steps + 8);
  GenerationContext gen(model, Sampler({1.0f, top_k}), CommandScheduler(), max_seq);

  std::vector<int> out;
  std::vector<double> gen_ms;
  for (int r = 0; r <= repeat; ++r) {  // run 0 warms every path up and is not reported
    const double t0 = now_ms();
    if (!gen.Generate(*context, &cache, prompt, static_cast<std::size_t>(max_new), -1, arena.get(), &out, &err)) {
      std::fprintf(stderr, "generate: %s\n", err.c_str());
      return 1;
    }
    if (r > 0) gen_ms.push_back(now_ms() - t0);
  }
  // prefill latency (Prefill alone), then decode latency through DecodeNextToken (each call: token upload,
  // ForwardLogitsCached, Sampler) continuing from the tail a Generate call leaves (generation_context.cpp:151-163)
  double prefill_ms = 0.0;
  std::vector<double> step_ms;
  {
    const double t0 = now_ms();
    if (!gen.Prefill(*context, &cache, prompt, arena.get(), &err)) {
      std::fprintf(stderr, "prefill: %s\n", err.c_str());
      return 1;
    }
    prefill_ms = now_ms() - t0;
    if (!gen.Generate(*context, &cache, prompt, static_cast<std::size_t>(max_new), -1, arena.get(), &out, &err)) {
      std::fprintf(stderr, "generate: %s\n", err.c_str());
      return 1;
    }
    for (int s = 0; s < decode_steps; ++s) {
      GenerationStepResult r;
      const int last = gen.running_token_ids().back();
      const double t1 = now_ms();
      if (!gen.DecodeNextToken(*context, &cache, last, arena.get(), &r, &err)) {
        std::fprintf(stderr, "decode: %s\n", err.c_str());
        return 1;
      }
      step_ms.push_back(now_ms() - t1);
    }
  }
  std::vector<double> sorted = step_ms;
  std::sort(sorted.begin(), sorted.end());
  const double median_step = sorted.empty() ? 0.0 : sorted[sorted.size() / 2];
  std::vector<double> gsorted = gen_ms;
  std::sort(gsorted.begin(), gsorted.end());
  const double median_gen = gsorted.empty() ? 0.0 : gsorted[gsorted.size() / 2];
  std::printf("{\"model\": \"%s\", \"prompt_len\": %d, \"new_tokens\": %d, \"tokens\": [", model_name.c_str(),
              prompt_len, max_new);
  for (std::size_t i = 0; i < out.size(); ++i) std::printf("%s%d", i ? ", " : "", out[i]);
  std::printf("], \"generate_ms\": [");
  for (std::size_t i = 0; i < gen_ms.size(); ++i) std::printf("%s%.3f", i ? ", " : "", gen_ms[i]);
  std::printf("], \"generate_ms_median\": %.3f, \"generate_tok_s\": %.1f, \"prefill_ms\": %.3f, "
              "\"decode_next_token_ms_median\": %.4f, \"decode_next_token_tok_s\": %.1f, \"decode_steps\": %d}\n",
              median_gen, median_gen > 0 ? max_new / (median_gen * 1e-3) : 0.0, prefill_ms, median_step,
              median_step > 0 ? 1000.0 / median_step : 0.0, decode_steps);
  return 0;
}
