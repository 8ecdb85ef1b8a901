// The reference harness's text-level flow (Mac/gpu/test/integration/test_real_bundle_regression.mm:192-200 options,
// :501-553 RunGpuGenerationContext, :706-724 bundle and prompts) on a bundle written by the test:
// RuntimePipeline::LoadBundle, GenerationOptionsFromManifest, PreparePrompt with the chat template, TokenizerRuntime
// encode, GenerationContext::Generate on the device, TokenizerRuntime decode.
//
// usage: test_text_generation OUT MANIFEST chat(0|1) thinking(0|1) PROMPT
// OUT (binary): n_prompt, prompt ids, n_generated, generated ids, n_text, text bytes (int32 counts and ids).
#include <cstdio>
#include <string>
#include <vector>

#include "soc/gpu/runtime.h"
#include "soc/tokenizer.h"

using namespace soc::gpu;

namespace {

int Die(const char* what, const std::string& err) {
  std::fprintf(stderr, "FAIL: %s: %s\n", what, err.c_str());
  return 1;
}

void WriteInts(FILE* f, const std::vector<int>& v) {
  const int32_t n = static_cast<int32_t>(v.size());
  std::fwrite(&n, 4, 1, f);
  for (const int x : v) {
    const int32_t y = x;
    std::fwrite(&y, 4, 1, f);
  }
}

}  // namespace

int main(int argc, char** argv) {
  if (argc != 6) {
    std::fprintf(stderr, "usage: %s OUT MANIFEST chat thinking PROMPT\n", argv[0]);
    return 2;
  }
  std::string err;
  auto context = MetalContext::CreateDefault("unused.metallib", "unused.metal", &err);
  if (!context) return Die("context", err);
  RuntimeBundle bundle;
  if (!RuntimePipeline::LoadBundle(*context, argv[2], &bundle, &err)) return Die("LoadBundle", err);
  const RuntimeGenerationOptions options = RuntimePipeline::GenerationOptionsFromManifest(bundle.manifest);
  RuntimePromptOptions prompt_options;
  prompt_options.apply_chat_template = std::string(argv[3]) == "1";
  prompt_options.enable_thinking = std::string(argv[4]) == "1";
  const std::string prompt = RuntimePipeline::PreparePrompt(bundle.tokenizer_runtime, argv[5], prompt_options);
  std::vector<int> prompt_ids;
  std::vector<int> generated;
  std::string text;
  try {
    const soc::TokenizerRuntime tokenizer(bundle.tokenizer_runtime);
    prompt_ids = tokenizer.Encode(prompt);
    PipelineCache pipeline_cache(*context);
    auto arena = BufferArena::CreateShared(*context, 1 << 20, "temp", &err);
    if (!arena) return Die("arena", err);
    GenerationContext generation(bundle.model, Sampler(options.sampler), CommandScheduler(),
                                 options.max_sequence_length);
    if (!generation.Generate(*context, &pipeline_cache, prompt_ids, options.max_new_tokens, options.eos_token_id,
                             arena.get(), &generated, &err))
      return Die("Generate", err);
    text = tokenizer.Decode(generated);
  } catch (const std::exception& e) {
    return Die("tokenizer", e.what());
  }
  FILE* f = std::fopen(argv[1], "wb");
  if (f == nullptr) return Die("open", argv[1]);
  WriteInts(f, prompt_ids);
  WriteInts(f, generated);
  const int32_t n = static_cast<int32_t>(text.size());
  std::fwrite(&n, 4, 1, f);
  std::fwrite(text.data(), 1, text.size(), f);
  std::fclose(f);
  std::printf("test_text_generation done: %zu prompt ids, %zu generated\n", prompt_ids.size(), generated.size());
  return 0;
}
