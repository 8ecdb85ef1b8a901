// The reference parity harness's call sequence (Mac/gpu/test/integration/test_real_bundle_regression.mm:127-168
// helpers, :278-318 first token, :377-466 manual generation), written against soc/gpu/runtime.h with only the
// context type renamed: a seeded model, KVCache::CreateShared from the model's dimensions, token ids uploaded into a
// device buffer, RunPrefill into an all-rows logits tensor, Sampler::SampleFromLogits on the last row, then
// RunDecode / SampleFromLogits per step. Writes the tokens, top-k lists and logit rows to a file that
// tests/test_gpu_host_api.py compares with the reference-emitted fixture of the same model.
//
// usage: test_harness_sequence OUT vocab hidden layers nq nkv inter tie seed top_k new_tokens id0 id1 ...
//        test_harness_sequence OUT --bundle MANIFEST top_k new_tokens id0 id1 ...   (model from a bundle on disk,
//        QwenModelLoader::LoadModelFromFile)
#include <cstdio>
#include <cstdlib>
#include <string>
#include <vector>

#include "soc/gpu/runtime.h"

using namespace soc::gpu;

namespace {

DeviceTensor UploadTokenIds(const MetalContext& context, const std::vector<int>& token_ids, const std::string& label,
                            std::string* error_message) {
  auto buffer = MetalBuffer::CreateShared(context, token_ids.size() * sizeof(std::int32_t), label, error_message);
  if (buffer == nullptr) return {};
  if (!token_ids.empty() && !buffer->Write(token_ids.data(), token_ids.size() * 4, 0, error_message)) return {};
  return DeviceTensor(buffer, 0, TensorDesc::CreateContiguous(DataType::kInt32, {token_ids.size()}));
}

DeviceTensor MakeLogitsTensor(const std::shared_ptr<MetalBuffer>& buffer, std::size_t rows, std::size_t vocab) {
  return DeviceTensor(buffer, 0, TensorDesc::CreateContiguous(DataType::kFloat32, {rows, vocab}));
}

int Die(const char* what, const std::string& err) {
  std::fprintf(stderr, "FAIL: %s: %s\n", what, err.c_str());
  return 1;
}

}  // namespace

int main(int argc, char** argv) {
  const bool from_bundle = argc > 2 && std::string(argv[2]) == "--bundle";
  if ((from_bundle && argc < 7) || (!from_bundle && argc < 13)) {
    std::fprintf(stderr, "usage: %s OUT (vocab hidden layers nq nkv inter tie seed | --bundle MANIFEST) top_k new id...\n",
                 argv[0]);
    return 2;
  }
  QwenCausalLMParams p;
  uint64_t seed = 0;
  std::string manifest_path;
  int a;  // first of: top_k new_tokens ids...
  if (from_bundle) {
    manifest_path = argv[3];
    a = 4;
  } else {
    p.vocab_size = std::strtoul(argv[2], nullptr, 10);
    p.hidden_size = std::strtoul(argv[3], nullptr, 10);
    p.num_hidden_layers = std::strtoul(argv[4], nullptr, 10);
    p.num_attention_heads = std::strtoul(argv[5], nullptr, 10);
    p.num_key_value_heads = std::strtoul(argv[6], nullptr, 10);
    p.head_dim = 128;
    p.intermediate_size = std::strtoul(argv[7], nullptr, 10);
    p.max_position_embeddings = 4096;
    p.tie_word_embeddings = std::atoi(argv[8]) != 0;
    seed = std::strtoull(argv[9], nullptr, 10);
    a = 10;
  }
  SamplerConfig sc;
  sc.top_k = std::strtoul(argv[a], nullptr, 10);
  const std::size_t max_new_tokens = std::strtoul(argv[a + 1], nullptr, 10);
  std::vector<int> prompt_token_ids;
  for (int i = a + 2; i < argc; ++i) prompt_token_ids.push_back(std::atoi(argv[i]));

  std::string err;
  auto context_holder = MetalContext::CreateDefault("unused.metallib", "unused.metal", &err);
  if (!context_holder) return Die("context", err);
  const MetalContext& context = *context_holder;
  PipelineCache pipeline_cache(context);
  auto temporary_arena = BufferArena::CreateShared(context, 1 << 20, "temp", &err);
  if (!temporary_arena) return Die("arena", err);
  QwenCausalLM model;
  if (from_bundle ? !QwenModelLoader::LoadModelFromFile(context, manifest_path, &model, &err)
                  : !QwenModelLoader::SynthesizeModel(context, p, seed, 0.02f, &model, &err))
    return Die("model", err);
  const CommandScheduler scheduler;
  const Sampler sampler(sc);

  // :377-386 KV cache from the model's dimensions
  auto kv_cache = KVCache::CreateShared(context, model.num_layers(), model.num_key_value_heads(), model.head_dim(),
                                        prompt_token_ids.size() + max_new_tokens + 8, "manual_generation_kv", &err);
  if (kv_cache == nullptr) return Die("kv cache", err);
  // :391-405 prompt upload, all-rows logits tensor
  const DeviceTensor prompt_tensor = UploadTokenIds(context, prompt_token_ids, "manual_prompt", &err);
  if (!prompt_tensor.IsValid()) return Die("upload", err);
  auto prefill_logits_buffer =
      MetalBuffer::CreateShared(context, prompt_token_ids.size() * model.vocab_size() * 4, "prefill_logits", &err);
  if (prefill_logits_buffer == nullptr) return Die("logits buffer", err);
  const DeviceTensor prefill_logits = MakeLogitsTensor(prefill_logits_buffer, prompt_token_ids.size(),
                                                       model.vocab_size());
  temporary_arena->Reset();
  temporary_arena->ClearTelemetry();
  context.ResetProfiling();
  // :409-418
  if (!scheduler.RunPrefill(context, &pipeline_cache, model, prompt_tensor, kv_cache.get(), prefill_logits,
                            temporary_arena.get(), 0, &err))
    return Die("RunPrefill", err);
  if (context.GetProfilingSnapshot().command_buffer_count != 1) return Die("profiling", "no forward recorded");
  // :420-428 first token from the last prompt row
  int first_token_id = -1;
  std::vector<float> first_top_logits;
  std::vector<int> first_top_ids;
  if (!sampler.SampleFromLogits(prefill_logits, prompt_token_ids.size() - 1, &first_token_id, &first_top_logits,
                                &first_top_ids, &err))
    return Die("sample", err);
  std::vector<std::vector<float>> rows(prompt_token_ids.size(), std::vector<float>(model.vocab_size()));
  for (std::size_t r = 0; r < rows.size(); ++r)
    if (!prefill_logits_buffer->Read(rows[r].data(), model.vocab_size() * 4, r * model.vocab_size() * 4, &err))
      return Die("read", err);
  std::vector<int> generated = {first_token_id};
  std::vector<std::vector<int>> top_ids = {first_top_ids};
  std::vector<std::vector<float>> top_vals = {first_top_logits};
  std::vector<int> running_token_ids = prompt_token_ids;
  running_token_ids.push_back(first_token_id);
  // :436-466 decode loop
  for (std::size_t step = 1; step < max_new_tokens; ++step) {
    const int last_token_id = running_token_ids.back();
    const DeviceTensor decode_input = UploadTokenIds(context, {last_token_id}, "manual_decode_token", &err);
    if (!decode_input.IsValid()) return Die("upload", err);
    auto decode_logits_buffer = MetalBuffer::CreateShared(context, model.vocab_size() * 4, "decode_logits", &err);
    if (decode_logits_buffer == nullptr) return Die("logits buffer", err);
    const DeviceTensor decode_logits = MakeLogitsTensor(decode_logits_buffer, 1, model.vocab_size());
    temporary_arena->Reset();
    if (!scheduler.RunDecode(context, &pipeline_cache, model, decode_input, kv_cache.get(), decode_logits,
                             temporary_arena.get(), running_token_ids.size() - 1, &err))
      return Die("RunDecode", err);
    int next_token_id = -1;
    std::vector<float> tl;
    std::vector<int> ti;
    if (!sampler.SampleFromLogits(decode_logits, 0, &next_token_id, &tl, &ti, &err)) return Die("sample", err);
    rows.emplace_back(model.vocab_size());
    if (!decode_logits_buffer->Read(rows.back().data(), model.vocab_size() * 4, 0, &err)) return Die("read", err);
    generated.push_back(next_token_id);
    top_ids.push_back(ti);
    top_vals.push_back(tl);
    running_token_ids.push_back(next_token_id);
  }
  // the layer views after generation: every layer holds prompt + new - 1 positions
  for (std::size_t l = 0; l < model.num_layers(); ++l) {
    const KVCacheLayerView view = kv_cache->ViewForLayer(l);
    if (!view.keys.IsValid() || view.sequence_length != prompt_token_ids.size() + max_new_tokens - 1)
      return Die("ViewForLayer", "unexpected view");
  }
  // output: n_generated, k, then per step: token, k ids, k values; then n_rows, vocab, rows
  FILE* f = std::fopen(argv[1], "wb");
  if (f == nullptr) return Die("open", argv[1]);
  const int32_t ng = static_cast<int32_t>(generated.size()), k = static_cast<int32_t>(top_ids[0].size());
  std::fwrite(&ng, 4, 1, f);
  std::fwrite(&k, 4, 1, f);
  for (std::size_t s = 0; s < generated.size(); ++s) {
    const int32_t t = generated[s];
    std::fwrite(&t, 4, 1, f);
    for (int j = 0; j < k; ++j) {
      const int32_t id = top_ids[s][j];
      std::fwrite(&id, 4, 1, f);
    }
    std::fwrite(top_vals[s].data(), 4, k, f);
  }
  const int32_t nr = static_cast<int32_t>(rows.size()), v = static_cast<int32_t>(model.vocab_size());
  std::fwrite(&nr, 4, 1, f);
  std::fwrite(&v, 4, 1, f);
  for (const auto& r : rows) std::fwrite(r.data(), 4, r.size(), f);
  std::fclose(f);
  std::printf("test_harness_sequence done: %d tokens\n", ng);
  return 0;
}
