// host_api.cpp - the reference GPU runtime's C++ classes (include/soc/gpu/runtime.h) implemented on the C ABI.
// Semantics follow Mac/gpu/src/runtime/generation_context.cpp, command_scheduler.cpp and sampler.cpp.
#include <algorithm>
#include <cstring>
#include <numeric>

#include "soc/gpu/runtime.h"

namespace soc::gpu {

namespace {

bool Fail(std::string* error_message, const std::string& msg) {
  if (error_message != nullptr) *error_message = msg;
  return false;
}

bool Check(int rc, std::string* error_message) {
  if (rc == SOC_OK) return true;
  return Fail(error_message, soc_last_error());
}

soc_qwen_config ToConfig(const QwenCausalLMParams& p) {
  soc_qwen_config c{};
  c.vocab_size = static_cast<int32_t>(p.vocab_size);
  c.hidden_size = static_cast<int32_t>(p.hidden_size);
  c.num_hidden_layers = static_cast<int32_t>(p.num_hidden_layers);
  c.num_attention_heads = static_cast<int32_t>(p.num_attention_heads);
  c.num_key_value_heads = static_cast<int32_t>(p.num_key_value_heads);
  c.head_dim = static_cast<int32_t>(p.head_dim);
  c.intermediate_size = static_cast<int32_t>(p.intermediate_size);
  c.max_position_embeddings = static_cast<int32_t>(p.max_position_embeddings);
  c.rope_theta = p.rope_theta;
  c.rms_norm_eps = p.rms_norm_eps;
  c.tie_word_embeddings = p.tie_word_embeddings ? 1 : 0;
  return c;
}

std::shared_ptr<soc_model> WrapModel(soc_model* m) {
  return std::shared_ptr<soc_model>(m, [](soc_model* p) { soc_model_destroy(p); });
}

}  // namespace

// ---- HipContext ----
std::unique_ptr<HipContext> HipContext::CreateDefault(int device, std::string* error_message) {
  soc_ctx* ctx = nullptr;
  if (!Check(soc_ctx_create(device, &ctx), error_message)) return nullptr;
  return std::unique_ptr<HipContext>(new HipContext(ctx));
}

HipContext::~HipContext() { soc_ctx_destroy(ctx_); }

bool HipContext::Synchronize(std::string* error_message) const {
  return Check(soc_ctx_synchronize(ctx_), error_message);
}

// ---- BufferArena ----
std::unique_ptr<BufferArena> BufferArena::CreateShared(const HipContext&, std::size_t capacity_bytes,
                                                       const std::string& label, std::string* error_message) {
  if (capacity_bytes == 0) {
    Fail(error_message, "BufferArena capacity must be positive");
    return nullptr;
  }
  return std::unique_ptr<BufferArena>(new BufferArena(capacity_bytes, label));
}

bool BufferArena::Reserve(std::size_t bytes, std::string* error_message) {
  const std::size_t aligned = (bytes + 255) / 256 * 256;
  if (offset_ + aligned > capacity_) return Fail(error_message, "BufferArena capacity exceeded");
  offset_ += aligned;
  peak_ = std::max(peak_, offset_);
  return true;
}

// ---- QwenModelLoader ----
bool QwenModelLoader::LoadModel(const HipContext& context, const QwenCausalLMParams& params,
                                const std::map<std::string, HostTensor>& tensors, QwenCausalLM* model,
                                std::string* error_message) {
  if (model == nullptr) return Fail(error_message, "QwenModelLoader requires a non-null model output");
  const soc_qwen_config cfg = ToConfig(params);
  soc_model* m = nullptr;
  if (!Check(soc_model_create(context.handle(), &cfg, &m), error_message)) return false;
  auto holder = WrapModel(m);
  for (const auto& kv : tensors)
    if (!Check(soc_model_load_tensor(m, kv.first.c_str(), kv.second.data, kv.second.numel), error_message))
      return false;
  if (!Check(soc_model_finalize(m), error_message)) return false;
  *model = QwenCausalLM(std::move(holder), params);
  return true;
}

bool QwenModelLoader::SynthesizeModel(const HipContext& context, const QwenCausalLMParams& params, uint64_t seed,
                                      float sigma, QwenCausalLM* model, std::string* error_message) {
  if (model == nullptr) return Fail(error_message, "QwenModelLoader requires a non-null model output");
  const soc_qwen_config cfg = ToConfig(params);
  soc_model* m = nullptr;
  if (!Check(soc_model_create(context.handle(), &cfg, &m), error_message)) return false;
  auto holder = WrapModel(m);
  if (!Check(soc_model_synthesize(m, seed, sigma), error_message)) return false;
  if (!Check(soc_model_finalize(m), error_message)) return false;
  *model = QwenCausalLM(std::move(holder), params);
  return true;
}

// ---- KVCache ----
std::unique_ptr<KVCache> KVCache::CreateShared(const HipContext&, const QwenCausalLM& model,
                                               std::size_t max_sequence_length, const std::string&,
                                               std::string* error_message) {
  if (!model.IsValid()) {
    Fail(error_message, "KVCache requires a loaded model");
    return nullptr;
  }
  soc_kv* kv = nullptr;
  if (!Check(soc_kv_create(model.handle(), 1, static_cast<int32_t>(max_sequence_length), &kv), error_message))
    return nullptr;
  return std::unique_ptr<KVCache>(
      new KVCache(kv, model.num_layers(), model.num_key_value_heads(), model.head_dim(), max_sequence_length));
}

KVCache::~KVCache() { soc_kv_destroy(kv_); }

std::size_t KVCache::GetSequenceLength() const {
  int32_t n = 0;
  soc_kv_length(kv_, 0, &n);
  return static_cast<std::size_t>(n);
}

// ---- CommandScheduler (command_scheduler.cpp:5-41: both paths are ForwardLogitsCached) ----
bool CommandScheduler::RunPrefill(const HipContext&, PipelineCache*, const QwenCausalLM& model,
                                  const std::vector<int>& token_ids, KVCache* kv_cache,
                                  std::vector<float>* logits_output, BufferArena*, std::size_t position_offset,
                                  int* greedy_token, std::string* error_message) const {
  if (kv_cache == nullptr) return Fail(error_message, "CommandScheduler requires a KV cache");
  if (logits_output != nullptr) logits_output->assign(model.vocab_size(), 0.0f);
  int32_t tok = -1;
  const int rc = soc_prefill(model.handle(), kv_cache->handle(), 0, token_ids.data(),
                             static_cast<int32_t>(token_ids.size()), static_cast<int32_t>(position_offset),
                             logits_output != nullptr ? 1 : 0, logits_output ? logits_output->data() : nullptr, &tok);
  if (!Check(rc, error_message)) return false;
  if (greedy_token) *greedy_token = tok;
  return true;
}

bool CommandScheduler::RunDecode(const HipContext&, PipelineCache*, const QwenCausalLM& model,
                                 const std::vector<int>& token_ids, KVCache* kv_cache,
                                 std::vector<float>* logits_output, BufferArena*, std::size_t position_offset,
                                 int* greedy_token, std::string* error_message) const {
  if (kv_cache == nullptr) return Fail(error_message, "CommandScheduler requires a KV cache");
  if (token_ids.size() != 1) return Fail(error_message, "CommandScheduler decode takes exactly one token");
  if (kv_cache->GetSequenceLength() != position_offset)
    return Fail(error_message, "CommandScheduler decode position does not match the KV cache length");
  if (logits_output != nullptr) logits_output->assign(model.vocab_size(), 0.0f);
  int32_t tok = -1;
  const int rc = soc_decode(model.handle(), kv_cache->handle(), 0, token_ids[0],
                            logits_output ? logits_output->data() : nullptr, &tok);
  if (!Check(rc, error_message)) return false;
  if (greedy_token) *greedy_token = tok;
  return true;
}

// ---- Sampler (Mac/gpu/src/runtime/sampler.cpp:14-71) ----
bool Sampler::SampleFromLogits(const std::vector<float>& row, int* token_id, std::vector<float>* top_logits,
                               std::vector<int>* top_token_ids, std::string* error_message) const {
  if (token_id == nullptr) return Fail(error_message, "Sampler requires a non-null token_id output");
  if (row.empty()) return Fail(error_message, "Sampler expects a non-empty logits row");
  const std::size_t vocab = row.size();
  std::vector<std::size_t> cand(vocab);
  std::iota(cand.begin(), cand.end(), std::size_t{0});
  const std::size_t k = std::max<std::size_t>(1, std::min<std::size_t>(config_.top_k, vocab));
  const float t = config_.temperature <= 0.0f ? 1.0f : config_.temperature;
  std::partial_sort(cand.begin(), cand.begin() + static_cast<std::ptrdiff_t>(k), cand.end(),
                    [&row, t](std::size_t l, std::size_t r) { return row[l] / t > row[r] / t; });
  *token_id = static_cast<int>(cand[0]);
  if (top_logits) {
    top_logits->clear();
    for (std::size_t i = 0; i < k; ++i) top_logits->push_back(row[cand[i]]);
  }
  if (top_token_ids) {
    top_token_ids->clear();
    for (std::size_t i = 0; i < k; ++i) top_token_ids->push_back(static_cast<int>(cand[i]));
  }
  return true;
}

// ---- GenerationContext (Mac/gpu/src/runtime/generation_context.cpp) ----
GenerationContext::GenerationContext(QwenCausalLM model, Sampler sampler, CommandScheduler scheduler,
                                     std::size_t max_sequence_length)
    : model_(std::move(model)),
      sampler_(sampler),
      scheduler_(scheduler),
      max_sequence_length_(max_sequence_length) {}

bool GenerationContext::Prefill(const HipContext& context, PipelineCache* pipeline_cache,
                                const std::vector<int>& token_ids, BufferArena* temporary_arena,
                                std::string* error_message) {
  if (token_ids.empty()) return Fail(error_message, "GenerationContext prefill requires at least one token");
  Reset();
  prompt_token_ids_ = token_ids;
  running_token_ids_ = token_ids;
  kv_cache_ = KVCache::CreateShared(context, model_, max_sequence_length_, "generation_kv_cache", error_message);
  if (kv_cache_ == nullptr) return false;
  std::vector<float>* logits = sampler_.greedy() ? nullptr : &last_logits_;
  return scheduler_.RunPrefill(context, pipeline_cache, model_, token_ids, kv_cache_.get(), logits, temporary_arena,
                               0, &prefill_token_, error_message);
}

bool GenerationContext::DecodeNextToken(const HipContext& context, PipelineCache* pipeline_cache, int last_token_id,
                                        BufferArena* temporary_arena, GenerationStepResult* result,
                                        std::string* error_message) {
  if (result == nullptr) return Fail(error_message, "GenerationContext decode requires a non-null result");
  if (kv_cache_ == nullptr) return Fail(error_message, "GenerationContext decode requires a prefilled KV cache");
  if (running_token_ids_.empty() || running_token_ids_.back() != last_token_id)
    return Fail(error_message, "GenerationContext decode requires last_token_id to match the current sequence tail");
  if (running_token_ids_.size() >= max_sequence_length_)
    return Fail(error_message, "GenerationContext sequence length would exceed max_sequence_length");
  std::vector<float>* logits = sampler_.greedy() ? nullptr : &last_logits_;
  int greedy = -1;
  if (!scheduler_.RunDecode(context, pipeline_cache, model_, std::vector<int>{last_token_id}, kv_cache_.get(),
                            logits, temporary_arena, running_token_ids_.size() - 1, &greedy, error_message))
    return false;
  if (sampler_.greedy()) {
    result->token_id = greedy;
    result->top_token_ids = {greedy};
    result->top_logits.clear();
  } else if (!sampler_.SampleFromLogits(last_logits_, &result->token_id, &result->top_logits,
                                        &result->top_token_ids, error_message)) {
    return false;
  }
  running_token_ids_.push_back(result->token_id);
  return true;
}

bool GenerationContext::Generate(const HipContext& context, PipelineCache* pipeline_cache,
                                 const std::vector<int>& prompt_token_ids, std::size_t max_new_tokens,
                                 int eos_token_id, BufferArena* temporary_arena, std::vector<int>* generated_token_ids,
                                 std::string* error_message) {
  if (generated_token_ids == nullptr)
    return Fail(error_message, "GenerationContext generate requires a non-null generated_token_ids output");
  generated_token_ids->clear();
  if (!Prefill(context, pipeline_cache, prompt_token_ids, temporary_arena, error_message)) return false;
  if (max_new_tokens == 0) return true;
  int first = prefill_token_;
  if (!sampler_.greedy()) {
    GenerationStepResult r;
    if (!sampler_.SampleFromLogits(last_logits_, &r.token_id, &r.top_logits, &r.top_token_ids, error_message))
      return false;
    first = r.token_id;
  }
  generated_token_ids->push_back(first);
  running_token_ids_.push_back(first);
  if (eos_token_id >= 0 && first == eos_token_id) return true;
  int last = first;
  for (std::size_t step = 1; step < max_new_tokens; ++step) {
    GenerationStepResult r;
    if (!DecodeNextToken(context, pipeline_cache, last, temporary_arena, &r, error_message)) return false;
    generated_token_ids->push_back(r.token_id);
    last = r.token_id;
    if (eos_token_id >= 0 && r.token_id == eos_token_id) break;
  }
  return true;
}

void GenerationContext::Reset() {
  kv_cache_.reset();
  prompt_token_ids_.clear();
  running_token_ids_.clear();
  last_logits_.clear();
  prefill_token_ = -1;
}

}  // namespace soc::gpu
