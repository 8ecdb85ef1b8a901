// runtime.h - the reference GPU runtime's C++ host interface, kept for callers, on top of the C ABI (soc_hip.h).
//
// Class and method names, argument meaning and error behaviour follow SongWooYoung/SoC Mac/gpu/include:
//   MetalContext        -> HipContext            (metal/metal_context.h)
//   PipelineCache       -> PipelineCache         (kernel/pipeline_cache.h; kernels are compiled ahead of time)
//   BufferArena         -> BufferArena           (buffer/buffer_arena.h; scratch is owned by the library, the
//                                                  arena keeps the reference's mark/reset/telemetry surface)
//   QwenCausalLM        -> QwenCausalLM          (model/qwen_causal_lm.h)
//   QwenModelLoader     -> QwenModelLoader       (model/qwen_model_loader.h; from named host fp16 tensors)
//   KVCache             -> KVCache               (runtime/kv_cache.h)
//   CommandScheduler    -> CommandScheduler      (runtime/command_scheduler.h)
//   Sampler             -> Sampler               (runtime/sampler.h)
//   GenerationContext   -> GenerationContext     (runtime/generation_context.h)
// Token ids and logits cross this interface as host vectors (the reference passes DeviceTensors that it fills from
// host vectors right before each call). Every method returns bool and fills an optional std::string* error message;
// nothing throws.
#pragma once

#include <cstddef>
#include <cstdint>
#include <map>
#include <memory>
#include <string>
#include <vector>

#include "soc_hip.h"

namespace soc::gpu {

class HipContext {
 public:
  static std::unique_ptr<HipContext> CreateDefault(int device, std::string* error_message);
  ~HipContext();
  HipContext(const HipContext&) = delete;
  HipContext& operator=(const HipContext&) = delete;

  soc_ctx* handle() const { return ctx_; }
  bool Synchronize(std::string* error_message) const;

 private:
  explicit HipContext(soc_ctx* ctx) : ctx_(ctx) {}
  soc_ctx* ctx_ = nullptr;
};

// Kernels are compiled for gfx950 when the library is built; the cache only keeps the reference's call shape.
class PipelineCache {
 public:
  explicit PipelineCache(const HipContext& context) : context_(&context) {}
  const HipContext& context() const { return *context_; }

 private:
  const HipContext* context_;
};

// Scratch bookkeeping with the reference's scope API (Mac/gpu/include/buffer/buffer_arena.h:71-80). The forward's
// device scratch is allocated and reused by the library; the arena records named scope peaks for telemetry.
class BufferArena {
 public:
  static std::unique_ptr<BufferArena> CreateShared(const HipContext& context, std::size_t capacity_bytes,
                                                   const std::string& label, std::string* error_message);
  std::size_t GetCapacityBytes() const { return capacity_; }
  std::size_t GetMark() const { return offset_; }
  void ResetToMark(std::size_t mark) { offset_ = mark; }
  void Reset() { offset_ = 0; }
  bool Reserve(std::size_t bytes, std::string* error_message);  // "BufferArena capacity exceeded" on overflow
  const std::string& label() const { return label_; }
  std::size_t peak_bytes() const { return peak_; }

 private:
  BufferArena(std::size_t capacity, std::string label) : capacity_(capacity), label_(std::move(label)) {}
  std::size_t capacity_ = 0, offset_ = 0, peak_ = 0;
  std::string label_;
};

// Mac/gpu/include/model/qwen_causal_lm.h:25-36
struct QwenCausalLMParams {
  std::size_t vocab_size = 0;
  std::size_t hidden_size = 0;
  std::size_t num_hidden_layers = 0;
  std::size_t num_attention_heads = 0;
  std::size_t num_key_value_heads = 0;
  std::size_t head_dim = 0;
  std::size_t intermediate_size = 0;
  std::size_t max_position_embeddings = 0;
  float rope_theta = 1000000.0f;
  float rms_norm_eps = 1.0e-6f;
  bool tie_word_embeddings = true;
};

class QwenCausalLM {
 public:
  QwenCausalLM() = default;
  QwenCausalLM(std::shared_ptr<soc_model> model, QwenCausalLMParams params)
      : model_(std::move(model)), params_(params) {}

  std::size_t num_layers() const { return params_.num_hidden_layers; }
  std::size_t num_key_value_heads() const { return params_.num_key_value_heads; }
  std::size_t head_dim() const { return params_.head_dim; }
  std::size_t vocab_size() const { return params_.vocab_size; }
  std::size_t max_position_embeddings() const { return params_.max_position_embeddings; }
  const QwenCausalLMParams& params() const { return params_; }
  soc_model* handle() const { return model_.get(); }
  bool IsValid() const { return model_ != nullptr; }

 private:
  std::shared_ptr<soc_model> model_;
  QwenCausalLMParams params_;
};

// Loads a model from named fp16 host tensors (Hugging Face names, Mac/cpu/src/qwen_model_loader.cpp:35-93).
class QwenModelLoader {
 public:
  struct HostTensor {
    const uint16_t* data = nullptr;
    int64_t numel = 0;
  };
  static bool LoadModel(const HipContext& context, const QwenCausalLMParams& params,
                        const std::map<std::string, HostTensor>& tensors, QwenCausalLM* model,
                        std::string* error_message);
  // Random-init weights from the seeded generator (norm gains 1.0, the rest N(0, sigma)).
  static bool SynthesizeModel(const HipContext& context, const QwenCausalLMParams& params, uint64_t seed, float sigma,
                              QwenCausalLM* model, std::string* error_message);
};

// Mac/gpu/include/runtime/kv_cache.h: one sequence, fp16, capacity fixed at creation.
class KVCache {
 public:
  static std::unique_ptr<KVCache> CreateShared(const HipContext& context, const QwenCausalLM& model,
                                               std::size_t max_sequence_length, const std::string& label,
                                               std::string* error_message);
  ~KVCache();
  KVCache(const KVCache&) = delete;
  KVCache& operator=(const KVCache&) = delete;
  std::size_t GetLayerCount() const { return layers_; }
  std::size_t GetKeyValueHeadCount() const { return kv_heads_; }
  std::size_t GetHeadDim() const { return head_dim_; }
  std::size_t GetMaxSequenceLength() const { return capacity_; }
  std::size_t GetSequenceLength() const;
  soc_kv* handle() const { return kv_; }

 private:
  KVCache(soc_kv* kv, std::size_t layers, std::size_t kv_heads, std::size_t head_dim, std::size_t capacity)
      : kv_(kv), layers_(layers), kv_heads_(kv_heads), head_dim_(head_dim), capacity_(capacity) {}
  soc_kv* kv_ = nullptr;
  std::size_t layers_, kv_heads_, head_dim_, capacity_;
};

// Mac/gpu/include/runtime/command_scheduler.h:14-35. logits_output (nullable) receives the last row [V].
class CommandScheduler {
 public:
  bool RunPrefill(const HipContext& context, PipelineCache* pipeline_cache, const QwenCausalLM& model,
                  const std::vector<int>& token_ids, KVCache* kv_cache, std::vector<float>* logits_output,
                  BufferArena* temporary_arena, std::size_t position_offset, int* greedy_token,
                  std::string* error_message) const;
  bool RunDecode(const HipContext& context, PipelineCache* pipeline_cache, const QwenCausalLM& model,
                 const std::vector<int>& token_ids, KVCache* kv_cache, std::vector<float>* logits_output,
                 BufferArena* temporary_arena, std::size_t position_offset, int* greedy_token,
                 std::string* error_message) const;
};

// Mac/gpu/include/runtime/sampler.h
struct SamplerConfig {
  float temperature = 1.0f;
  std::size_t top_k = 1;
};

class Sampler {
 public:
  explicit Sampler(SamplerConfig config = {}) : config_(config) {}
  const SamplerConfig& config() const { return config_; }
  // Mac/gpu/src/runtime/sampler.cpp:14-71 on a host logits row.
  bool SampleFromLogits(const std::vector<float>& logits_row, int* token_id, std::vector<float>* top_logits,
                        std::vector<int>* top_token_ids, std::string* error_message) const;
  bool greedy() const { return config_.top_k <= 1; }

 private:
  SamplerConfig config_;
};

struct GenerationStepResult {
  int token_id = -1;
  std::vector<float> top_logits;
  std::vector<int> top_token_ids;
};

// Mac/gpu/include/runtime/generation_context.h:23-74
class GenerationContext {
 public:
  GenerationContext(QwenCausalLM model, Sampler sampler, CommandScheduler scheduler,
                    std::size_t max_sequence_length);

  bool Prefill(const HipContext& context, PipelineCache* pipeline_cache, const std::vector<int>& token_ids,
               BufferArena* temporary_arena, std::string* error_message);
  bool DecodeNextToken(const HipContext& context, PipelineCache* pipeline_cache, int last_token_id,
                       BufferArena* temporary_arena, GenerationStepResult* result, std::string* error_message);
  bool Generate(const HipContext& context, PipelineCache* pipeline_cache, const std::vector<int>& prompt_token_ids,
                std::size_t max_new_tokens, int eos_token_id, BufferArena* temporary_arena,
                std::vector<int>* generated_token_ids, std::string* error_message);
  void Reset();
  const std::vector<int>& prompt_token_ids() const { return prompt_token_ids_; }
  const std::vector<int>& running_token_ids() const { return running_token_ids_; }
  const QwenCausalLM& model() const { return model_; }

 private:
  QwenCausalLM model_;
  Sampler sampler_;
  CommandScheduler scheduler_;
  std::size_t max_sequence_length_ = 0;
  std::unique_ptr<KVCache> kv_cache_;
  std::vector<int> prompt_token_ids_;
  std::vector<int> running_token_ids_;
  std::vector<float> last_logits_;
  int prefill_token_ = -1;
};

}  // namespace soc::gpu
