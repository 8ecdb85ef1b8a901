// runtime.h - the reference GPU runtime's C++ host interface, kept for its callers, on top of the C ABI (soc_hip.h).
//
// Class and method names, signatures, argument meaning and error behaviour follow SongWooYoung/SoC Mac/gpu/include:
//   MetalContext        -> HipContext            (metal/metal_context.h; kernels are compiled into the library)
//   MetalBuffer         -> HipBuffer             (buffer/metal_buffer.h; device memory, Write/Read copy)
//   TensorDesc          -> TensorDesc            (tensor/tensor_desc.h)
//   DeviceTensor        -> DeviceTensor          (tensor/device_tensor.h)
//   PipelineCache       -> PipelineCache         (kernel/pipeline_cache.h)
//   BufferArena         -> BufferArena           (buffer/buffer_arena.h; the forward's scratch is the library's own)
//   QwenCausalLM        -> QwenCausalLM          (model/qwen_causal_lm.h)
//   QwenModelLoader     -> QwenModelLoader       (model/qwen_model_loader.h; from a bundle's manifest, or from
//                                                  named host fp16 tensors)
//   KVCache             -> KVCache               (runtime/kv_cache.h)
//   CommandScheduler    -> CommandScheduler      (runtime/command_scheduler.h)
//   Sampler             -> Sampler               (runtime/sampler.h)
//   GenerationContext   -> GenerationContext     (runtime/generation_context.h)
//   RuntimePipeline     -> RuntimePipeline       (Mac/cpu/header/runtime_pipeline.h; the text-level helpers, with
//                                                  the bundle's model loaded on the device)
// The tokenizer runtime and chat template are soc::TokenizerRuntime / soc::Qwen3TemplateBuilder (soc/tokenizer.h).
// MetalContext, MetalBuffer and MetalProfilingSnapshot are also declared under their reference names (aliases at the
// end of this file), so that reference callers compile unchanged. Every method returns bool (or a null pointer) and
// fills an optional std::string* error message; nothing throws.
//
// Differences a caller can observe (storage is fp16 where the reference stores fp32):
//   * KVCache keeps fp16 keys/values [kv_head][max_sequence_length][head_dim] per layer; ViewForLayer describes that
//     (kFloat16, shape {kv_heads, length, head_dim}, strides {max_len * head_dim, head_dim, 1}); AppendPrefill and
//     AppendDecodeToken take fp32 (as the reference) or fp16 rows [rows][kv_heads * head_dim] and round to fp16.
//   * CommandScheduler writes the logits of the last r token rows when logits_output has r <= n rows (r = n is the
//     reference's all-rows output); an invalid (empty) logits_output skips the logits.
#pragma once

#include <cstddef>
#include <cstdint>
#include <map>
#include <memory>
#include <string>
#include <vector>

#include "soc/assets.h"
#include "soc/tokenizer.h"
#include "soc_hip.h"

namespace soc::gpu {

struct HipProfilingSnapshot {  // metal_context.h:19-22
  double gpu_ms = 0.0;         // GPU time of the forwards run since ResetProfiling (HIP events)
  std::size_t command_buffer_count = 0;
};

class HipContext {
 public:
  static std::unique_ptr<HipContext> CreateDefault(int device, std::string* error_message);
  // The reference's factory (metal_context.h:26-28): the kernel paths are not needed (the kernels are compiled into
  // the library); device 0.
  static std::unique_ptr<HipContext> CreateDefault(const std::string& kernel_library_path,
                                                   const std::string& kernel_source_path,
                                                   std::string* error_message);
  ~HipContext();
  HipContext(const HipContext&) = delete;
  HipContext& operator=(const HipContext&) = delete;

  soc_ctx* handle() const { return ctx_; }
  bool Synchronize(std::string* error_message) const;
  void ResetProfiling() const { profile_ = {}; }
  HipProfilingSnapshot GetProfilingSnapshot() const { return profile_; }
  void AddProfile(double gpu_ms) const {
    profile_.gpu_ms += gpu_ms;
    profile_.command_buffer_count += 1;
  }

 private:
  explicit HipContext(soc_ctx* ctx) : ctx_(ctx) {}
  soc_ctx* ctx_ = nullptr;
  mutable HipProfilingSnapshot profile_;
};

// Device memory (metal_buffer.h:13-37). Write/Read copy between host memory and the buffer and return when done.
class HipBuffer {
 public:
  static std::shared_ptr<HipBuffer> CreateShared(const HipContext& context, std::size_t size_bytes,
                                                 const std::string& label, std::string* error_message);
  // A view of device memory that `owner` keeps alive (the KV cache's layer planes).
  static std::shared_ptr<HipBuffer> Wrap(const HipContext& context, void* device_ptr, std::size_t size_bytes,
                                         std::shared_ptr<void> owner);
  ~HipBuffer();
  HipBuffer(const HipBuffer&) = delete;
  HipBuffer& operator=(const HipBuffer&) = delete;

  std::size_t GetSizeBytes() const { return size_; }
  bool IsHostVisible() const { return false; }
  bool Write(const void* source, std::size_t size_bytes, std::size_t offset_bytes, std::string* error_message);
  bool Read(void* destination, std::size_t size_bytes, std::size_t offset_bytes, std::string* error_message) const;
  const void* GetNativeHandle() const { return ptr_; }  // the device address
  void* data() const { return ptr_; }
  soc_ctx* context() const { return ctx_; }

 private:
  HipBuffer(soc_ctx* ctx, void* ptr, std::size_t size, std::shared_ptr<void> owner)
      : ctx_(ctx), ptr_(ptr), size_(size), owner_(std::move(owner)) {}
  soc_ctx* ctx_ = nullptr;
  void* ptr_ = nullptr;
  std::size_t size_ = 0;
  std::shared_ptr<void> owner_;  // null: this buffer owns ptr_
};

enum class DataType { kFloat16, kFloat32, kInt32 };  // tensor_desc.h:8-12
std::size_t GetDataTypeSize(DataType data_type);

class TensorDesc {  // tensor_desc.h:14-32
 public:
  static TensorDesc CreateContiguous(DataType data_type, const std::vector<std::size_t>& shape);
  // Element strides given explicitly (views of the KV cache).
  static TensorDesc CreateStrided(DataType data_type, const std::vector<std::size_t>& shape,
                                  const std::vector<std::size_t>& strides);
  DataType GetDataType() const { return data_type_; }
  const std::vector<std::size_t>& GetShape() const { return shape_; }
  const std::vector<std::size_t>& GetStrides() const { return strides_; }
  std::size_t Rank() const { return shape_.size(); }
  std::size_t ElementCount() const;
  std::size_t ByteSize() const;  // bytes spanned from element 0 to the last element
  bool IsContiguous() const { return contiguous_; }

 private:
  DataType data_type_ = DataType::kFloat32;
  std::vector<std::size_t> shape_;
  std::vector<std::size_t> strides_;
  bool contiguous_ = false;
};

class DeviceTensor {  // device_tensor.h:11-25
 public:
  DeviceTensor() = default;
  DeviceTensor(std::shared_ptr<HipBuffer> buffer, std::size_t byte_offset, TensorDesc desc)
      : buffer_(std::move(buffer)), byte_offset_(byte_offset), desc_(std::move(desc)) {}
  bool IsValid() const;  // a buffer, and the tensor's bytes lie inside it
  const std::shared_ptr<HipBuffer>& GetBuffer() const { return buffer_; }
  std::size_t GetByteOffset() const { return byte_offset_; }
  const TensorDesc& GetDesc() const { return desc_; }
  void* data() const { return buffer_ ? static_cast<char*>(buffer_->data()) + byte_offset_ : nullptr; }

 private:
  std::shared_ptr<HipBuffer> buffer_;
  std::size_t byte_offset_ = 0;
  TensorDesc desc_;
};

// Kernels are compiled for gfx950 when the library is built; the cache only keeps the reference's call shape.
class PipelineCache {
 public:
  explicit PipelineCache(const HipContext& context) : context_(&context) {}
  const HipContext& context() const { return *context_; }

 private:
  const HipContext* context_;
};

// buffer_arena.h:15-80: a bump allocator over one device buffer with marks and per-scope telemetry. The forward
// passes keep their scratch inside the library, so the arena serves callers' own temporaries.
using BufferArenaMark = std::size_t;

struct BufferArenaSlice {
  std::shared_ptr<HipBuffer> buffer;
  std::size_t offset_bytes = 0;
  std::size_t size_bytes = 0;
  bool IsValid() const { return buffer != nullptr && size_bytes > 0; }
};

struct BufferArenaScopeTelemetry {
  std::string name;
  std::size_t invocation_count = 0;
  std::size_t peak_delta_bytes = 0;
  std::size_t peak_used_bytes = 0;
  std::size_t peak_allocation_count = 0;
};

class BufferArena {
 public:
  static std::unique_ptr<BufferArena> CreateShared(const HipContext& context, std::size_t capacity_bytes,
                                                   const std::string& label, std::string* error_message);
  bool Allocate(std::size_t size_bytes, std::size_t alignment_bytes, BufferArenaSlice* slice,
                std::string* error_message);
  BufferArenaMark GetMark() const { return used_; }
  bool ResetToMark(BufferArenaMark mark, std::string* error_message);
  void Reset() { used_ = 0; }
  void ClearTelemetry();
  std::size_t GetCapacityBytes() const { return capacity_; }
  std::size_t GetUsedBytes() const { return used_; }
  std::size_t GetPeakUsedBytes() const { return peak_; }
  const std::vector<BufferArenaScopeTelemetry>& GetTelemetrySnapshot() const { return telemetry_; }

 private:
  struct ActiveScope {
    std::string name;
    std::size_t start_used;  // usage when the scope began
    std::size_t peak_used;
    std::size_t allocations;
  };
  BufferArena(std::shared_ptr<HipBuffer> buffer, std::size_t capacity)
      : buffer_(std::move(buffer)), capacity_(capacity) {}
  void BeginScope(const std::string& scope_name);
  void EndScope();
  std::shared_ptr<HipBuffer> buffer_;
  std::size_t capacity_ = 0, used_ = 0, peak_ = 0;
  std::vector<ActiveScope> active_scopes_;
  std::vector<BufferArenaScopeTelemetry> telemetry_;
  friend class BufferArenaMarkGuard;
};

class BufferArenaMarkGuard {  // buffer_arena.h:71-80: resets the arena to its mark when the scope ends
 public:
  explicit BufferArenaMarkGuard(BufferArena* arena, const std::string& scope_name = {});
  ~BufferArenaMarkGuard();

 private:
  BufferArena* arena_ = nullptr;
  BufferArenaMark mark_ = 0;
  bool has_scope_ = false;
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

class KVCache;

// The model's weights as device tensors (qwen_attention.h:16-23, qwen_mlp.h:13-17, qwen_block.h:15-20,
// qwen_causal_lm.h:17-23). A model built from them (the constructor below) copies them into its own fp16 storage; a
// model from QwenModelLoader reports fp16 views of that storage here.
struct QwenAttentionWeights {
  DeviceTensor q_proj_weight;
  DeviceTensor k_proj_weight;
  DeviceTensor v_proj_weight;
  DeviceTensor o_proj_weight;
  DeviceTensor q_norm_weight;
  DeviceTensor k_norm_weight;
};

struct QwenMlpWeights {
  DeviceTensor gate_proj_weight;
  DeviceTensor up_proj_weight;
  DeviceTensor down_proj_weight;
};

struct QwenBlockWeights {
  DeviceTensor input_layernorm_weight;
  QwenAttentionWeights attention;
  DeviceTensor post_attention_layernorm_weight;
  QwenMlpWeights mlp;
};

struct QwenCausalLMWeights {
  DeviceTensor embed_tokens_weight;
  std::vector<QwenBlockWeights> blocks;
  DeviceTensor final_norm_weight;
  DeviceTensor lm_head_weight;
  bool tie_word_embeddings = true;
};

// Mac/gpu/include/model/qwen_causal_lm.h:38-95. Every forward runs the hot-path kernels through soc_forward; token
// ids and outputs are device tensors, and the ids are never read back to the host.
class QwenCausalLM {
 public:
  QwenCausalLM() = default;
  // qwen_causal_lm.cpp:31-32: a model over the given weights (float32 or float16 device tensors, shapes of
  // Mac/cpu/src/qwen_model_loader.cpp:57-100; lm_head_weight is used only without tied embeddings). The weights are
  // converted to fp16 device storage here; the layer count is weights.blocks.size(). A constructor cannot fail in the
  // reference's interface: a weight of the wrong shape, dtype or memory leaves the model invalid (IsValid() false)
  // and every forward then fails with the reason.
  QwenCausalLM(QwenCausalLMWeights weights, QwenCausalLMParams params);
  // A model over library storage (QwenModelLoader); `weights` holds fp16 views of it.
  QwenCausalLM(std::shared_ptr<soc_model> model, QwenCausalLMParams params, QwenCausalLMWeights weights = {})
      : model_(std::move(model)), params_(params), weights_(std::move(weights)) {}

  std::size_t num_layers() const { return params_.num_hidden_layers; }
  std::size_t num_key_value_heads() const { return params_.num_key_value_heads; }
  std::size_t head_dim() const { return params_.head_dim; }
  std::size_t vocab_size() const { return params_.vocab_size; }
  std::size_t max_position_embeddings() const { return params_.max_position_embeddings; }
  const QwenCausalLMParams& params() const { return params_; }
  const QwenCausalLMWeights& weights() const { return weights_; }
  soc_model* handle() const { return model_.get(); }
  bool IsValid() const { return model_ != nullptr; }

  // qwen_causal_lm.cpp:37-129: the uncached forward of token_ids [n] (kInt32) at positions position_offset.. (causal
  // over the n tokens alone), the final-RMSNorm rows into output [n][hidden_size] (kFloat32).
  bool ForwardHidden(const HipContext& context, PipelineCache* pipeline_cache, const DeviceTensor& token_ids,
                     const DeviceTensor& output, BufferArena* temporary_arena, std::size_t position_offset,
                     std::string* error_message) const;
  // qwen_causal_lm.cpp:130-229: the same over kv_cache (position_offset must equal its length), appending K/V.
  bool ForwardHiddenCached(const HipContext& context, PipelineCache* pipeline_cache, const DeviceTensor& token_ids,
                           KVCache* kv_cache, const DeviceTensor& output, BufferArena* temporary_arena,
                           std::size_t position_offset, std::string* error_message) const;
  // qwen_causal_lm.cpp:231-248: uncached logits of the last rows into logits_output [r][vocab] (r <= n; the
  // reference's all-rows output is r = n).
  bool ForwardLogits(const HipContext& context, PipelineCache* pipeline_cache, const DeviceTensor& token_ids,
                     const DeviceTensor& logits_output, BufferArena* temporary_arena, std::size_t position_offset,
                     std::string* error_message) const;
  // qwen_causal_lm.cpp:250-268: the cached forward, logits of the last rows into logits_output [r][vocab] (r <= n).
  bool ForwardLogitsCached(const HipContext& context, PipelineCache* pipeline_cache, const DeviceTensor& token_ids,
                           KVCache* kv_cache, const DeviceTensor& logits_output, BufferArena* temporary_arena,
                           std::size_t position_offset, std::string* error_message) const;

 private:
  bool Forward(const HipContext& context, const DeviceTensor& token_ids, KVCache* kv_cache, const DeviceTensor* hidden,
               const DeviceTensor* logits, std::size_t position_offset, std::string* error_message) const;

  std::shared_ptr<soc_model> model_;
  QwenCausalLMParams params_;
  QwenCausalLMWeights weights_;
  std::string build_error_;  // why the weights constructor left the model invalid
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
  // Mac/gpu/src/model/qwen_model_loader.cpp:100-192 over a manifest (soc/assets.h): validates it and its config
  // (StartupValidator), reads every weight (float32, float16 or bfloat16 files; kept as fp16) and builds the model;
  // lm_head.weight only when the embeddings are not tied.
  static bool LoadModel(const HipContext& context, const soc::ManifestData& manifest, QwenCausalLM* model,
                        std::string* error_message);
  static bool LoadModelFromFile(const HipContext& context, const std::string& manifest_path, QwenCausalLM* model,
                                std::string* error_message);
  // Random-init weights from the seeded generator (norm gains 1.0, the rest N(0, sigma)).
  static bool SynthesizeModel(const HipContext& context, const QwenCausalLMParams& params, uint64_t seed, float sigma,
                              QwenCausalLM* model, std::string* error_message);
};

// kv_cache.h:15-19
struct KVCacheLayerView {
  DeviceTensor keys;
  DeviceTensor values;
  std::size_t sequence_length = 0;
};

// kv_cache.h:21-79: one sequence, capacity fixed at creation, a length per layer.
class KVCache {
 public:
  static std::unique_ptr<KVCache> CreateShared(const HipContext& context, std::size_t layer_count,
                                               std::size_t key_value_head_count, std::size_t head_dim,
                                               std::size_t max_sequence_length, const std::string& label,
                                               std::string* error_message);
  ~KVCache() = default;
  KVCache(const KVCache&) = delete;
  KVCache& operator=(const KVCache&) = delete;

  bool Reserve(std::size_t sequence_length, std::string* error_message);
  bool AppendPrefill(const HipContext& context, std::size_t layer_index, const DeviceTensor& keys,
                     const DeviceTensor& values, std::string* error_message);
  bool AppendDecodeToken(const HipContext& context, std::size_t layer_index, const DeviceTensor& key,
                         const DeviceTensor& value, std::string* error_message);
  KVCacheLayerView ViewForLayer(std::size_t layer_index) const;
  std::size_t GetLayerCount() const { return layer_count_; }
  std::size_t GetKeyValueHeadCount() const { return kv_heads_; }
  std::size_t GetHeadDim() const { return head_dim_; }
  std::size_t GetMaxSequenceLength() const { return capacity_; }

  // Length of layer 0 (every layer after a forward).
  std::size_t GetSequenceLength() const { return sequence_lengths_.empty() ? 0 : sequence_lengths_[0]; }
  soc_kv* handle() const { return kv_.get(); }
  // After a forward that appended `rows` positions to every layer.
  void OnForward(std::size_t rows);
  // True when every layer holds the same number of positions (required by a forward).
  bool LayersAligned() const;

 private:
  KVCache(const HipContext& context, std::shared_ptr<soc_kv> kv, std::size_t layers, std::size_t kv_heads,
          std::size_t head_dim, std::size_t capacity)
      : context_(&context), kv_(std::move(kv)), layer_count_(layers), kv_heads_(kv_heads), head_dim_(head_dim),
        capacity_(capacity), sequence_lengths_(layers, 0) {}
  const HipContext* context_;
  std::shared_ptr<soc_kv> kv_;
  std::size_t layer_count_, kv_heads_, head_dim_, capacity_;
  std::vector<std::size_t> sequence_lengths_;
};

// command_scheduler.h:14-35 (both run QwenCausalLM::ForwardLogitsCached).
class CommandScheduler {
 public:
  bool RunPrefill(const HipContext& context, PipelineCache* pipeline_cache, const QwenCausalLM& model,
                  const DeviceTensor& token_ids, KVCache* kv_cache, const DeviceTensor& logits_output,
                  BufferArena* temporary_arena, std::size_t position_offset, std::string* error_message) const;
  bool RunDecode(const HipContext& context, PipelineCache* pipeline_cache, const QwenCausalLM& model,
                 const DeviceTensor& token_ids, KVCache* kv_cache, const DeviceTensor& logits_output,
                 BufferArena* temporary_arena, std::size_t position_offset, std::string* error_message) const;
};

// sampler.h:10-27
struct SamplerConfig {
  float temperature = 1.0f;
  std::size_t top_k = 1;
};

class Sampler {
 public:
  explicit Sampler(SamplerConfig config = {}) : config_(config) {}
  const SamplerConfig& config() const { return config_; }
  // sampler.cpp:14-71: top-k of row `row_index` of logits [rows][vocab] (kFloat32), selected on the device.
  bool SampleFromLogits(const DeviceTensor& logits, std::size_t row_index, int* token_id,
                        std::vector<float>* top_logits, std::vector<int>* top_token_ids,
                        std::string* error_message) const;

 private:
  SamplerConfig config_;
};

struct GenerationStepResult {  // generation_context.h:17-21
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
  bool EnsureLogitsBuffer(const HipContext& context, std::string* error_message);
  bool UploadTokenIds(const HipContext& context, const std::vector<int>& token_ids, DeviceTensor* token_tensor,
                      std::string* error_message);

  QwenCausalLM model_;
  Sampler sampler_;
  CommandScheduler scheduler_;
  std::size_t max_sequence_length_ = 0;
  std::unique_ptr<KVCache> kv_cache_;
  std::vector<int> prompt_token_ids_;
  std::vector<int> running_token_ids_;
  std::shared_ptr<HipBuffer> logits_buffer_;  // one logits row: generation samples only the last row
  std::shared_ptr<HipBuffer> token_buffer_;
  std::vector<int> uploaded_ids_;  // source of the last asynchronous token upload, kept until the forward has run
};

// ---- text-level helpers (Mac/cpu/header/runtime_pipeline.h:13-43) ----
struct RuntimeGenerationOptions {  // runtime_pipeline.h:13-18
  std::size_t max_new_tokens = 32;
  SamplerConfig sampler;
  int eos_token_id = -1;
  std::size_t max_sequence_length = 256;
};

struct RuntimePromptOptions {  // runtime_pipeline.h:26-31
  bool apply_chat_template = false;
  bool add_generation_prompt = true;
  bool enable_thinking = true;
  std::string system_prompt;
};

// A bundle loaded for generation: its manifest, tokenizer runtime and the model on the device (the reference's
// RuntimeBundle holds the CPU model; runtime_pipeline.h:20-24).
struct RuntimeBundle {
  soc::ManifestData manifest;
  soc::TokenizerRuntimeData tokenizer_runtime;
  QwenCausalLM model;
};

class RuntimePipeline {
 public:
  // runtime_pipeline.cpp:35-40: manifest, the tokenizer runtime it names, StartupValidator::
  // ValidateManifestAndTokenizer, then the weights (QwenModelLoader::LoadModel).
  static bool LoadBundle(const HipContext& context, const std::string& manifest_path, RuntimeBundle* bundle,
                         std::string* error_message);
  // runtime_pipeline.cpp:42-54: max_new_tokens, temperature, top_k, eos_token_id (first entry of a list) and
  // max_length from the manifest's generation_config, defaults otherwise. Throws std::runtime_error on a value of
  // the wrong JSON type, as the reference does.
  static RuntimeGenerationOptions GenerationOptionsFromManifest(const soc::ManifestData& manifest);
  // runtime_pipeline.cpp:56-70: the prompt itself, or one user turn through the Qwen3 chat template.
  static std::string PreparePrompt(const soc::TokenizerRuntimeData& tokenizer_runtime, const std::string& prompt,
                                   const RuntimePromptOptions& options = {});
};

}  // namespace soc::gpu

#include "soc/gpu/ops.h"

namespace soc::gpu {

// The reference's names for the platform classes.
using MetalContext = HipContext;
using MetalBuffer = HipBuffer;
using MetalProfilingSnapshot = HipProfilingSnapshot;

}  // namespace soc::gpu
