// host_api.cpp - the reference GPU runtime's C++ classes (include/soc/gpu/runtime.h) implemented on the C ABI.
// Semantics follow Mac/gpu/src: runtime/generation_context.cpp, command_scheduler.cpp, sampler.cpp, kv_cache.mm,
// tensor/tensor_desc.cpp, device_tensor.cpp, buffer/buffer_arena.cpp, metal_buffer.mm; and the text-level helpers of
// Mac/cpu/src/runtime_pipeline.cpp.
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

struct WeightSlot {
  std::string name;                // Hugging Face name (Mac/cpu/src/qwen_model_loader.cpp:57-100)
  DeviceTensor* tensor;            // its place in QwenCausalLMWeights
  std::vector<std::size_t> shape;  // expected shape
};

// Every weight of a model of params.num_hidden_layers layers (w.blocks already sized), lm_head only when untied.
std::vector<WeightSlot> WeightSlots(QwenCausalLMWeights& w, const QwenCausalLMParams& p) {
  const std::size_t H = p.hidden_size, I = p.intermediate_size, q = p.num_attention_heads * p.head_dim,
                    kv = p.num_key_value_heads * p.head_dim;
  std::vector<WeightSlot> out;
  out.push_back({"model.embed_tokens.weight", &w.embed_tokens_weight, {p.vocab_size, H}});
  for (std::size_t l = 0; l < w.blocks.size(); ++l) {
    const std::string n = "model.layers." + std::to_string(l) + ".";
    QwenBlockWeights& b = w.blocks[l];
    out.push_back({n + "input_layernorm.weight", &b.input_layernorm_weight, {H}});
    out.push_back({n + "self_attn.q_proj.weight", &b.attention.q_proj_weight, {q, H}});
    out.push_back({n + "self_attn.k_proj.weight", &b.attention.k_proj_weight, {kv, H}});
    out.push_back({n + "self_attn.v_proj.weight", &b.attention.v_proj_weight, {kv, H}});
    out.push_back({n + "self_attn.o_proj.weight", &b.attention.o_proj_weight, {H, q}});
    out.push_back({n + "self_attn.q_norm.weight", &b.attention.q_norm_weight, {p.head_dim}});
    out.push_back({n + "self_attn.k_norm.weight", &b.attention.k_norm_weight, {p.head_dim}});
    out.push_back({n + "post_attention_layernorm.weight", &b.post_attention_layernorm_weight, {H}});
    out.push_back({n + "mlp.gate_proj.weight", &b.mlp.gate_proj_weight, {I, H}});
    out.push_back({n + "mlp.up_proj.weight", &b.mlp.up_proj_weight, {I, H}});
    out.push_back({n + "mlp.down_proj.weight", &b.mlp.down_proj_weight, {H, I}});
  }
  out.push_back({"model.norm.weight", &w.final_norm_weight, {H}});
  if (!w.tie_word_embeddings) out.push_back({"lm_head.weight", &w.lm_head_weight, {p.vocab_size, H}});
  return out;
}

std::string ShapeText(const std::vector<std::size_t>& s) {
  std::string t = "[";
  for (std::size_t i = 0; i < s.size(); ++i) t += (i ? ", " : "") + std::to_string(s[i]);
  return t + "]";
}

// fp16 views of a loaded model's device storage, kept alive by the model (QwenCausalLM::weights()).
QwenCausalLMWeights ViewWeights(const HipContext& context, const std::shared_ptr<soc_model>& holder,
                                const QwenCausalLMParams& p) {
  QwenCausalLMWeights w;
  w.blocks.resize(p.num_hidden_layers);
  w.tie_word_embeddings = p.tie_word_embeddings;
  for (const WeightSlot& slot : WeightSlots(w, p)) {
    void* ptr = nullptr;
    int64_t numel = 0;
    if (soc_model_tensor(holder.get(), slot.name.c_str(), &ptr, &numel) != SOC_OK) continue;
    *slot.tensor = DeviceTensor(HipBuffer::Wrap(context, ptr, static_cast<std::size_t>(numel) * 2, holder), 0,
                                TensorDesc::CreateContiguous(DataType::kFloat16, slot.shape));
  }
  if (w.tie_word_embeddings) w.lm_head_weight = w.embed_tokens_weight;
  return w;
}

}  // namespace

// ---- HipContext (metal_context.h) ----
std::unique_ptr<HipContext> HipContext::CreateDefault(int device, std::string* error_message) {
  soc_ctx* ctx = nullptr;
  if (!Check(soc_ctx_create(device, &ctx), error_message)) return nullptr;
  return std::unique_ptr<HipContext>(new HipContext(ctx));
}

std::unique_ptr<HipContext> HipContext::CreateDefault(const std::string&, const std::string&,
                                                      std::string* error_message) {
  return CreateDefault(0, error_message);
}

HipContext::~HipContext() { soc_ctx_destroy(ctx_); }

bool HipContext::Synchronize(std::string* error_message) const {
  return Check(soc_ctx_synchronize(ctx_), error_message);
}

// ---- HipBuffer (metal_buffer.mm: bounds-checked copies) ----
std::shared_ptr<HipBuffer> HipBuffer::CreateShared(const HipContext& context, std::size_t size_bytes,
                                                   const std::string&, std::string* error_message) {
  void* p = nullptr;
  if (!Check(soc_buffer_alloc(context.handle(), std::max<std::size_t>(size_bytes, 1), &p), error_message))
    return nullptr;
  return std::shared_ptr<HipBuffer>(new HipBuffer(context.handle(), p, size_bytes, nullptr));
}

std::shared_ptr<HipBuffer> HipBuffer::Wrap(const HipContext& context, void* device_ptr, std::size_t size_bytes,
                                           std::shared_ptr<void> owner) {
  return std::shared_ptr<HipBuffer>(new HipBuffer(context.handle(), device_ptr, size_bytes, std::move(owner)));
}

HipBuffer::~HipBuffer() {
  if (owner_ == nullptr && ptr_ != nullptr) soc_buffer_free(ctx_, ptr_);
}

bool HipBuffer::Write(const void* source, std::size_t size_bytes, std::size_t offset_bytes,
                      std::string* error_message) {
  if (source == nullptr) return Fail(error_message, "Write source must not be null");
  if (offset_bytes > size_ || size_bytes > size_ - offset_bytes)
    return Fail(error_message, "Write range exceeds buffer size");
  if (size_bytes == 0) return true;
  return Check(soc_buffer_write(ctx_, static_cast<char*>(ptr_) + offset_bytes, source, size_bytes), error_message);
}

bool HipBuffer::Read(void* destination, std::size_t size_bytes, std::size_t offset_bytes,
                     std::string* error_message) const {
  if (destination == nullptr) return Fail(error_message, "Read destination must not be null");
  if (offset_bytes > size_ || size_bytes > size_ - offset_bytes)
    return Fail(error_message, "Read range exceeds buffer size");
  if (size_bytes == 0) return true;
  return Check(soc_buffer_read(ctx_, destination, static_cast<const char*>(ptr_) + offset_bytes, size_bytes),
               error_message);
}

// ---- TensorDesc / DeviceTensor (tensor_desc.cpp, device_tensor.cpp) ----
std::size_t GetDataTypeSize(DataType data_type) {
  switch (data_type) {
    case DataType::kFloat16:
      return 2;
    case DataType::kFloat32:
    case DataType::kInt32:
      return 4;
  }
  return 0;
}

TensorDesc TensorDesc::CreateContiguous(DataType data_type, const std::vector<std::size_t>& shape) {
  TensorDesc d;
  d.data_type_ = data_type;
  d.shape_ = shape;
  d.strides_.assign(shape.size(), 1);
  for (std::size_t i = shape.size(); i-- > 1;) d.strides_[i - 1] = d.strides_[i] * shape[i];  // row-major
  d.contiguous_ = true;
  return d;
}

TensorDesc TensorDesc::CreateStrided(DataType data_type, const std::vector<std::size_t>& shape,
                                     const std::vector<std::size_t>& strides) {
  TensorDesc d = CreateContiguous(data_type, shape);
  if (strides.size() == shape.size() && strides != d.strides_) {
    d.strides_ = strides;
    d.contiguous_ = false;
  }
  return d;
}

std::size_t TensorDesc::ElementCount() const {
  std::size_t n = 1;
  for (std::size_t s : shape_) n *= s;
  return n;
}

std::size_t TensorDesc::ByteSize() const {
  if (ElementCount() == 0) return 0;
  std::size_t last = 0;  // element offset of the last element
  for (std::size_t i = 0; i < shape_.size(); ++i) last += (shape_[i] - 1) * strides_[i];
  return (last + 1) * GetDataTypeSize(data_type_);
}

bool DeviceTensor::IsValid() const {
  return buffer_ != nullptr && byte_offset_ + desc_.ByteSize() <= buffer_->GetSizeBytes();
}

// ---- BufferArena (buffer_arena.cpp) ----
std::unique_ptr<BufferArena> BufferArena::CreateShared(const HipContext& context, std::size_t capacity_bytes,
                                                       const std::string& label, std::string* error_message) {
  auto buffer = HipBuffer::CreateShared(context, capacity_bytes, label, error_message);
  if (buffer == nullptr) return nullptr;
  return std::unique_ptr<BufferArena>(new BufferArena(std::move(buffer), capacity_bytes));
}

bool BufferArena::Allocate(std::size_t size_bytes, std::size_t alignment_bytes, BufferArenaSlice* slice,
                           std::string* error_message) {
  if (slice == nullptr) return Fail(error_message, "Arena allocation slice must not be null");
  const std::size_t a = std::max<std::size_t>(alignment_bytes, 1);
  const std::size_t start = (used_ + a - 1) / a * a;
  if (start + size_bytes > capacity_) return Fail(error_message, "BufferArena capacity exceeded");
  *slice = BufferArenaSlice{buffer_, start, size_bytes};
  used_ = start + size_bytes;
  peak_ = std::max(peak_, used_);
  for (ActiveScope& sc : active_scopes_) {
    sc.peak_used = std::max(sc.peak_used, used_);
    ++sc.allocations;
  }
  return true;
}

bool BufferArena::ResetToMark(BufferArenaMark mark, std::string* error_message) {
  if (mark > used_) return Fail(error_message, "BufferArena mark is ahead of current usage");
  used_ = mark;
  return true;
}

void BufferArena::ClearTelemetry() { telemetry_.clear(); }

void BufferArena::BeginScope(const std::string& scope_name) {
  if (!scope_name.empty()) active_scopes_.push_back(ActiveScope{scope_name, used_, used_, 0});
}

void BufferArena::EndScope() {
  if (active_scopes_.empty()) return;
  const ActiveScope sc = active_scopes_.back();
  active_scopes_.pop_back();
  const std::size_t delta = sc.peak_used - std::min(sc.peak_used, sc.start_used);
  auto it = std::find_if(telemetry_.begin(), telemetry_.end(),
                         [&sc](const BufferArenaScopeTelemetry& t) { return t.name == sc.name; });
  if (it == telemetry_.end()) {
    telemetry_.push_back(BufferArenaScopeTelemetry{sc.name, 1, delta, sc.peak_used, sc.allocations});
    return;
  }
  it->invocation_count += 1;
  it->peak_delta_bytes = std::max(it->peak_delta_bytes, delta);
  it->peak_used_bytes = std::max(it->peak_used_bytes, sc.peak_used);
  it->peak_allocation_count = std::max(it->peak_allocation_count, sc.allocations);
}

BufferArenaMarkGuard::BufferArenaMarkGuard(BufferArena* arena, const std::string& scope_name)
    : arena_(arena), has_scope_(!scope_name.empty()) {
  if (arena_ == nullptr) return;
  mark_ = arena_->GetMark();
  if (has_scope_) arena_->BeginScope(scope_name);
}

BufferArenaMarkGuard::~BufferArenaMarkGuard() {
  if (arena_ == nullptr) return;
  if (has_scope_) arena_->EndScope();
  std::string ignored;
  arena_->ResetToMark(mark_, &ignored);
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
  QwenCausalLMWeights views = ViewWeights(context, holder, params);
  *model = QwenCausalLM(std::move(holder), params, std::move(views));
  return true;
}

bool QwenModelLoader::LoadModel(const HipContext& context, const soc::ManifestData& manifest, QwenCausalLM* model,
                                std::string* error_message) {
  if (model == nullptr) return Fail(error_message, "QwenModelLoader requires a non-null model output");
  try {
    const soc::Qwen3Config c = soc::StartupValidator::ValidateManifest(manifest);
    QwenCausalLMParams p;
    p.vocab_size = c.vocab_size;
    p.hidden_size = c.hidden_size;
    p.num_hidden_layers = c.num_hidden_layers;
    p.num_attention_heads = c.num_attention_heads;
    p.num_key_value_heads = c.num_key_value_heads;
    p.head_dim = c.head_dim;
    p.intermediate_size = c.intermediate_size;
    p.max_position_embeddings = c.max_position_embeddings;
    p.rope_theta = static_cast<float>(c.rope_theta);
    p.rms_norm_eps = static_cast<float>(c.rms_norm_eps);
    p.tie_word_embeddings = c.tie_word_embeddings;
    const soc_qwen_config cfg = ToConfig(p);
    soc_model* m = nullptr;
    if (!Check(soc_model_create(context.handle(), &cfg, &m), error_message)) return false;
    auto holder = WrapModel(m);
    for (const auto& [name, shape] : soc::Qwen3TensorShapes(c)) {
      const std::vector<uint16_t> w = soc::WeightLoader::LoadFloat16(manifest, name, shape);
      if (!Check(soc_model_load_tensor(m, name.c_str(), w.data(), static_cast<int64_t>(w.size())), error_message))
        return false;
    }
    if (!Check(soc_model_finalize(m), error_message)) return false;
    QwenCausalLMWeights views = ViewWeights(context, holder, p);
    *model = QwenCausalLM(std::move(holder), p, std::move(views));
    return true;
  } catch (const std::exception& e) {
    return Fail(error_message, e.what());
  }
}

bool QwenModelLoader::LoadModelFromFile(const HipContext& context, const std::string& manifest_path,
                                        QwenCausalLM* model, std::string* error_message) {
  try {
    return LoadModel(context, soc::ManifestLoader::LoadFromFile(manifest_path), model, error_message);
  } catch (const std::exception& e) {
    return Fail(error_message, e.what());
  }
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
  QwenCausalLMWeights views = ViewWeights(context, holder, params);
  *model = QwenCausalLM(std::move(holder), params, std::move(views));
  return true;
}

// ---- KVCache (kv_cache.mm) ----
std::unique_ptr<KVCache> KVCache::CreateShared(const HipContext& context, std::size_t layer_count,
                                               std::size_t key_value_head_count, std::size_t head_dim,
                                               std::size_t max_sequence_length, const std::string&,
                                               std::string* error_message) {
  if (layer_count == 0 || key_value_head_count == 0 || head_dim == 0 || max_sequence_length == 0) {
    Fail(error_message, "KVCache dimensions must be non-zero");
    return nullptr;
  }
  soc_kv* kv = nullptr;
  if (!Check(soc_kv_create_dims(context.handle(), static_cast<int32_t>(layer_count),
                                static_cast<int32_t>(key_value_head_count), static_cast<int32_t>(head_dim), 1,
                                static_cast<int32_t>(max_sequence_length), &kv),
             error_message))
    return nullptr;
  std::shared_ptr<soc_kv> holder(kv, [](soc_kv* p) { soc_kv_destroy(p); });
  return std::unique_ptr<KVCache>(
      new KVCache(context, std::move(holder), layer_count, key_value_head_count, head_dim, max_sequence_length));
}

bool KVCache::Reserve(std::size_t sequence_length, std::string* error_message) {
  if (sequence_length > capacity_) return Fail(error_message, "KVCache reserve length exceeds max_sequence_length");
  return true;
}

bool KVCache::AppendPrefill(const HipContext&, std::size_t layer_index, const DeviceTensor& keys,
                            const DeviceTensor& values, std::string* error_message) {
  if (layer_index >= layer_count_) return Fail(error_message, "KVCache layer index is out of range");
  const std::size_t width = kv_heads_ * head_dim_;
  for (const DeviceTensor* t : {&keys, &values}) {
    const TensorDesc& d = t->GetDesc();
    if (!t->IsValid() || d.Rank() != 2 || !d.IsContiguous() ||
        (d.GetDataType() != DataType::kFloat32 && d.GetDataType() != DataType::kFloat16))
      return Fail(error_message, "KVCache append expects a valid rank-2 float32 or float16 tensor");
    if (d.GetShape()[1] != width)
      return Fail(error_message, "KVCache append tensor hidden size does not match cache configuration");
  }
  if (keys.GetDesc().GetShape() != values.GetDesc().GetShape() ||
      keys.GetDesc().GetDataType() != values.GetDesc().GetDataType())
    return Fail(error_message, "KVCache key/value append tensors must have matching shapes");
  const std::size_t rows = keys.GetDesc().GetShape()[0];
  if (sequence_lengths_[layer_index] + rows > capacity_)
    return Fail(error_message, "KVCache append would exceed max_sequence_length");
  const int32_t dtype = keys.GetDesc().GetDataType() == DataType::kFloat16 ? SOC_DTYPE_F16 : SOC_DTYPE_F32;
  if (!Check(soc_kv_append(kv_.get(), 0, static_cast<int32_t>(layer_index),
                           static_cast<int32_t>(sequence_lengths_[layer_index]), static_cast<int32_t>(rows),
                           keys.data(), values.data(), dtype),
             error_message))
    return false;
  sequence_lengths_[layer_index] += rows;
  // a forward attends over the positions every layer holds
  const std::size_t common = *std::min_element(sequence_lengths_.begin(), sequence_lengths_.end());
  return Check(soc_kv_set_length(kv_.get(), 0, static_cast<int32_t>(common)), error_message);
}

bool KVCache::AppendDecodeToken(const HipContext& context, std::size_t layer_index, const DeviceTensor& key,
                                const DeviceTensor& value, std::string* error_message) {
  if (key.GetDesc().Rank() != 2 || value.GetDesc().Rank() != 2 || key.GetDesc().GetShape()[0] != 1 ||
      value.GetDesc().GetShape()[0] != 1)
    return Fail(error_message, "KVCache decode append expects single-row key/value tensors");
  return AppendPrefill(context, layer_index, key, value, error_message);
}

KVCacheLayerView KVCache::ViewForLayer(std::size_t layer_index) const {
  if (layer_index >= layer_count_) return {};
  void* k = nullptr;
  void* v = nullptr;
  if (soc_kv_layer_planes(kv_.get(), 0, static_cast<int32_t>(layer_index), &k, &v) != SOC_OK) return {};
  const std::size_t n = sequence_lengths_[layer_index];
  const std::size_t bytes = kv_heads_ * capacity_ * head_dim_ * 2;
  const TensorDesc desc = TensorDesc::CreateStrided(DataType::kFloat16, {kv_heads_, n, head_dim_},
                                                    {capacity_ * head_dim_, head_dim_, 1});
  return {DeviceTensor(HipBuffer::Wrap(*context_, k, bytes, kv_), 0, desc),
          DeviceTensor(HipBuffer::Wrap(*context_, v, bytes, kv_), 0, desc), n};
}

void KVCache::OnForward(std::size_t rows) {
  for (std::size_t& n : sequence_lengths_) n += rows;
}

bool KVCache::LayersAligned() const {
  return std::all_of(sequence_lengths_.begin(), sequence_lengths_.end(),
                     [this](std::size_t n) { return n == sequence_lengths_[0]; });
}

// ---- QwenCausalLM (qwen_causal_lm.cpp) ----
QwenCausalLM::QwenCausalLM(QwenCausalLMWeights weights, QwenCausalLMParams params)
    : params_(params), weights_(std::move(weights)) {
  params_.num_hidden_layers = weights_.blocks.size();  // qwen_causal_lm.cpp:34: the layer count is the blocks'
  params_.tie_word_embeddings = weights_.tie_word_embeddings;
  const std::shared_ptr<HipBuffer>& eb = weights_.embed_tokens_weight.GetBuffer();
  if (eb == nullptr) {
    build_error_ = "QwenCausalLM weight model.embed_tokens.weight is not a valid device tensor";
    return;
  }
  const soc_qwen_config cfg = ToConfig(params_);
  soc_model* m = nullptr;
  if (soc_model_create(eb->context(), &cfg, &m) != SOC_OK) {
    build_error_ = soc_last_error();
    return;
  }
  std::shared_ptr<soc_model> holder = WrapModel(m);
  for (const WeightSlot& slot : WeightSlots(weights_, params_)) {
    const DeviceTensor& t = *slot.tensor;
    const TensorDesc& d = t.GetDesc();
    if (!t.IsValid()) {
      build_error_ = "QwenCausalLM weight " + slot.name + " is not a valid device tensor";
      return;
    }
    if (d.GetDataType() != DataType::kFloat32 && d.GetDataType() != DataType::kFloat16) {
      build_error_ = "QwenCausalLM weight " + slot.name + " must be float32 or float16";
      return;
    }
    if (!d.IsContiguous() || d.GetShape() != slot.shape) {
      build_error_ = "QwenCausalLM weight " + slot.name + " has shape " + ShapeText(d.GetShape()) + ", expected " +
                     ShapeText(slot.shape) + " (contiguous)";
      return;
    }
    const int32_t dtype = d.GetDataType() == DataType::kFloat32 ? SOC_DTYPE_F32 : SOC_DTYPE_F16;
    if (soc_model_load_tensor_device(m, slot.name.c_str(), t.data(), dtype, static_cast<int64_t>(d.ElementCount())) !=
        SOC_OK) {
      build_error_ = soc_last_error();
      return;
    }
  }
  if (soc_model_finalize(m) != SOC_OK) {
    build_error_ = soc_last_error();
    return;
  }
  model_ = std::move(holder);
}

// The forwards: token ids stay on the device (soc_forward checks them there), one host synchronisation per call, and
// the GPU time of the call is recorded inside it for the context's profiling snapshot.
bool QwenCausalLM::Forward(const HipContext& context, const DeviceTensor& token_ids, KVCache* kv_cache,
                           const DeviceTensor* hidden, const DeviceTensor* logits, std::size_t position_offset,
                           std::string* error_message) const {
  if (!IsValid())
    return Fail(error_message, build_error_.empty() ? "QwenCausalLM is not loaded" : build_error_);
  const TensorDesc& td = token_ids.GetDesc();
  if (!token_ids.IsValid() || td.GetDataType() != DataType::kInt32 || td.Rank() != 1 || td.GetShape()[0] == 0)
    return Fail(error_message, "token_ids must be a valid non-empty rank-1 int32 tensor");
  const std::size_t n = td.GetShape()[0];
  float* hp = nullptr;
  if (hidden != nullptr) {
    const TensorDesc& hd = hidden->GetDesc();
    if (!hidden->IsValid() || hd.GetDataType() != DataType::kFloat32 || hd.Rank() != 2)
      return Fail(error_message, "QwenCausalLM hidden forward expects rank-1 int32 token ids and rank-2 float32 output");
    if (hd.GetShape() != std::vector<std::size_t>{n, params_.hidden_size})
      return Fail(error_message, "QwenCausalLM hidden output shape must be [token_count, hidden_size]");
    hp = static_cast<float*>(hidden->data());
  }
  int32_t rows = 0;
  float* lp = nullptr;
  if (logits != nullptr && logits->GetBuffer() != nullptr) {
    const TensorDesc& ld = logits->GetDesc();
    if (!logits->IsValid() || ld.GetDataType() != DataType::kFloat32 || ld.Rank() != 2 ||
        ld.GetShape()[1] != vocab_size() || ld.GetShape()[0] == 0 || ld.GetShape()[0] > n)
      return Fail(error_message, "logits_output must be a valid float32 tensor [rows <= token count][vocab]");
    rows = static_cast<int32_t>(ld.GetShape()[0]);
    lp = static_cast<float*>(logits->data());
  }
  if (kv_cache != nullptr) {
    if (!kv_cache->LayersAligned())
      return Fail(error_message, "KV cache layers hold different numbers of positions");
    if (position_offset != kv_cache->GetSequenceLength())
      return Fail(error_message, "position_offset must equal the KV cache length");
  }
  soc_ctx* ctx = context.handle();
  if (!Check(soc_ctx_timer_start(ctx), error_message)) return false;
  const int rc = soc_forward(model_.get(), kv_cache != nullptr ? kv_cache->handle() : nullptr, 0,
                             static_cast<const int32_t*>(token_ids.data()), static_cast<int32_t>(n),
                             static_cast<int32_t>(position_offset), hp, rows, lp, nullptr);
  const std::string err = rc == SOC_OK ? std::string() : soc_last_error();
  float ms = 0.0f;
  const bool timed = soc_ctx_timer_stop(ctx, &ms) == SOC_OK;
  if (rc != SOC_OK) return Fail(error_message, err);
  if (timed) context.AddProfile(ms);
  if (kv_cache != nullptr) kv_cache->OnForward(n);
  return true;
}

bool QwenCausalLM::ForwardHidden(const HipContext& context, PipelineCache*, const DeviceTensor& token_ids,
                                 const DeviceTensor& output, BufferArena*, std::size_t position_offset,
                                 std::string* error_message) const {
  if (!token_ids.IsValid() || !output.IsValid())
    return Fail(error_message, "QwenCausalLM hidden forward expects valid tensors");
  return Forward(context, token_ids, nullptr, &output, nullptr, position_offset, error_message);
}

bool QwenCausalLM::ForwardHiddenCached(const HipContext& context, PipelineCache*, const DeviceTensor& token_ids,
                                       KVCache* kv_cache, const DeviceTensor& output, BufferArena*,
                                       std::size_t position_offset, std::string* error_message) const {
  if (kv_cache == nullptr) return Fail(error_message, "QwenCausalLM cached forward requires a KVCache");
  if (!token_ids.IsValid() || !output.IsValid())
    return Fail(error_message, "QwenCausalLM cached hidden forward expects valid tensors");
  return Forward(context, token_ids, kv_cache, &output, nullptr, position_offset, error_message);
}

bool QwenCausalLM::ForwardLogits(const HipContext& context, PipelineCache*, const DeviceTensor& token_ids,
                                 const DeviceTensor& logits_output, BufferArena*, std::size_t position_offset,
                                 std::string* error_message) const {
  return Forward(context, token_ids, nullptr, nullptr, &logits_output, position_offset, error_message);
}

bool QwenCausalLM::ForwardLogitsCached(const HipContext& context, PipelineCache*, const DeviceTensor& token_ids,
                                       KVCache* kv_cache, const DeviceTensor& logits_output, BufferArena*,
                                       std::size_t position_offset, std::string* error_message) const {
  if (kv_cache == nullptr) return Fail(error_message, "ForwardLogitsCached requires a KV cache");
  return Forward(context, token_ids, kv_cache, nullptr, &logits_output, position_offset, error_message);
}

// ---- CommandScheduler (command_scheduler.cpp:5-41: both paths are ForwardLogitsCached) ----
bool CommandScheduler::RunPrefill(const HipContext& context, PipelineCache* pipeline_cache, const QwenCausalLM& model,
                                  const DeviceTensor& token_ids, KVCache* kv_cache, const DeviceTensor& logits_output,
                                  BufferArena* temporary_arena, std::size_t position_offset,
                                  std::string* error_message) const {
  return model.ForwardLogitsCached(context, pipeline_cache, token_ids, kv_cache, logits_output, temporary_arena,
                                   position_offset, error_message);
}

bool CommandScheduler::RunDecode(const HipContext& context, PipelineCache* pipeline_cache, const QwenCausalLM& model,
                                 const DeviceTensor& token_ids, KVCache* kv_cache, const DeviceTensor& logits_output,
                                 BufferArena* temporary_arena, std::size_t position_offset,
                                 std::string* error_message) const {
  return model.ForwardLogitsCached(context, pipeline_cache, token_ids, kv_cache, logits_output, temporary_arena,
                                   position_offset, error_message);
}

// ---- Sampler (sampler.cpp:14-71; candidates found on the device by soc_sample_topk) ----
bool Sampler::SampleFromLogits(const DeviceTensor& logits, std::size_t row_index, int* token_id,
                               std::vector<float>* top_logits, std::vector<int>* top_token_ids,
                               std::string* error_message) const {
  if (token_id == nullptr) return Fail(error_message, "Sampler requires a non-null token_id output");
  const TensorDesc& d = logits.GetDesc();
  if (!logits.IsValid() || d.GetDataType() != DataType::kFloat32 || d.Rank() != 2)
    return Fail(error_message, "Sampler expects a valid rank-2 float32 logits tensor");
  if (row_index >= d.GetShape()[0]) return Fail(error_message, "Sampler row_index is out of range");
  const std::size_t vocab = d.GetShape()[1];
  const std::size_t k = std::max<std::size_t>(1, std::min<std::size_t>(config_.top_k, vocab));
  std::vector<int32_t> ids(k);
  std::vector<float> vals(k);
  int32_t tok = -1;
  const float* row = static_cast<const float*>(logits.data()) + row_index * vocab;
  if (!Check(soc_sample_topk(logits.GetBuffer()->context(), row, static_cast<int32_t>(vocab),
                             static_cast<int32_t>(k), config_.temperature, &tok, ids.data(), vals.data()),
             error_message))
    return false;
  *token_id = tok;
  if (top_logits) top_logits->assign(vals.begin(), vals.end());
  if (top_token_ids) top_token_ids->assign(ids.begin(), ids.end());
  return true;
}

// ---- GenerationContext (generation_context.cpp) ----
GenerationContext::GenerationContext(QwenCausalLM model, Sampler sampler, CommandScheduler scheduler,
                                     std::size_t max_sequence_length)
    : model_(std::move(model)),
      sampler_(sampler),
      scheduler_(scheduler),
      max_sequence_length_(max_sequence_length) {}

bool GenerationContext::EnsureLogitsBuffer(const HipContext& context, std::string* error_message) {
  if (logits_buffer_ != nullptr) return true;
  logits_buffer_ = HipBuffer::CreateShared(context, model_.vocab_size() * 4, "generation_logits", error_message);
  return logits_buffer_ != nullptr;
}

bool GenerationContext::UploadTokenIds(const HipContext& context, const std::vector<int>& token_ids,
                                       DeviceTensor* token_tensor, std::string* error_message) {
  const std::size_t bytes = token_ids.size() * 4;
  if (token_buffer_ == nullptr || token_buffer_->GetSizeBytes() < bytes) {
    token_buffer_ = HipBuffer::CreateShared(context, std::max<std::size_t>(bytes, 256), "generation_tokens",
                                            error_message);
    if (token_buffer_ == nullptr) return false;
  }
  // queued without waiting: the forward that reads the ids synchronises the stream before the next upload replaces
  // uploaded_ids_, the copy's source
  uploaded_ids_ = token_ids;
  if (!Check(soc_buffer_write_async(context.handle(), token_buffer_->data(), uploaded_ids_.data(), bytes),
             error_message))
    return false;
  *token_tensor = DeviceTensor(token_buffer_, 0, TensorDesc::CreateContiguous(DataType::kInt32, {token_ids.size()}));
  return true;
}

bool GenerationContext::Prefill(const HipContext& context, PipelineCache* pipeline_cache,
                                const std::vector<int>& token_ids, BufferArena* temporary_arena,
                                std::string* error_message) {
  if (token_ids.empty()) return Fail(error_message, "GenerationContext prefill requires at least one token");
  Reset();
  prompt_token_ids_ = token_ids;
  running_token_ids_ = token_ids;
  kv_cache_ = KVCache::CreateShared(context, model_.num_layers(), model_.num_key_value_heads(), model_.head_dim(),
                                    max_sequence_length_, "generation_kv_cache", error_message);
  if (kv_cache_ == nullptr) return false;
  if (!EnsureLogitsBuffer(context, error_message)) return false;
  DeviceTensor tokens;
  if (!UploadTokenIds(context, token_ids, &tokens, error_message)) return false;
  // generation samples the last row only: the logits tensor holds that row
  const DeviceTensor logits(logits_buffer_, 0, TensorDesc::CreateContiguous(DataType::kFloat32, {1, model_.vocab_size()}));
  return scheduler_.RunPrefill(context, pipeline_cache, model_, tokens, kv_cache_.get(), logits, temporary_arena, 0,
                               error_message);
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
  if (!EnsureLogitsBuffer(context, error_message)) return false;
  DeviceTensor tokens;
  if (!UploadTokenIds(context, std::vector<int>{last_token_id}, &tokens, error_message)) return false;
  const DeviceTensor logits(logits_buffer_, 0, TensorDesc::CreateContiguous(DataType::kFloat32, {1, model_.vocab_size()}));
  if (!scheduler_.RunDecode(context, pipeline_cache, model_, tokens, kv_cache_.get(), logits, temporary_arena,
                            running_token_ids_.size() - 1, error_message))
    return false;
  if (!sampler_.SampleFromLogits(logits, 0, &result->token_id, &result->top_logits, &result->top_token_ids,
                                 error_message))
    return false;
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
  GenerationStepResult first;
  const DeviceTensor logits(logits_buffer_, 0, TensorDesc::CreateContiguous(DataType::kFloat32, {1, model_.vocab_size()}));
  if (!sampler_.SampleFromLogits(logits, 0, &first.token_id, &first.top_logits, &first.top_token_ids, error_message))
    return false;
  generated_token_ids->push_back(first.token_id);
  running_token_ids_.push_back(first.token_id);
  if (eos_token_id >= 0 && first.token_id == eos_token_id) return true;
  int last = first.token_id;
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
}

// ---- RuntimePipeline (Mac/cpu/src/runtime_pipeline.cpp) ----
bool RuntimePipeline::LoadBundle(const HipContext& context, const std::string& manifest_path, RuntimeBundle* bundle,
                                 std::string* error_message) {
  if (bundle == nullptr) return Fail(error_message, "RuntimePipeline requires a non-null bundle output");
  try {
    RuntimeBundle b;
    b.manifest = soc::ManifestLoader::LoadFromFile(manifest_path);
    b.tokenizer_runtime = soc::TokenizerRuntimeLoader::LoadFromFile(b.manifest.tokenizer_runtime_file);
    soc::StartupValidator::ValidateManifestAndTokenizer(b.manifest, b.tokenizer_runtime);
    if (!QwenModelLoader::LoadModel(context, b.manifest, &b.model, error_message)) return false;
    *bundle = std::move(b);
    return true;
  } catch (const std::exception& e) {
    return Fail(error_message, e.what());
  }
}

RuntimeGenerationOptions RuntimePipeline::GenerationOptionsFromManifest(const soc::ManifestData& manifest) {
  RuntimeGenerationOptions o;
  const soc::JsonValue& g = manifest.generation_config;
  if (!g.is_object()) return o;
  if (const soc::JsonValue* v = g.find("max_new_tokens")) o.max_new_tokens = static_cast<std::size_t>(v->as_int64());
  if (const soc::JsonValue* v = g.find("temperature")) o.sampler.temperature = static_cast<float>(v->as_number());
  if (const soc::JsonValue* v = g.find("top_k")) o.sampler.top_k = static_cast<std::size_t>(v->as_int64());
  if (const soc::JsonValue* v = g.find("eos_token_id")) {
    if (!v->is_array())
      o.eos_token_id = v->as_int();
    else if (!v->as_array().empty())
      o.eos_token_id = v->as_array().front().as_int();  // a list names several; the first one stops generation
  }
  if (const soc::JsonValue* v = g.find("max_length")) o.max_sequence_length = static_cast<std::size_t>(v->as_int64());
  return o;
}

std::string RuntimePipeline::PreparePrompt(const soc::TokenizerRuntimeData& tokenizer_runtime, const std::string& prompt,
                                           const RuntimePromptOptions& options) {
  if (!options.apply_chat_template) return prompt;
  return soc::Qwen3TemplateBuilder(tokenizer_runtime.template_runtime)
      .BuildPrompt({soc::ChatMessage{"user", prompt}}, options.add_generation_prompt, options.enable_thinking,
                   options.system_prompt);
}

}  // namespace soc::gpu
