// assets.h - the model bundle on disk: JSON values, the export manifest, the Qwen3 config and tensor files.
//
// The bundle is the reference's export format (Mac/cpu/header/runtime_assets.h, json_value.h, json_parser.h,
// qwen3_config.h, startup_validator.h, weight_loader.h): a manifest.json whose "tensors" list names one raw
// little-endian file per tensor (dtype float32, float16 or bfloat16, row-major shape, byte_size) relative to the
// manifest, plus the Hugging Face config under "config". The classes keep the reference's names and throw
// std::runtime_error with the reference's messages, as its CPU-side loaders do; the GPU model loader
// (soc::gpu::QwenModelLoader, soc/gpu/runtime.h) turns those into bool + message.
#pragma once

#include <cstddef>
#include <cstdint>
#include <string>
#include <map>
#include <memory>
#include <vector>

namespace soc {

class JsonValue {  // json_value.h
 public:
  enum class Type { Null, Bool, Number, String, Array, Object };
  using Array = std::vector<JsonValue>;
  using Object = std::map<std::string, JsonValue>;

  JsonValue() = default;
  explicit JsonValue(bool b) : type_(Type::Bool), bool_(b) {}
  explicit JsonValue(double n) : type_(Type::Number), number_(n) {}
  explicit JsonValue(std::string s) : type_(Type::String), string_(std::move(s)) {}
  explicit JsonValue(Array a);
  explicit JsonValue(Object o);

  Type type() const { return type_; }
  bool is_null() const { return type_ == Type::Null; }
  bool is_bool() const { return type_ == Type::Bool; }
  bool is_number() const { return type_ == Type::Number; }
  bool is_string() const { return type_ == Type::String; }
  bool is_array() const { return type_ == Type::Array; }
  bool is_object() const { return type_ == Type::Object; }

  bool as_bool() const;
  double as_number() const;
  int as_int() const;
  std::int64_t as_int64() const;
  const std::string& as_string() const;
  const Array& as_array() const;
  const Object& as_object() const;

  bool contains(const std::string& key) const;
  const JsonValue& at(const std::string& key) const;  // throws when absent
  const JsonValue* find(const std::string& key) const;

 private:
  Type type_ = Type::Null;
  bool bool_ = false;
  double number_ = 0.0;
  std::string string_;
  std::shared_ptr<const Array> array_;  // values are immutable once parsed: copies share them
  std::shared_ptr<const Object> object_;
};

class JsonParser {  // json_parser.h
 public:
  static JsonValue Parse(const std::string& text);
  static JsonValue ParseFile(const std::string& path);
};

struct TensorRecord {  // runtime_assets.h:10-17
  std::string name;
  std::string file;  // resolved against the manifest's directory
  std::string dtype;
  std::vector<std::size_t> shape;
  std::size_t byte_size = 0;
  std::string source_shard;
};

struct ManifestData {  // runtime_assets.h:19-32
  std::string format;
  int format_version = 0;
  std::string model_id;
  std::string source_dir;
  std::string export_dtype;
  std::string manifest_dir;
  std::string tokenizer_runtime_file;
  JsonValue config;
  JsonValue generation_config;
  std::vector<TensorRecord> tensors;

  const TensorRecord& FindTensor(const std::string& name) const;  // throws "missing tensor in manifest: <name>"
};

class ManifestLoader {  // runtime_assets.cpp:138-168
 public:
  static ManifestData LoadFromFile(const std::string& manifest_path);
};

struct Qwen3Config {  // qwen3_config.h
  std::string model_type;
  std::size_t hidden_size = 0;
  std::size_t intermediate_size = 0;
  std::size_t num_hidden_layers = 0;
  std::size_t num_attention_heads = 0;
  std::size_t num_key_value_heads = 0;
  std::size_t head_dim = 0;
  double rms_norm_eps = 0.0;
  double rope_theta = 0.0;
  bool tie_word_embeddings = false;
  std::string torch_dtype;
  std::size_t vocab_size = 0;
  std::size_t max_position_embeddings = 0;  // config value when present, else kDefaultMaxPositions

  static constexpr std::size_t kDefaultMaxPositions = 32768;
  static Qwen3Config FromJson(const JsonValue& config_json);
  void Validate() const;
};

struct TokenizerRuntimeData;  // soc/tokenizer.h

class StartupValidator {  // startup_validator.h:8-17
 public:
  static Qwen3Config ValidateManifest(const ManifestData& manifest);  // startup_validator.cpp:5-23
  // The tokenizer runtime's format, chat boundary tokens, BPE model and byte table (startup_validator.cpp:25-72),
  // and its vocabulary against the model config (:74-100). Defined with the tokenizer.
  static void ValidateTokenizerRuntime(const TokenizerRuntimeData& tokenizer_runtime);
  static void ValidateManifestAndTokenizer(const ManifestData& manifest, const TokenizerRuntimeData& tokenizer_runtime);
};

// Tensor files (weight_loader.cpp:17-30): checks byte_size against dtype and shape and the file against byte_size.
class WeightLoader {
 public:
  static std::size_t DTypeByteWidth(const std::string& dtype);  // throws for an unknown dtype
  static bool DTypeIsFloatLike(const std::string& dtype);       // float32, float16, bfloat16
  // The tensor as fp16 bits (float16 as stored; float32 and bfloat16 rounded to nearest even), after checking
  // that it is floating point and has `expected_shape` (qwen_model_loader.cpp:17-25).
  static std::vector<uint16_t> LoadFloat16(const ManifestData& manifest, const std::string& name,
                                           const std::vector<std::size_t>& expected_shape);
};

// Names and shapes of every weight a Qwen3 model of this config needs (qwen_model_loader.cpp:35-93), in load order.
std::vector<std::pair<std::string, std::vector<std::size_t>>> Qwen3TensorShapes(const Qwen3Config& config);

}  // namespace soc
