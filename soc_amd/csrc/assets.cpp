// assets.cpp - JSON, the export manifest, the Qwen3 config and tensor files of a model bundle (include/soc/assets.h),
// and the C entry points that read a bundle (soc_bundle_*). Host only; soc_model_load_bundle is in model_bundle.cpp.
// Follows Mac/cpu/src/json_parser.cpp (messages), runtime_assets.cpp:138-168, qwen3_config.cpp:20-67,
// startup_validator.cpp:5-23, weight_loader.cpp:17-30, qwen_model_loader.cpp:17-93.
#include <cmath>
#include <cstdio>
#include <cstring>
#include <filesystem>
#include <fstream>
#include <memory>
#include <sstream>
#include <stdexcept>

#include "soc/assets.h"
#include "soc_hip.h"
#include "status.h"

namespace soc {

// ---- JsonValue ----
JsonValue::JsonValue(Array a) : type_(Type::Array), array_(std::make_shared<const Array>(std::move(a))) {}
JsonValue::JsonValue(Object o) : type_(Type::Object), object_(std::make_shared<const Object>(std::move(o))) {}

bool JsonValue::as_bool() const {
  if (type_ != Type::Bool) throw std::runtime_error("JSON value is not a bool");
  return bool_;
}
double JsonValue::as_number() const {
  if (type_ != Type::Number) throw std::runtime_error("JSON value is not a number");
  return number_;
}
// Integers are the number truncated toward zero, as a cast does; a number outside the target range is an error
// rather than an out-of-range conversion.
int JsonValue::as_int() const {
  const double d = as_number();
  if (!(d > -2147483649.0 && d < 2147483648.0)) throw std::runtime_error("JSON number out of int range");
  return static_cast<int>(d);
}
std::int64_t JsonValue::as_int64() const {
  const double d = as_number();
  if (!(d >= -9223372036854775808.0 && d < 9223372036854775808.0))
    throw std::runtime_error("JSON number out of int64 range");
  return static_cast<std::int64_t>(d);
}
const std::string& JsonValue::as_string() const {
  if (type_ != Type::String) throw std::runtime_error("JSON value is not a string");
  return string_;
}
const JsonValue::Array& JsonValue::as_array() const {
  if (type_ != Type::Array) throw std::runtime_error("JSON value is not an array");
  return *array_;
}
const JsonValue::Object& JsonValue::as_object() const {
  if (type_ != Type::Object) throw std::runtime_error("JSON value is not an object");
  return *object_;
}
bool JsonValue::contains(const std::string& key) const { return find(key) != nullptr; }
const JsonValue* JsonValue::find(const std::string& key) const {
  if (type_ != Type::Object) return nullptr;
  auto it = object_->find(key);
  return it == object_->end() ? nullptr : &it->second;
}
const JsonValue& JsonValue::at(const std::string& key) const {
  as_object();  // "JSON value is not an object"
  const JsonValue* v = find(key);
  if (v == nullptr) throw std::runtime_error("missing JSON object key: " + key);
  return *v;
}

// ---- JsonParser: recursive descent over the text ----
namespace {

class Reader {
 public:
  explicit Reader(const std::string& t) : t_(t) {}

  JsonValue Document() {
    JsonValue v = Value();
    Skip();
    if (i_ != t_.size()) throw std::runtime_error("unexpected trailing JSON content");
    return v;
  }

 private:
  void Skip() {
    while (i_ < t_.size() && (t_[i_] == ' ' || t_[i_] == '\t' || t_[i_] == '\n' || t_[i_] == '\r')) ++i_;
  }
  char Peek() {
    Skip();
    if (i_ >= t_.size()) throw std::runtime_error("unexpected end of JSON input");
    return t_[i_];
  }
  bool Consume(const char* lit) {
    const size_t n = std::strlen(lit);
    if (t_.compare(i_, n, lit) != 0) return false;
    i_ += n;
    return true;
  }

  JsonValue Value() {
    const char c = Peek();
    if (c == '{' || c == '[') {
      if (++depth_ > kMaxDepth) throw std::runtime_error("JSON nesting too deep");
      JsonValue v = c == '{' ? Object() : ArrayValue();
      --depth_;
      return v;
    }
    if (c == '"') return JsonValue(String());
    if (c == '-' || (c >= '0' && c <= '9')) return Number();
    if (c == 't' || c == 'f' || c == 'n') {
      if (Consume("true")) return JsonValue(true);
      if (Consume("false")) return JsonValue(false);
      if (Consume("null")) return JsonValue();
      throw std::runtime_error("invalid JSON literal");
    }
    throw std::runtime_error("unexpected token in JSON input");
  }

  JsonValue Number() {
    const size_t start = i_;
    if (t_[i_] == '-') ++i_;
    while (i_ < t_.size() && std::strchr("0123456789+-.eE", t_[i_]) != nullptr) ++i_;
    const std::string s = t_.substr(start, i_ - start);
    char* end = nullptr;
    const double d = std::strtod(s.c_str(), &end);
    if (end == s.c_str() || *end != '\0') throw std::runtime_error("unexpected token in JSON input");
    return JsonValue(d);
  }

  static void AppendUtf8(std::string& out, uint32_t cp) {
    if (cp < 0x80) {
      out += static_cast<char>(cp);
    } else if (cp < 0x800) {
      out += static_cast<char>(0xC0 | (cp >> 6));
      out += static_cast<char>(0x80 | (cp & 0x3F));
    } else if (cp < 0x10000) {
      out += static_cast<char>(0xE0 | (cp >> 12));
      out += static_cast<char>(0x80 | ((cp >> 6) & 0x3F));
      out += static_cast<char>(0x80 | (cp & 0x3F));
    } else {
      out += static_cast<char>(0xF0 | (cp >> 18));
      out += static_cast<char>(0x80 | ((cp >> 12) & 0x3F));
      out += static_cast<char>(0x80 | ((cp >> 6) & 0x3F));
      out += static_cast<char>(0x80 | (cp & 0x3F));
    }
  }

  uint32_t Hex4() {
    if (i_ + 4 > t_.size()) throw std::runtime_error("invalid unicode escape in JSON string");
    uint32_t v = 0;
    for (int k = 0; k < 4; ++k) {
      const char h = t_[i_++];
      v <<= 4;
      if (h >= '0' && h <= '9') v |= h - '0';
      else if (h >= 'a' && h <= 'f') v |= h - 'a' + 10;
      else if (h >= 'A' && h <= 'F') v |= h - 'A' + 10;
      else throw std::runtime_error("invalid unicode escape in JSON string");
    }
    return v;
  }

  std::string String() {
    if (Peek() != '"') throw std::runtime_error("expected JSON string");
    ++i_;
    std::string out;
    while (i_ < t_.size()) {
      const char c = t_[i_++];
      if (c == '"') return out;
      if (c != '\\') {
        out += c;
        continue;
      }
      if (i_ >= t_.size()) break;
      const char e = t_[i_++];
      switch (e) {
        case '"': out += '"'; break;
        case '\\': out += '\\'; break;
        case '/': out += '/'; break;
        case 'b': out += '\b'; break;
        case 'f': out += '\f'; break;
        case 'n': out += '\n'; break;
        case 'r': out += '\r'; break;
        case 't': out += '\t'; break;
        case 'u': {
          uint32_t cp = Hex4();
          if (cp >= 0xD800 && cp <= 0xDBFF) {  // surrogate pair
            if (!Consume("\\u")) throw std::runtime_error("invalid unicode escape in JSON string");
            const uint32_t lo = Hex4();
            if (lo < 0xDC00 || lo > 0xDFFF) throw std::runtime_error("invalid unicode escape in JSON string");
            cp = 0x10000 + ((cp - 0xD800) << 10) + (lo - 0xDC00);
          }
          AppendUtf8(out, cp);
          break;
        }
        default:
          throw std::runtime_error("unsupported JSON escape sequence");
      }
    }
    throw std::runtime_error("unterminated JSON string");
  }

  JsonValue ArrayValue() {
    if (Peek() != '[') throw std::runtime_error("expected JSON array");
    ++i_;
    JsonValue::Array a;
    if (Peek() == ']') {
      ++i_;
      return JsonValue(std::move(a));
    }
    while (true) {
      a.push_back(Value());
      Skip();
      if (i_ >= t_.size()) throw std::runtime_error("unterminated JSON array");
      if (t_[i_] == ']') {
        ++i_;
        return JsonValue(std::move(a));
      }
      if (t_[i_] != ',') throw std::runtime_error("expected comma in JSON array");
      ++i_;
    }
  }

  JsonValue Object() {
    if (Peek() != '{') throw std::runtime_error("expected JSON object");
    ++i_;
    JsonValue::Object o;
    if (Peek() == '}') {
      ++i_;
      return JsonValue(std::move(o));
    }
    while (true) {
      std::string key = String();
      if (Peek() != ':') throw std::runtime_error("expected colon in JSON object");
      ++i_;
      o[key] = Value();
      Skip();
      if (i_ >= t_.size()) throw std::runtime_error("unterminated JSON object");
      if (t_[i_] == '}') {
        ++i_;
        return JsonValue(std::move(o));
      }
      if (t_[i_] != ',') throw std::runtime_error("expected comma in JSON object");
      ++i_;
    }
  }

  static constexpr int kMaxDepth = 256;  // bundle files nest a few levels; bounded recursion keeps the stack safe
  const std::string& t_;
  size_t i_ = 0;
  int depth_ = 0;
};

}  // namespace

JsonValue JsonParser::Parse(const std::string& text) { return Reader(text).Document(); }

JsonValue JsonParser::ParseFile(const std::string& path) {
  std::ifstream f(path, std::ios::binary);
  if (!f) throw std::runtime_error("failed to open JSON file: " + path);
  std::stringstream ss;
  ss << f.rdbuf();
  return Parse(ss.str());
}

// ---- manifest ----
const TensorRecord& ManifestData::FindTensor(const std::string& name) const {
  for (const TensorRecord& t : tensors)
    if (t.name == name) return t;
  throw std::runtime_error("missing tensor in manifest: " + name);
}

ManifestData ManifestLoader::LoadFromFile(const std::string& manifest_path) {
  namespace fs = std::filesystem;
  const JsonValue root = JsonParser::ParseFile(manifest_path);
  const fs::path dir = fs::path(manifest_path).lexically_normal().parent_path();
  auto resolve = [&dir](const std::string& rel) { return (dir / rel).lexically_normal().string(); };
  ManifestData m;
  m.format = root.at("format").as_string();
  m.format_version = root.at("format_version").as_int();
  const JsonValue* id = root.find("model_id");
  m.model_id = id != nullptr && !id->is_null() ? id->as_string() : "";
  m.source_dir = root.contains("source_dir") ? root.at("source_dir").as_string() : "";
  m.export_dtype = root.at("export_dtype").as_string();
  m.manifest_dir = dir.string();
  m.tokenizer_runtime_file =
      root.contains("tokenizer_runtime_file") ? resolve(root.at("tokenizer_runtime_file").as_string()) : "";
  if (root.contains("config")) m.config = root.at("config");
  if (root.contains("generation_config")) m.generation_config = root.at("generation_config");
  for (const JsonValue& tv : root.at("tensors").as_array()) {
    TensorRecord t;
    t.name = tv.at("name").as_string();
    t.file = resolve(tv.at("file").as_string());
    t.dtype = tv.at("dtype").as_string();
    for (const JsonValue& d : tv.at("shape").as_array()) t.shape.push_back(static_cast<std::size_t>(d.as_int64()));
    t.byte_size = static_cast<std::size_t>(tv.at("byte_size").as_int64());
    t.source_shard = tv.at("source_shard").as_string();
    m.tensors.push_back(std::move(t));
  }
  return m;
}

// ---- config and validation ----
Qwen3Config Qwen3Config::FromJson(const JsonValue& j) {
  Qwen3Config c;
  auto size = [&j](const char* k) { return static_cast<std::size_t>(j.at(k).as_int64()); };
  c.model_type = j.at("model_type").as_string();
  c.hidden_size = size("hidden_size");
  c.intermediate_size = size("intermediate_size");
  c.num_hidden_layers = size("num_hidden_layers");
  c.num_attention_heads = size("num_attention_heads");
  c.num_key_value_heads = size("num_key_value_heads");
  c.head_dim = size("head_dim");
  c.rms_norm_eps = j.at("rms_norm_eps").as_number();
  c.rope_theta = j.at("rope_theta").as_number();
  c.tie_word_embeddings = j.at("tie_word_embeddings").as_bool();
  c.torch_dtype = j.at("torch_dtype").as_string();
  c.vocab_size = size("vocab_size");
  const JsonValue* mp = j.find("max_position_embeddings");
  c.max_position_embeddings =
      mp != nullptr && !mp->is_null() ? static_cast<std::size_t>(mp->as_int64()) : kDefaultMaxPositions;
  c.Validate();
  return c;
}

void Qwen3Config::Validate() const {
  if (model_type != "qwen3") throw std::runtime_error("config model_type must be qwen3");
  if (hidden_size == 0 || intermediate_size == 0 || num_hidden_layers == 0)
    throw std::runtime_error("qwen3 config dimensions must be non-zero");
  if (num_attention_heads == 0 || num_key_value_heads == 0 || head_dim == 0)
    throw std::runtime_error("qwen3 attention dimensions must be non-zero");
  if (hidden_size % num_attention_heads != 0)
    throw std::runtime_error("hidden_size must be divisible by num_attention_heads");
  if (num_attention_heads % num_key_value_heads != 0)
    throw std::runtime_error("num_attention_heads must be divisible by num_key_value_heads");
  if (rms_norm_eps <= 0.0 || rope_theta <= 0.0)
    throw std::runtime_error("qwen3 normalization and rope parameters must be positive");
  if (vocab_size == 0) throw std::runtime_error("vocab_size must be non-zero");
  if (torch_dtype.empty()) throw std::runtime_error("torch_dtype must not be empty");
}

Qwen3Config StartupValidator::ValidateManifest(const ManifestData& m) {
  if (m.format != "soc.cpp.llm_export") throw std::runtime_error("manifest format must be soc.cpp.llm_export");
  if (m.format_version < 2) throw std::runtime_error("manifest format_version must be at least 2");
  if (!m.config.is_object()) throw std::runtime_error("manifest config must be a JSON object");
  if (m.tensors.empty()) throw std::runtime_error("manifest must contain at least one tensor");
  if (m.tokenizer_runtime_file.empty()) throw std::runtime_error("manifest must reference tokenizer_runtime_file");
  return Qwen3Config::FromJson(m.config);
}

// ---- tensor files ----
std::size_t WeightLoader::DTypeByteWidth(const std::string& dtype) {
  if (dtype == "float32" || dtype == "int32") return 4;
  if (dtype == "float16" || dtype == "bfloat16" || dtype == "uint16") return 2;
  if (dtype == "int64") return 8;
  if (dtype == "int8" || dtype == "uint8") return 1;
  throw std::runtime_error("unsupported dtype: " + dtype);
}

bool WeightLoader::DTypeIsFloatLike(const std::string& dtype) {
  return dtype == "float32" || dtype == "float16" || dtype == "bfloat16";
}

namespace {
std::size_t Product(const std::vector<std::size_t>& v) {
  std::size_t p = 1;
  for (std::size_t x : v) p *= x;
  return p;
}
}  // namespace

std::vector<uint16_t> WeightLoader::LoadFloat16(const ManifestData& manifest, const std::string& name,
                                                const std::vector<std::size_t>& expected_shape) {
  const TensorRecord& r = manifest.FindTensor(name);
  const std::size_t n = Product(r.shape);
  if (n * DTypeByteWidth(r.dtype) != r.byte_size)
    throw std::runtime_error("tensor record byte_size does not match dtype and shape for: " + name);
  if (!DTypeIsFloatLike(r.dtype))
    throw std::runtime_error("model loader requires floating-point weights for: " + name);
  if (r.shape != expected_shape) throw std::runtime_error("model loader encountered unexpected shape for: " + name);
  std::ifstream f(r.file, std::ios::binary);
  if (!f) throw std::runtime_error("failed to open tensor file: " + r.file);
  f.seekg(0, std::ios::end);
  if (static_cast<std::size_t>(f.tellg()) < r.byte_size)
    throw std::runtime_error("tensor file is smaller than expected byte_size for: " + name);
  f.seekg(0);
  std::vector<uint16_t> out(n);
  if (r.dtype == "float16") {
    f.read(reinterpret_cast<char*>(out.data()), static_cast<std::streamsize>(n * 2));
  } else {
    std::vector<uint8_t> raw(r.byte_size);
    f.read(reinterpret_cast<char*>(raw.data()), static_cast<std::streamsize>(raw.size()));
    for (std::size_t i = 0; i < n; ++i) {
      uint32_t bits;
      if (r.dtype == "float32") {
        std::memcpy(&bits, raw.data() + 4 * i, 4);
      } else {  // bfloat16: the upper half of an fp32
        uint16_t b;
        std::memcpy(&b, raw.data() + 2 * i, 2);
        bits = static_cast<uint32_t>(b) << 16;
      }
      float v;
      std::memcpy(&v, &bits, 4);
      out[i] = soc_f64_to_f16_rne(static_cast<double>(v));  // exact in double, one rounding to fp16
      // the device keeps fp16: a finite weight beyond fp16's range (|w| >= 65520 rounds to inf) is refused rather
      // than stored as inf; non-finite source values pass through unchanged, as the reference's fp32 copy keeps them
      if (std::isfinite(v) && (out[i] & 0x7c00u) == 0x7c00u)
        throw std::runtime_error("tensor value outside the float16 range (|w| >= 65520) in: " + name);
    }
  }
  if (!f) throw std::runtime_error("failed to read tensor file: " + r.file);
  return out;
}

std::vector<std::pair<std::string, std::vector<std::size_t>>> Qwen3TensorShapes(const Qwen3Config& c) {
  const std::size_t H = c.hidden_size, I = c.intermediate_size, q = c.num_attention_heads * c.head_dim,
                    kv = c.num_key_value_heads * c.head_dim;
  std::vector<std::pair<std::string, std::vector<std::size_t>>> out;
  out.push_back({"model.embed_tokens.weight", {c.vocab_size, H}});
  for (std::size_t l = 0; l < c.num_hidden_layers; ++l) {
    const std::string p = "model.layers." + std::to_string(l) + ".";
    out.push_back({p + "input_layernorm.weight", {H}});
    out.push_back({p + "self_attn.q_proj.weight", {q, H}});
    out.push_back({p + "self_attn.k_proj.weight", {kv, H}});
    out.push_back({p + "self_attn.v_proj.weight", {kv, H}});
    out.push_back({p + "self_attn.o_proj.weight", {H, q}});
    out.push_back({p + "self_attn.q_norm.weight", {c.head_dim}});
    out.push_back({p + "self_attn.k_norm.weight", {c.head_dim}});
    out.push_back({p + "post_attention_layernorm.weight", {H}});
    out.push_back({p + "mlp.gate_proj.weight", {I, H}});
    out.push_back({p + "mlp.up_proj.weight", {I, H}});
    out.push_back({p + "mlp.down_proj.weight", {H, I}});
  }
  out.push_back({"model.norm.weight", {H}});
  if (!c.tie_word_embeddings) out.push_back({"lm_head.weight", {c.vocab_size, H}});
  return out;
}

}  // namespace soc

// ---- C entry points ----
struct soc_bundle {
  soc::ManifestData manifest;
  soc::Qwen3Config config;
};

extern "C" {

int soc_bundle_open(const char* manifest_path, soc_bundle** out) {
  if (manifest_path == nullptr || out == nullptr) return soc::fail(SOC_ERR_INVALID, "null argument");
  *out = nullptr;
  try {
    std::unique_ptr<soc_bundle> b(new soc_bundle());
    b->manifest = soc::ManifestLoader::LoadFromFile(manifest_path);
    b->config = soc::StartupValidator::ValidateManifest(b->manifest);
    *out = b.release();
    return SOC_OK;
  } catch (const std::exception& e) {
    return soc::fail(SOC_ERR_INVALID, e.what());
  }
}

int soc_bundle_close(soc_bundle* b) {
  delete b;
  return SOC_OK;
}

int soc_bundle_config(const soc_bundle* b, soc_qwen_config* out) {
  if (b == nullptr || out == nullptr) return soc::fail(SOC_ERR_INVALID, "null argument");
  const soc::Qwen3Config& c = b->config;
  *out = soc_qwen_config{};
  out->vocab_size = static_cast<int32_t>(c.vocab_size);
  out->hidden_size = static_cast<int32_t>(c.hidden_size);
  out->num_hidden_layers = static_cast<int32_t>(c.num_hidden_layers);
  out->num_attention_heads = static_cast<int32_t>(c.num_attention_heads);
  out->num_key_value_heads = static_cast<int32_t>(c.num_key_value_heads);
  out->head_dim = static_cast<int32_t>(c.head_dim);
  out->intermediate_size = static_cast<int32_t>(c.intermediate_size);
  out->max_position_embeddings = static_cast<int32_t>(c.max_position_embeddings);
  out->rope_theta = c.rope_theta;
  out->rms_norm_eps = static_cast<float>(c.rms_norm_eps);
  out->tie_word_embeddings = c.tie_word_embeddings ? 1 : 0;
  return SOC_OK;
}

int soc_bundle_tensor_f16(const soc_bundle* b, const char* name, uint16_t* out, int64_t numel) {
  if (b == nullptr || name == nullptr || out == nullptr) return soc::fail(SOC_ERR_INVALID, "null argument");
  try {
    for (const auto& [n, shape] : soc::Qwen3TensorShapes(b->config)) {
      if (n != name) continue;
      std::vector<uint16_t> v = soc::WeightLoader::LoadFloat16(b->manifest, n, shape);
      if (static_cast<int64_t>(v.size()) != numel)
        return soc::fail(SOC_ERR_INVALID, "soc_bundle_tensor_f16: numel does not match " + n);
      std::memcpy(out, v.data(), v.size() * 2);
      return SOC_OK;
    }
    return soc::fail(SOC_ERR_INVALID, std::string("not a weight of this model: ") + name);
  } catch (const std::exception& e) {
    return soc::fail(SOC_ERR_INVALID, e.what());
  }
}

}  // extern "C"
