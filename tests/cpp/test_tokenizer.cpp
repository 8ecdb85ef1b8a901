// The reference's tokenizer, chat-template and startup-validation tests (Mac/cpu/test/test_model_bootstrap.cpp:
// 130-290, Mac/cpu/test/test_runtime_assets.cpp:80-239), restated against soc/tokenizer.h and soc/gpu/runtime.h.
// Host only: needs the library, not a GPU. Exits non-zero with the failed requirement on stderr.
#include <algorithm>
#include <cstdio>
#include <filesystem>
#include <fstream>
#include <stdexcept>
#include <string>
#include <vector>

#include "soc/gpu/runtime.h"
#include "soc/tokenizer.h"

using namespace soc;

namespace {

void require(bool ok, const char* what) {
  if (!ok) throw std::runtime_error(what);
}

template <typename F>
bool throws(F&& f) {
  try {
    f();
  } catch (const std::runtime_error&) {
    return true;
  }
  return false;
}

// GPT-2 byte-level table, UTF-8 encoded (test_model_bootstrap.cpp:19-64).
std::vector<std::string> ByteTable() {
  std::vector<int> keep;
  for (int b = '!'; b <= '~'; ++b) keep.push_back(b);
  for (int b = 161; b <= 172; ++b) keep.push_back(b);
  for (int b = 174; b <= 255; ++b) keep.push_back(b);
  std::vector<std::string> t(256);
  int extra = 0;
  for (int b = 0; b < 256; ++b) {
    const bool kept = std::find(keep.begin(), keep.end(), b) != keep.end();
    const int cp = kept ? b : 256 + extra++;
    std::string u;
    if (cp < 0x80) {
      u.push_back(static_cast<char>(cp));
    } else {
      u.push_back(static_cast<char>(0xC0 | (cp >> 6)));
      u.push_back(static_cast<char>(0x80 | (cp & 0x3F)));
    }
    t[b] = u;
  }
  return t;
}

ManifestData Manifest() {  // test_model_bootstrap.cpp:66-100
  ManifestData m;
  m.format = "soc.cpp.llm_export";
  m.format_version = 2;
  m.model_id = "Qwen/Qwen3-0.6B";
  m.export_dtype = "float16";
  m.tokenizer_runtime_file = "tokenizer/tokenizer_runtime.json";
  m.config = JsonParser::Parse(
      R"({"model_type":"qwen3","hidden_size":1024,"intermediate_size":3072,"num_hidden_layers":28,)"
      R"("num_attention_heads":16,"num_key_value_heads":8,"head_dim":128,"rms_norm_eps":1e-6,"rope_theta":1000000,)"
      R"("tie_word_embeddings":true,"torch_dtype":"bfloat16","vocab_size":16})");
  m.tensors.push_back(TensorRecord{"model.embed_tokens.weight", "weights/embed.bin", "float16", {16, 1024},
                                   16 * 1024 * 2, "model-00001-of-00001.safetensors"});
  return m;
}

TokenizerRuntimeData Runtime() {  // test_model_bootstrap.cpp:102-137
  TokenizerRuntimeData r;
  r.format = "soc.cpp.tokenizer_runtime";
  r.format_version = 1;
  r.tokenizer_class = "Qwen2TokenizerFast";
  r.vocab_size = 16;
  r.model_max_length = 32768;
  r.chat_template = "qwen3-template";
  r.template_runtime = {"qwen3", "<|im_start|>", "<|im_end|>", "<think>", "</think>", "You are a helpful assistant."};
  for (const auto& [id, content] : std::vector<std::pair<int, std::string>>{
           {10, "<|im_start|>"}, {11, "<|im_end|>"}, {12, "<think>"}, {13, "</think>"}})
    r.added_tokens.push_back(AddedTokenRecord{id, content, true, false, false, false, false});
  r.vocab = {{0, "system\n"}, {1, "assistant\n"}, {2, "user\n"}, {3, "You are a helpful assistant."},
             {4, "Hello"},     {5, " world"},      {6, "Say hello."}, {7, "Now think first."},
             {8, "\n"},        {9, "Hello."}};
  return r;
}

void TestStartupValidator() {  // test_model_bootstrap.cpp:150-167
  const ManifestData m = Manifest();
  const TokenizerRuntimeData r = Runtime();
  require(StartupValidator::ValidateManifest(m).vocab_size == 16, "validator returns the parsed config");
  StartupValidator::ValidateTokenizerRuntime(r);
  StartupValidator::ValidateManifestAndTokenizer(m, r);
  TokenizerRuntimeData bad = r;
  bad.vocab_size = 17;
  require(throws([&] { StartupValidator::ValidateManifestAndTokenizer(m, bad); }), "vocab mismatch is rejected");
  bad = r;
  bad.added_tokens.pop_back();  // no </think>
  require(throws([&] { StartupValidator::ValidateTokenizerRuntime(bad); }), "missing think_end is rejected");
  bad = r;
  bad.decoder.enabled = bad.decoder.byte_level.enabled = true;
  bad.decoder.byte_level.byte_to_unicode = {"!", "\""};
  require(throws([&] { StartupValidator::ValidateTokenizerRuntime(bad); }), "a partial byte table is rejected");
}

void TestMinimalEncodeDecode() {  // test_model_bootstrap.cpp:169-187
  const TokenizerRuntime tok(Runtime());
  const std::string text = "<|im_start|>user\nSay hello.<|im_end|>\n<|im_start|>assistant\nHello world<|im_end|>\n";
  const std::vector<int> ids = tok.Encode(text);
  require(ids == std::vector<int>({10, 2, 6, 11, 8, 10, 1, 4, 5, 11, 8}), "longest-match ids");
  require(tok.Decode(ids) == text, "decode reconstructs the text");
  require(tok.TokenToId("<|im_start|>") == 10, "TokenToId");
  require(tok.IdToToken(5) == " world", "IdToToken");
  require(throws([&] { tok.Encode("unencodable-token"); }), "unmatched text is rejected without BPE");
  require(throws([&] { tok.IdToToken(99); }), "unknown id is rejected");
}

void TestBpeFallback() {  // test_model_bootstrap.cpp:189-226
  TokenizerRuntimeData r = Runtime();
  r.added_tokens.clear();
  r.vocab = {{0, "h"}, {1, "e"},  {2, "l"},    {3, "o"},     {4, " "},     {5, "w"},     {6, "r"},
             {7, "d"}, {8, "he"}, {9, "ll"},   {10, "hell"}, {11, "hello"}, {12, " world"}};
  r.vocab_size = 13;
  r.bpe_model.enabled = true;
  r.bpe_model.type = "bpe";
  r.bpe_model.merges = {{"h", "e"},  {"l", "l"},   {"he", "ll"},   {"hell", "o"},   {" ", "w"},
                        {" w", "o"}, {" wo", "r"}, {" wor", "l"}, {" worl", "d"}};
  const TokenizerRuntime tok(r);
  const std::vector<int> ids = tok.Encode("hello world");
  require(ids == std::vector<int>({11, 12}), "BPE merges into [hello, ' world']");
  require(tok.Decode(ids) == "hello world", "BPE decode");
}

void TestByteLevelPrefixSpace() {  // test_model_bootstrap.cpp:228-280
  TokenizerRuntimeData r = Runtime();
  r.added_tokens.clear();
  r.vocab = {{0, "Ġh"},     {1, "e"},      {2, "l"},       {3, "o"},       {4, "Ġw"},
             {5, "r"},      {6, "d"},      {7, "Ġhe"},     {8, "ll"},      {9, "Ġhell"},
             {10, "Ġhello"}, {11, "Ġwo"},  {12, "Ġwor"},   {13, "Ġworl"},  {14, "Ġworld"}};
  r.vocab_size = 15;
  r.bpe_model.enabled = true;
  r.bpe_model.type = "bpe";
  r.bpe_model.merges = {{"Ġ", "h"},  {"Ġh", "e"},  {"l", "l"},    {"Ġhe", "ll"},  {"Ġhell", "o"},
                        {"Ġ", "w"},  {"Ġw", "o"},  {"Ġwo", "r"},  {"Ġwor", "l"},  {"Ġworl", "d"}};
  r.pre_tokenizer.enabled = true;
  r.pre_tokenizer.type = "ByteLevel";
  r.pre_tokenizer.byte_level.enabled = true;
  r.pre_tokenizer.byte_level.add_prefix_space = true;
  r.pre_tokenizer.byte_level.use_regex = true;
  r.decoder.enabled = true;
  r.decoder.type = "ByteLevel";
  r.decoder.byte_level.enabled = true;
  r.decoder.byte_level.byte_to_unicode = ByteTable();
  const TokenizerRuntime tok(r);
  const std::vector<int> ids = tok.Encode("hello world");
  require(ids == std::vector<int>({10, 14}), "byte-level pieces with a prefix space");
  require(tok.Decode(ids) == " hello world", "byte-level decode keeps the stored leading space");
  const TokenizerRuntime copy = tok;  // copies rebuild their lookup tables
  require(copy.Encode("hello world") == ids, "a copied tokenizer encodes the same");
}

void TestLoader(const std::filesystem::path& dir) {  // test_runtime_assets.cpp:80-164
  const std::filesystem::path p = dir / "tokenizer_runtime.json";
  std::ofstream(p) << R"({
  "format": "soc.cpp.tokenizer_runtime", "format_version": 1, "tokenizer_class": "Qwen2TokenizerFast",
  "vocab_size": 151936, "model_max_length": 131072,
  "special_tokens_map": {"bos_token": "<|endoftext|>"}, "special_token_ids": {"bos_token": 151643},
  "added_tokens": [{"id": 151644, "content": "<|im_start|>", "special": true, "single_word": false, "lstrip": false,
                    "rstrip": false, "normalized": false}],
  "vocab": [{"id": 0, "token": "!"}, {"id": 1, "token": "\""}],
  "bpe_model": {"type": "bpe", "unk_token": null, "continuing_subword_prefix": "", "end_of_word_suffix": "",
                "merges": [{"left": "h", "right": "e"}, {"left": "he", "right": "llo"}]},
  "pre_tokenizer": {"type": "ByteLevel", "byte_level": {"enabled": true, "add_prefix_space": true, "use_regex": true}},
  "decoder": {"type": "Sequence",
              "byte_level": {"enabled": true, "add_prefix_space": false, "trim_offsets": false, "use_regex": true,
                             "byte_to_unicode": ["!", "\""]},
              "bpe": {"enabled": true, "suffix": "</w>"}},
  "chat_template": "dummy-template",
  "template_runtime": {"type": "qwen3", "im_start": "<|im_start|>", "im_end": "<|im_end|>", "think_start": "<think>",
                       "think_end": "</think>", "default_system_prompt": "You are a helpful assistant."},
  "copied_files": ["tokenizer.json"]
})";
  const TokenizerRuntimeData r = TokenizerRuntimeLoader::LoadFromFile(p.string());
  require(r.format == "soc.cpp.tokenizer_runtime", "loader reads format");
  require(r.vocab_size == 151936, "loader reads vocab size");
  require(r.model_max_length == 131072, "loader reads model_max_length");
  require(r.template_runtime.im_start == "<|im_start|>", "loader reads the template runtime");
  require(r.added_tokens.size() == 1 && r.added_tokens[0].id == 151644 && r.added_tokens[0].special,
          "loader reads added tokens");
  require(r.vocab.size() == 2 && r.vocab[1].token == "\"", "loader reads vocab entries");
  require(r.bpe_model.enabled && r.bpe_model.merges.size() == 2 && r.bpe_model.unk_token.empty(),
          "loader reads the optional BPE model");
  require(r.pre_tokenizer.enabled && r.pre_tokenizer.byte_level.add_prefix_space, "loader reads the pre-tokenizer");
  require(r.decoder.enabled && r.decoder.bpe.suffix == "</w>", "loader reads the BPE decoder suffix");
  require(r.decoder.byte_level.byte_to_unicode.size() == 2, "loader reads the byte table");
  require(r.chat_template == "dummy-template", "loader reads chat_template");
  require(r.special_token_ids.at("bos_token").as_int() == 151643, "loader keeps special_token_ids");
}

void TestTemplateBuilder() {  // test_runtime_assets.cpp:166-197
  const Qwen3TemplateBuilder b({"qwen3", "<|im_start|>", "<|im_end|>", "<think>", "</think>",
                                "You are a helpful assistant."});
  const std::vector<ChatMessage> msgs = {{"user", "Say hello."}, {"assistant", "Hello."}, {"user", "Now think first."}};
  const std::string p = b.BuildPrompt(msgs, true, true);
  require(p ==
              "<|im_start|>system\nYou are a helpful assistant.<|im_end|>\n"
              "<|im_start|>user\nSay hello.<|im_end|>\n<|im_start|>assistant\nHello.<|im_end|>\n"
              "<|im_start|>user\nNow think first.<|im_end|>\n<|im_start|>assistant\n<think>\n",
          "template layout with the default system prompt and thinking");
  const std::string q = b.BuildPrompt(msgs, true, false, "Custom system prompt.");
  require(q.find("Custom system prompt.") != std::string::npos, "system prompt override");
  require(q.find("<think>") == std::string::npos, "no think tag without thinking");
  const std::string s = b.BuildPrompt({{"system", "S."}, {"user", "U."}}, false, true);
  require(s == "<|im_start|>system\nS.<|im_end|>\n<|im_start|>user\nU.<|im_end|>\n",
          "an explicit system turn replaces the default and no generation prompt is added");
}

void TestPipelineHelpers() {  // test_runtime_assets.cpp:199-239
  ManifestData m;
  m.generation_config =
      JsonParser::Parse(R"({"max_new_tokens":12,"temperature":0.7,"top_k":4,"eos_token_id":[151645],"max_length":1024})");
  const gpu::RuntimeGenerationOptions o = gpu::RuntimePipeline::GenerationOptionsFromManifest(m);
  require(o.max_new_tokens == 12, "max_new_tokens from generation_config");
  require(o.sampler.top_k == 4, "top_k from generation_config");
  require(o.sampler.temperature == 0.7f, "temperature from generation_config");
  require(o.eos_token_id == 151645, "eos_token_id list");
  require(o.max_sequence_length == 1024, "max_length");
  const gpu::RuntimeGenerationOptions d = gpu::RuntimePipeline::GenerationOptionsFromManifest(ManifestData{});
  require(d.max_new_tokens == 32 && d.sampler.top_k == 1 && d.eos_token_id == -1 && d.max_sequence_length == 256,
          "defaults without generation_config");
  TokenizerRuntimeData r;
  r.template_runtime = {"qwen3", "<|im_start|>", "<|im_end|>", "<think>", "</think>", "You are a helpful assistant."};
  gpu::RuntimePromptOptions po;
  po.apply_chat_template = true;
  po.enable_thinking = false;
  po.system_prompt = "System override.";
  const std::string pp = gpu::RuntimePipeline::PreparePrompt(r, "Hello", po);
  require(pp.find("System override.") != std::string::npos, "system override passes through");
  require(pp.find("<|im_start|>user\nHello<|im_end|>") != std::string::npos, "prompt becomes a user turn");
  require(pp.find("<think>") == std::string::npos, "no think tag");
  require(gpu::RuntimePipeline::PreparePrompt(r, "Hello", {}) == "Hello", "raw prompt without the template");
}

}  // namespace

int main(int argc, char** argv) {
  const std::filesystem::path dir = argc > 1 ? argv[1] : std::filesystem::temp_directory_path();
  try {
    TestStartupValidator();
    TestMinimalEncodeDecode();
    TestBpeFallback();
    TestByteLevelPrefixSpace();
    TestLoader(dir);
    TestTemplateBuilder();
    TestPipelineHelpers();
  } catch (const std::exception& e) {
    std::fprintf(stderr, "FAIL: %s\n", e.what());
    return 1;
  }
  std::printf("test_tokenizer: all passed\n");
  return 0;
}
