// tokenizer.h - the bundle's tokenizer runtime (tokenizer/tokenizer_runtime.json), text <-> token ids, and the
// Qwen3 chat template.
//
// Data types and class names are the reference's (Mac/cpu/header/runtime_assets.h:34-155, tokenizer_runtime.h:12-44,
// startup_validator.h:8-17) so that code written against them compiles unchanged; errors are std::runtime_error
// with the reference's messages. Encoding follows Mac/cpu/src/tokenizer_runtime.cpp:54-304:
//   * protected (added) tokens are matched greedily, longest first, at every offset; without a BPE model every token
//     of the vocabulary is matched that way and unmatched text is an error;
//   * with a BPE model, the text between protected tokens is split by the byte-level pre-tokenizer (whitespace run
//     + a run of letters, of digits or of other bytes, in the C locale; optional prefix space), mapped to byte-level
//     symbols and merged lowest-rank-first (leftmost among equal ranks) until no ranked pair is left.
// Decoding concatenates added tokens verbatim and maps model tokens back through the byte-level table.
#pragma once

#include <cstddef>
#include <memory>
#include <string>
#include <vector>

#include "soc/assets.h"

namespace soc {

struct AddedTokenRecord {  // runtime_assets.h:34-42
  int id = 0;
  std::string content;
  bool special = false;
  bool single_word = false;
  bool lstrip = false;
  bool rstrip = false;
  bool normalized = false;
};

struct TemplateRuntimeData {  // runtime_assets.h:44-51
  std::string type;
  std::string im_start;
  std::string im_end;
  std::string think_start;
  std::string think_end;
  std::string default_system_prompt;
};

struct VocabEntry {  // runtime_assets.h:53-56
  int id = 0;
  std::string token;
};

struct BPEMergeRecord {  // runtime_assets.h:58-61
  std::string left;
  std::string right;
};

struct BPETokenizerModelData {  // runtime_assets.h:63-70
  bool enabled = false;
  std::string type;
  std::string unk_token;
  std::string continuing_subword_prefix;
  std::string end_of_word_suffix;
  std::vector<BPEMergeRecord> merges;
};

struct ByteLevelPreTokenizerData {  // runtime_assets.h:72-76
  bool enabled = false;
  bool add_prefix_space = false;
  bool use_regex = true;
};

struct PreTokenizerRuntimeData {  // runtime_assets.h:78-82
  bool enabled = false;
  std::string type;
  ByteLevelPreTokenizerData byte_level;
};

struct ByteLevelDecoderData {  // runtime_assets.h:84-90
  bool enabled = false;
  bool add_prefix_space = false;
  bool trim_offsets = false;
  bool use_regex = true;
  std::vector<std::string> byte_to_unicode;
};

struct BPEDecoderData {  // runtime_assets.h:92-95
  bool enabled = false;
  std::string suffix;
};

struct DecoderRuntimeData {  // runtime_assets.h:97-102
  bool enabled = false;
  std::string type;
  ByteLevelDecoderData byte_level;
  BPEDecoderData bpe;
};

struct TokenizerRuntimeData {  // runtime_assets.h:104-119
  std::string format;
  int format_version = 0;
  std::string tokenizer_class;
  int vocab_size = 0;
  std::size_t model_max_length = 0;
  std::string chat_template;
  TemplateRuntimeData template_runtime;
  std::vector<AddedTokenRecord> added_tokens;
  std::vector<VocabEntry> vocab;
  BPETokenizerModelData bpe_model;
  PreTokenizerRuntimeData pre_tokenizer;
  DecoderRuntimeData decoder;
  JsonValue special_tokens_map;
  JsonValue special_token_ids;
};

struct ChatMessage {  // runtime_assets.h:121-124
  std::string role;
  std::string content;
};

class TokenizerRuntimeLoader {  // runtime_assets.cpp:170-216
 public:
  static TokenizerRuntimeData LoadFromFile(const std::string& runtime_path);
};

// The Qwen3 chat layout (runtime_assets.cpp:218-257): "<im_start>role\ncontent<im_end>\n" per message, a system turn
// first when no message has the system role (the override, else the default prompt), then "<im_start>assistant\n"
// and, with thinking, "<think>\n".
class Qwen3TemplateBuilder {
 public:
  explicit Qwen3TemplateBuilder(TemplateRuntimeData template_runtime);
  std::string BuildPrompt(const std::vector<ChatMessage>& messages, bool add_generation_prompt, bool enable_thinking,
                          const std::string& system_prompt_override = "") const;

 private:
  TemplateRuntimeData template_runtime_;
};

class TokenizerRuntime {  // tokenizer_runtime.h:12-44
 public:
  explicit TokenizerRuntime(TokenizerRuntimeData runtime_data);
  ~TokenizerRuntime();
  TokenizerRuntime(const TokenizerRuntime& other);
  TokenizerRuntime& operator=(const TokenizerRuntime& other);
  TokenizerRuntime(TokenizerRuntime&&) noexcept;
  TokenizerRuntime& operator=(TokenizerRuntime&&) noexcept;

  const TokenizerRuntimeData& runtime_data() const;
  std::vector<int> Encode(const std::string& text) const;
  std::string Decode(const std::vector<int>& token_ids) const;
  int TokenToId(const std::string& token) const;    // throws "unknown token content: <token>"
  std::string IdToToken(int token_id) const;        // throws "unknown token id: <id>"

 private:
  struct Tables;  // lookup tables built once from the runtime data
  TokenizerRuntimeData runtime_data_;
  std::unique_ptr<Tables> tables_;
};

}  // namespace soc
