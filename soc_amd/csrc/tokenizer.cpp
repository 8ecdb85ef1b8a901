// tokenizer.cpp - the tokenizer runtime of a model bundle (include/soc/tokenizer.h): loader, validation, the Qwen3
// chat template, encode/decode, and the C entry points soc_tokenizer_*.
//
// Behaviour follows Mac/cpu/src/tokenizer_runtime.cpp:54-304, runtime_assets.cpp:170-257 and
// startup_validator.cpp:25-100. Host code only: nothing here touches the GPU.
//
// Encoding is organised for lookups rather than scans: longest-first matching tries each distinct token length once
// against a hash set (the reference walks the length-sorted token list), and BPE merging keeps the adjacent pairs in a
// min-heap ordered by (merge rank, position) with stale entries discarded on pop (the reference rescans every pair
// after each merge). Both choose exactly what the reference chooses: at one offset only one token of a given length
// can match, and the heap's minimum is the lowest-ranked pair, leftmost among equal ranks.
#include <algorithm>
#include <cstdint>
#include <cstring>
#include <deque>
#include <queue>
#include <stdexcept>
#include <string_view>
#include <unordered_map>
#include <unordered_set>

#include "soc/tokenizer.h"
#include "soc_hip.h"
#include "status.h"

namespace soc {
namespace {

// Character classes of the pre-tokenizer: std::isspace / isalpha / isdigit in the "C" locale, on unsigned bytes
// (bytes >= 0x80 are none of them).
enum ByteClass { kSpace, kAlpha, kDigit, kOther };
inline ByteClass byte_class(unsigned char c) {
  if (c == ' ' || (c >= '\t' && c <= '\r')) return kSpace;
  if ((c | 0x20) >= 'a' && (c | 0x20) <= 'z') return kAlpha;
  if (c >= '0' && c <= '9') return kDigit;
  return kOther;
}

// Width of the UTF-8 sequence a lead byte starts; 1 for bytes that start none (tokenizer_runtime.cpp:344-359).
inline std::size_t utf8_width(unsigned char lead) {
  if ((lead & 0x80u) == 0) return 1;
  if ((lead & 0xE0u) == 0xC0u) return 2;
  if ((lead & 0xF0u) == 0xE0u) return 3;
  if ((lead & 0xF8u) == 0xF0u) return 4;
  return 1;
}

inline bool starts_with(std::string_view v, std::string_view p) { return v.size() >= p.size() && v.substr(0, p.size()) == p; }
inline bool ends_with(std::string_view v, std::string_view s) {
  return v.size() >= s.size() && v.substr(v.size() - s.size()) == s;
}

// The longest member of a string set that starts at an offset. Members are owned by the matcher.
class LongestMatch {
 public:
  void add(const std::string& s) {
    if (s.empty() || set_.count(s) != 0) return;
    set_.insert(store_.emplace_back(s));
  }
  void finish() {
    std::unordered_set<std::size_t> seen;
    for (std::string_view s : set_) seen.insert(s.size());
    lengths_.assign(seen.begin(), seen.end());
    std::sort(lengths_.rbegin(), lengths_.rend());
  }
  std::size_t at(std::string_view text, std::size_t off) const {  // 0 when nothing matches
    for (const std::size_t n : lengths_)
      if (off + n <= text.size() && set_.count(text.substr(off, n)) != 0) return n;
    return 0;
  }
  // The first offset >= off at which any member starts, text.size() if none does.
  std::size_t next(std::string_view text, std::size_t off) const {
    std::size_t best = text.size();
    for (std::string_view s : set_) {
      const std::size_t p = text.find(s, off);
      if (p < best) best = p;
    }
    return best;
  }
  bool empty() const { return set_.empty(); }

 private:
  std::deque<std::string> store_;  // stable addresses for the views below
  std::unordered_set<std::string_view> set_;
  std::vector<std::size_t> lengths_;
};

// Merge-table key of an adjacent pair. The separator is the reference's (tokenizer_runtime.cpp:375-377), so pairs
// that only differ in where a newline sits collide exactly as they do there.
inline std::string pair_key(const std::string& left, const std::string& right) {
  std::string k;
  k.reserve(left.size() + 1 + right.size());
  k.append(left).push_back('\n');
  k.append(right);
  return k;
}

}  // namespace

struct TokenizerRuntime::Tables {
  std::unordered_map<std::string, int> id_of;     // content -> id; the first record wins (added tokens, then vocab)
  std::unordered_map<int, std::string> token_of;  // id -> content; the first record wins
  std::unordered_set<int> added_ids;
  LongestMatch protected_tokens;  // added tokens: matched whole before any BPE
  LongestMatch all_tokens;        // every token: the matcher when there is no BPE model
  std::unordered_map<std::string, std::size_t> merge_rank;  // pair_key -> merge index; the first occurrence wins
  std::unordered_map<std::string, unsigned char> byte_of;   // byte-level symbol -> byte; the lowest byte wins

  explicit Tables(const TokenizerRuntimeData& d) {
    for (const AddedTokenRecord& t : d.added_tokens) {
      id_of.emplace(t.content, t.id);
      token_of.emplace(t.id, t.content);
      added_ids.insert(t.id);
      protected_tokens.add(t.content);
      all_tokens.add(t.content);
    }
    for (const VocabEntry& t : d.vocab) {
      id_of.emplace(t.token, t.id);
      token_of.emplace(t.id, t.token);
      all_tokens.add(t.token);
    }
    protected_tokens.finish();
    all_tokens.finish();
    for (std::size_t i = 0; i < d.bpe_model.merges.size(); ++i)
      merge_rank.emplace(pair_key(d.bpe_model.merges[i].left, d.bpe_model.merges[i].right), i);
    const std::vector<std::string>& b2u = d.decoder.byte_level.byte_to_unicode;
    for (std::size_t b = 0; b < b2u.size(); ++b) byte_of.emplace(b2u[b], static_cast<unsigned char>(b));
  }
};

TokenizerRuntime::TokenizerRuntime(TokenizerRuntimeData runtime_data)
    : runtime_data_(std::move(runtime_data)), tables_(std::make_unique<Tables>(runtime_data_)) {}
TokenizerRuntime::~TokenizerRuntime() = default;
TokenizerRuntime::TokenizerRuntime(const TokenizerRuntime& o)
    : runtime_data_(o.runtime_data_), tables_(std::make_unique<Tables>(runtime_data_)) {}
TokenizerRuntime& TokenizerRuntime::operator=(const TokenizerRuntime& o) {
  if (this != &o) {
    runtime_data_ = o.runtime_data_;
    tables_ = std::make_unique<Tables>(runtime_data_);
  }
  return *this;
}
TokenizerRuntime::TokenizerRuntime(TokenizerRuntime&&) noexcept = default;
TokenizerRuntime& TokenizerRuntime::operator=(TokenizerRuntime&&) noexcept = default;

const TokenizerRuntimeData& TokenizerRuntime::runtime_data() const { return runtime_data_; }

int TokenizerRuntime::TokenToId(const std::string& token) const {
  const auto it = tables_->id_of.find(token);
  if (it == tables_->id_of.end()) throw std::runtime_error("unknown token content: " + token);
  return it->second;
}

std::string TokenizerRuntime::IdToToken(int token_id) const {
  const auto it = tables_->token_of.find(token_id);
  if (it == tables_->token_of.end()) throw std::runtime_error("unknown token id: " + std::to_string(token_id));
  return it->second;
}

namespace {

// Pre-tokenizer (tokenizer_runtime.cpp:185-231): each piece is a whitespace run followed by one run of letters, of
// digits or of other non-space bytes; trailing whitespace is a piece of its own. Optionally a space is put in front
// of the first piece when it does not start with whitespace.
std::vector<std::string> pre_tokenize(const TokenizerRuntimeData& d, const std::string& text) {
  const ByteLevelPreTokenizerData& bl = d.pre_tokenizer.byte_level;
  if (!d.pre_tokenizer.enabled || !bl.enabled) return {text};
  std::vector<std::string> pieces;
  if (!bl.use_regex) {
    pieces.push_back(text);
  } else {
    const auto* s = reinterpret_cast<const unsigned char*>(text.data());
    const std::size_t n = text.size();
    std::size_t i = 0;
    while (i < n) {
      const std::size_t start = i;
      while (i < n && byte_class(s[i]) == kSpace) ++i;
      if (i < n) {
        const ByteClass run = byte_class(s[i]);
        do ++i;
        while (i < n && byte_class(s[i]) == run);
      }
      pieces.push_back(text.substr(start, i - start));
    }
  }
  if (bl.add_prefix_space && !pieces.empty() && !pieces[0].empty() &&
      byte_class(static_cast<unsigned char>(pieces[0][0])) != kSpace)
    pieces[0].insert(pieces[0].begin(), ' ');
  return pieces;
}

// One symbol per byte (tokenizer_runtime.cpp:233-269): the byte-level table's string when the pre-tokenizer is
// byte-level and the table is present, else the byte itself; the continuing-subword prefix on every symbol after the
// first and the end-of-word suffix on the last.
std::vector<std::string> piece_symbols(const TokenizerRuntimeData& d, const std::string& piece) {
  const std::vector<std::string>& b2u = d.decoder.byte_level.byte_to_unicode;
  const bool byte_level = d.pre_tokenizer.byte_level.enabled && !b2u.empty();
  const std::string& prefix = d.bpe_model.continuing_subword_prefix;
  const std::string& suffix = d.bpe_model.end_of_word_suffix;
  std::vector<std::string> out;
  out.reserve(piece.size());
  for (std::size_t i = 0; i < piece.size(); ++i) {
    const unsigned char b = static_cast<unsigned char>(piece[i]);
    std::string sym;
    if (i > 0) sym = prefix;
    if (byte_level) {
      if (b >= b2u.size())
        throw std::runtime_error("tokenizer byte_to_unicode mapping has no entry for byte " + std::to_string(b));
      sym += b2u[b];
    } else {
      sym.push_back(static_cast<char>(b));
    }
    if (i + 1 == piece.size()) sym += suffix;
    out.push_back(std::move(sym));
  }
  return out;
}

// BPE merging (tokenizer_runtime.cpp:271-304): repeatedly joins the adjacent pair with the lowest merge rank, the
// leftmost among equal ranks, until no adjacent pair has a rank.
void merge_symbols(const std::unordered_map<std::string, std::size_t>& rank, std::vector<std::string>& sym) {
  const std::size_t n = sym.size();
  if (n < 2 || rank.empty()) return;
  struct Cand {
    std::size_t rank, left, right;
    uint32_t vl, vr;
  };
  const auto later = [](const Cand& a, const Cand& b) { return a.rank != b.rank ? a.rank > b.rank : a.left > b.left; };
  std::priority_queue<Cand, std::vector<Cand>, decltype(later)> heap(later);
  constexpr std::size_t kNone = ~std::size_t{0};
  std::vector<std::size_t> prev(n), next(n);
  std::vector<uint32_t> version(n, 0);
  std::vector<char> alive(n, 1);
  for (std::size_t i = 0; i < n; ++i) {
    prev[i] = i == 0 ? kNone : i - 1;
    next[i] = i + 1 == n ? kNone : i + 1;
  }
  const auto offer = [&](std::size_t l, std::size_t r) {
    if (l == kNone || r == kNone) return;
    const auto it = rank.find(pair_key(sym[l], sym[r]));
    if (it != rank.end()) heap.push(Cand{it->second, l, r, version[l], version[r]});
  };
  for (std::size_t i = 0; i + 1 < n; ++i) offer(i, i + 1);
  while (!heap.empty()) {
    const Cand c = heap.top();
    heap.pop();
    if (!alive[c.left] || !alive[c.right] || next[c.left] != c.right || version[c.left] != c.vl ||
        version[c.right] != c.vr)
      continue;  // stale: one side has merged since this pair was offered
    sym[c.left] += sym[c.right];
    sym[c.right].clear();
    alive[c.right] = 0;
    next[c.left] = next[c.right];
    if (next[c.left] != kNone) prev[next[c.left]] = c.left;
    ++version[c.left];
    offer(prev[c.left], c.left);
    offer(c.left, next[c.left]);
  }
  std::size_t w = 0;
  for (std::size_t i = 0; i < n; ++i) {
    if (!alive[i]) continue;
    if (i != w) sym[w] = std::move(sym[i]);  // never a self-move: that may leave the string empty
    ++w;
  }
  sym.resize(w);
}

}  // namespace

std::vector<int> TokenizerRuntime::Encode(const std::string& text) const {
  const Tables& t = *tables_;
  const bool bpe = runtime_data_.bpe_model.enabled;
  const LongestMatch& whole = bpe ? t.protected_tokens : t.all_tokens;
  std::vector<int> ids;
  std::size_t off = 0;
  while (off < text.size()) {
    if (const std::size_t n = whole.at(text, off)) {
      ids.push_back(t.id_of.at(text.substr(off, n)));
      off += n;
      continue;
    }
    if (!bpe) throw std::runtime_error("tokenizer runtime cannot encode input at byte offset " + std::to_string(off));
    // BPE over the text up to the next protected token (tokenizer_runtime.cpp:158-183).
    const std::size_t end = t.protected_tokens.next(text, off);
    for (const std::string& piece : pre_tokenize(runtime_data_, text.substr(off, end - off))) {
      std::vector<std::string> sym = piece_symbols(runtime_data_, piece);
      merge_symbols(t.merge_rank, sym);
      for (const std::string& s : sym) {
        const auto it = t.id_of.find(s);
        if (it != t.id_of.end()) {
          ids.push_back(it->second);
        } else if (!runtime_data_.bpe_model.unk_token.empty()) {
          ids.push_back(TokenToId(runtime_data_.bpe_model.unk_token));
        } else {
          throw std::runtime_error("tokenizer runtime cannot encode BPE symbol: " + s);
        }
      }
    }
    off = end;
  }
  return ids;
}

std::string TokenizerRuntime::Decode(const std::vector<int>& token_ids) const {
  const Tables& t = *tables_;
  const TokenizerRuntimeData& d = runtime_data_;
  const bool byte_level = d.decoder.byte_level.enabled && !t.byte_of.empty();
  const bool strip_suffix = d.decoder.bpe.enabled && !d.decoder.bpe.suffix.empty();
  const std::string& prefix = d.bpe_model.continuing_subword_prefix;
  std::string text;
  bool first_model_token = true;
  for (const int id : token_ids) {
    const std::string tok = IdToToken(id);
    if (t.added_ids.count(id) != 0) {  // added tokens are copied verbatim (tokenizer_runtime.cpp:82-96)
      text += tok;
      continue;
    }
    // Model tokens (tokenizer_runtime.cpp:306-342): the decoder suffix becomes a trailing space, the subword prefix
    // is dropped after the first model token, byte-level symbols map back to bytes (others are kept as they are).
    std::string_view v = tok;
    const bool space = strip_suffix && ends_with(v, d.decoder.bpe.suffix);
    if (space) v.remove_suffix(d.decoder.bpe.suffix.size());
    if (!first_model_token && !prefix.empty() && starts_with(v, prefix)) v.remove_prefix(prefix.size());
    first_model_token = false;
    if (byte_level) {
      std::size_t off = 0;
      while (off < v.size()) {  // a sequence cut short by the token's end is taken as it is
        const std::size_t w = utf8_width(static_cast<unsigned char>(v[off]));
        const std::string cp(v.substr(off, w));
        const auto it = t.byte_of.find(cp);
        if (it != t.byte_of.end())
          text.push_back(static_cast<char>(it->second));
        else
          text += cp;
        off += w;
      }
    } else {
      text.append(v);
    }
    if (space) text.push_back(' ');
  }
  return text;
}

// ---- loader (runtime_assets.cpp:29-137, 170-216) ----
namespace {

std::string opt_string(const JsonValue& o, const char* key) {
  const JsonValue* v = o.find(key);
  return v != nullptr && !v->is_null() ? v->as_string() : std::string();
}
bool opt_bool(const JsonValue& o, const char* key, bool fallback) {
  const JsonValue* v = o.find(key);
  return v != nullptr ? v->as_bool() : fallback;
}
const JsonValue* present(const JsonValue& o, const char* key) {  // the member unless it is absent or null
  const JsonValue* v = o.find(key);
  return v != nullptr && !v->is_null() ? v : nullptr;
}

}  // namespace

TokenizerRuntimeData TokenizerRuntimeLoader::LoadFromFile(const std::string& runtime_path) {
  const JsonValue root = JsonParser::ParseFile(runtime_path);
  TokenizerRuntimeData d;
  d.format = root.at("format").as_string();
  d.format_version = root.at("format_version").as_int();
  d.tokenizer_class = root.at("tokenizer_class").as_string();
  d.vocab_size = root.at("vocab_size").as_int();
  d.model_max_length = static_cast<std::size_t>(root.at("model_max_length").as_int64());
  d.chat_template = opt_string(root, "chat_template");
  const JsonValue& tr = root.at("template_runtime");
  d.template_runtime = TemplateRuntimeData{tr.at("type").as_string(),        tr.at("im_start").as_string(),
                                           tr.at("im_end").as_string(),      tr.at("think_start").as_string(),
                                           tr.at("think_end").as_string(),   tr.at("default_system_prompt").as_string()};
  if (const JsonValue* v = root.find("special_tokens_map")) d.special_tokens_map = *v;
  if (const JsonValue* v = root.find("special_token_ids")) d.special_token_ids = *v;
  for (const JsonValue& a : root.at("added_tokens").as_array())
    d.added_tokens.push_back(AddedTokenRecord{a.at("id").as_int(), a.at("content").as_string(),
                                              a.at("special").as_bool(), a.at("single_word").as_bool(),
                                              a.at("lstrip").as_bool(), a.at("rstrip").as_bool(),
                                              a.at("normalized").as_bool()});
  for (const JsonValue& v : root.at("vocab").as_array())
    d.vocab.push_back(VocabEntry{v.at("id").as_int(), v.at("token").as_string()});
  if (const JsonValue* m = present(root, "bpe_model")) {
    d.bpe_model.enabled = true;
    d.bpe_model.type = m->at("type").as_string();
    d.bpe_model.unk_token = opt_string(*m, "unk_token");
    d.bpe_model.continuing_subword_prefix = opt_string(*m, "continuing_subword_prefix");
    d.bpe_model.end_of_word_suffix = opt_string(*m, "end_of_word_suffix");
    for (const JsonValue& r : m->at("merges").as_array())
      d.bpe_model.merges.push_back(BPEMergeRecord{r.at("left").as_string(), r.at("right").as_string()});
  }
  if (const JsonValue* p = present(root, "pre_tokenizer")) {
    d.pre_tokenizer.enabled = true;
    d.pre_tokenizer.type = opt_string(*p, "type");
    if (const JsonValue* bl = present(*p, "byte_level")) {
      d.pre_tokenizer.byte_level.enabled = opt_bool(*bl, "enabled", true);
      d.pre_tokenizer.byte_level.add_prefix_space = opt_bool(*bl, "add_prefix_space", false);
      d.pre_tokenizer.byte_level.use_regex = opt_bool(*bl, "use_regex", true);
    }
  }
  if (const JsonValue* dec = present(root, "decoder")) {
    d.decoder.enabled = true;
    d.decoder.type = opt_string(*dec, "type");
    if (const JsonValue* bl = present(*dec, "byte_level")) {
      ByteLevelDecoderData& b = d.decoder.byte_level;
      b.enabled = opt_bool(*bl, "enabled", true);
      b.add_prefix_space = opt_bool(*bl, "add_prefix_space", false);
      b.trim_offsets = opt_bool(*bl, "trim_offsets", false);
      b.use_regex = opt_bool(*bl, "use_regex", true);
      if (const JsonValue* map = present(*bl, "byte_to_unicode"))
        for (const JsonValue& s : map->as_array()) b.byte_to_unicode.push_back(s.as_string());
    }
    if (const JsonValue* bpe = present(*dec, "bpe")) {
      d.decoder.bpe.enabled = opt_bool(*bpe, "enabled", true);
      d.decoder.bpe.suffix = opt_string(*bpe, "suffix");
    }
  }
  return d;
}

// ---- chat template (runtime_assets.cpp:218-257) ----
Qwen3TemplateBuilder::Qwen3TemplateBuilder(TemplateRuntimeData template_runtime)
    : template_runtime_(std::move(template_runtime)) {}

std::string Qwen3TemplateBuilder::BuildPrompt(const std::vector<ChatMessage>& messages, bool add_generation_prompt,
                                              bool enable_thinking, const std::string& system_prompt_override) const {
  const TemplateRuntimeData& t = template_runtime_;
  const auto turn = [&t](const std::string& role, const std::string& content) {
    return t.im_start + role + '\n' + content + t.im_end + '\n';
  };
  bool has_system = false;
  std::string turns;
  for (const ChatMessage& m : messages) {
    has_system = has_system || m.role == "system";
    turns += turn(m.role, m.content);
  }
  std::string prompt;
  if (!has_system) prompt = turn("system", system_prompt_override.empty() ? t.default_system_prompt : system_prompt_override);
  prompt += turns;
  if (add_generation_prompt) {
    prompt += t.im_start + "assistant\n";
    if (enable_thinking) prompt += t.think_start + '\n';
  }
  return prompt;
}

// ---- validation (startup_validator.cpp:25-100) ----
namespace {

int find_token_id(const TokenizerRuntimeData& d, const std::string& content) {  // added tokens first, then vocab
  for (const AddedTokenRecord& t : d.added_tokens)
    if (t.content == content) return t.id;
  for (const VocabEntry& t : d.vocab)
    if (t.token == content) return t.id;
  return -1;
}

}  // namespace

void StartupValidator::ValidateTokenizerRuntime(const TokenizerRuntimeData& d) {
  const auto require = [](bool ok, const char* msg) {
    if (!ok) throw std::runtime_error(msg);
  };
  require(d.format == "soc.cpp.tokenizer_runtime", "tokenizer runtime format must be soc.cpp.tokenizer_runtime");
  require(d.format_version == 1, "tokenizer runtime format_version must be 1");
  require(d.vocab_size > 0, "tokenizer runtime vocab_size must be positive");
  const TemplateRuntimeData& t = d.template_runtime;
  require(t.type == "qwen3", "tokenizer template runtime type must be qwen3");
  require(!t.im_start.empty() && !t.im_end.empty(), "tokenizer runtime must define chat boundary tokens");
  require(find_token_id(d, t.im_start) >= 0, "tokenizer runtime is missing im_start token id");
  require(find_token_id(d, t.im_end) >= 0, "tokenizer runtime is missing im_end token id");
  require(find_token_id(d, t.think_start) >= 0, "tokenizer runtime is missing think_start token id");
  require(find_token_id(d, t.think_end) >= 0, "tokenizer runtime is missing think_end token id");
  if (d.bpe_model.enabled) {
    require(d.bpe_model.type == "bpe", "tokenizer bpe_model type must be bpe");
    require(!d.bpe_model.merges.empty(), "tokenizer bpe_model must define merges");
    require(d.bpe_model.unk_token.empty() || find_token_id(d, d.bpe_model.unk_token) >= 0,
            "tokenizer bpe_model unk_token must exist in tokenizer vocab");
  }
  if (d.pre_tokenizer.enabled && d.pre_tokenizer.byte_level.enabled)
    require(!d.pre_tokenizer.type.empty(), "tokenizer pre_tokenizer must define a type when enabled");
  const std::vector<std::string>& b2u = d.decoder.byte_level.byte_to_unicode;
  if (d.decoder.enabled && d.decoder.byte_level.enabled)
    require(b2u.empty() || b2u.size() == 256,
            "tokenizer decoder byte_to_unicode mapping must contain 256 entries when provided");
}

void StartupValidator::ValidateManifestAndTokenizer(const ManifestData& manifest, const TokenizerRuntimeData& d) {
  const Qwen3Config config = ValidateManifest(manifest);
  ValidateTokenizerRuntime(d);
  if (d.vocab_size <= 0) throw std::runtime_error("tokenizer vocab_size must be positive");
  if (static_cast<std::size_t>(d.vocab_size) > config.vocab_size)
    throw std::runtime_error("tokenizer vocab_size must not exceed qwen3 config vocab_size");
  int max_id = -1;
  for (const AddedTokenRecord& t : d.added_tokens) max_id = std::max(max_id, t.id);
  for (const VocabEntry& t : d.vocab) max_id = std::max(max_id, t.id);
  if (max_id < 0 || static_cast<std::size_t>(max_id) >= config.vocab_size)
    throw std::runtime_error("tokenizer token ids must fit within qwen3 config vocab_size");
}

}  // namespace soc

// ---- C entry points ----
struct soc_tokenizer {
  soc::TokenizerRuntime runtime;
};

namespace {

// Copies `n` items to a caller buffer of `cap` items, reporting the full size in *size either way.
template <typename T>
int copy_out(const T* src, std::size_t n, T* dst, int64_t cap, int64_t* size) {
  *size = static_cast<int64_t>(n);
  if (static_cast<int64_t>(n) > cap) return soc::fail(SOC_ERR_INVALID, "output buffer too small");
  if (n != 0) std::memcpy(dst, src, n * sizeof(T));
  return SOC_OK;
}

}  // namespace

extern "C" {

int soc_tokenizer_load(const char* runtime_path, soc_tokenizer** out) {
  if (runtime_path == nullptr || out == nullptr) return soc::fail(SOC_ERR_INVALID, "null argument");
  *out = nullptr;
  try {
    *out = new soc_tokenizer{soc::TokenizerRuntime(soc::TokenizerRuntimeLoader::LoadFromFile(runtime_path))};
    return SOC_OK;
  } catch (const std::exception& e) {
    return soc::fail(SOC_ERR_INVALID, e.what());
  }
}

int soc_tokenizer_load_bundle(const char* manifest_path, soc_tokenizer** out) {
  if (manifest_path == nullptr || out == nullptr) return soc::fail(SOC_ERR_INVALID, "null argument");
  *out = nullptr;
  try {
    const soc::ManifestData manifest = soc::ManifestLoader::LoadFromFile(manifest_path);
    soc::TokenizerRuntimeData d = soc::TokenizerRuntimeLoader::LoadFromFile(manifest.tokenizer_runtime_file);
    soc::StartupValidator::ValidateManifestAndTokenizer(manifest, d);
    *out = new soc_tokenizer{soc::TokenizerRuntime(std::move(d))};
    return SOC_OK;
  } catch (const std::exception& e) {
    return soc::fail(SOC_ERR_INVALID, e.what());
  }
}

int soc_tokenizer_destroy(soc_tokenizer* tok) {
  delete tok;
  return SOC_OK;
}

int soc_tokenizer_encode(const soc_tokenizer* tok, const char* text, int64_t len, int32_t* ids, int64_t cap,
                         int64_t* n_ids) {
  if (tok == nullptr || (text == nullptr && len != 0) || len < 0 || n_ids == nullptr || (ids == nullptr && cap != 0))
    return soc::fail(SOC_ERR_INVALID, "null argument");
  try {
    const std::vector<int> v = tok->runtime.Encode(std::string(text == nullptr ? "" : text, static_cast<size_t>(len)));
    const std::vector<int32_t> v32(v.begin(), v.end());
    return copy_out(v32.data(), v32.size(), ids, cap, n_ids);
  } catch (const std::exception& e) {
    return soc::fail(SOC_ERR_INVALID, e.what());
  }
}

int soc_tokenizer_decode(const soc_tokenizer* tok, const int32_t* ids, int64_t n, char* text, int64_t cap,
                         int64_t* len) {
  if (tok == nullptr || (ids == nullptr && n != 0) || n < 0 || len == nullptr || (text == nullptr && cap != 0))
    return soc::fail(SOC_ERR_INVALID, "null argument");
  try {
    const std::string s = tok->runtime.Decode(std::vector<int>(ids, ids + n));
    return copy_out(s.data(), s.size(), text, cap, len);
  } catch (const std::exception& e) {
    return soc::fail(SOC_ERR_INVALID, e.what());
  }
}

int soc_tokenizer_token_to_id(const soc_tokenizer* tok, const char* token, int64_t len, int32_t* id) {
  if (tok == nullptr || token == nullptr || len < 0 || id == nullptr) return soc::fail(SOC_ERR_INVALID, "null argument");
  try {
    *id = tok->runtime.TokenToId(std::string(token, static_cast<size_t>(len)));
    return SOC_OK;
  } catch (const std::exception& e) {
    return soc::fail(SOC_ERR_INVALID, e.what());
  }
}

int soc_tokenizer_chat_prompt(const soc_tokenizer* tok, const char* const* roles, const char* const* contents,
                              int32_t n_messages, int add_generation_prompt, int enable_thinking,
                              const char* system_prompt_override, char* text, int64_t cap, int64_t* len) {
  if (tok == nullptr || n_messages < 0 || (n_messages > 0 && (roles == nullptr || contents == nullptr)) ||
      len == nullptr || (text == nullptr && cap != 0))
    return soc::fail(SOC_ERR_INVALID, "null argument");
  try {
    std::vector<soc::ChatMessage> msgs;
    for (int32_t i = 0; i < n_messages; ++i) {
      if (roles[i] == nullptr || contents[i] == nullptr) return soc::fail(SOC_ERR_INVALID, "null message");
      msgs.push_back(soc::ChatMessage{roles[i], contents[i]});
    }
    const soc::Qwen3TemplateBuilder b(tok->runtime.runtime_data().template_runtime);
    const std::string s = b.BuildPrompt(msgs, add_generation_prompt != 0, enable_thinking != 0,
                                        system_prompt_override == nullptr ? "" : system_prompt_override);
    return copy_out(s.data(), s.size(), text, cap, len);
  } catch (const std::exception& e) {
    return soc::fail(SOC_ERR_INVALID, e.what());
  }
}

}  // extern "C"
