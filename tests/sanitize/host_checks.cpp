// host_checks.cpp - drives the library's host-only code and the CPU oracle under AddressSanitizer and
// UndefinedBehaviorSanitizer (built by tests/sanitize/Makefile; run by tests/test_sanitize_cpu.py).
//
// Covered: the JSON parser on valid and mutated documents, the manifest / config / tensor-file loaders on bundles
// written here (valid, truncated, mislabelled), the tokenizer runtime (loader, encode, decode, template, the C entry
// points with short output buffers), the group-64 packer (against the oracle's, bit for bit), the seeded generators,
// and the oracle's forward, cached forward, generation, sampling, attention and quantized matmul on a tiny model.
// Any sanitizer report aborts the program (-fno-sanitize-recover=all); the last line printed names the step.
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <filesystem>
#include <fstream>
#include <random>
#include <stdexcept>
#include <string>
#include <vector>

#include "../../oracle/soc_oracle.h"
#include "soc/assets.h"
#include "soc/tokenizer.h"
#include "soc_hip.h"

namespace fs = std::filesystem;
using soc::JsonParser;

namespace {

int g_fail = 0;
void check(bool ok, const char* what) {
  if (!ok) {
    std::fprintf(stderr, "FAIL: %s\n", what);
    ++g_fail;
  }
}
void step(const char* name) {
  std::printf("step: %s\n", name);
  std::fflush(stdout);
}

template <typename F>
bool throws(F&& f) {
  try {
    f();
  } catch (const std::exception&) {
    return true;
  }
  return false;
}

std::string b2u(int b) {  // GPT-2 byte-level symbol of byte b, UTF-8
  const bool kept = (b >= '!' && b <= '~') || (b >= 161 && b <= 172) || (b >= 174);
  int cp = b;
  if (!kept) {
    int extra = 0;
    for (int x = 0; x < b; ++x)
      if (!((x >= '!' && x <= '~') || (x >= 161 && x <= 172) || (x >= 174))) ++extra;
    cp = 256 + extra;
  }
  std::string u;
  if (cp < 0x80) {
    u.push_back(static_cast<char>(cp));
  } else {
    u.push_back(static_cast<char>(0xC0 | (cp >> 6)));
    u.push_back(static_cast<char>(0x80 | (cp & 0x3F)));
  }
  return u;
}

void json_checks(std::mt19937_64& rng) {
  step("json");
  const std::vector<std::string> docs = {
      R"({"a":[1,2.5e3,-0.0,true,false,null,"xé😀\n"],"b":{"c":{"d":[[],{}]}}})",
      R"([{"id":1,"token":"\"q\""},{"id":2,"token":"\\"}])",
      R"({"format":"soc.cpp.llm_export","format_version":2,"tensors":[{"name":"w","shape":[2,3]}]})"};
  for (const std::string& d : docs) check(!throws([&] { JsonParser::Parse(d); }), "valid JSON parses");
  std::uniform_int_distribution<int> byte(0, 255);
  const std::string alphabet = "{}[]\",:0123456789.eE+-truefalsn \\u";
  for (int it = 0; it < 20000; ++it) {
    std::string s = docs[it % docs.size()];
    const int edits = 1 + static_cast<int>(rng() % 4);
    for (int e = 0; e < edits && !s.empty(); ++e) {
      const size_t pos = rng() % s.size();
      switch (rng() % 4) {
        case 0: s[pos] = static_cast<char>(byte(rng)); break;
        case 1: s.erase(pos, 1 + rng() % 3); break;
        case 2: s.insert(pos, 1, alphabet[rng() % alphabet.size()]); break;
        default: s.resize(pos); break;
      }
    }
    try {
      const soc::JsonValue v = JsonParser::Parse(s);
      if (v.is_object() && v.contains("a")) (void)v.at("a");
    } catch (const std::exception&) {
    }
  }
  check(throws([] { JsonParser::Parse(std::string(100000, '[')); }), "deep nesting is rejected, not recursed into");
  check(throws([] { JsonParser::Parse("1e400").as_int(); }) || true, "huge numbers");
  check(throws([] { JsonParser::Parse("1e30").as_int64(); }), "out-of-range int64 is an error");
  check(throws([] { JsonParser::Parse("-3e9").as_int(); }), "out-of-range int is an error");
  check(JsonParser::Parse("-7.9").as_int() == -7, "as_int truncates toward zero");
}

void write_file(const fs::path& p, const void* data, size_t n) {
  fs::create_directories(p.parent_path());
  std::ofstream f(p, std::ios::binary);
  f.write(static_cast<const char*>(data), static_cast<std::streamsize>(n));
}

void bundle_checks(const fs::path& dir) {
  step("bundle");
  const int V = 32, H = 128, I = 64;
  const std::string config = R"({"model_type":"qwen3","hidden_size":128,"intermediate_size":64,"num_hidden_layers":1,)"
                             R"("num_attention_heads":1,"num_key_value_heads":1,"head_dim":128,"rms_norm_eps":1e-6,)"
                             R"("rope_theta":1000000,"tie_word_embeddings":true,"torch_dtype":"float16","vocab_size":32})";
  soc::Qwen3Config cfg = soc::Qwen3Config::FromJson(JsonParser::Parse(config));
  std::string tensors;
  int idx = 0;
  for (const auto& [name, shape] : soc::Qwen3TensorShapes(cfg)) {
    size_t n = 1;
    for (size_t d : shape) n *= d;
    const std::string dtype = idx % 3 == 0 ? "float32" : idx % 3 == 1 ? "bfloat16" : "float16";
    const size_t width = dtype == "float32" ? 4 : 2;
    std::vector<uint8_t> bytes(n * width);
    for (size_t i = 0; i < bytes.size(); ++i) bytes[i] = static_cast<uint8_t>((i * 37 + idx) & 0x3F);
    const std::string file = "weights/t" + std::to_string(idx) + ".bin";
    write_file(dir / file, bytes.data(), bytes.size() - (name == "model.norm.weight" ? 2 : 0));  // one short file
    tensors += std::string(idx ? "," : "") + R"({"name":")" + name + R"(","file":")" + file + R"(","dtype":")" +
               dtype + R"(","shape":[)";
    for (size_t d = 0; d < shape.size(); ++d) tensors += (d ? "," : "") + std::to_string(shape[d]);
    tensors += R"(],"byte_size":)" + std::to_string(bytes.size()) + R"(,"source_shard":"s"})";
    ++idx;
  }
  const std::string manifest = R"({"format":"soc.cpp.llm_export","format_version":2,"export_dtype":"float16",)"
                               R"("tokenizer_runtime_file":"tokenizer/tokenizer_runtime.json","config":)" +
                               config + R"(,"tensors":[)" + tensors + "]}";
  write_file(dir / "manifest.json", manifest.data(), manifest.size());
  const soc::ManifestData m = soc::ManifestLoader::LoadFromFile((dir / "manifest.json").string());
  check(soc::StartupValidator::ValidateManifest(m).vocab_size == static_cast<size_t>(V), "manifest validates");
  int loaded = 0, rejected = 0;
  for (const auto& [name, shape] : soc::Qwen3TensorShapes(cfg)) {
    try {
      const std::vector<uint16_t> v = soc::WeightLoader::LoadFloat16(m, name, shape);
      loaded += v.empty() ? 0 : 1;
    } catch (const std::exception&) {
      ++rejected;
    }
  }
  check(rejected == 1 && loaded + rejected == idx, "the short file is rejected, the rest load");
  check(throws([&] { soc::WeightLoader::LoadFloat16(m, "model.embed_tokens.weight", {V, H + 1}); }),
        "a wrong expected shape is rejected");
  soc_bundle* b = nullptr;
  check(soc_bundle_open((dir / "manifest.json").string().c_str(), &b) == SOC_OK, "soc_bundle_open");
  std::vector<uint16_t> e(static_cast<size_t>(V) * H);
  check(soc_bundle_tensor_f16(b, "model.embed_tokens.weight", e.data(), static_cast<int64_t>(e.size())) == SOC_OK,
        "soc_bundle_tensor_f16");
  check(soc_bundle_tensor_f16(b, "model.embed_tokens.weight", e.data(), 5) != SOC_OK, "numel mismatch rejected");
  soc_bundle_close(b);
  (void)I;
}

soc::TokenizerRuntimeData random_runtime(std::mt19937_64& rng, bool byte_level) {
  soc::TokenizerRuntimeData d;
  d.format = "soc.cpp.tokenizer_runtime";
  d.format_version = 1;
  d.template_runtime = {"qwen3", "<|im_start|>", "<|im_end|>", "<think>", "</think>", "You are helpful."};
  std::vector<std::string> syms;
  for (int b = 0; b < 256; ++b) syms.push_back(byte_level ? b2u(b) : std::string(1, static_cast<char>(b)));
  const std::string pre = rng() % 3 == 0 ? "##" : "";
  const std::string suf = rng() % 3 == 0 ? "</w>" : "";
  d.bpe_model.enabled = true;
  d.bpe_model.type = "bpe";
  d.bpe_model.continuing_subword_prefix = pre;
  d.bpe_model.end_of_word_suffix = suf;
  std::vector<std::string> toks = syms;
  for (const std::string& s : syms) {
    toks.push_back(pre + s);
    toks.push_back(s + suf);
    toks.push_back(pre + s + suf);
  }
  for (int i = 0; i < 300; ++i) {  // random merges over existing tokens; results join the vocabulary
    const std::string& l = toks[rng() % toks.size()];
    const std::string& r = toks[rng() % toks.size()];
    d.bpe_model.merges.push_back({l, r});
    toks.push_back(l + r);
  }
  if (rng() % 2) {
    d.bpe_model.unk_token = "<unk>";
    toks.push_back("<unk>");
  }
  for (size_t i = 0; i < toks.size(); ++i)
    if (rng() % 50 != 0 || toks[i] == "<unk>") d.vocab.push_back({static_cast<int>(i), toks[i]});
  const int n = static_cast<int>(toks.size());
  d.added_tokens = {{n, "<|im_start|>"}, {n + 1, "<|im_end|>"}, {n + 2, "<think>"}, {n + 3, "</think>"}};
  d.vocab_size = n + 4;
  d.pre_tokenizer.enabled = true;
  d.pre_tokenizer.type = "ByteLevel";
  d.pre_tokenizer.byte_level.enabled = byte_level;
  d.pre_tokenizer.byte_level.add_prefix_space = rng() % 2;
  d.pre_tokenizer.byte_level.use_regex = rng() % 4 != 0;
  d.decoder.enabled = true;
  d.decoder.byte_level.enabled = byte_level;
  if (byte_level)
    for (int b = 0; b < 256; ++b) d.decoder.byte_level.byte_to_unicode.push_back(b2u(b));
  d.decoder.bpe.enabled = !suf.empty();
  d.decoder.bpe.suffix = suf;
  return d;
}

void tokenizer_checks(std::mt19937_64& rng) {
  step("tokenizer");
  int encoded = 0, errors = 0;
  for (int t = 0; t < 40; ++t) {
    const soc::TokenizerRuntime tok(random_runtime(rng, t % 3 != 0));
    for (int it = 0; it < 200; ++it) {
      std::string text;
      const int len = static_cast<int>(rng() % 40);
      for (int i = 0; i < len; ++i) {
        const uint64_t r = rng() % 10;
        if (r == 0) text += "<|im_start|>";
        else if (r == 1) text += "<think>";
        else text.push_back(static_cast<char>(rng() & 0xFF));  // any byte, invalid UTF-8 included
      }
      try {
        const std::vector<int> ids = tok.Encode(text);
        const std::string back = tok.Decode(ids);
        (void)back;
        ++encoded;
      } catch (const std::exception&) {
        ++errors;
      }
      std::vector<int> ids;
      for (int i = 0; i < 8; ++i) ids.push_back(static_cast<int>(rng() % (tok.runtime_data().vocab_size + 3)) - 1);
      try {
        (void)tok.Decode(ids);
      } catch (const std::exception&) {
      }
    }
  }
  check(encoded > 1000, "most random texts encode");
  const soc::TokenizerRuntime tok(random_runtime(rng, true));
  const soc::TokenizerRuntime copy = tok;
  check(copy.Encode("hello <think> world") == tok.Encode("hello <think> world"), "copies encode alike");
  soc::Qwen3TemplateBuilder tb(tok.runtime_data().template_runtime);
  check(!tb.BuildPrompt({{"user", "x"}}, true, true).empty(), "template builds");

  // the C entry points, including short output buffers
  const fs::path p = fs::temp_directory_path() / "soc_sanitize_tok.json";
  {
    std::ofstream f(p);
    f << R"({"format":"soc.cpp.tokenizer_runtime","format_version":1,"tokenizer_class":"X","vocab_size":6,)"
      << R"("model_max_length":1e30,"added_tokens":[{"id":5,"content":"<|im_start|>","special":true,)"
      << R"("single_word":false,"lstrip":false,"rstrip":false,"normalized":false}],"vocab":[{"id":0,"token":"a"},)"
      << R"({"id":1,"token":"b"}],"template_runtime":{"type":"qwen3","im_start":"<|im_start|>","im_end":"<|im_end|>",)"
      << R"("think_start":"<think>","think_end":"</think>","default_system_prompt":"S"}})";
  }
  soc_tokenizer* h = nullptr;
  check(soc_tokenizer_load(p.string().c_str(), &h) != SOC_OK, "model_max_length 1e30 is rejected, not cast");
  {
    std::ofstream f(p);
    f << R"({"format":"soc.cpp.tokenizer_runtime","format_version":1,"tokenizer_class":"X","vocab_size":6,)"
      << R"("model_max_length":128,"added_tokens":[{"id":5,"content":"<|im_start|>","special":true,)"
      << R"("single_word":false,"lstrip":false,"rstrip":false,"normalized":false}],"vocab":[{"id":0,"token":"a"},)"
      << R"({"id":1,"token":"b"}],"template_runtime":{"type":"qwen3","im_start":"<|im_start|>","im_end":"<|im_end|>",)"
      << R"("think_start":"<think>","think_end":"</think>","default_system_prompt":"S"}})";
  }
  check(soc_tokenizer_load(p.string().c_str(), &h) == SOC_OK, "soc_tokenizer_load");
  int32_t ids[4];
  int64_t n = 0;
  check(soc_tokenizer_encode(h, "ab<|im_start|>a", 15, ids, 2, &n) != SOC_OK && n == 4, "short id buffer");
  check(soc_tokenizer_encode(h, "ab<|im_start|>a", 15, ids, 4, &n) == SOC_OK && ids[2] == 5, "encode");
  char text[8];
  check(soc_tokenizer_decode(h, ids, 4, text, 3, &n) != SOC_OK && n == 15, "short text buffer");
  const char* roles[] = {"user"};
  const char* contents[] = {"hi"};
  check(soc_tokenizer_chat_prompt(h, roles, contents, 1, 1, 1, nullptr, nullptr, 0, &n) != SOC_OK && n > 0,
        "chat prompt size query");
  std::vector<char> buf(static_cast<size_t>(n));
  check(soc_tokenizer_chat_prompt(h, roles, contents, 1, 1, 1, nullptr, buf.data(), n, &n) == SOC_OK, "chat");
  soc_tokenizer_destroy(h);
  fs::remove(p);
}

void quant_checks(std::mt19937_64& rng) {
  step("quantize");
  for (const int bits : {8, 4}) {
    const int64_t N = 37, K = 192;
    std::vector<uint16_t> w(N * K);
    for (auto& x : w) {
      const uint64_t r = rng() % 100;
      x = r < 5 ? 0 : r < 10 ? static_cast<uint16_t>(rng() % 0x400) : static_cast<uint16_t>(rng() & 0x7BFF);
      if (rng() % 2) x |= 0x8000;
    }
    for (int64_t i = 0; i < K; ++i) w[3 * K + i] = 0;  // an all-zero row
    const size_t cb = bits == 8 ? N * K : N * K / 2;
    std::vector<uint8_t> c1(cb), c2(cb);
    std::vector<uint16_t> s1(N * K / 64), s2(N * K / 64);
    check(soc_quantize_group(w.data(), N, K, bits, c1.data(), s1.data()) == SOC_OK, "soc_quantize_group");
    check(orc_quantize_group(w.data(), N, K, bits, c2.data(), s2.data()) == 0, "orc_quantize_group");
    check(c1 == c2 && s1 == s2, "packer equals the oracle bit for bit");
    w[7] = 0x7C00;  // inf
    check(soc_quantize_group(w.data(), N, K, bits, c1.data(), s1.data()) != SOC_OK, "inf is rejected");
    w[7] = 0x7E00;  // NaN
    check(orc_quantize_group(w.data(), N, K, bits, c2.data(), s2.data()) != 0, "NaN is rejected by the oracle");
  }
  std::vector<uint16_t> a(4 * 128), sc(8 * 2);
  std::vector<uint8_t> codes(8 * 128);
  for (auto& x : a) x = static_cast<uint16_t>(rng() & 0x3BFF);
  for (auto& x : sc) x = static_cast<uint16_t>(0x1000 + rng() % 0x800);
  for (auto& x : codes) x = static_cast<uint8_t>(rng());
  std::vector<float> y(4 * 8), wd(8 * 128);
  check(orc_qmm_group(a.data(), 4, 128, codes.data(), 8, sc.data(), 64, 8, y.data()) == 0, "orc_qmm_group int8");
  check(orc_qmm_group(a.data(), 4, 128, codes.data(), 4, sc.data(), 64, 8, y.data()) == 0, "orc_qmm_group int4");
  check(orc_dequant_group(codes.data(), 4, sc.data(), 64, 8, 128, wd.data()) == 0, "orc_dequant_group");
}

void synth_checks() {
  step("synth");
  std::vector<uint16_t> h(1000);
  std::vector<int32_t> t(1000);
  std::vector<uint8_t> c(1000);
  check(soc_synth_normal_f16(1, "w", 0.02f, 17, 1000, h.data()) == SOC_OK, "normal");
  check(soc_synth_uniform_f16(1, "u", -1.0f, 1.0f, 0, 1000, h.data()) == SOC_OK, "uniform");
  check(soc_synth_tokens(1, "t", 151936, 1000, t.data()) == SOC_OK, "tokens");
  check(soc_synth_int_uniform(1, "i", 64, 4096, 1000, t.data()) == SOC_OK, "int uniform");
  check(soc_synth_codes(1, "c", 4, 1000, c.data()) == SOC_OK, "codes");
  check(soc_synth_tokens(1, "t", 0, 10, t.data()) != SOC_OK, "empty vocabulary rejected");
}

void oracle_checks(std::mt19937_64& rng) {
  step("oracle model");
  orc_set_threads(4);
  const int64_t V = 96, H = 128, L = 2, NQ = 2, NKV = 1, D = 128, I = 96;
  for (const int tie : {1, 0}) {
    orc_model* m = orc_model_create(V, H, L, NQ, NKV, D, I, 1e6, 1e-6f, tie);
    check(m != nullptr, "orc_model_create");
    std::vector<std::vector<uint16_t>> keep;
    const auto put = [&](const std::string& name, int64_t n, bool gain) {
      keep.emplace_back(static_cast<size_t>(n));
      if (gain)
        std::fill(keep.back().begin(), keep.back().end(), static_cast<uint16_t>(0x3C00));
      else
        soc_synth_normal_f16(7, name.c_str(), 0.05f, 0, n, keep.back().data());
      check(orc_model_set(m, name.c_str(), keep.back().data(), n) == 0, name.c_str());
    };
    put("model.embed_tokens.weight", V * H, false);
    put("model.norm.weight", H, true);
    if (!tie) put("lm_head.weight", V * H, false);
    for (int64_t l = 0; l < L; ++l) {
      const std::string p = "model.layers." + std::to_string(l) + ".";
      put(p + "input_layernorm.weight", H, true);
      put(p + "post_attention_layernorm.weight", H, true);
      put(p + "self_attn.q_norm.weight", D, true);
      put(p + "self_attn.k_norm.weight", D, true);
      put(p + "self_attn.q_proj.weight", NQ * D * H, false);
      put(p + "self_attn.k_proj.weight", NKV * D * H, false);
      put(p + "self_attn.v_proj.weight", NKV * D * H, false);
      put(p + "self_attn.o_proj.weight", H * NQ * D, false);
      put(p + "mlp.gate_proj.weight", I * H, false);
      put(p + "mlp.up_proj.weight", I * H, false);
      put(p + "mlp.down_proj.weight", H * I, false);
    }
    check(orc_model_check(m) == 0, "orc_model_check");
    std::vector<int32_t> ids(9);
    for (auto& x : ids) x = static_cast<int32_t>(rng() % V);
    std::vector<float> logits(ids.size() * V), hidden(ids.size() * H);
    check(orc_forward_logits(m, ids.data(), 9, 0, logits.data(), hidden.data()) == 0, "orc_forward_logits");
    orc_cache* c = orc_cache_create(m, 32);
    std::vector<float> last(V);
    check(orc_forward_logits_cached(m, c, ids.data(), 9, 0, 1, last.data()) == 0, "cached prefill");
    check(orc_cache_length(c) == 9, "cache length");
    const int32_t one = ids[0];
    check(orc_forward_logits_cached(m, c, &one, 1, 9, 1, last.data()) == 0, "cached decode");
    check(orc_forward_logits_cached(m, c, ids.data(), 9, 30, 1, last.data()) != 0, "cache overflow rejected");
    orc_cache_destroy(c);
    std::vector<int32_t> out(6);
    std::vector<float> steps(6 * V);
    check(orc_generate(m, ids.data(), 9, 6, -1, 16, 1.0f, 1, out.data(), steps.data()) == 6, "greedy generate");
    check(orc_generate(m, ids.data(), 9, 6, out[2], 16, 0.7f, 5, out.data(), nullptr) >= 1, "top-k generate");
    int32_t bad = static_cast<int32_t>(V);
    check(orc_forward_logits(m, &bad, 1, 0, logits.data(), nullptr) != 0, "out-of-range id rejected");
    orc_model_destroy(m);
  }
  step("oracle ops");
  std::vector<float> row(1000);
  for (auto& x : row) x = static_cast<float>(rng() % 7);  // many ties
  std::vector<int32_t> tid(50);
  std::vector<float> tv(50);
  check(orc_sample(row.data(), 1000, 1.0f, 1) >= 0, "orc_sample");
  check(orc_sample_topk(row.data(), 1000, 0.5f, 50, tid.data(), tv.data()) >= 0, "orc_sample_topk");
  const int64_t T = 5, S = 8, nq = 4, nkv = 2, d = 16;
  std::vector<float> q(T * nq * d), k(S * nkv * d), v(S * nkv * d), o(T * nq * d);
  for (auto* vec : {&q, &k, &v})
    for (auto& x : *vec) x = static_cast<float>(static_cast<int64_t>(rng() % 200) - 100) / 50.0f;
  check(orc_gqa(q.data(), k.data(), v.data(), T, S, nq, nkv, d, 3, 1, o.data()) == 0, "orc_gqa causal");
  check(orc_gqa(q.data(), k.data(), v.data(), T, S, nq, nkv, d, 0, 0, o.data()) == 0, "orc_gqa full");
  std::vector<float> x(3 * 64), y(3 * 64);
  std::vector<uint16_t> g(64, 0x3C00);
  orc_rmsnorm_f16(x.data(), 3, 64, g.data(), 1e-6f, y.data());  // all-zero rows
  orc_rope(q.data(), T, nq, d, 1e6, 4093);
  for (uint32_t h = 0; h < 65536; ++h) (void)orc_f16_to_f32(static_cast<uint16_t>(h));
  for (const float f : {0.0f, -0.0f, 1e-8f, 65504.0f, 65520.0f, 1e10f, INFINITY, NAN}) (void)orc_f32_to_f16(f);
}

}  // namespace

int main(int argc, char** argv) {
  const fs::path dir = argc > 1 ? fs::path(argv[1]) : fs::temp_directory_path() / "soc_sanitize";
  std::mt19937_64 rng(12345);
  try {
    json_checks(rng);
    bundle_checks(dir / "bundle");
    tokenizer_checks(rng);
    quant_checks(rng);
    synth_checks();
    oracle_checks(rng);
  } catch (const std::exception& e) {
    std::fprintf(stderr, "FAIL: unexpected exception: %s\n", e.what());
    return 1;
  }
  if (g_fail != 0) {
    std::fprintf(stderr, "%d checks failed\n", g_fail);
    return 1;
  }
  std::printf("host_checks: all passed\n");
  return 0;
}
