"""Pure-Python restatement of the reference tokenizer runtime and chat template. TEST INFRASTRUCTURE ONLY.

Only tests/ may import this module; the product tokenizer is soc_amd/csrc/tokenizer.cpp behind the C ABI.

It follows the reference statement by statement, in its own loop structure (a scan of the length-sorted token list
for longest matches, a full rescan of adjacent pairs after every BPE merge), so that it checks the product's
hash-set and heap formulation rather than repeating it:
  * TokenizerRuntime            Mac/cpu/src/tokenizer_runtime.cpp:8-379
  * Qwen3TemplateBuilder        Mac/cpu/src/runtime_assets.cpp:218-257
  * TokenizerRuntimeLoader      Mac/cpu/src/runtime_assets.cpp:29-137, 170-216
  * GenerationOptionsFromManifest / PreparePrompt   Mac/cpu/src/runtime_pipeline.cpp:5-74

The reference's C++ cannot be compiled here (its JSON layer, which the tokenizer headers include, needs a standard
library that accepts a map of an incomplete type), so this restatement is pinned instead by the reference's own test
expectations (Mac/cpu/test/test_model_bootstrap.cpp:168-290, test_runtime_assets.cpp:80-239), by the GPT-2 byte table
and BPE merge order of the `tokenizers` library where the two algorithms coincide, and by a regular-expression
statement of the pre-tokenizer split (tests/test_tokenizer_cpu.py).

Text is handled as bytes throughout, as the reference handles std::string.
"""
from __future__ import annotations

import json
from dataclasses import dataclass, field
from pathlib import Path


@dataclass
class TemplateRuntime:  # runtime_assets.h:44-51
    type: str = "qwen3"
    im_start: str = "<|im_start|>"
    im_end: str = "<|im_end|>"
    think_start: str = "<think>"
    think_end: str = "</think>"
    default_system_prompt: str = "You are a helpful assistant."


@dataclass
class RuntimeData:  # runtime_assets.h:104-119, only the fields encoding and decoding read
    added_tokens: list = field(default_factory=list)   # [(id, content bytes)]
    vocab: list = field(default_factory=list)          # [(id, token bytes)]
    bpe_enabled: bool = False
    unk_token: bytes = b""
    continuing_subword_prefix: bytes = b""
    end_of_word_suffix: bytes = b""
    merges: list = field(default_factory=list)         # [(left bytes, right bytes)]
    pre_enabled: bool = False
    pre_byte_level: bool = False
    add_prefix_space: bool = False
    use_regex: bool = True
    dec_byte_level: bool = False
    byte_to_unicode: list = field(default_factory=list)  # 256 bytes objects (UTF-8 of the mapped code point)
    dec_bpe_enabled: bool = False
    dec_bpe_suffix: bytes = b""
    template: TemplateRuntime = field(default_factory=TemplateRuntime)


def gpt2_byte_to_unicode() -> list[bytes]:
    """The byte-level table (Mac/cpu/test/test_model_bootstrap.cpp:19-64, convert_py_to_cpp.py:27-42): printable
    Latin-1 bytes map to themselves, the other 68 bytes to U+0100.. in byte order; UTF-8 encoded."""
    keep = list(range(ord("!"), ord("~") + 1)) + list(range(161, 173)) + list(range(174, 256))
    out = [b""] * 256
    extra = 0
    for b in range(256):
        if b in keep:
            out[b] = chr(b).encode()
        else:
            out[b] = chr(256 + extra).encode()
            extra += 1
    return out


def _isspace(c: int) -> bool:  # std::isspace in the "C" locale
    return c in (0x20, 0x09, 0x0A, 0x0B, 0x0C, 0x0D)


def _isalpha(c: int) -> bool:
    return 0x41 <= c <= 0x5A or 0x61 <= c <= 0x7A


def _isdigit(c: int) -> bool:
    return 0x30 <= c <= 0x39


class Tokenizer:
    """TokenizerRuntime (tokenizer_runtime.cpp)."""

    def __init__(self, d: RuntimeData):
        self.d = d
        self.token_to_id: dict[bytes, int] = {}
        self.id_to_token: dict[int, bytes] = {}
        ordered, protected = [], []
        self.added_ids = set()
        for tid, content in d.added_tokens:  # :8-15, emplace keeps the first
            self.token_to_id.setdefault(content, tid)
            self.id_to_token.setdefault(tid, content)
            ordered.append(content)
            protected.append(content)
            self.added_ids.add(tid)
        for tid, tok in d.vocab:  # :17-21
            self.token_to_id.setdefault(tok, tid)
            self.id_to_token.setdefault(tid, tok)
            ordered.append(tok)
        key = lambda t: (-len(t), t)  # :23-28 longer first, then lexicographic
        self.ordered = sorted(set(ordered), key=key)
        self.protected = sorted(set(protected), key=key)
        self.merge_ranks: dict[bytes, int] = {}
        for i, (l, r) in enumerate(d.merges):  # :40-43
            self.merge_ranks.setdefault(l + b"\n" + r, i)
        self.unicode_to_byte: dict[bytes, int] = {}
        for b, u in enumerate(d.byte_to_unicode):  # :45-47
            self.unicode_to_byte.setdefault(u, b)

    def token_to_id_of(self, tok: bytes) -> int:  # :98-104
        if tok not in self.token_to_id:
            raise ValueError("unknown token content: " + tok.decode(errors="replace"))
        return self.token_to_id[tok]

    @staticmethod
    def _match(tokens, text: bytes, off: int) -> bytes:  # :114-144
        for t in tokens:
            if not t or off + len(t) > len(text):
                continue
            if text[off:off + len(t)] == t:
                return t
        return b""

    def encode(self, text: bytes) -> list[int]:  # :54-80
        ids, off = [], 0
        while off < len(text):
            m = self._match(self.protected if self.d.bpe_enabled else self.ordered, text, off)
            if m:
                ids.append(self.token_to_id_of(m))
                off += len(m)
                continue
            if not self.d.bpe_enabled:
                raise ValueError(f"tokenizer runtime cannot encode input at byte offset {off}")
            nxt = len(text)  # :146-156
            for t in self.protected:
                if not t:
                    continue
                p = text.find(t, off)
                if p != -1 and p < nxt:
                    nxt = p
            ids += self._encode_bpe(text[off:nxt])
            off = nxt
        return ids

    def _encode_bpe(self, text: bytes) -> list[int]:  # :158-183
        if not text:
            return []
        ids = []
        for piece in self._pre_tokenize(text):
            for sym in self._merge(self._symbols(piece)):
                if sym in self.token_to_id:
                    ids.append(self.token_to_id[sym])
                elif self.d.unk_token:
                    ids.append(self.token_to_id_of(self.d.unk_token))
                else:
                    raise ValueError("tokenizer runtime cannot encode BPE symbol: " + sym.decode(errors="replace"))
        return ids

    def _pre_tokenize(self, text: bytes) -> list[bytes]:  # :185-231
        d = self.d
        if not d.pre_enabled or not d.pre_byte_level:
            return [text]
        pieces = []
        if not d.use_regex:
            pieces.append(text)
        else:
            i = 0
            while i < len(text):
                start = i
                while i < len(text) and _isspace(text[i]):
                    i += 1
                if i == len(text):
                    pieces.append(text[start:])
                    break
                if _isalpha(text[i]):
                    while i < len(text) and _isalpha(text[i]):
                        i += 1
                elif _isdigit(text[i]):
                    while i < len(text) and _isdigit(text[i]):
                        i += 1
                else:
                    while i < len(text) and not _isspace(text[i]) and not (_isalpha(text[i]) or _isdigit(text[i])):
                        i += 1
                pieces.append(text[start:i])
        if pieces and d.add_prefix_space and pieces[0] and not _isspace(pieces[0][0]):
            pieces[0] = b" " + pieces[0]
        return pieces

    def _symbols(self, text: bytes) -> list[bytes]:  # :233-269
        d = self.d
        byte_level = d.pre_byte_level and len(d.byte_to_unicode) > 0
        out = []
        for i, b in enumerate(text):
            s = d.byte_to_unicode[b] if byte_level else bytes([b])
            if d.continuing_subword_prefix and out:
                s = d.continuing_subword_prefix + s
            if d.end_of_word_suffix and i + 1 == len(text):
                s = s + d.end_of_word_suffix
            out.append(s)
        return out

    def _merge(self, sym: list[bytes]) -> list[bytes]:  # :271-304
        if len(sym) < 2 or not self.merge_ranks:
            return sym
        sym = list(sym)
        while len(sym) > 1:
            best_i, best_r = len(sym), None
            for i in range(len(sym) - 1):
                r = self.merge_ranks.get(sym[i] + b"\n" + sym[i + 1])
                if r is None:
                    continue
                if best_r is None or r < best_r:
                    best_r, best_i = r, i
            if best_i == len(sym):
                break
            sym[best_i] = sym[best_i] + sym[best_i + 1]
            del sym[best_i + 1]
        return sym

    def decode(self, ids) -> bytes:  # :82-96
        out = b""
        first = True
        for tid in ids:
            if tid not in self.id_to_token:
                raise ValueError(f"unknown token id: {tid}")
            tok = self.id_to_token[tid]
            if tid in self.added_ids:
                out += tok
                continue
            out += self._decode_model_token(tok, first)
            first = False
        return out

    def _decode_model_token(self, tok: bytes, first: bool) -> bytes:  # :306-342
        d = self.d
        append_space = False
        if d.dec_bpe_enabled and d.dec_bpe_suffix and tok.endswith(d.dec_bpe_suffix):
            tok = tok[: len(tok) - len(d.dec_bpe_suffix)]
            append_space = True
        if not first and d.continuing_subword_prefix and tok.startswith(d.continuing_subword_prefix):
            tok = tok[len(d.continuing_subword_prefix):]
        if d.dec_byte_level and self.unicode_to_byte:
            out, off = b"", 0
            while off < len(tok):
                lead = tok[off]
                w = 1 if lead & 0x80 == 0 else 2 if lead & 0xE0 == 0xC0 else 3 if lead & 0xF0 == 0xE0 else \
                    4 if lead & 0xF8 == 0xF0 else 1
                cp = tok[off:off + w]
                out += bytes([self.unicode_to_byte[cp]]) if cp in self.unicode_to_byte else cp
                off += w
            tok = out
        if append_space:
            tok += b" "
        return tok


def build_prompt(t: TemplateRuntime, messages, add_generation_prompt: bool, enable_thinking: bool,
                 system_prompt_override: str = "") -> str:
    """Qwen3TemplateBuilder::BuildPrompt (runtime_assets.cpp:221-257)."""
    prompt = ""
    has_system = False
    for role, content in messages:
        if role == "system":
            has_system = True
        prompt += t.im_start + role + "\n" + content + t.im_end + "\n"
    if not has_system:
        sp = system_prompt_override if system_prompt_override else t.default_system_prompt
        prompt = t.im_start + "system\n" + sp + t.im_end + "\n" + prompt
    if add_generation_prompt:
        prompt += t.im_start + "assistant\n"
        if enable_thinking:
            prompt += t.think_start + "\n"
    return prompt


def runtime_from_json(obj: dict) -> RuntimeData:
    """RuntimeData from a parsed tokenizer_runtime.json (runtime_assets.cpp:170-216), byte strings UTF-8 encoded."""
    e = lambda s: s.encode()
    d = RuntimeData()
    d.added_tokens = [(a["id"], e(a["content"])) for a in obj["added_tokens"]]
    d.vocab = [(v["id"], e(v["token"])) for v in obj["vocab"]]
    tr = obj["template_runtime"]
    d.template = TemplateRuntime(tr["type"], tr["im_start"], tr["im_end"], tr["think_start"], tr["think_end"],
                                 tr["default_system_prompt"])
    m = obj.get("bpe_model")
    if m is not None:
        d.bpe_enabled = True
        d.unk_token = e(m.get("unk_token") or "")
        d.continuing_subword_prefix = e(m.get("continuing_subword_prefix") or "")
        d.end_of_word_suffix = e(m.get("end_of_word_suffix") or "")
        d.merges = [(e(r["left"]), e(r["right"])) for r in m["merges"]]
    p = obj.get("pre_tokenizer")
    if p is not None:
        d.pre_enabled = True
        bl = p.get("byte_level")
        if bl is not None:
            d.pre_byte_level = bl.get("enabled", True)
            d.add_prefix_space = bl.get("add_prefix_space", False)
            d.use_regex = bl.get("use_regex", True)
    dec = p2 = obj.get("decoder")
    if dec is not None:
        bl = dec.get("byte_level")
        if bl is not None:
            d.dec_byte_level = bl.get("enabled", True)
            d.byte_to_unicode = [e(s) for s in (bl.get("byte_to_unicode") or [])]
        b = p2.get("bpe")
        if b is not None:
            d.dec_bpe_enabled = b.get("enabled", True)
            d.dec_bpe_suffix = e(b.get("suffix") or "")
    return d


def load_runtime(path) -> RuntimeData:
    return runtime_from_json(json.loads(Path(path).read_text(encoding="utf-8")))


def generation_options(generation_config) -> dict:
    """RuntimePipeline::GenerationOptionsFromManifest (runtime_pipeline.cpp:5-56): defaults 32 new tokens,
    temperature 1, top_k 1, eos -1 (the first entry of a list), max_length 256."""
    o = {"max_new_tokens": 32, "temperature": 1.0, "top_k": 1, "eos_token_id": -1, "max_sequence_length": 256}
    g = generation_config
    if not isinstance(g, dict):
        return o
    if "max_new_tokens" in g:
        o["max_new_tokens"] = int(g["max_new_tokens"])
    if "temperature" in g:
        o["temperature"] = float(g["temperature"])
    if "top_k" in g:
        o["top_k"] = int(g["top_k"])
    if "eos_token_id" in g:
        v = g["eos_token_id"]
        o["eos_token_id"] = (int(v[0]) if v else -1) if isinstance(v, list) else int(v)
    if "max_length" in g:
        o["max_sequence_length"] = int(g["max_length"])
    return o
