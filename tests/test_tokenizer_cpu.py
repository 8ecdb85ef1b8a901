"""Tokenizer runtime and chat template: the oracle pinned, then the product (soc_tokenizer_* through the C ABI, and the
C++ classes through tests/cpp/test_tokenizer.cpp) checked against it. Host only.

The oracle (oracle/tokenizer.py) restates Mac/cpu/src/tokenizer_runtime.cpp and runtime_assets.cpp:218-257; it is
pinned here by
  * the reference's own expectations (test_model_bootstrap.cpp:169-280, test_runtime_assets.cpp:166-239);
  * the GPT-2 byte table of `transformers` (convert_slow_tokenizer.bytes_to_unicode);
  * the BPE of the `tokenizers` library, whose merge order (lowest rank, leftmost first) the reference shares, on
    random merge tables over one byte-level piece;
  * a regular expression that states the pre-tokenizer split independently of its loop.
"""
from __future__ import annotations

import json
import random
import re
import shutil
import subprocess
from pathlib import Path

import pytest

from oracle import tokenizer as OT

ROOT = Path(__file__).resolve().parents[1]
B2U = OT.gpt2_byte_to_unicode()


# ---------------------------------------------------------------- the oracle against fixed points
def minimal_runtime() -> OT.RuntimeData:  # test_model_bootstrap.cpp:102-137
    d = OT.RuntimeData()
    d.added_tokens = [(10, b"<|im_start|>"), (11, b"<|im_end|>"), (12, b"<think>"), (13, b"</think>")]
    d.vocab = list(enumerate([b"system\n", b"assistant\n", b"user\n", b"You are a helpful assistant.", b"Hello",
                              b" world", b"Say hello.", b"Now think first.", b"\n", b"Hello."]))
    return d


def test_oracle_reference_minimal_case():
    t = OT.Tokenizer(minimal_runtime())
    text = b"<|im_start|>user\nSay hello.<|im_end|>\n<|im_start|>assistant\nHello world<|im_end|>\n"
    ids = t.encode(text)
    assert ids == [10, 2, 6, 11, 8, 10, 1, 4, 5, 11, 8]
    assert t.decode(ids) == text
    with pytest.raises(ValueError, match="byte offset 0"):
        t.encode(b"unencodable-token")


def test_oracle_reference_bpe_cases():
    d = minimal_runtime()  # test_model_bootstrap.cpp:189-226
    d.added_tokens = []
    d.vocab = list(enumerate([b"h", b"e", b"l", b"o", b" ", b"w", b"r", b"d", b"he", b"ll", b"hell", b"hello",
                              b" world"]))
    d.bpe_enabled = True
    d.merges = [(b"h", b"e"), (b"l", b"l"), (b"he", b"ll"), (b"hell", b"o"), (b" ", b"w"), (b" w", b"o"),
                (b" wo", b"r"), (b" wor", b"l"), (b" worl", b"d")]
    t = OT.Tokenizer(d)
    assert t.encode(b"hello world") == [11, 12]
    assert t.decode([11, 12]) == b"hello world"

    g = "Ġ".encode()  # test_model_bootstrap.cpp:228-280
    d.vocab = list(enumerate([g + b"h", b"e", b"l", b"o", g + b"w", b"r", b"d", g + b"he", b"ll", g + b"hell",
                              g + b"hello", g + b"wo", g + b"wor", g + b"worl", g + b"world"]))
    d.merges = [(g, b"h"), (g + b"h", b"e"), (b"l", b"l"), (g + b"he", b"ll"), (g + b"hell", b"o"), (g, b"w"),
                (g + b"w", b"o"), (g + b"wo", b"r"), (g + b"wor", b"l"), (g + b"worl", b"d")]
    d.pre_enabled = d.pre_byte_level = d.add_prefix_space = d.use_regex = True
    d.dec_byte_level = True
    d.byte_to_unicode = B2U
    t = OT.Tokenizer(d)
    assert t.encode(b"hello world") == [10, 14]
    assert t.decode([10, 14]) == b" hello world"


def test_oracle_template_reference_case():  # test_runtime_assets.cpp:166-197
    tr = OT.TemplateRuntime()
    msgs = [("user", "Say hello."), ("assistant", "Hello."), ("user", "Now think first.")]
    p = OT.build_prompt(tr, msgs, True, True)
    assert "<|im_start|>system\nYou are a helpful assistant.<|im_end|>" in p
    assert "<|im_start|>user\nSay hello.<|im_end|>" in p
    assert p.endswith("<|im_start|>assistant\n<think>\n")
    q = OT.build_prompt(tr, msgs, True, False, "Custom system prompt.")
    assert "Custom system prompt." in q and "<think>" not in q


def test_oracle_generation_options_reference_case():  # test_runtime_assets.cpp:199-214
    o = OT.generation_options({"max_new_tokens": 12, "temperature": 0.7, "top_k": 4, "eos_token_id": [151645],
                               "max_length": 1024})
    assert (o["max_new_tokens"], o["top_k"], o["eos_token_id"], o["max_sequence_length"]) == (12, 4, 151645, 1024)


def test_oracle_byte_table_is_gpt2():
    from transformers.convert_slow_tokenizer import bytes_to_unicode

    ref = bytes_to_unicode()
    assert [ref[b].encode() for b in range(256)] == B2U
    assert len(set(B2U)) == 256


def test_oracle_pretokenizer_matches_regex():
    """Each piece is optional whitespace plus one run of letters, digits or other non-space bytes; whitespace at the
    end stands alone (C-locale classes, which is what re.ASCII gives on bytes)."""
    split = re.compile(rb"\s*(?:[A-Za-z]+|[0-9]+|[^\sA-Za-z0-9]+)|\s+", re.ASCII)
    d = OT.RuntimeData(pre_enabled=True, pre_byte_level=True, use_regex=True)
    t = OT.Tokenizer(d)
    rng = random.Random(5)
    alphabet = [b" ", b"\t", b"\n", b"\r", b"\x0b", b"\x0c", b"a", b"Z", b"q", b"0", b"7", b".", b"!", b"_",
                b"\xc3", b"\xa9", b"\x00", b"\x7f"]
    for _ in range(3000):
        s = b"".join(rng.choice(alphabet) for _ in range(rng.randint(1, 24)))
        assert t._pre_tokenize(s) == split.findall(s), s
    # prefix space: added in front of a first piece that does not start with whitespace
    d.add_prefix_space = True
    assert OT.Tokenizer(d)._pre_tokenize(b"ab cd") == [b" ab", b" cd"]
    assert OT.Tokenizer(d)._pre_tokenize(b" ab") == [b" ab"]


def _random_merges(rng, n_words=40, n_merges=120):
    """A merge table learned greedily from random words over a small alphabet (all results in the vocabulary)."""
    words = ["".join(rng.choice("abcdeé中 ") for _ in range(rng.randint(2, 9))) for _ in range(n_words)]
    seqs = [[B2U[b].decode() for b in w.encode()] for w in words]
    merges = []
    for _ in range(n_merges):
        counts = {}
        for s in seqs:
            for p in zip(s, s[1:]):
                counts[p] = counts.get(p, 0) + 1
        if not counts:
            break
        best = max(counts.items(), key=lambda kv: (kv[1], kv[0]))[0]
        merges.append(best)
        for s in seqs:
            i = 0
            while i < len(s) - 1:
                if (s[i], s[i + 1]) == best:
                    s[i:i + 2] = [s[i] + s[i + 1]]
                i += 1
    return merges


def test_oracle_bpe_merge_matches_tokenizers_library():
    tokenizers = pytest.importorskip("tokenizers")
    from tokenizers import models, pre_tokenizers

    rng = random.Random(11)
    for trial in range(6):
        merges = _random_merges(rng)
        vocab = {u.decode(): i for i, u in enumerate(B2U)}
        for l, r in merges:
            vocab.setdefault(l + r, len(vocab))
        hf = tokenizers.Tokenizer(models.BPE(vocab=vocab, merges=merges))
        hf.pre_tokenizer = pre_tokenizers.ByteLevel(add_prefix_space=False, use_regex=False)
        d = OT.RuntimeData(bpe_enabled=True, pre_enabled=True, pre_byte_level=True, use_regex=False,
                           dec_byte_level=True, byte_to_unicode=B2U,
                           vocab=[(i, t.encode()) for t, i in vocab.items()],
                           merges=[(l.encode(), r.encode()) for l, r in merges])
        t = OT.Tokenizer(d)
        for _ in range(150):
            s = "".join(rng.choice("abcdeé中 xy") for _ in range(rng.randint(1, 30)))
            assert t.encode(s.encode()) == hf.encode(s).ids, (trial, s)
            assert t.decode(t.encode(s.encode())) == s.encode()


# ---------------------------------------------------------------- the product against the oracle
def _json_runtime(d: OT.RuntimeData, vocab_size: int) -> dict:
    s = lambda b: b.decode("utf-8", errors="surrogateescape") if isinstance(b, bytes) else b
    obj = {
        "format": "soc.cpp.tokenizer_runtime", "format_version": 1, "tokenizer_class": "Qwen2TokenizerFast",
        "vocab_size": vocab_size, "model_max_length": 4096,
        "added_tokens": [{"id": i, "content": s(c), "special": True, "single_word": False, "lstrip": False,
                          "rstrip": False, "normalized": False} for i, c in d.added_tokens],
        "vocab": [{"id": i, "token": s(t)} for i, t in d.vocab],
        "chat_template": None,
        "template_runtime": {"type": "qwen3", "im_start": "<|im_start|>", "im_end": "<|im_end|>",
                             "think_start": "<think>", "think_end": "</think>",
                             "default_system_prompt": "You are a helpful assistant."},
    }
    if d.bpe_enabled:
        obj["bpe_model"] = {"type": "bpe", "unk_token": s(d.unk_token) or None,
                            "continuing_subword_prefix": s(d.continuing_subword_prefix),
                            "end_of_word_suffix": s(d.end_of_word_suffix),
                            "merges": [{"left": s(l), "right": s(r)} for l, r in d.merges]}
    if d.pre_enabled:
        obj["pre_tokenizer"] = {"type": "ByteLevel", "byte_level": {
            "enabled": d.pre_byte_level, "add_prefix_space": d.add_prefix_space, "use_regex": d.use_regex}}
    obj["decoder"] = {"type": "ByteLevel",
                      "byte_level": {"enabled": d.dec_byte_level, "byte_to_unicode": [s(u) for u in d.byte_to_unicode]},
                      "bpe": {"enabled": d.dec_bpe_enabled, "suffix": s(d.dec_bpe_suffix)}}
    return obj


def _random_runtime(rng: random.Random) -> OT.RuntimeData:
    """A random byte-level or plain BPE tokenizer with optional prefix/suffix markers, unk token and added tokens.
    All strings are valid UTF-8 so that they survive JSON."""
    byte_level = rng.random() < 0.7
    prefix = rng.choice([b"", b"", b"##"])
    suffix = rng.choice([b"", b"", b"</w>"])
    merges = _random_merges(rng, n_merges=rng.randint(10, 150))
    if not byte_level:  # plain mode: symbols are raw ASCII bytes, so keep to ASCII words
        merges = [(l, r) for l, r in merges if all(ord(c) < 128 for c in l + r)]
    d = OT.RuntimeData(bpe_enabled=True, pre_enabled=True, pre_byte_level=byte_level,
                       add_prefix_space=rng.random() < 0.5, use_regex=rng.random() < 0.7,
                       dec_byte_level=byte_level, byte_to_unicode=B2U if byte_level else [],
                       continuing_subword_prefix=prefix, end_of_word_suffix=suffix,
                       dec_bpe_enabled=bool(suffix), dec_bpe_suffix=suffix)
    d.merges = [(l.encode(), r.encode()) for l, r in merges]
    base = [u for u in B2U] if byte_level else [bytes([b]) for b in range(32, 127)] + [b"\n", b"\t"]
    toks = []
    for b in base:  # every symbol shape the marker rules can produce
        toks += [b, prefix + b, b + suffix, prefix + b + suffix]
    for l, r in d.merges:
        toks.append(l + r)
    if rng.random() < 0.5:
        d.unk_token = b"<unk>"
        toks.append(b"<unk>")
        if not byte_level:  # leave some bytes out so that unk is used
            toks = [t for t in toks if b"q" not in t]
    seen, vocab = set(), []
    for t in toks:
        if t not in seen:
            seen.add(t)
            vocab.append((len(vocab), t))
    d.vocab = vocab
    n = len(vocab)
    d.added_tokens = [(n, b"<|im_start|>"), (n + 1, b"<|im_end|>"), (n + 2, b"<think>"), (n + 3, b"</think>")]
    return d


def _random_text(rng: random.Random, byte_level: bool) -> bytes:
    parts = ["ab", "cde", " ", "  ", "\n", "\t", "x", "7", "42", ".", "!?", "<|im_start|>", "<|im_end|>", "<think>",
             "q", "Q"]
    if byte_level:
        parts += ["é", "中", "\U0001F600"]
    return "".join(rng.choice(parts) for _ in range(rng.randint(0, 14))).encode()


@pytest.fixture(scope="module")
def product():
    import soc_amd as S

    return S


def test_product_tokenizer_matches_oracle_on_random_tokenizers(product, tmp_path):
    rng = random.Random(2024)
    checked = 0
    for trial in range(30):
        d = _random_runtime(rng)
        path = tmp_path / f"tok{trial}.json"
        path.write_text(json.dumps(_json_runtime(d, len(d.vocab) + 4), ensure_ascii=False), encoding="utf-8")
        ours = product.Tokenizer(path)
        ref = OT.Tokenizer(OT.load_runtime(path))
        for _ in range(60):
            text = _random_text(rng, bool(d.byte_to_unicode))
            try:
                want = ref.encode(text)
            except ValueError as e:
                with pytest.raises(product.SocError, match=re.escape(str(e).split(":")[0])):
                    ours.encode(text)
                continue
            got = ours.encode(text)
            assert got == want, (trial, text)
            assert ours.decode(got) == ref.decode(want), (trial, text)
            checked += 1
        ids = [i for i, _ in d.vocab[:50]] + [i for i, _ in d.added_tokens]
        rng.shuffle(ids)
        assert ours.decode(ids) == ref.decode(ids)
    assert checked > 1000


def test_product_tokenizer_plain_longest_match_and_errors(product, tmp_path):
    d = minimal_runtime()
    path = tmp_path / "minimal.json"
    path.write_text(json.dumps(_json_runtime(d, 16)), encoding="utf-8")
    tok = product.Tokenizer(path)
    text = b"<|im_start|>user\nSay hello.<|im_end|>\n<|im_start|>assistant\nHello world<|im_end|>\n"
    assert tok.encode(text) == [10, 2, 6, 11, 8, 10, 1, 4, 5, 11, 8]
    assert tok.decode(tok.encode(text)) == text
    assert tok.token_to_id("<|im_start|>") == 10
    assert tok.encode(b"") == []
    with pytest.raises(product.SocError, match="cannot encode input at byte offset 5"):
        tok.encode(b"Hello-")
    with pytest.raises(product.SocError, match="unknown token id: 99"):
        tok.decode([4, 99])
    with pytest.raises(product.SocError, match="unknown token content"):
        tok.token_to_id("nope")


def test_product_chat_prompt_matches_oracle(product, tmp_path):
    d = minimal_runtime()
    path = tmp_path / "minimal.json"
    path.write_text(json.dumps(_json_runtime(d, 16)), encoding="utf-8")
    tok = product.Tokenizer(path)
    tr = OT.TemplateRuntime()
    cases = [([("user", "Say hello.")], True, True, None),
             ([("user", "Say hello."), ("assistant", "Hello."), ("user", "Now think first.")], True, False, "Sys."),
             ([("system", "S"), ("user", "U")], False, True, None),
             ([], True, True, None)]
    for msgs, gen, think, sp in cases:
        want = OT.build_prompt(tr, msgs, gen, think, sp or "").encode()
        assert tok.chat_prompt(msgs, gen, think, sp) == want
    # the chat layout of the reference's minimal case round-trips through the longest-match tokenizer
    p = tok.chat_prompt([("user", "Say hello.")], True, False)
    assert tok.decode(tok.encode(p)) == p


def test_product_tokenizer_from_bundle_validates(product, tmp_path):
    import numpy as np

    from tests.bundle import config_dict, write_bundle

    d = minimal_runtime()
    cfg = product.QwenConfig(vocab_size=16, hidden_size=128, num_hidden_layers=1, num_attention_heads=1,
                             num_key_value_heads=1, intermediate_size=64, head_dim=128)
    embed = {"model.embed_tokens.weight": (np.zeros((16, 128), np.float32), "float16")}
    man = write_bundle(tmp_path / "b", config_dict(cfg), embed, tokenizer_runtime=_json_runtime(d, 16))
    tok = product.Tokenizer.from_bundle(man)
    assert tok.encode(b"Hello world") == [4, 5]
    man2 = write_bundle(tmp_path / "b2", config_dict(cfg), embed, tokenizer_runtime=_json_runtime(d, 17))
    with pytest.raises(product.SocError, match="must not exceed qwen3 config vocab_size"):
        product.Tokenizer.from_bundle(man2)
    d.added_tokens.append((16, b"<extra>"))  # an id outside the model's vocabulary
    man3 = write_bundle(tmp_path / "b3", config_dict(cfg), embed, tokenizer_runtime=_json_runtime(d, 16))
    with pytest.raises(product.SocError, match="token ids must fit"):
        product.Tokenizer.from_bundle(man3)


def test_cpp_tokenizer_program(tmp_path):
    """tests/cpp/test_tokenizer.cpp: the reference's tokenizer, template, loader and pipeline-helper tests restated
    against the C++ headers."""
    exe = ROOT / "tests" / "cpp" / "test_tokenizer"
    if not exe.exists():
        if shutil.which("g++") is None:
            pytest.skip("g++ not available to build tests/cpp/test_tokenizer.cpp")
        pkg = ROOT / "soc_amd"
        exe = tmp_path / "test_tokenizer"
        subprocess.run(["g++", "-O1", "-std=c++17", f"-I{ROOT / 'include'}", str(ROOT / "tests/cpp/test_tokenizer.cpp"),
                        f"-L{pkg}", "-lsoc_hip", f"-Wl,-rpath,{pkg}", "-o", str(exe)], check=True)
    r = subprocess.run([str(exe), str(tmp_path)], capture_output=True, text=True, timeout=60)
    assert r.returncode == 0, r.stderr + r.stdout
