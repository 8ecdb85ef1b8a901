"""Text in, text out on the GPU: a bundle with a byte-level BPE tokenizer runtime and a seeded model.

The prompt goes through the Qwen3 chat template and the tokenizer (soc_tokenizer_*), the model generates greedily on
the device, and the generated ids are decoded back to text. The same steps through the oracle (oracle/tokenizer.py
for the text, the CPU restatement of the forward for the tokens) must give the same prompt ids, generated ids and
text. The C++ program tests/cpp/test_text_generation.cpp runs the reference harness's flow (RuntimePipeline::
LoadBundle, PreparePrompt, TokenizerRuntime, GenerationContext::Generate) on the same bundle and must agree too.
"""
import random
import subprocess
from pathlib import Path

import numpy as np
import pytest

import soc_amd as S
from oracle import tokenizer as OT
from tests.bundle import config_dict, write_bundle
from tests.test_tokenizer_cpu import _json_runtime, _random_merges

pytestmark = pytest.mark.gpu

CPP = Path(__file__).resolve().parent / "cpp"
CFG = S.QwenConfig(vocab_size=768, hidden_size=256, num_hidden_layers=3, num_attention_heads=4,
                   num_key_value_heads=2, intermediate_size=384, tie_word_embeddings=False)
ADDED = [b"<|endoftext|>", b"<|im_start|>", b"<|im_end|>", b"<think>", b"</think>"]


def _runtime(vocab_size: int) -> OT.RuntimeData:
    """Byte-level BPE covering exactly the ids 0..vocab_size-1: 256 byte symbols, learned merges, filler tokens,
    then the added tokens."""
    b2u = OT.gpt2_byte_to_unicode()
    merges = _random_merges(random.Random(3), n_words=120, n_merges=300)
    vocab = [u for u in b2u]
    for l, r in merges:
        t = (l + r).encode()
        if t not in vocab:
            vocab.append(t)
    n_fill = vocab_size - len(ADDED) - len(vocab)
    assert n_fill >= 0
    vocab += [f"<fill{i}>".encode() for i in range(n_fill)]
    d = OT.RuntimeData(bpe_enabled=True, pre_enabled=True, pre_byte_level=True, add_prefix_space=False,
                       use_regex=True, dec_byte_level=True, byte_to_unicode=b2u)
    d.vocab = list(enumerate(vocab))
    d.added_tokens = [(len(vocab) + i, t) for i, t in enumerate(ADDED)]
    d.merges = [(l.encode(), r.encode()) for l, r in merges]
    return d


@pytest.fixture(scope="module")
def text_bundle(tmp_path_factory):
    d = _runtime(CFG.vocab_size)
    im_end = dict((t, i) for i, t in d.added_tokens)[b"<|im_end|>"]
    w = S.synth_weights(CFG, 31)
    root = tmp_path_factory.mktemp("text_bundle")
    man = write_bundle(root, config_dict(CFG), {n: (a.view(np.uint16), "float16") for n, a in w.items()},
                       tokenizer_runtime=_json_runtime(d, CFG.vocab_size),
                       generation_config={"max_new_tokens": 10, "eos_token_id": [im_end], "max_length": 160,
                                          "top_k": 1, "temperature": 1.0})
    return man, d, w, im_end


def _oracle_run(oracle_mod, d, w, text: str, chat: bool, thinking: bool, max_new: int, eos: int):
    tr = OT.TemplateRuntime()
    prompt = OT.build_prompt(tr, [("user", text)], True, thinking) if chat else text
    tok = OT.Tokenizer(d)
    ids = tok.encode(prompt.encode())
    om = oracle_mod.OracleModel(CFG, w)
    try:
        gen, _ = om.generate(np.array(ids, np.int32), max_new, max_seq=160, eos=eos)
    finally:
        om.close()
    gen = gen.tolist()
    return ids, gen, tok.decode(gen)


PROMPTS = [("Say hello to the world, then count 1 2 3.", True, True),
           ("abc  dé 中 x!", True, False),
           ("plain text prompt 42", False, False)]


@pytest.mark.parametrize("text,chat,thinking", PROMPTS)
def test_text_generation_matches_oracle(gpu_ctx, oracle_mod, text_bundle, text, chat, thinking):
    man, d, w, im_end = text_bundle
    tok = S.Tokenizer.from_bundle(man)
    prompt = tok.chat_prompt([("user", text)], True, thinking) if chat else text.encode()
    ids = tok.encode(prompt)
    want_ids, want_gen, want_text = _oracle_run(oracle_mod, d, w, text, chat, thinking, 10, im_end)
    assert ids == want_ids
    m = S.load_bundle(gpu_ctx, man)
    kv = S.KVCache(m, 1, 160)
    try:
        _, t = S.prefill(m, kv, 0, np.array(ids, np.int32))
        gen = [t]
        while len(gen) < 10 and gen[-1] != im_end:
            _, t = S.decode(m, kv, 0, gen[-1])
            gen.append(t)
    finally:
        kv.close()
        m.close()
    print(f"[text] prompt {len(ids)} ids, generated {gen}")
    assert gen == want_gen
    assert tok.decode(gen) == want_text


@pytest.mark.parametrize("text,chat,thinking", PROMPTS[:2])
def test_cpp_text_generation_matches_oracle(oracle_mod, text_bundle, tmp_path, text, chat, thinking):
    exe = CPP / "test_text_generation"
    assert exe.exists(), "build it with `python -m soc_amd.build` (build_cpp_tests)"
    man, d, w, im_end = text_bundle
    out = tmp_path / "t.bin"
    r = subprocess.run([str(exe), str(out), str(man), "1" if chat else "0", "1" if thinking else "0", text],
                       capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stdout + r.stderr
    raw = out.read_bytes()
    ints = lambda off, n: np.frombuffer(raw, np.int32, count=n, offset=4 * off).tolist()
    n0 = ints(0, 1)[0]
    ids = ints(1, n0)
    n1 = ints(1 + n0, 1)[0]
    gen = ints(2 + n0, n1)
    nt = ints(2 + n0 + n1, 1)[0]
    txt = raw[4 * (3 + n0 + n1):4 * (3 + n0 + n1) + nt]
    assert len(raw) == 4 * (3 + n0 + n1) + nt
    want_ids, want_gen, want_text = _oracle_run(oracle_mod, d, w, text, chat, thinking, 10, im_end)
    assert ids == want_ids
    assert gen == want_gen
    assert txt == want_text
