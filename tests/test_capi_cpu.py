"""CPU-side checks of the drop-in boundary: the C-ABI library loads, exports every declared symbol, rejects bad
arguments without a GPU, and the seeded generator follows its written specification."""
import re
import shutil
import subprocess
from pathlib import Path

import numpy as np
import pytest

import soc_amd as S
from soc_amd import capi

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "soc_hip.h"
CPP_HEADER = ROOT / "include" / "soc" / "gpu" / "runtime.h"


def declared_c_functions():
    text = HEADER.read_text()
    return sorted(set(re.findall(r"^\s*(?:int|const char\*|uint16_t)\s+(soc_\w+)\s*\(", text, re.M)))


def test_library_exports_every_declared_c_symbol():
    L = S.lib()
    names = declared_c_functions()
    assert len(names) >= 30
    missing = [n for n in names if not hasattr(L, n)]
    assert not missing, missing


@pytest.mark.skipif(shutil.which("nm") is None, reason="nm not available")
def test_library_exports_cpp_host_interface():
    out = subprocess.run(["nm", "-DC", "--defined-only", str(capi.LIB_PATH)], capture_output=True, text=True,
                         check=True).stdout
    text = CPP_HEADER.read_text()
    # every out-of-line method declared in runtime.h (those ending in ';' with a parameter list and no body)
    methods = {
        "soc::gpu::HipContext::CreateDefault", "soc::gpu::HipContext::Synchronize",
        "soc::gpu::HipBuffer::CreateShared", "soc::gpu::HipBuffer::Wrap", "soc::gpu::HipBuffer::Write",
        "soc::gpu::HipBuffer::Read", "soc::gpu::GetDataTypeSize", "soc::gpu::TensorDesc::CreateContiguous",
        "soc::gpu::TensorDesc::CreateStrided", "soc::gpu::TensorDesc::ElementCount", "soc::gpu::TensorDesc::ByteSize",
        "soc::gpu::DeviceTensor::IsValid",
        "soc::gpu::BufferArena::CreateShared", "soc::gpu::BufferArena::Allocate", "soc::gpu::BufferArena::ResetToMark",
        "soc::gpu::BufferArena::ClearTelemetry", "soc::gpu::BufferArenaMarkGuard::BufferArenaMarkGuard",
        "soc::gpu::QwenModelLoader::LoadModel", "soc::gpu::QwenModelLoader::SynthesizeModel",
        "soc::gpu::QwenCausalLM::ForwardLogitsCached",
        "soc::gpu::KVCache::CreateShared", "soc::gpu::KVCache::Reserve", "soc::gpu::KVCache::AppendPrefill",
        "soc::gpu::KVCache::AppendDecodeToken", "soc::gpu::KVCache::ViewForLayer", "soc::gpu::KVCache::OnForward",
        "soc::gpu::KVCache::LayersAligned",
        "soc::gpu::CommandScheduler::RunPrefill", "soc::gpu::CommandScheduler::RunDecode",
        "soc::gpu::Sampler::SampleFromLogits", "soc::gpu::GenerationContext::Prefill",
        "soc::gpu::GenerationContext::DecodeNextToken", "soc::gpu::GenerationContext::Generate",
        "soc::gpu::GenerationContext::Reset", "soc::gpu::GenerationContext::GenerationContext",
        "soc::gpu::RuntimePipeline::LoadBundle", "soc::gpu::RuntimePipeline::GenerationOptionsFromManifest",
        "soc::gpu::RuntimePipeline::PreparePrompt",
    }
    for m in methods:
        assert m.split("::")[-1] in text
        assert m + "(" in out, m
    # the tokenizer classes of soc/tokenizer.h and the validator of soc/assets.h
    out = out.replace("[abi:cxx11]", "")
    tok_text = (ROOT / "include" / "soc" / "tokenizer.h").read_text() + (ROOT / "include" / "soc" / "assets.h").read_text()
    for m in ("soc::TokenizerRuntimeLoader::LoadFromFile", "soc::TokenizerRuntime::Encode",
              "soc::TokenizerRuntime::Decode", "soc::TokenizerRuntime::TokenToId", "soc::TokenizerRuntime::IdToToken",
              "soc::TokenizerRuntime::TokenizerRuntime", "soc::Qwen3TemplateBuilder::BuildPrompt",
              "soc::StartupValidator::ValidateTokenizerRuntime", "soc::StartupValidator::ValidateManifestAndTokenizer",
              "soc::StartupValidator::ValidateManifest", "soc::ManifestLoader::LoadFromFile"):
        assert m.split("::")[-1] in tok_text
        assert m + "(" in out, m


def test_calls_without_gpu_fail_cleanly():
    """No GPU in this container: context creation must return an error status, not crash."""
    import ctypes as C

    h = C.c_void_p()
    rc = S.lib().soc_ctx_create(0, C.byref(h))
    if rc == capi.SOC_OK:  # a GPU is present
        S.lib().soc_ctx_destroy(h)
        pytest.skip("GPU present")
    assert rc in (capi.SOC_ERR_HIP, capi.SOC_ERR_INVALID)
    assert S.lib().soc_last_error()
    assert S.lib().soc_ctx_synchronize(None) == capi.SOC_ERR_INVALID


def test_synth_argument_errors():
    with pytest.raises(S.SocError):
        S.synth_codes(1, "x", 3, 16)
    with pytest.raises(S.SocError):
        S.synth_tokens(1, "x", 0, 4)


# ---- the generator specification (soc_amd/csrc/synth.cpp header), restated in numpy ----
M64 = (1 << 64) - 1


def mix64(z):
    z = np.uint64(z)
    with np.errstate(over="ignore"):
        z = (z ^ (z >> np.uint64(30))) * np.uint64(0xBF58476D1CE4E5B9)
        z = (z ^ (z >> np.uint64(27))) * np.uint64(0x94D049BB133111EB)
    return z ^ (z >> np.uint64(31))


def fnv1a64(s: str) -> int:
    h = 0xCBF29CE484222325
    for b in s.encode():
        h ^= b
        h = (h * 0x100000001B3) & M64
    return h


def draws(seed: int, name: str, n: int, offset: int = 0) -> np.ndarray:
    key = int(mix64(np.uint64(seed) ^ mix64(np.uint64(fnv1a64(name)))))
    i = np.arange(offset, offset + n, dtype=np.uint64) + np.uint64(1)
    with np.errstate(over="ignore"):
        return mix64(np.uint64(key) + i * np.uint64(0x9E3779B97F4A7C15))


def test_generator_tokens_and_codes_follow_spec():
    d = draws(7, "prompt", 1000)
    want = ((d >> np.uint64(32)) * np.uint64(151936)) >> np.uint64(32)
    assert np.array_equal(S.synth_tokens(7, "prompt", 151936, 1000), want.astype(np.int32))
    d = draws(3, "c8", 512)
    assert np.array_equal(S.synth_codes(3, "c8", 8, 512), (d & np.uint64(0xFF)).astype(np.uint8))
    d = draws(3, "c4", 512)
    nib = (d & np.uint64(0xF)).astype(np.uint8)
    assert np.array_equal(S.synth_codes(3, "c4", 4, 512), nib[0::2] | (nib[1::2] << 4))


def test_generator_normal_follows_spec():
    from math import erfc, sqrt

    n = 20000
    got = S.synth_normal_f16(11, "model.layers.0.mlp.up_proj.weight", 0.02, n)
    d = draws(11, "model.layers.0.mlp.up_proj.weight", n)
    j = (d >> np.uint64(48)).astype(np.int64)
    vals = got.view(np.float16).astype(np.float64)
    # NORMAL[j] = f16(0.02 * Phi^-1((j + 0.5) / 65536)): Phi(value / 0.02) lands within fp16 rounding of the quantile
    phi = np.array([0.5 * erfc(-v / 0.02 / sqrt(2)) for v in vals[:2000]])
    q = (j[:2000] + 0.5) / 65536.0
    dens = np.exp(-0.5 * (vals[:2000] / 0.02) ** 2) / np.sqrt(2 * np.pi)
    tol = dens * (np.abs(vals[:2000]) / 0.02 * 2.0 ** -10 + 2.0 ** -14 / 0.02) + 1e-9
    assert np.all(np.abs(phi - q) <= tol)
    # monotone in j, antisymmetric table, offsets give the same stream
    order = np.argsort(j)
    assert np.all(np.diff(vals[order]) >= 0)
    assert np.array_equal(S.synth_normal_f16(11, "model.layers.0.mlp.up_proj.weight", 0.02, 100, offset=500),
                          got[500:600])
    # moments of N(0, 0.02)
    assert abs(vals.mean()) < 0.02 * 0.03 and abs(vals.std() / 0.02 - 1) < 0.03


def test_f64_to_f16_rne_matches_numpy():
    rng = np.random.default_rng(0)
    x = np.concatenate([rng.normal(0, 1, 5000), rng.normal(0, 1e-5, 3000), rng.normal(0, 3e4, 2000),
                        [0.0, -0.0, 65504.0, 65519.99, 65520.0, 1e9, 2.0 ** -24, 2.0 ** -25, 3 * 2.0 ** -26,
                         1 + 2.0 ** -11, 1 + 3 * 2.0 ** -11]])
    got = np.array([S.lib().soc_f64_to_f16_rne(float(v)) for v in x], dtype=np.uint16)
    want = x.astype(np.float16).view(np.uint16)
    assert np.array_equal(got, want)
