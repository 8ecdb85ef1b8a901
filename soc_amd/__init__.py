"""soc_amd - MI355X (gfx950) implementation of the SoC runtime's Qwen3 forward hot path.

The product is the C ABI in include/soc_hip.h, implemented by soc_amd/libsoc_hip.so (hand-written HIP kernels plus
a C++ host runtime), with the reference's C++ host classes on top of it in include/soc/. This package holds the
sources, the in-tree build, and a ctypes binding used by the tests and the benchmark.
"""
from .capi import (  # noqa: F401
    QWEN3_0_6B, QWEN3_1_7B, QWEN3_4B, QWEN3_8B, Bundle, Context, Tokenizer, KVCache, Model, QwenConfig, SocError, decode, decode_batch, decode_batch_steps,
    attention_decode, attention_prefill, decode_steps, decode_steps_noalloc, dequant, forward, gemm_f16, gemv_f16,
    lib, load_bundle, prefill, qmm, quantize_group, sample_topk, synth_codes, synth_int_uniform, synth_normal_f16, synth_tokens, synth_uniform_f16,
    synth_weights, tensor_specs,
)
