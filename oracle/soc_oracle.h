/*
 * soc_oracle.h - CPU oracle for the Qwen3 forward hot path.
 *
 * TEST INFRASTRUCTURE ONLY. This library restates, in plain C++, the arithmetic of the reference CPU runtime
 * (SongWooYoung/SoC, Mac/cpu/src) so that the HIP path can be checked against it. Only tests/, the smoke check in
 * __graft_entry__.py and the cpu_baseline leg of bench.py may load it. The product path never calls it.
 *
 * Every function follows the reference's operation order exactly: fp32 activations, fp16 weights decoded to fp32
 * element by element, sequential accumulation from 0.0f with the inner index ascending, double-precision RoPE
 * angles, divide-by-sum softmax. Row loops that are independent of each other may run on several threads; the
 * value of each output element does not depend on the thread count.
 *
 * Parity pins (see tests/test_oracle.py):
 *   orc_f16_to_f32 / orc_f32_to_f16 : exhaustive over all 65,536 codes vs closed form and the compiled reference.
 *   orc_linear_f16, orc_rmsnorm, orc_rope, orc_gqa, orc_sample, model forward / generate :
 *       reference KATs (Mac/cpu/test/test_nn_modules.cpp), closed forms, and golden vectors emitted by the
 *       compiled reference sources (oracle/_ref, fixtures under tests/golden/).
 *   orc_sample_topk : the first id equals orc_sample (pinned above); the ids' values are the k largest of
 *       logit / temperature in non-increasing order; the order among equal values is std::partial_sort's, the very
 *       call the reference makes (Mac/gpu/src/runtime/sampler.cpp:50-55).
 *   orc_quantize_group : matrix_ops.h:42-74 per group of 64 with an fp16 scale; pinned where the fp16 scale is exact
 *       (the int8 codes then equal the reference per-column quantizer's on that group), by the round-trip bound
 *       |w - code * s| <= s / 2 away from the clamp, and against the library's packer bit for bit.
 *   orc_qmm_group : the group-quantized format is not in the reference; pinned by the closed-form dequant
 *       (exact products), by group size 64 == per-row scale when all scales of a row are equal, and by the int8
 *       per-column reference quantizer (Mac/cpu/header/matrix_ops.h:42-74,308-350) through orc_quant_int8_percol.
 */
#ifndef SOC_ORACLE_H
#define SOC_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Mac/cpu/src/dtype.cpp:76-106 */
float orc_f16_to_f32(uint16_t value);
/* Mac/cpu/src/dtype.cpp:115-156 */
uint16_t orc_f32_to_f16(float value);
void orc_f16_to_f32_array(const uint16_t* in, float* out, int64_t n);

/* Mac/cpu/src/linear.cpp:51-84 (no bias; Qwen3 projections have none). x [rows][in], w fp16 [out][in]. */
void orc_linear_f16(const float* x, int64_t rows, int64_t in_dim, const uint16_t* w, int64_t out_dim, float* y);
/* Same loop with an fp32 weight matrix (used for KATs written with fp32 weights). */
void orc_linear_f32(const float* x, int64_t rows, int64_t in_dim, const float* w, int64_t out_dim, float* y);

/* Mac/cpu/src/rms_norm_module.cpp:37-69. x [rows][n], gain fp16 [n]. */
void orc_rmsnorm_f16(const float* x, int64_t rows, int64_t n, const uint16_t* gain, float eps, float* y);
void orc_rmsnorm_f32(const float* x, int64_t rows, int64_t n, const float* gain, float eps, float* y);

/* Mac/cpu/src/rope.cpp:54-89, in place. x [seq][heads][head_dim] (batch 1). */
void orc_rope(float* x, int64_t seq, int64_t heads, int64_t head_dim, double theta, int64_t position_offset);

/* Mac/cpu/src/grouped_query_attention.cpp:59-142 (batch 1).
 * q [T][nq][d], k/v [S][nkv][d], out [T][nq][d]. prefix = number of keys that precede query row 0. */
int orc_gqa(const float* q, const float* k, const float* v, int64_t T, int64_t S, int64_t nq, int64_t nkv,
            int64_t d, int64_t prefix, int causal, float* out);

/* Mac/cpu/src/sampler.cpp:26-61 on one logits row. Returns the token id (-1 on invalid arguments). */
int orc_sample(const float* logits_row, int64_t vocab, float temperature, int64_t top_k);
int orc_quantize_group(const uint16_t* w, int64_t N, int64_t K, int bits, void* codes, uint16_t* scales);
int orc_sample_topk(const float* logits_row, int64_t vocab, float temperature, int64_t top_k, int32_t* ids,
                    float* vals);

/* Mac/cpu/src/qwen_mlp.cpp:20-74 with fp16 weights. x [rows][H] -> y [rows][H]. */
void orc_mlp_f16(const float* x, int64_t rows, int64_t hidden, int64_t inter, const uint16_t* gate,
                 const uint16_t* up, const uint16_t* down, float* y);

/* ---- Model (Mac/cpu/src/qwen_causal_lm.cpp, qwen_block.cpp, qwen_attention.cpp, kv_cache.cpp) ---- */
typedef struct orc_model orc_model;
typedef struct orc_cache orc_cache;

orc_model* orc_model_create(int64_t vocab, int64_t hidden, int64_t layers, int64_t nq, int64_t nkv, int64_t head_dim,
                            int64_t inter, double rope_theta, float eps, int tie_word_embeddings);
void orc_model_destroy(orc_model* m);
/* Borrow an fp16 tensor by its Hugging Face name (Mac/cpu/src/qwen_model_loader.cpp:35-93). 0 = ok. */
int orc_model_set(orc_model* m, const char* name, const uint16_t* data, int64_t numel);
/* fp32 projection weights (dequantized group-quantized ones) that replace the layer's fp16 projection. */
int orc_model_set_f32(orc_model* m, const char* name, const float* data, int64_t numel);
/* 0 when every tensor the config needs is present. */
int orc_model_check(const orc_model* m);

/* Mac/cpu/src/kv_cache.cpp (fp32 store, batch 1). */
orc_cache* orc_cache_create(const orc_model* m, int64_t max_seq);
void orc_cache_destroy(orc_cache* c);
void orc_cache_clear(orc_cache* c);
int64_t orc_cache_length(const orc_cache* c);
/* Set position `pos` of layer `layer` from fp32 key/value rows [nkv][d] (used to seed long KV prefixes). */
int orc_cache_write(orc_cache* c, int64_t layer, int64_t pos, const float* key, const float* value);

/* QwenCausalLM::ForwardLogits (uncached), qwen_causal_lm.cpp:50-70; logits [T][V]; NULL skips them.
 * hidden_out (nullable) receives the final-norm hidden states [T][H]. */
int orc_forward_logits(const orc_model* m, const int32_t* ids, int64_t T, int64_t position_offset, float* logits,
                       float* hidden_out);
/* QwenCausalLM::ForwardLogitsCached, qwen_causal_lm.cpp:74-80. Only the last `logit_rows` rows are computed
 * (the reference computes every row; each row is independent, so the values of the kept rows are unchanged). */
int orc_forward_logits_cached(const orc_model* m, orc_cache* c, const int32_t* ids, int64_t T,
                              int64_t position_offset, int64_t logit_rows, float* logits);

/* GenerationSession::Generate with a greedy sampler (generation_session.cpp:46-79, sampler.cpp:26-61).
 * The first token comes from the prompt's last row; then one cached decode per step.
 * step_logits (nullable) receives [max_new][V]: row 0 = prompt last row, row i = decode step i. */
int orc_generate(const orc_model* m, const int32_t* prompt, int64_t T, int64_t max_new, int eos, int64_t max_seq,
                 float temperature, int64_t top_k, int32_t* out_tokens, float* step_logits);

/* ---- Group-quantized matmul (format defined by this project; see header comment) ----
 * a fp16 [M][K]; codes [N][K] int8, or int4 packed two per byte (even k in the low nibble) -> [N][K/2];
 * scales fp16 [N][K/group]; y fp32 [M][N] = sum_k a[m][k] * (float(code[n][k]) * float(scale[n][k/group])). */
int orc_qmm_group(const uint16_t* a, int64_t M, int64_t K, const void* codes, int bits, const uint16_t* scales,
                  int64_t group, int64_t N, float* y);
/* Dequantize a whole matrix to fp32 [N][K] (the bit-exact dequant contract). */
int orc_dequant_group(const void* codes, int bits, const uint16_t* scales, int64_t group, int64_t N, int64_t K,
                      float* w);

/* Mac/cpu/header/matrix_ops.h:42-74. rhs fp32 [K][N] (row-major, shared_dim rows); codes [N][K]; scales [N]. */
void orc_quant_int8_percol(const float* rhs, int64_t K, int64_t N, int8_t* codes, float* scales);
/* Mac/cpu/header/matrix_ops.h:308-350. a [M][K] fp32. */
void orc_matmul_quant_int8(const float* a, int64_t M, int64_t K, const int8_t* codes, const float* scales, int64_t N,
                           float* y);

/* Threads used by the row-parallel loops (default: 1). Returns the previous value. */
int orc_set_threads(int n);

#ifdef __cplusplus
}
#endif

#endif
