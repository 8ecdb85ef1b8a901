/*
 * soc_hip.h - C ABI of the MI355X (gfx950) Qwen3 forward hot path.
 *
 * Plain C types only (pointers, sizes, integers); no exceptions cross this boundary. Every call returns a status
 * code (SOC_OK == 0) and, on failure, leaves a message for soc_last_error() on the calling thread.
 *
 * The reference runtime (SongWooYoung/SoC, Mac/gpu) exposes these operations as C++ classes; each declaration below
 * names the reference interface it replaces. The C++ host layer in include/soc/ keeps those class names and
 * signatures and calls into this ABI.
 *
 * Data contract: weights are fp16 in the Hugging Face [out][in] layout, activations and logits fp32, token ids
 * int32. Device memory is owned by the library unless an entry point says it takes caller device pointers.
 * Not thread-safe per context; all work of one context runs in order on that context's HIP stream.
 */
#ifndef SOC_HIP_H
#define SOC_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- status ------------------------------------------------------------------------------------------------ */
enum {
  SOC_OK = 0,
  SOC_ERR_INVALID = 1,   /* bad argument, shape, name or dtype (e.g. matmul_op.mm:29-100 validation)          */
  SOC_ERR_STATE = 2,     /* call out of order (decode before prefill, token mismatch: generation_context.cpp:73-84) */
  SOC_ERR_CAPACITY = 3,  /* sequence/KV capacity exceeded (generation_context.cpp:85-90, kv_cache.mm:103-108)   */
  SOC_ERR_HIP = 4,       /* HIP runtime error                                                                  */
  SOC_ERR_NOMEM = 5      /* device allocation failed (buffer_arena.cpp:59-65 "capacity exceeded" analogue)     */
};

/* Element types of caller tensors (Mac/gpu/include/tensor/tensor_desc.h DataType kFloat32 / kFloat16). */
enum { SOC_DTYPE_F32 = 0, SOC_DTYPE_F16 = 1 };

/* Message of the calling thread's last failed call ("" if none). Replaces the `std::string* error_message`
 * out-parameter of every reference GPU entry point (e.g. Mac/gpu/include/runtime/generation_context.h:30-50). */
const char* soc_last_error(void);

/* ---- device context: replaces MetalContext (Mac/gpu/include/metal/metal_context.h; metal_context.mm:78-216) ---- */
typedef struct soc_ctx soc_ctx;
int soc_ctx_create(int device, soc_ctx** out);
int soc_ctx_destroy(soc_ctx* ctx);
/* Host waits for all work queued on the context stream (MetalContext::FinalizeCommandBuffer's wait). */
int soc_ctx_synchronize(soc_ctx* ctx);
/* GPU time between two points of the context stream, from HIP events (metal_context.mm:206-214 GPU ms). */
int soc_ctx_timer_start(soc_ctx* ctx);
int soc_ctx_timer_stop(soc_ctx* ctx, float* ms);

/* ---- device buffers: replaces MetalBuffer::CreateShared / Write / Read (Mac/gpu/include/buffer/metal_buffer.h) ---- */
int soc_buffer_alloc(soc_ctx* ctx, size_t bytes, void** device_ptr);
int soc_buffer_free(soc_ctx* ctx, void* device_ptr);
int soc_buffer_write(soc_ctx* ctx, void* device_dst, const void* host_src, size_t bytes);
int soc_buffer_read(soc_ctx* ctx, void* host_dst, const void* device_src, size_t bytes);
/* soc_buffer_write queued on the context stream without waiting: host_src must stay unchanged until the stream has
 * been synchronised (by soc_ctx_synchronize or any call that returns results). */
int soc_buffer_write_async(soc_ctx* ctx, void* device_dst, const void* host_src, size_t bytes);

/* ---- model: replaces QwenCausalLM + QwenModelLoader (Mac/gpu/include/model/qwen_causal_lm.h:17-95,
 *      Mac/gpu/src/model/qwen_model_loader.cpp:57-192; names/shapes of Mac/cpu/src/qwen_model_loader.cpp:35-93) ---- */
typedef struct soc_qwen_config {
  int32_t vocab_size;
  int32_t hidden_size;
  int32_t num_hidden_layers;
  int32_t num_attention_heads;
  int32_t num_key_value_heads;
  int32_t head_dim;               /* must be 128 */
  int32_t intermediate_size;
  int32_t max_position_embeddings;
  double rope_theta;
  float rms_norm_eps;
  int32_t tie_word_embeddings;
} soc_qwen_config;

typedef struct soc_model soc_model;
int soc_model_create(soc_ctx* ctx, const soc_qwen_config* cfg, soc_model** out);
int soc_model_destroy(soc_model* model);
/* Upload one fp16 tensor by its Hugging Face name ("model.layers.3.self_attn.q_proj.weight", ...). */
int soc_model_load_tensor(soc_model* model, const char* name, const uint16_t* host_fp16, int64_t numel);
/* The same from device memory: `src` holds numel fp32 (SOC_DTYPE_F32, rounded to fp16 to nearest even) or fp16
 * (SOC_DTYPE_F16) elements of one allocation; the copy is finished when the call returns. Serves the reference's model
 * constructor from device tensors (QwenCausalLM(QwenCausalLMWeights, QwenCausalLMParams),
 * Mac/gpu/include/model/qwen_causal_lm.h:40-41). */
int soc_model_load_tensor_device(soc_model* model, const char* name, const void* src, int32_t dtype, int64_t numel);
/* The device address (fp16 storage, Hugging Face [out][in] layout) and element count of one named tensor of the model;
 * the memory belongs to the model. Serves QwenCausalLM::weights() (qwen_causal_lm.h:82) for loaded models. */
int soc_model_tensor(const soc_model* model, const char* name, void** device_ptr, int64_t* numel);
/* Fill every tensor with the seeded generator (soc_synth_normal_f16 with `sigma`; norm gains = 1.0). */
int soc_model_synthesize(soc_model* model, uint64_t seed, float sigma);
/* Validates that every tensor the config needs is present (StartupValidator / loader checks). */
int soc_model_finalize(soc_model* model);
/* A model bundle on disk (the reference's export format: manifest.json + one raw tensor file per weight;
 * Mac/cpu/src/runtime_assets.cpp:138-168, startup_validator.cpp:5-23, qwen3_config.cpp:20-67). Opening parses the
 * manifest and validates it and its Qwen3 config; it needs no GPU. Messages are the reference loaders'. */
typedef struct soc_bundle soc_bundle;
int soc_bundle_open(const char* manifest_path, soc_bundle** out);
int soc_bundle_close(soc_bundle* bundle);
/* The config the bundle describes (max_position_embeddings: the config's value, else 32768). */
int soc_bundle_config(const soc_bundle* bundle, soc_qwen_config* out);
/* One weight of the model as fp16 bits: float16 as stored, float32 and bfloat16 rounded to nearest even, after the
 * checks of weight_loader.cpp:17-30 and qwen_model_loader.cpp:17-25 (byte_size, floating dtype, expected shape). */
int soc_bundle_tensor_f16(const soc_bundle* bundle, const char* name, uint16_t* out, int64_t numel);
/* Creates, fills and finalizes a model from a bundle (QwenModelLoader::LoadModelFromFile, qwen_model_loader.cpp:
 * 35-97): every weight of the config's layer count, lm_head.weight only when the embeddings are not tied. */
int soc_model_load_bundle(soc_ctx* ctx, const char* manifest_path, soc_model** out);
/* The bundle's tokenizer runtime (tokenizer/tokenizer_runtime.json; TokenizerRuntimeLoader and TokenizerRuntime,
 * Mac/cpu/src/runtime_assets.cpp:170-216, tokenizer_runtime.cpp:8-379) and its Qwen3 chat template
 * (Qwen3TemplateBuilder, runtime_assets.cpp:218-257). Host only. soc_tokenizer_load reads one runtime file;
 * soc_tokenizer_load_bundle reads a manifest and the runtime file it names and applies
 * StartupValidator::ValidateManifestAndTokenizer (startup_validator.cpp:74-100). Text is UTF-8 bytes with an explicit
 * length. Outputs go to caller buffers of `cap` items; the full size is always stored (*n_ids, *len) and a buffer that
 * is too small fails with SOC_ERR_INVALID without writing, so a caller can ask with cap 0 first. */
typedef struct soc_tokenizer soc_tokenizer;
int soc_tokenizer_load(const char* runtime_path, soc_tokenizer** out);
int soc_tokenizer_load_bundle(const char* manifest_path, soc_tokenizer** out);
int soc_tokenizer_destroy(soc_tokenizer* tok);
/* TokenizerRuntime::Encode (tokenizer_runtime.cpp:54-80). At most 2 * len + 1 ids (one per byte, plus a prefix
 * space per BPE segment). */
int soc_tokenizer_encode(const soc_tokenizer* tok, const char* text, int64_t len, int32_t* ids, int64_t cap,
                         int64_t* n_ids);
/* TokenizerRuntime::Decode (tokenizer_runtime.cpp:82-96). */
int soc_tokenizer_decode(const soc_tokenizer* tok, const int32_t* ids, int64_t n, char* text, int64_t cap,
                         int64_t* len);
/* TokenizerRuntime::TokenToId (tokenizer_runtime.cpp:98-104). */
int soc_tokenizer_token_to_id(const soc_tokenizer* tok, const char* token, int64_t len, int32_t* id);
/* Qwen3TemplateBuilder::BuildPrompt over n_messages (role, content) pairs; system_prompt_override may be NULL. */
int soc_tokenizer_chat_prompt(const soc_tokenizer* tok, const char* const* roles, const char* const* contents,
                              int32_t n_messages, int add_generation_prompt, int enable_thinking,
                              const char* system_prompt_override, char* text, int64_t cap, int64_t* len);
/* Group-64 weight packer (the reference's only quantizer, QuantizeMatMulRhs8, Mac/cpu/header/matrix_ops.h:42-74,
 * applied per 64 weights of a row with the scale kept in fp16): for each row of w [n][k] (fp16 bits, k % 64 == 0) and
 * group of 64, s = fp16(max |w| / Q) with Q = 127 (bits 8) or 7 (bits 4), code = clamp(round(w / s), -Q, Q) (round
 * half away from zero; an all-zero group, or one whose scale rounds to 0, gets scale 0 and codes 0). codes: int8
 * [n][k], or int4 [n][k / 2] two per byte with the even k in the low nibble; scales: fp16 [n][k / 64]. Host only. */
int soc_quantize_group(const uint16_t* w, int64_t n, int64_t k, int32_t bits, void* codes, uint16_t* scales);
/* Packs every projection of a finalized model (q/k/v, o, gate/up, down) with soc_quantize_group; afterwards prefill
 * and decode run those projections as group-quantized matmuls (soc_qmm's kernels) on fp16 activation rows, with
 * the embedding, norms, attention and LM head unchanged. Quantized models decode on the per-operator path (no
 * one-launch kernels) and do not support the ragged batch. No counterpart in the reference. */
int soc_model_quantize(soc_model* model, int32_t bits);
/* Bytes of weights held on the device. */
int soc_model_weight_bytes(const soc_model* model, int64_t* bytes);
/* Which decode implementation soc_decode / soc_decode_steps use on this device: 2 = one kernel launch per token
 * (soc_decode) or per up to 128 tokens (soc_decode_steps) with every layer split over the 8 XCDs (k_decode_xcd;
 * models with 8 KV heads), 1 = one kernel launch per token with
 * dedicated attention blocks (k_decode_persistent), 0 = the per-operator kernel sequence replayed as a HIP graph.
 * Diagnostics only; the reference has no counterpart (it has one decode implementation per backend). */
int soc_model_decode_path(soc_model* model, int32_t* path);

/* ---- KV cache: replaces KVCache (Mac/gpu/include/runtime/kv_cache.h:23-79; kv_cache.mm:32-204).
 *      fp16, `num_slots` independent sequences of `capacity` positions each. ---- */
typedef struct soc_kv soc_kv;
int soc_kv_create(soc_model* model, int32_t num_slots, int32_t capacity, soc_kv** out);
/* The same from dimensions alone (KVCache::CreateShared(context, layers, kv_heads, head_dim, max_sequence_length),
 * kv_cache.h:23-30): the cache is bound to the first model that runs a forward on it, which must have these
 * dimensions; head_dim must be 128. */
int soc_kv_create_dims(soc_ctx* ctx, int32_t layers, int32_t kv_heads, int32_t head_dim, int32_t num_slots,
                       int32_t capacity, soc_kv** out);
int soc_kv_destroy(soc_kv* kv);
/* Length (number of cached positions) of one slot; reset sets it to 0 (GenerationContext::Reset). */
int soc_kv_length(const soc_kv* kv, int32_t slot, int32_t* length);
int soc_kv_reset(soc_kv* kv, int32_t slot);
/* Write fp32 key/value rows [nkv][head_dim] of one position (stored as fp16) and extend the length to pos+1
 * (TensorKVCache::Write, Mac/cpu/src/kv_cache.cpp:50-78). Used to seed long prefixes. */
int soc_kv_write(soc_kv* kv, int32_t slot, int32_t layer, int32_t pos, const float* key, const float* value);
/* Fill positions [0, length) of a slot in every layer with seeded N(0,1) fp16 keys/values and set the length. */
int soc_kv_fill_synthetic(soc_kv* kv, int32_t slot, int32_t length, uint64_t seed);
/* Read back fp16 K and V of one (slot, layer) as [nkv][length][head_dim] (nullable destinations). */
int soc_kv_read(const soc_kv* kv, int32_t slot, int32_t layer, uint16_t* keys, uint16_t* values);
/* Device rows keys/values [rows][kv_heads * head_dim] (SOC_DTYPE_F32 or _F16, device memory) into positions
 * [pos, pos + rows) of one (slot, layer), stored as fp16 (KVCache::AppendPrefill / AppendDecodeToken,
 * kv_cache.mm:78-131). The slot length is not changed (soc_kv_set_length); returns when the copy is done. */
int soc_kv_append(soc_kv* kv, int32_t slot, int32_t layer, int32_t pos, int32_t rows, const void* keys,
                  const void* values, int32_t dtype);
/* Sets the cached length of a slot (0 <= length <= capacity). */
int soc_kv_set_length(soc_kv* kv, int32_t slot, int32_t length);
/* Device addresses of one (slot, layer)'s fp16 key and value planes, [kv_heads][capacity][head_dim] each
 * (KVCache::ViewForLayer, kv_cache.mm:133-143; nullable outputs). */
int soc_kv_layer_planes(const soc_kv* kv, int32_t slot, int32_t layer, void** keys, void** values);

/* ---- forward: replaces CommandScheduler::RunPrefill / RunDecode (Mac/gpu/include/runtime/command_scheduler.h:14-35)
 *      -> QwenCausalLM::ForwardLogitsCached (Mac/gpu/src/model/qwen_causal_lm.cpp:250-268) ---- */
/* Runs `n` tokens of one slot at positions [position_offset, position_offset + n), appending their K/V.
 * position_offset must equal the slot's current length. Writes the fp32 logits of the last `logit_rows` rows
 * (nullable; host or device memory) and the greedy next token from the last row (nullable). */
int soc_prefill(soc_model* model, soc_kv* kv, int32_t slot, const int32_t* token_ids, int32_t n,
                int32_t position_offset, int32_t logit_rows, float* logits, int32_t* next_token);
/* The model's forward in every form of QwenCausalLM (Mac/gpu/include/model/qwen_causal_lm.h:47-80,
 * qwen_causal_lm.cpp:37-268): ForwardHidden / ForwardLogits with kv == NULL, ForwardHiddenCached / ForwardLogitsCached
 * with a cache. token_ids [n] may be in host or device memory; ids in device memory are checked on the device (an id
 * outside [0, vocab) fails the call with SOC_ERR_INVALID after it ran, leaving the slot length unchanged) and are never
 * read back to the host.
 *   kv == NULL: the uncached forward: causal attention over the n tokens alone, RoPE at positions position_offset ..
 *     (qwen_attention.cpp:103-140), on a private cache of the model; position_offset + n <= max_position_embeddings.
 *   kv set: the cached forward of `slot`; position_offset must equal the slot's length; the n tokens' K/V are appended.
 * hidden [n][hidden_size] (nullable): the final-RMSNorm rows (ForwardHidden*); logits [logit_rows][vocab] (nullable):
 * the last logit_rows rows (ForwardLogits* with logit_rows = n); next_token (nullable): greedy id of the last row.
 * Outputs may be host or device memory. One host synchronisation per call; a cached single token without hidden rows
 * runs the decode path. */
int soc_forward(soc_model* model, soc_kv* kv, int32_t slot, const int32_t* token_ids, int32_t n,
                int32_t position_offset, float* hidden, int32_t logit_rows, float* logits, int32_t* next_token);
/* One decode step of one slot: feeds `last_token` at position = current length. Logits [V] nullable, in host or
 * device memory. */
int soc_decode(soc_model* model, soc_kv* kv, int32_t slot, int32_t last_token, float* logits, int32_t* next_token);
/* `steps` greedy decode steps of one slot with the token fed back on the device (no host round trip per step).
 * tokens_out[steps] receives the generated ids. */
int soc_decode_steps(soc_model* model, soc_kv* kv, int32_t slot, int32_t last_token, int32_t steps,
                     int32_t* tokens_out);
/* No counterpart in the reference: for callers that cannot allocate device memory (tight serving loops, harnesses
 * that forbid hipMalloc). soc_decode_steps with the same results, its device buffers (exchange state of the
 * one-launch decode kernel, token ring) taken from a 4 MiB array compiled into the library, one per device, held
 * until the process ends, instead of hipMalloc'd scratch; it allocates nothing. Needs a model that
 * soc_model_decode_path reports as 1 or 2 (else SOC_ERR_INVALID); fails with SOC_ERR_CAPACITY when the model's
 * exchange state plus 4 bytes per step exceed 4 MiB (about 900k steps at Qwen3-0.6B shape). Every call re-initialises
 * the array. Calls on one device are serialised by a per-device flag held from the array's initialisation to the
 * end of the call: a call made while another one holds it (another thread, another context or model on the same
 * device) fails at once with SOC_ERR_STATE and touches nothing. */
int soc_decode_steps_noalloc(soc_model* model, soc_kv* kv, int32_t slot, int32_t last_token, int32_t steps,
                             int32_t* tokens_out);

/* ---- Ragged multi-sequence decode. The reference decodes one sequence per call (GenerationContext::
 *      DecodeNextToken, Mac/gpu/src/runtime/generation_context.cpp:68-172, one token at pos = len - 1); a batch of n
 *      rows gives each row exactly that semantics for its own slot, in one pass over the weights: row i feeds
 *      tokens[i] to slot slots[i] at position = that slot's current length (per-sequence KV length, any mix of
 *      lengths) and appends its K/V. Slots must be distinct; 1 <= n <= 1024. ---- */
/* One step. logits: nullable [n][vocab]; next_tokens [n]: greedy ids (lowest index on ties, sampler.cpp:42-48). */
int soc_decode_batch(soc_model* model, soc_kv* kv, int32_t n, const int32_t* slots, const int32_t* tokens,
                     float* logits, int32_t* next_tokens);
/* `steps` greedy steps with each row's token fed back on the device; tokens_out [steps][n]. */
int soc_decode_batch_steps(soc_model* model, soc_kv* kv, int32_t n, const int32_t* slots, const int32_t* tokens,
                           int32_t steps, int32_t* tokens_out);

/* ---- sampler: replaces Sampler::SampleFromLogits (Mac/gpu/src/runtime/sampler.cpp:14-71) ---- */
/* Top-k sampling of one fp32 logits row, with the reference's results: k = top_k clamped to [1, vocab], temperature
 * <= 0 taken as 1, candidates ordered as std::partial_sort(0..vocab-1, by logit / temperature, greater first) orders
 * them, ties included; *token_id = the first. top_ids / top_logits (nullable, k entries) receive the candidates and
 * their raw logits. The row may be in device memory (hipMalloc'd or managed), pinned host memory or pageable host
 * memory: the pointer is classified with hipPointerGetAttributes first. For k <= 64 and a row a kernel may read
 * (device or pinned memory, the whole row inside one allocation) the candidates are found on the device and only
 * they are copied back; larger k, a row holding NaN, or a row in pageable host memory is sorted whole on the host as
 * the reference does (a kernel never reads pageable host memory). */
int soc_sample_topk(soc_ctx* ctx, const float* logits_row, int32_t vocab, int32_t top_k, float temperature,
                    int32_t* token_id, int32_t* top_ids, float* top_logits);

/* ---- op-level entry points on caller device pointers, queued on the context stream (tests, microbenchmarks).
 *      These replace the reference's op wrappers (the static Run(...) of the headers under Mac/gpu/include/op/). ---- */
/* y[N] = W[N][K] . x[K]; W fp16, x fp16, y fp32 (LinearOp/MatMulOp decode mode, matmul_op.mm:143-163). */
int soc_gemv_f16(soc_ctx* ctx, const void* w, const void* x, float* y, int32_t n, int32_t k);
/* Prefill projection: y[M][N] = x[M][K] . W[N][K]^T; x and W fp16 (16-byte aligned), y fp32; K % 32 == 0. The
 * prefill GEMM of the model (MFMA 32x32x16, direct-to-LDS tiles; LinearOp / MatMulOp prefill mode, matmul_op.mm). */
int soc_gemm_f16(soc_ctx* ctx, const void* x, const void* w, float* y, int32_t m, int32_t n, int32_t k);
/* Causal GQA attention of a prefill chunk (GroupedQueryAttention::ForwardWithPrefix, grouped_query_attention.cpp:
 * 59-142): q fp32 [rows][nq * 128] (already normed and rotated), keys / values fp16 [nkv][cap][128] (one layer's cache
 * planes, holding the chunk's own keys), out fp32 [rows][nq * 128]; row t sees keys 0 .. pos_base + t; head_dim must be
 * 128 and nq / nkv in {1, 2, 4, 8}. */
int soc_attention_prefill(soc_ctx* ctx, const float* q, const void* keys, const void* values, float* out, int32_t rows,
                          int32_t pos_base, int32_t nq, int32_t nkv, int32_t head_dim, int32_t cap);
/* Decode attention of one token over keys 0 .. kv_len - 1 of the same planes (QwenAttention::RunDecode's attention,
 * Mac/gpu/src/module/qwen_attention.mm): q fp32 [nq * 128], out fp32 [nq * 128]. */
int soc_attention_decode(soc_ctx* ctx, const float* q, const void* keys, const void* values, float* out,
                         int32_t kv_len, int32_t nq, int32_t nkv, int32_t head_dim, int32_t cap);
/* Group-quantized matmul: y[M][N] = x[M][K] . dequant(codes, scales)^T; bits 8 or 4; group 64 along K. */
int soc_qmm(soc_ctx* ctx, const void* x_f16, const void* codes, int32_t bits, const void* scales_f16, float* y,
            int32_t m, int32_t n, int32_t k);
/* Dequantize to fp32 [N][K] (bit-exact contract: w = float(code) * float(scale)). */
int soc_dequant(soc_ctx* ctx, const void* codes, int32_t bits, const void* scales_f16, float* w, int32_t n, int32_t k);

/* ---- the reference's fp32 op kernels (the static Run of the headers under Mac/gpu/include/op/; kernels in
 *      Mac/gpu/shaders/gpu_kernels.metal:82-289) on caller device pointers, row-major; each validates that every
 *      operand lies in device memory inside one allocation before launching, and returns when the result is written.
 *      The C++ classes MatMulOp, LinearOp, RmsNormOp, RopeOp, SoftmaxOp, EmbeddingOp and ElementwiseMulOp
 *      (include/soc/gpu/ops.h) call these. ---- */
/* MatMulOp::Run (matmul_op.mm:196-330): out[r][c] = sum_i lhs[r][i] rhs'[i][c] (+ bias[c]) (+ residual[r][c]), then
 * SiLU when `silu`; rhs' = rhs [inner][cols], or rhs [cols][inner] read transposed when transpose_rhs. bias and
 * residual nullable; residual may alias out. fp32 operands and accumulation (MFMA 16x16x4 fp32). */
int soc_op_matmul(soc_ctx* ctx, const float* lhs, const float* rhs, const float* bias, const float* residual,
                  float* out, int32_t rows, int32_t inner, int32_t cols, int32_t transpose_rhs, int32_t silu);
/* RmsNormOp::Run: y = x / sqrt(mean(x^2) + eps) * weight per row of n (rms_norm_module.cpp:56-64). */
int soc_op_rmsnorm(soc_ctx* ctx, const float* x, const float* weight, float* y, int32_t rows, int32_t n, float eps);
/* RopeOp::Run over [rows][heads * head_dim]: rotate-half of the first rotary_dim dims of each head at position
 * position_offset + row, angle (position) / theta^(2i / rotary_dim) in double (rope.cpp:72-79); other dims copied.
 * In place (x == y) allowed. */
int soc_op_rope(soc_ctx* ctx, const float* x, float* y, int32_t rows, int32_t heads, int32_t head_dim,
                int32_t rotary_dim, int32_t position_offset, double theta);
/* SoftmaxOp::Run per row of n: exp(x - max) / sum. */
int soc_op_softmax(soc_ctx* ctx, const float* x, float* y, int32_t rows, int32_t n);
/* EmbeddingOp::Run: out[t] = table[ids[t]] (fp32 or fp16 table [vocab][hidden]); an id outside [0, vocab) gives a zero
 * row, as the reference's kernel (gpu_kernels.metal:104-136). */
int soc_op_embedding(soc_ctx* ctx, const int32_t* ids, const void* table, int32_t table_dtype, float* out,
                     int32_t tokens, int32_t hidden, int32_t vocab);
/* ElementwiseMulOp::Run: y = a * b elementwise over rows * n. */
int soc_op_mul(soc_ctx* ctx, const float* a, const float* b, float* y, int32_t rows, int32_t n);

/* ---- seeded synthetic data (this project's generator; the reference has none) ---- */
int soc_synth_normal_f16(uint64_t seed, const char* name, float sigma, int64_t offset, int64_t n, uint16_t* out);
int soc_synth_uniform_f16(uint64_t seed, const char* name, float lo, float hi, int64_t offset, int64_t n,
                          uint16_t* out);
int soc_synth_tokens(uint64_t seed, const char* name, int32_t vocab, int64_t n, int32_t* out);
int soc_synth_int_uniform(uint64_t seed, const char* name, int32_t lo, int32_t hi, int64_t n, int32_t* out);
int soc_synth_codes(uint64_t seed, const char* name, int32_t bits, int64_t n_codes, uint8_t* out);
uint16_t soc_f64_to_f16_rne(double x);

#ifdef __cplusplus
}
#endif

#endif /* SOC_HIP_H */
