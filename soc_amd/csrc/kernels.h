// kernels.h - argument blocks and launchers of the HIP kernels (all launched on the caller's stream).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "device_common.h"

namespace soc {

enum { EPI_STORE = 0, EPI_RESIDUAL = 1, EPI_SWIGLU = 2, EPI_QKV = 3 };

// ---- decode GEMV (batch 1) ----
struct GemvArgs {
  const float* x;    // [K] fp32 activations (or nullptr when xh is given)
  const f16* xh;     // [K] fp16 activations (op-level entry point)
  const f16* gain;   // RMSNorm gain [K] or nullptr (no normalisation)
  float eps;
  const f16* w;      // [N][K]
  const f16* w2;     // EPI_SWIGLU: up-projection rows [N][K]
  float* y;          // [N]
  int N, K;
};
hipError_t launch_gemv(const GemvArgs& a, int epi, hipStream_t s);

struct LmHeadArgs {
  const float* x;     // [K] residual stream (pre final norm)
  const f16* gain;    // final norm gain [K]
  float eps;
  const f16* w;       // [N][K] embedding table (tied) or lm_head
  float* logits;      // [N] or nullptr
  float* part_val;    // [blocks]
  int* part_idx;      // [blocks]
  int* counter;       // zero-initialised; the last block resets it
  int* token_out;     // nullable: argmax token
  int* state;         // nullable: {token, pos} decode state; token <- argmax, pos += 1
  int* ring;          // nullable: ring[ring_pos[0]] = token
  int* ring_pos;      // nullable
  int N, K;
};
int lm_head_blocks(int N);
hipError_t launch_lm_head_argmax(const LmHeadArgs& a, hipStream_t s);

struct QmmArgs {
  const f16* x;        // [M][K] fp16 activations
  const void* codes;   // int8 [N][K] or packed int4 [N][K/2]
  const f16* scales;   // [N][K/64]
  float* y;            // [M][N]
  int M, N, K;
};
hipError_t launch_qmm(const QmmArgs& a, int bits, hipStream_t s);
hipError_t launch_dequant(const void* codes, int bits, const f16* scales, int N, int K, float* w, hipStream_t s);
// The same weights rounded to fp16 (nearest) [N][K], for the prefill GEMMs of a quantized model (K % 64 == 0).
hipError_t launch_dequant_f16(const void* codes, int bits, const f16* scales, int N, int K, f16* w, hipStream_t s);

// ---- attention ----
struct AttnArgs {
  const float* qkv;      // fused mode: raw projections [B][ld_qkv] (q | k | v); else normed+roped q [B][ld_qkv]
  int ld_qkv;
  const f16* q_gain;     // [d] (fused mode)
  const f16* k_gain;     // [d] (fused mode)
  float eps;
  const float* rope_cos; // [max_pos][d/2]
  const float* rope_sin;
  f16* kcache;           // layer-0 base of slot 0; element (slot, layer, head, pos, i) at
  f16* vcache;           //   slot*slot_stride + layer*layer_stride + head*cap*d + pos*d + i
  long long slot_stride, layer_stride;
  int layer, cap;
  const int32_t* pos;    // [B] query position (== number of earlier keys)
  const int32_t* slot;   // [B] KV slot of each row, nullptr = slot_base for every row
  int slot_base;
  int pos_base;          // added to pos[] (prefill rows use pos = nullptr and pos_base + row)
  float* out;            // [B][nq*d] (prefill MFMA kernel: may be null when out_hi / out_lo are set)
  int ld_out;
  f16* out_hi;           // prefill MFMA kernel: optional hi = f16(o), lo = f16((o - hi) * 2^11) copies [B][ld_out]
  f16* out_lo;
  float* part;           // split partials [B][nq][max_split][d + 2]
  int* counters;         // [B][nkv] zero-initialised
  int B, nq, nkv, max_split, chunk;
  float scale;
};
// fused = 1: q/k norm + RoPE + KV append of the new token are done inside (decode).
hipError_t launch_attention(const AttnArgs& a, int fused, hipStream_t s);
// Prefill chunk (pos == slot == nullptr) on MFMA: causal over keys 0..pos_base+row of the slot's cache, which must
// already hold the chunk's own keys. Supports nq/nkv in {1, 2, 4}; `part`, `counters`, `max_split`, `chunk` unused.
hipError_t launch_attention_prefill_mfma(const AttnArgs& a, hipStream_t s);
bool attention_prefill_mfma_supported(int nq, int nkv);
// Same contract, load-balanced over pairs of query tiles; nq/nkv in {2, 4}.
hipError_t launch_attention_prefill_pairs(const AttnArgs& a, hipStream_t s);
bool attention_prefill_pairs_supported(int nq, int nkv);

// q/k RMSNorm over each head + RoPE + KV-cache append for T new rows at positions pos_base + t (prefill).
struct QkNormRopeArgs {
  const float* qkv;      // [T][ld_qkv] raw projections
  int ld_qkv;
  const f16* q_gain;
  const f16* k_gain;
  float eps;
  const float* rope_cos;
  const float* rope_sin;
  float* q_out;          // [T][nq*d]
  f16* kcache;
  f16* vcache;
  long long slot_stride, layer_stride;
  int slot, layer, cap, pos_base;
  int T, nq, nkv;
  const int32_t* pos;    // nullable [T]: row t sits at position pos[t] of slot slots[t] (ragged decode batch);
  const int32_t* slots;  //   nullptr: row t at position pos_base + t of `slot` (prefill chunk)
};
hipError_t launch_qk_norm_rope_append(const QkNormRopeArgs& a, hipStream_t s);

// Greedy token of each of n logit rows (lowest index among equal maxima) for a ragged decode batch: writes it as
// the row's next input id, records it at ring[row * ring_stride + (pos[row] - start[row])] and advances pos[row].
// Each row is scanned by argmax_chunks(V, n) blocks; with more than one, part_val / part_idx hold
// [n][kArgmaxMaxChunks] candidates and counters[n] (zero before the first call) count arrivals per row.
constexpr int kArgmaxMaxChunks = 64;
int argmax_chunks(int V, int n);
hipError_t launch_argmax_rows(const float* logits, int V, int n, int32_t* ids, int32_t* pos, const int32_t* start,
                              int32_t* ring, int ring_stride, float* part_val, int32_t* part_idx, int32_t* counters,
                              hipStream_t s);

// K/V rows [rows][nkv * hd] (fp32, or fp16 when `fp16`) into positions pos .. pos + rows - 1 of one (slot, layer)
// of the cache, whose [nkv][cap][hd] fp16 planes start at kdst / vdst.
hipError_t launch_kv_append_rows(const void* keys, const void* values, bool fp16, int rows, int nkv, int hd, int cap,
                                 int pos, f16* kdst, f16* vdst, hipStream_t s);

// Token ids in device memory [n] -> dst [n], ids outside [0, vocab) replaced by 0 with *err set to 1 (ops.hip).
hipError_t launch_stage_ids(const int32_t* src, int n, int vocab, int32_t* dst, int* err, hipStream_t s);
// A decode step's inputs in one launch: state[0] = dev_last ? *dev_last (checked like launch_stage_ids) : host_last,
// state[1] = pos, *ring = 0 (ops.hip).
hipError_t launch_decode_prologue(const int32_t* dev_last, int32_t host_last, int32_t pos, int vocab, int32_t* state,
                                  int32_t* ring, int* err, hipStream_t s);
// host[0] = state[0], host[1] = *wait_err, host[2] = id_err ? *id_err : 0; host is a device address of pinned host
// memory (ops.hip).
hipError_t launch_decode_readback(const int32_t* state, const int32_t* wait_err, const int* id_err, int32_t* host,
                                  hipStream_t s);
// dst[0..n) = src[0..n) for n <= 16 words read from the host at launch (the words travel as kernel arguments).
hipError_t launch_write_words(int32_t* dst, const int32_t* src, int n, hipStream_t s);

// ---- quantized-model forward steps (qpath.hip) ----
hipError_t launch_f32_to_f16(const float* x, size_t n, f16* y, hipStream_t s);
hipError_t launch_add_f32(float* x, const float* y, size_t n, hipStream_t s);  // x += y
// gu [T][2 I] (gate | up) -> h [T][I] = fp16(silu(gate) * up)
hipError_t launch_swiglu_f16(const float* gu, int T, int I, f16* h, hipStream_t s);

// ---- sampler: top-k candidates of one logits row (sample.hip) ----
constexpr int kSampleChunk = 2048, kSampleMaxK = 64;
// LDS bound on the prefix lists one block merges: ceil(V / kSampleChunk) * k floats.
constexpr size_t kSampleTreeBytes = 48 * 1024;
// Whether a row of V logits at this k is searched on the device (k <= kSampleMaxK and the lists fit).
bool sample_device_fits(int V, int k);
// Device workspace bytes for a row of V logits; zero-filled when allocated (its first word is an arrival counter
// that every k = 1 search leaves at zero).
size_t sample_ws_bytes(int V);
// Finds the candidates that std::partial_sort(top k of row / t) over 0..V-1 moves into its heap, in index order:
// out[0] = count, out[1] = NaN seen, then for j < min(count, max_out): out[2 + 2 j] = index,
// out[3 + 2 j] = the bits of its raw logit. Requires sample_device_fits(V, k).
hipError_t launch_sample_topk(const float* row, int V, float t, int k, void* ws, int* out, int max_out,
                              hipStream_t s);

// ---- persistent batch-1 decode step (one launch per token) ----
struct PersistArgs {
  const f16* const* layer_w;  // device array [L][9]: in_norm, post_norm, q_norm, k_norm, wqkv, wo, wgate, wup, wdown
  const f16* embed;
  const f16* final_norm;
  const f16* lm_head;
  const float* rope_cos;
  const float* rope_sin;
  f16* kcache;                // base of this slot's layer 0
  f16* vcache;
  long long layer_stride;
  int cap;
  int L, H, I, V, nq, nkv, qkv_rows, qd, xs_cap;
  float eps, scale;
  uint32_t* xa;               // exchange vectors: one tagged 32-bit word per element (value, 2-bit phase tag)
  uint32_t* xb;
  uint32_t* qkv;
  uint32_t* attn;
  uint32_t* h;
  float* logits;              // [V] or nullptr
  float* part_val;            // [nblocks]
  int* part_idx;              // [nblocks]
  int* counter;               // zero; reset by the last block
  int* state;                 // {token, pos, step of k_decode_persistent, step of k_decode_xcd}; steps start at 1
  int* ring;                  // nullable
  int* ring_pos;
  int* err;                   // raised when a wait times out
  uint64_t* trace;            // nullable: phase timestamps (diagnostics)
  int spin_sleep;             // back-off between polling rounds, in units of s_sleep 1 (about 64 clocks)
  uint64_t spin_ticks;        // bound of every cross-block wait, in ticks of the 100 MHz counter (kSpinTicks)
  int cooperative;            // launch with hipLaunchCooperativeKernel (the runtime refuses a grid that cannot be
                              // co-resident instead of leaving its blocks to time out)
  // XCD-partitioned kernel only (k_decode_xcd):
  uint32_t* xo;               // [8][H] tagged partial o_proj outputs of the eight XCDs (cross-XCD)
  uint32_t* xd;               // [8][H] tagged partial down_proj outputs (cross-XCD)
  uint32_t* xp;               // [H] tagged residual x' of the last layer, for the other block group
  uint32_t* loc;              // [8][loc_stride] per-XCD hand-off regions (q/k/v, attention partials, h)
  int loc_stride;             // words per region
  int* xcd_ctr;               // [2][8] arrivals per XCD, by step parity (zero; the next step's pair is reset)
  int steps;                  // decode steps one launch of k_decode_xcd runs (>= 1; the token of each is released to
                              // the next through state[3])
};
bool persistent_supported(int H, int qd, int I, int qkv_rows, int nq, int nkv, int nblocks);
size_t persistent_lds_bytes(const PersistArgs& a, int G);
hipError_t persistent_blocks_per_cu(int G, int* blocks);
hipError_t launch_decode_persistent(const PersistArgs& a, int nblocks, hipStream_t s);

// XCD-partitioned one-launch decode step: 256 blocks, 32 on each of the 8 XCDs, XCD g owns KV head g; two groups of
// 16 blocks per XCD take alternate layers.
constexpr int kXcdGroups = 8, kXcdBlocks = 32;
constexpr int kTracePts = 32;  // diagnostic timestamps per block of k_decode_xcd
// then 128 per-layer slots, then kTracePts timestamps per wave (8 waves per block) of the middle layer
constexpr int kTraceWaveBase = kXcdGroups * kXcdBlocks * kTracePts + 128;
constexpr int kTraceTotal = kTraceWaveBase + kXcdGroups * kXcdBlocks * 8 * kTracePts;
bool xcd_supported(int H, int I, int nq, int nkv, int head_dim, int num_cus);
int xcd_loc_stride(int G, int I);  // words per per-XCD hand-off region
hipError_t xcd_blocks_per_cu(int G, int* blocks);
hipError_t launch_decode_xcd(const PersistArgs& a, hipStream_t s);

// ---- prefill helpers ----
// x[t][:] = float(table[ids[t]][:]) for t < T (Mac/cpu/src/embedding.cpp:51-77).
hipError_t launch_embed(const int32_t* ids, int T, const f16* table, int H, float* x, hipStream_t s);
// y[t] = RMSNorm(x[t]) with an fp16 gain; y may be fp32 (yf) or fp16 (yh), whichever is non-null.
hipError_t launch_rmsnorm_rows(const float* x, int T, int H, const f16* gain, float eps, float* yf, f16* yh,
                               f16* ylo, hipStream_t s);
// hi = f16(x), lo = f16((x - hi) * 2^11) of n fp32 values (the activation split of the MFMA GEMMs).
hipError_t launch_split_f16(const float* x, size_t n, f16* hi, f16* lo, hipStream_t s);

// C[M][N] (epilogue) = A[M][K] . W[N][K]^T, fp32 activations, fp16 weights, fp32 accumulation.
struct GemmArgs {
  const float* a;   // [M][lda]
  int lda;
  const f16* w;     // [N][K]
  const f16* w2;    // EPI_SWIGLU up rows
  float* c;         // [M][ldc]
  int ldc;
  int M, N, K;
};
// MFMA (fp16 inputs, fp32 accumulation); split = hi/lo fp16 parts of the fp32 activations. Requires K % 32 == 0.
bool gemm_mfma_supported(const GemmArgs& g);
hipError_t launch_gemm_mfma(const GemmArgs& g, int epi, bool split, hipStream_t s);
// Same products on activations pre-split into hi = f16(a) and lo = f16((a - hi) * 2^11) arrays [M][lda]
// (lda % 8 == 0, K % 32 == 0, 16-byte aligned); with al = null, on the single fp16 activations ah alone (the
// products of launch_gemm_mfma with split = false). EPI_SWIGLU writes c, or ch (and cl when set) in the same form.
struct GemmSplitArgs {
  const f16* ah;
  const f16* al;
  int lda;
  const f16* w;     // [N][K]
  const f16* w2;    // EPI_SWIGLU up rows
  float* c;         // [M][ldc]
  f16* ch;          // EPI_SWIGLU split output [M][ldc] (or null)
  f16* cl;
  int ldc;
  int M, N, K;
  // EPI_QKV (fused projection rows q | k | v, 128-column heads): per-head RMSNorm + RoPE of the q and k heads at
  // positions pos_base + row; q -> q_out [M][nq * 128] (fp32), k and v -> the fp16 cache rows of `slot`
  struct Qkv {
    float* q_out;
    f16* kcache;
    f16* vcache;
    const f16* q_gain;
    const f16* k_gain;
    const float* rope_cos;
    const float* rope_sin;
    long long slot_stride, layer_stride;
    int slot, layer, cap, pos_base, nq, nkv;
    float eps;
  } qkv;
};
bool gemm_split_supported(const GemmSplitArgs& g);
hipError_t launch_gemm_split(const GemmSplitArgs& g, int epi, hipStream_t s);

// Skinny projection of a ragged decode batch: x[M][K] . [w | w2]^T for 1 <= M <= 16 rows, K % 256 == 0, split over
// K, then an epilogue kernel that adds the splits in order. Rows 0..N0-1 come from w, rows N0..Ntot-1 from w2.
//   gain set: the input is RMSNorm(x) with that gain: x * gain enters the products, and the row's 1 / rms (from the
//     sum of squares of x over all K) scales the sums.
//   EPI_STORE: c = y (Ntot = N0). EPI_RESIDUAL: c += y (Ntot = N0). EPI_SWIGLU: c = silu(gate) * up over N0 outputs
//   (Ntot = 2 N0, N0 % 64 == 0). EPI_QKV: rows are q | k | v heads of 128; per head RMSNorm (q_gain / k_gain) and
//   rotate-half RoPE at pos[m] of q and k; q -> q_out [M][nq * 128], k and v -> the fp16 cache of slots[m] at pos[m].
// part: scratch of skinny_part_floats(Ntot, K) floats.
struct SkinnyArgs {
  const float* x;
  int ldx;
  const f16* w;
  const f16* w2;
  int N0, Ntot, K, M;
  float* part;
  float* c;
  int ldc;
  const f16* gain;  // nullable: RMSNorm gain of the input
  float eps;
  // EPI_QKV
  float* q_out;
  f16* kcache;
  f16* vcache;
  const f16* q_gain;
  const f16* k_gain;
  const float* rope_cos;
  const float* rope_sin;
  const int32_t* pos;
  const int32_t* slots;
  long long slot_stride, layer_stride;
  int layer, cap, nq, nkv;
  int KS, Kb;  // set by the launcher
};
bool skinny_supported(int M, int K);
int skinny_splits(int rows, int K);
size_t skinny_part_floats(int rows, int K);
hipError_t skinny_configure();
hipError_t launch_skinny(const SkinnyArgs& a, int epi, hipStream_t s);

}  // namespace soc
