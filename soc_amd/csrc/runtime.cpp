// runtime.cpp - host side of the C ABI: device context, weight placement and upload, fp16 KV cache, prefill and
// decode orchestration (decode steps replay one captured HIP graph; the sampled token and the position live in
// device memory so that consecutive steps need no host round trip).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <atomic>
#include <cmath>
#include <cstdlib>
#include <cstdio>
#include <cstring>
#include <map>
#include <memory>
#include <new>
#include <numeric>
#include <string>
#include <thread>
#include <vector>

#include "kernels.h"
#include "soc_hip.h"
#include "status.h"
#include "capi_internal.h"

using soc::f16;

// ------------------------------------------------------------------------------------------------------------
// objects
// ------------------------------------------------------------------------------------------------------------

// Device memory of soc_decode_steps_noalloc: the exchange state of the one-launch decode kernels and the token ring
// live here instead of in hipMalloc'd buffers. One copy per device for the whole process; every call re-initialises
// what it uses, and calls that overlap on one device race on it. Host code never passes `scratch` itself (the host
// symbol is only a stand-in): it uses the address hipGetSymbolAddress returned for the device, kept in soc_ctx.
constexpr size_t kNoAllocScratchBytes = size_t{4} << 20;
static __device__ __align__(256) uint32_t scratch[kNoAllocScratchBytes / 4];

// One flag per device: set while a soc_decode_steps_noalloc call uses that device's `scratch` (from its
// initialisation to the synchronisation that ends the call). A call that finds it set fails with SOC_ERR_STATE
// instead of racing on the array.
constexpr int kNoAllocMaxDevices = 64;
static std::atomic<bool> g_noalloc_busy[kNoAllocMaxDevices];

// Fills words [0, n_zero) with zero except the four decode-state words at `state_at` ({token, pos, 1, 1}: the step
// counters of both one-launch kernels start at 1) and words [ff_at, ff_at + n_ff) with 0xffffffff (tag 3 in every
// exchange word; the first phase of a step expects tag 0).
__global__ void k_noalloc_init(uint32_t* base, int n_zero, int state_at, int ff_at, int n_ff, int32_t token,
                               int32_t pos) {
  const int stride = gridDim.x * blockDim.x;
  for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < n_zero; i += stride) {
    uint32_t v = 0;
    if (i == state_at) v = static_cast<uint32_t>(token);
    else if (i == state_at + 1) v = static_cast<uint32_t>(pos);
    else if (i == state_at + 2 || i == state_at + 3) v = 1u;
    base[i] = v;
  }
  for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < n_ff; i += stride) base[ff_at + i] = 0xffffffffu;
}

namespace {

struct DevLayer {
  f16 *in_norm, *post_norm, *q_norm, *k_norm, *wqkv, *wo, *wgate, *wup, *wdown;
};

// Group-quantized copies of a layer's projections (soc_model_quantize): codes and fp16 scales per 64 weights.
struct QLayer {
  uint8_t *qkv = nullptr, *o = nullptr, *gu = nullptr, *down = nullptr;  // gu: gate rows then up rows
  f16 *qkv_s = nullptr, *o_s = nullptr, *gu_s = nullptr, *down_s = nullptr;
};

struct TensorSlot {
  f16* ptr;
  int64_t numel;
  bool loaded;
};

// Device scratch of one forward kind; pointers stay fixed once allocated (captured graphs refer to them).
struct DecodeWs {
  bool ready = false;
  float *x = nullptr, *qkv = nullptr, *attn = nullptr, *h = nullptr, *logits = nullptr, *part = nullptr,
        *lm_val = nullptr;
  int *lm_idx = nullptr, *lm_counter = nullptr, *attn_counters = nullptr, *state = nullptr, *ring = nullptr,
      *ring_pos = nullptr;
  int max_split = 0, ring_cap = 0;
  // persistent decode kernel: exchange vectors (tagged 32-bit word per element), argmax partials, error flag
  uint32_t *xa = nullptr, *xb = nullptr, *qkv_x = nullptr, *attn_x = nullptr, *h_x = nullptr;
  // XCD-partitioned decode kernel: cross-XCD partial vectors, per-XCD hand-off regions, arrival counters
  uint32_t *xo = nullptr, *xd = nullptr, *xp = nullptr, *loc = nullptr;
  int loc_stride = 0;
  int* xcd_ctr = nullptr;
  float* pv = nullptr;
  int *pi = nullptr, *err = nullptr;
  int nblocks = 0;
  // quantized models: fp16 activation row and fp32 projection output of the per-op decode
  f16* qx = nullptr;
  float* qy = nullptr;
  std::vector<void*> allocs;
};

struct PrefillWs {
  int cap_rows = 0, cap_split = 0;
  float *x = nullptr, *xn = nullptr, *qkv = nullptr, *q = nullptr, *attn = nullptr, *h = nullptr,
        *logits = nullptr, *part = nullptr, *lm_val = nullptr;
  int *ids = nullptr, *attn_counters = nullptr, *lm_idx = nullptr, *lm_counter = nullptr, *token = nullptr;
  int cap_logit_rows = 0;
  std::vector<void*> allocs;
  float* skpart = nullptr;  // split-K partials of the skinny batch projections
  // hi/lo fp16 activation pairs of the prefill projections: p = normed input / attention output, q = SwiGLU output
  soc::f16 *ph = nullptr, *pl = nullptr, *qh = nullptr, *ql = nullptr;
  // quantized models: fp16 activation rows and fp32 projection outputs of one chunk of kQChunk rows
  soc::f16* qx = nullptr;
  float* qy = nullptr;
};

// Per-row state of a ragged decode batch (device arrays of `cap` rows).
struct BatchWs {
  int cap = 0;
  int32_t *ids = nullptr, *pos = nullptr, *start = nullptr, *slots = nullptr, *ring1 = nullptr;
  // per-row candidates and arrival counters of the split greedy argmax ([cap][kArgmaxMaxChunks], [cap])
  float* am_val = nullptr;
  int32_t *am_idx = nullptr, *am_cnt = nullptr;
  std::vector<void*> allocs;
  int32_t* ring = nullptr;  // [rows][steps] tokens of soc_decode_batch_steps
  size_t ring_cap = 0;
};

constexpr int kAttnChunk = 256;
// Decode steps per launch of the XCD-partitioned one-launch kernel (its blocks stay resident from step to step: the
// next token's first layer streams while the last layer of the current one runs).
constexpr int kXcdStepsPerLaunch = 128;

// Keys per attention chunk of single-sequence per-op decode for a cache of `cap` positions: the smallest of 64, 128,
// 256 that keeps a full cache within 160 chunks (the kernel's combine limit). Smaller chunks give a short context
// more blocks (at batch 1 every block is one chunk of one KV head). SOC_DECODE_CHUNK overrides (64, 128 or 256).
int decode_attn_chunk(int cap) {
  if (const char* e = std::getenv("SOC_DECODE_CHUNK")) {
    const int v = std::atoi(e);
    if ((v == 64 || v == 128 || v == 256) && (cap + v - 1) / v <= 160) return v;
  }
  for (int c = 64; c < kAttnChunk; c *= 2)
    if ((cap + c - 1) / c <= 160) return c;
  return kAttnChunk;
}
constexpr int kQChunk = 8;  // rows per group-quantized projection call in a quantized model's prefill (k_qmm M <= 8)
constexpr int kMaxBatchRows = 1024;

}  // namespace

struct soc_model {
  soc_ctx* ctx = nullptr;
  soc_qwen_config cfg{};
  int qd = 0, kvd = 0, qkv_rows = 0;
  char* wbuf = nullptr;
  size_t wbytes = 0;
  f16 *embed = nullptr, *final_norm = nullptr, *lm_head = nullptr;
  std::vector<DevLayer> layers;
  std::map<std::string, TensorSlot> tensors;
  float *rope_cos = nullptr, *rope_sin = nullptr;
  int rope_len = 0;
  const f16** d_layer_w = nullptr;  // device copy of the per-layer weight pointers [L][9]
  DecodeWs dws;
  int dws_gen = 0;  // bumped whenever the decode scratch is reallocated (captured graphs refer to it)
  int bws_gen = 0;  // bumped whenever the prefill/batch scratch is reallocated (captured batch graphs refer to it)
  PrefillWs pws;
  BatchWs bws;
  bool finalized = false;
  bool xcd_off = false;  // the XCD-partitioned decode step failed its block placement once: not used again
  int qbits = 0;         // 8 or 4 after soc_model_quantize: the projections run on the group-quantized copies
  std::vector<QLayer> qlayers;
  std::vector<void*> qallocs;
  f16* qdeq = nullptr;    // quantized models: one layer's projections dequantized to fp16 for prefill GEMMs
  soc_kv* ukv = nullptr;  // private one-slot cache of the uncached forward (soc_forward with kv == NULL)
};

struct soc_kv {
  soc_ctx* ctx = nullptr;
  soc_model* model = nullptr;  // bound by its first forward when created from dimensions alone
  int layers = 0, nkv = 0, hd = 0;
  int slots = 0, cap = 0;
  f16 *k = nullptr, *v = nullptr;
  long long slot_stride = 0, layer_stride = 0;
  std::vector<int32_t> len;
  std::map<int, std::pair<int, hipGraphExec_t>> graphs;  // decode graph per slot, tagged with the scratch generation
  // batch-step graphs keyed by (rows, steps), tagged with the scratch generation
  std::map<std::pair<int, int>, std::pair<int, hipGraphExec_t>> batch_graphs;
};

namespace {

int hip_fail(hipError_t e, const char* what) {
  return soc::fail(SOC_ERR_HIP, std::string(what) + ": " + hipGetErrorString(e));
}

// Records the stop event of soc_ctx_timer_start / _stop on the stream before a forward's final synchronisation, so
// that reading the timer costs no further round trip.
void record_timer_stop(soc_ctx* ctx) {
  if (ctx->timing && !ctx->stop_recorded && hipEventRecord(ctx->ev1, ctx->stream) == hipSuccess)
    ctx->stop_recorded = true;
}

// A KV cache serves one model. One created from dimensions alone (soc_kv_create_dims, the reference's
// KVCache::CreateShared) is bound to the first model that runs a forward on it, if the shapes agree.
int bind_kv(soc_kv* kv, soc_model* m) {
  if (kv->model == m) return SOC_OK;
  if (kv->model != nullptr) return soc::fail(SOC_ERR_INVALID, "KV cache belongs to another model");
  const soc_qwen_config& c = m->cfg;
  if (kv->ctx != m->ctx) return soc::fail(SOC_ERR_INVALID, "KV cache belongs to another context");
  if (kv->layers != c.num_hidden_layers || kv->nkv != c.num_key_value_heads || kv->hd != c.head_dim)
    return soc::fail(SOC_ERR_INVALID, "KV cache dimensions do not match the model (layers, KV heads, head_dim)");
  if (kv->cap > m->rope_len) return soc::fail(SOC_ERR_CAPACITY, "KV capacity exceeds max_position_embeddings");
  kv->model = m;
  return SOC_OK;
}

int dev_alloc(std::vector<void*>& owner, size_t bytes, void** p) {
  hipError_t e = hipMalloc(p, bytes == 0 ? 256 : bytes);
  if (e != hipSuccess) {
    (void)hipGetLastError();
    return soc::fail(SOC_ERR_NOMEM, "hipMalloc of " + std::to_string(bytes) + " bytes failed");
  }
  owner.push_back(*p);
  return SOC_OK;
}

template <typename T>
int dev_alloc_t(std::vector<void*>& owner, size_t count, T** p) {
  return dev_alloc(owner, count * sizeof(T), reinterpret_cast<void**>(p));
}

void free_all(std::vector<void*>& v) {
  for (void* p : v) (void)hipFree(p);
  v.clear();
}

bool env_flag(const char* name) {
  const char* v = std::getenv(name);
  return v != nullptr && v[0] != '\0' && v[0] != '0';
}

int check_config(const soc_qwen_config& c) {
  if (c.vocab_size <= 0 || c.hidden_size <= 0 || c.num_hidden_layers <= 0 || c.num_attention_heads <= 0 ||
      c.num_key_value_heads <= 0 || c.intermediate_size <= 0 || c.max_position_embeddings <= 0)
    return soc::fail(SOC_ERR_INVALID, "qwen config: sizes must be positive");
  if (c.head_dim != 128) return soc::fail(SOC_ERR_INVALID, "qwen config: head_dim must be 128");
  if (c.num_attention_heads % c.num_key_value_heads != 0)
    return soc::fail(SOC_ERR_INVALID, "qwen config: num_attention_heads must be divisible by num_key_value_heads");
  const int G = c.num_attention_heads / c.num_key_value_heads;
  if (G != 1 && G != 2 && G != 4 && G != 8)
    return soc::fail(SOC_ERR_INVALID, "qwen config: query heads per KV head must be 1, 2, 4 or 8");
  if (c.hidden_size % 32 != 0 || c.intermediate_size % 32 != 0)
    return soc::fail(SOC_ERR_INVALID, "qwen config: hidden and intermediate sizes must be multiples of 32");
  if (!(c.rms_norm_eps > 0.0f) || !(c.rope_theta > 0.0))
    return soc::fail(SOC_ERR_INVALID, "qwen config: eps and rope_theta must be positive");
  if (static_cast<size_t>(c.hidden_size) * 4 > 64 * 1024 || static_cast<size_t>(c.intermediate_size) * 4 > 64 * 1024)
    return soc::fail(SOC_ERR_INVALID, "qwen config: hidden/intermediate size too large for the decode kernels");
  return SOC_OK;
}

int ensure_decode_ws(soc_model* m, int cap) {
  DecodeWs& w = m->dws;
  const int need_split = (cap + decode_attn_chunk(cap) - 1) / decode_attn_chunk(cap);
  if (w.ready && w.max_split >= need_split && w.ring_cap >= cap) return SOC_OK;
  hipError_t se = hipStreamSynchronize(m->ctx->stream);
  if (se != hipSuccess) return hip_fail(se, "hipStreamSynchronize");
  free_all(w.allocs);
  w = DecodeWs();
  ++m->dws_gen;
  const soc_qwen_config& c = m->cfg;
  w.max_split = need_split;
  w.ring_cap = cap;
  SOC_TRY(dev_alloc_t(w.allocs, c.hidden_size, &w.x));
  SOC_TRY(dev_alloc_t(w.allocs, m->qkv_rows, &w.qkv));
  SOC_TRY(dev_alloc_t(w.allocs, m->qd, &w.attn));
  SOC_TRY(dev_alloc_t(w.allocs, c.intermediate_size, &w.h));
  SOC_TRY(dev_alloc_t(w.allocs, c.vocab_size, &w.logits));
  SOC_TRY(dev_alloc_t(w.allocs, static_cast<size_t>(c.num_attention_heads) * w.max_split * (128 + 2), &w.part));
  SOC_TRY(dev_alloc_t(w.allocs, 1024, &w.lm_val));
  SOC_TRY(dev_alloc_t(w.allocs, 1024, &w.lm_idx));
  SOC_TRY(dev_alloc_t(w.allocs, 64, &w.lm_counter));
  SOC_TRY(dev_alloc_t(w.allocs, c.num_key_value_heads, &w.attn_counters));
  SOC_TRY(dev_alloc_t(w.allocs, 64, &w.state));
  SOC_TRY(dev_alloc_t(w.allocs, cap, &w.ring));
  SOC_TRY(dev_alloc_t(w.allocs, 64, &w.ring_pos));
  {
    const size_t kmax = std::max({c.hidden_size, m->qd, c.intermediate_size});
    const size_t nmax = std::max({m->qkv_rows, 2 * c.intermediate_size, c.hidden_size});
    SOC_TRY(dev_alloc_t(w.allocs, kmax, &w.qx));
    SOC_TRY(dev_alloc_t(w.allocs, nmax, &w.qy));
  }
  hipError_t e;
  if ((e = hipMemset(w.lm_counter, 0, 64 * sizeof(int))) != hipSuccess) return hip_fail(e, "hipMemset");
  if ((e = hipMemset(w.attn_counters, 0, c.num_key_value_heads * sizeof(int))) != hipSuccess)
    return hip_fail(e, "hipMemset");
  if ((e = hipMemset(w.state, 0, 64 * sizeof(int))) != hipSuccess) return hip_fail(e, "hipMemset");
  if ((e = hipMemset(w.ring_pos, 0, 64 * sizeof(int))) != hipSuccess) return hip_fail(e, "hipMemset");
  // persistent-kernel state: exchange vectors filled with 0xff bytes (tag 3; the first phase expects tag 0), step
  // counter starts at 1
  w.nblocks = m->ctx->num_cus;
  SOC_TRY(dev_alloc_t(w.allocs, c.hidden_size, &w.xa));
  SOC_TRY(dev_alloc_t(w.allocs, c.hidden_size, &w.xb));
  SOC_TRY(dev_alloc_t(w.allocs, m->qkv_rows, &w.qkv_x));
  SOC_TRY(dev_alloc_t(w.allocs, m->qd, &w.attn_x));
  SOC_TRY(dev_alloc_t(w.allocs, c.intermediate_size, &w.h_x));
  const int G = c.num_attention_heads / c.num_key_value_heads;
  w.loc_stride = soc::xcd_loc_stride(G, c.intermediate_size);
  SOC_TRY(dev_alloc_t(w.allocs, static_cast<size_t>(soc::kXcdGroups) * c.hidden_size, &w.xo));
  SOC_TRY(dev_alloc_t(w.allocs, static_cast<size_t>(soc::kXcdGroups) * c.hidden_size, &w.xd));
  SOC_TRY(dev_alloc_t(w.allocs, static_cast<size_t>(c.hidden_size), &w.xp));
  SOC_TRY(dev_alloc_t(w.allocs, static_cast<size_t>(soc::kXcdGroups) * w.loc_stride, &w.loc));
  SOC_TRY(dev_alloc_t(w.allocs, 2 * soc::kXcdGroups, &w.xcd_ctr));
  SOC_TRY(dev_alloc_t(w.allocs, std::max(w.nblocks, soc::kXcdGroups * soc::kXcdBlocks), &w.pv));
  SOC_TRY(dev_alloc_t(w.allocs, std::max(w.nblocks, soc::kXcdGroups * soc::kXcdBlocks), &w.pi));
  SOC_TRY(dev_alloc_t(w.allocs, 64, &w.err));
  for (auto pr : {std::make_pair((void*)w.xa, (size_t)c.hidden_size), std::make_pair((void*)w.xb, (size_t)c.hidden_size),
                  std::make_pair((void*)w.qkv_x, (size_t)m->qkv_rows), std::make_pair((void*)w.attn_x, (size_t)m->qd),
                  std::make_pair((void*)w.h_x, (size_t)c.intermediate_size),
                  std::make_pair((void*)w.xo, (size_t)soc::kXcdGroups * c.hidden_size),
                  std::make_pair((void*)w.xd, (size_t)soc::kXcdGroups * c.hidden_size),
                  std::make_pair((void*)w.xp, (size_t)c.hidden_size),
                  std::make_pair((void*)w.loc, (size_t)soc::kXcdGroups * w.loc_stride)})
    if ((e = hipMemset(pr.first, 0xff, pr.second * sizeof(uint32_t))) != hipSuccess) return hip_fail(e, "hipMemset");
  if ((e = hipMemset(w.err, 0, 64 * sizeof(int))) != hipSuccess) return hip_fail(e, "hipMemset");
  if ((e = hipMemset(w.xcd_ctr, 0, 2 * soc::kXcdGroups * sizeof(int))) != hipSuccess) return hip_fail(e, "hipMemset");
  // step counters of the two one-launch kernels (state[2]: k_decode_persistent, state[3]: k_decode_xcd): each kernel
  // derives its exchange tags from its own count, so the tags of its regions advance by one per layer whichever
  // decode implementation ran in between
  const int32_t step1[2] = {1, 1};
  if ((e = hipMemcpy(w.state + 2, step1, sizeof(step1), hipMemcpyHostToDevice)) != hipSuccess)
    return hip_fail(e, "hipMemcpy");
  w.ready = true;
  return SOC_OK;
}

size_t skinny_scratch_floats(const soc_model* m);

int ensure_prefill_ws(soc_model* m, int rows, int total_len, int logit_rows) {
  PrefillWs& w = m->pws;
  const int need_split = (total_len + kAttnChunk - 1) / kAttnChunk;
  if (w.cap_rows >= rows && w.cap_split >= need_split && w.cap_logit_rows >= logit_rows) return SOC_OK;
  hipError_t e = hipStreamSynchronize(m->ctx->stream);
  if (e != hipSuccess) return hip_fail(e, "hipStreamSynchronize");
  free_all(w.allocs);
  ++m->bws_gen;
  const int R = std::max(rows, w.cap_rows), SP = std::max(need_split, w.cap_split),
            LR = std::max(std::max(logit_rows, 1), w.cap_logit_rows);
  w = PrefillWs();
  const soc_qwen_config& c = m->cfg;
  const size_t H = c.hidden_size;
  SOC_TRY(dev_alloc_t(w.allocs, R * H, &w.x));
  SOC_TRY(dev_alloc_t(w.allocs, R * H, &w.xn));
  SOC_TRY(dev_alloc_t(w.allocs, static_cast<size_t>(R) * m->qkv_rows, &w.qkv));
  SOC_TRY(dev_alloc_t(w.allocs, static_cast<size_t>(R) * m->qd, &w.q));
  SOC_TRY(dev_alloc_t(w.allocs, static_cast<size_t>(R) * m->qd, &w.attn));
  SOC_TRY(dev_alloc_t(w.allocs, static_cast<size_t>(R) * c.intermediate_size, &w.h));
  const size_t pw = static_cast<size_t>(R) * std::max<size_t>(H, m->qd);
  SOC_TRY(dev_alloc_t(w.allocs, pw, &w.ph));
  SOC_TRY(dev_alloc_t(w.allocs, pw, &w.pl));
  SOC_TRY(dev_alloc_t(w.allocs, static_cast<size_t>(R) * c.intermediate_size, &w.qh));
  SOC_TRY(dev_alloc_t(w.allocs, static_cast<size_t>(R) * c.intermediate_size, &w.ql));
  SOC_TRY(dev_alloc_t(w.allocs, static_cast<size_t>(LR) * c.vocab_size, &w.logits));
  SOC_TRY(dev_alloc_t(w.allocs, static_cast<size_t>(R) * c.num_attention_heads * SP * (128 + 2), &w.part));
  SOC_TRY(dev_alloc_t(w.allocs, R, &w.ids));
  SOC_TRY(dev_alloc_t(w.allocs, static_cast<size_t>(R) * c.num_key_value_heads, &w.attn_counters));
  SOC_TRY(dev_alloc_t(w.allocs, 1024, &w.lm_val));
  SOC_TRY(dev_alloc_t(w.allocs, 1024, &w.lm_idx));
  SOC_TRY(dev_alloc_t(w.allocs, 64, &w.lm_counter));
  SOC_TRY(dev_alloc_t(w.allocs, 64, &w.token));
  {
    const size_t kmax = std::max({c.hidden_size, m->qd, c.intermediate_size});
    const size_t nmax = std::max({m->qkv_rows, 2 * c.intermediate_size, c.hidden_size});
    SOC_TRY(dev_alloc_t(w.allocs, kQChunk * kmax, &w.qx));
    SOC_TRY(dev_alloc_t(w.allocs, kQChunk * nmax, &w.qy));
    if ((e = hipMemset(w.qx, 0, kQChunk * kmax * sizeof(soc::f16))) != hipSuccess) return hip_fail(e, "hipMemset");
  }
  if (const size_t sk = skinny_scratch_floats(m)) {
    SOC_TRY(dev_alloc_t(w.allocs, sk, &w.skpart));
    if ((e = soc::skinny_configure()) != hipSuccess) return hip_fail(e, "skinny kernel attributes");
  }
  if ((e = hipMemset(w.attn_counters, 0, static_cast<size_t>(R) * c.num_key_value_heads * sizeof(int))) != hipSuccess)
    return hip_fail(e, "hipMemset");
  if ((e = hipMemset(w.lm_counter, 0, 64 * sizeof(int))) != hipSuccess) return hip_fail(e, "hipMemset");
  w.cap_rows = R;
  w.cap_split = SP;
  w.cap_logit_rows = LR;
  return SOC_OK;
}

// RoPE table: angle = pos / theta^(2i/d) in double, cos/sin rounded to float (Mac/cpu/src/rope.cpp:72-79).
int build_rope_table(soc_model* m, int len) {
  const int half = m->cfg.head_dim / 2;
  std::vector<float> c(static_cast<size_t>(len) * half), s(c.size());
  for (int p = 0; p < len; ++p) {
    const double abs_pos = static_cast<double>(p);
    for (int i = 0; i < half; ++i) {
      const double exponent = static_cast<double>(i * 2) / static_cast<double>(m->cfg.head_dim);
      const double angle = abs_pos / std::pow(m->cfg.rope_theta, exponent);
      c[static_cast<size_t>(p) * half + i] = static_cast<float>(std::cos(angle));
      s[static_cast<size_t>(p) * half + i] = static_cast<float>(std::sin(angle));
    }
  }
  hipError_t e;
  if ((e = hipMalloc(&m->rope_cos, c.size() * 4)) != hipSuccess) return hip_fail(e, "hipMalloc rope");
  if ((e = hipMalloc(&m->rope_sin, s.size() * 4)) != hipSuccess) return hip_fail(e, "hipMalloc rope");
  if ((e = hipMemcpy(m->rope_cos, c.data(), c.size() * 4, hipMemcpyHostToDevice)) != hipSuccess)
    return hip_fail(e, "hipMemcpy rope");
  if ((e = hipMemcpy(m->rope_sin, s.data(), s.size() * 4, hipMemcpyHostToDevice)) != hipSuccess)
    return hip_fail(e, "hipMemcpy rope");
  m->rope_len = len;
  return SOC_OK;
}

soc::AttnArgs attn_args(soc_model* m, soc_kv* kv, int layer) {
  soc::AttnArgs a{};
  a.q_gain = m->layers[layer].q_norm;
  a.k_gain = m->layers[layer].k_norm;
  a.eps = m->cfg.rms_norm_eps;
  a.rope_cos = m->rope_cos;
  a.rope_sin = m->rope_sin;
  a.kcache = kv->k;
  a.vcache = kv->v;
  a.slot_stride = kv->slot_stride;
  a.layer_stride = kv->layer_stride;
  a.layer = layer;
  a.cap = kv->cap;
  a.nq = m->cfg.num_attention_heads;
  a.nkv = m->cfg.num_key_value_heads;
  a.chunk = kAttnChunk;
  a.scale = 1.0f / std::sqrt(static_cast<float>(m->cfg.head_dim));  // grouped_query_attention.cpp:81
  return a;
}

// y[M][N] = x[M][K] . W^T on the model's group-quantized codes (M in 1, 2, 4, 8).
hipError_t qmm_rows(const soc_model* m, const soc::f16* x, int M, const uint8_t* codes, const soc::f16* scales, int N,
                    int K, float* y, hipStream_t s) {
  soc::QmmArgs q{};
  q.x = x;
  q.codes = codes;
  q.scales = scales;
  q.y = y;
  q.M = M;
  q.N = N;
  q.K = K;
  return soc::launch_qmm(q, m->qbits, s);
}

// One layer of a quantized model on T rows x (fp32 [T][H]) whose attention input comes out of `qkv_out` (rows of
// [T][qkv_rows], M >= T the projection row count): input RMSNorm -> fp16, QKV projection; the caller's attention
// writes attn (fp32 [T][qd]); then o projection + residual, post RMSNorm -> fp16, gate/up projection, SwiGLU -> fp16,
// down projection + residual. `attend` enqueues the attention.
template <typename Attend>
int enqueue_layer_q(soc_model* m, int l, float* x, int T, int M, soc::f16* qx, float* qy, float* qkv_out,
                    const float* attn, Attend attend, hipStream_t s) {
  const soc_qwen_config& c = m->cfg;
  const DevLayer& L = m->layers[l];
  const QLayer& Q = m->qlayers[l];
  const int H = c.hidden_size, I = c.intermediate_size;
  hipError_t e;
  if ((e = soc::launch_rmsnorm_rows(x, T, H, L.in_norm, c.rms_norm_eps, nullptr, qx, nullptr, s)) != hipSuccess)
    return hip_fail(e, "rmsnorm");
  if ((e = qmm_rows(m, qx, M, Q.qkv, Q.qkv_s, m->qkv_rows, H, qkv_out, s)) != hipSuccess) return hip_fail(e, "qmm qkv");
  SOC_TRY(attend());
  if ((e = soc::launch_f32_to_f16(attn, static_cast<size_t>(T) * m->qd, qx, s)) != hipSuccess)
    return hip_fail(e, "f32 -> f16");
  if ((e = qmm_rows(m, qx, M, Q.o, Q.o_s, H, m->qd, qy, s)) != hipSuccess) return hip_fail(e, "qmm o");
  if ((e = soc::launch_add_f32(x, qy, static_cast<size_t>(T) * H, s)) != hipSuccess) return hip_fail(e, "residual");
  if ((e = soc::launch_rmsnorm_rows(x, T, H, L.post_norm, c.rms_norm_eps, nullptr, qx, nullptr, s)) != hipSuccess)
    return hip_fail(e, "rmsnorm");
  if ((e = qmm_rows(m, qx, M, Q.gu, Q.gu_s, 2 * I, H, qy, s)) != hipSuccess) return hip_fail(e, "qmm gate/up");
  if ((e = soc::launch_swiglu_f16(qy, T, I, qx, s)) != hipSuccess) return hip_fail(e, "swiglu");
  if ((e = qmm_rows(m, qx, M, Q.down, Q.down_s, H, I, qy, s)) != hipSuccess) return hip_fail(e, "qmm down");
  if ((e = soc::launch_add_f32(x, qy, static_cast<size_t>(T) * H, s)) != hipSuccess) return hip_fail(e, "residual");
  return SOC_OK;
}

// Queues one decode step for `slot` reading {token, pos} from dws.state. Used eagerly and under graph capture.
int enqueue_decode(soc_model* m, soc_kv* kv, int slot, const int32_t* d_slot) {
  const soc_qwen_config& c = m->cfg;
  DecodeWs& w = m->dws;
  hipStream_t s = m->ctx->stream;
  hipError_t e;
  if (m->qbits != 0) {  // quantized model: the same steps with group-quantized projections
    if ((e = soc::launch_embed(w.state, 1, m->embed, c.hidden_size, w.x, s)) != hipSuccess)
      return hip_fail(e, "embed");
    for (int l = 0; l < c.num_hidden_layers; ++l) {
      auto attend = [&]() -> int {
        soc::AttnArgs a = attn_args(m, kv, l);
        a.qkv = w.qkv;
        a.ld_qkv = m->qkv_rows;
        a.pos = w.state + 1;
        a.slot = d_slot;
        a.slot_base = slot;
        a.pos_base = 0;
        a.out = w.attn;
        a.ld_out = m->qd;
        a.part = w.part;
        a.counters = w.attn_counters;
        a.B = 1;
        a.chunk = decode_attn_chunk(kv->cap);
        a.max_split = (kv->cap + a.chunk - 1) / a.chunk;
        const hipError_t ea = soc::launch_attention(a, 1, s);
        return ea == hipSuccess ? SOC_OK : hip_fail(ea, "attention decode");
      };
      SOC_TRY(enqueue_layer_q(m, l, w.x, 1, 1, w.qx, w.qy, w.qkv, w.attn, attend, s));
    }
  } else {
    if ((e = soc::launch_embed(w.state, 1, m->embed, c.hidden_size, w.x, s)) != hipSuccess) return hip_fail(e, "embed");
    for (int l = 0; l < c.num_hidden_layers; ++l) {
      const DevLayer& L = m->layers[l];
      soc::GemvArgs g{};
      g.x = w.x;
      g.gain = L.in_norm;
      g.eps = c.rms_norm_eps;
      g.w = L.wqkv;
      g.y = w.qkv;
      g.N = m->qkv_rows;
      g.K = c.hidden_size;
      if ((e = soc::launch_gemv(g, soc::EPI_STORE, s)) != hipSuccess) return hip_fail(e, "gemv qkv");
      soc::AttnArgs a = attn_args(m, kv, l);
      a.qkv = w.qkv;
      a.ld_qkv = m->qkv_rows;
      a.pos = w.state + 1;
      a.slot = d_slot;
      a.slot_base = slot;
      a.pos_base = 0;
      a.out = w.attn;
      a.ld_out = m->qd;
      a.part = w.part;
      a.counters = w.attn_counters;
      a.B = 1;
      a.chunk = decode_attn_chunk(kv->cap);
      a.max_split = (kv->cap + a.chunk - 1) / a.chunk;
      if ((e = soc::launch_attention(a, 1, s)) != hipSuccess) return hip_fail(e, "attention decode");
      g = soc::GemvArgs{};
      g.x = w.attn;
      g.w = L.wo;
      g.y = w.x;
      g.N = c.hidden_size;
      g.K = m->qd;
      if ((e = soc::launch_gemv(g, soc::EPI_RESIDUAL, s)) != hipSuccess) return hip_fail(e, "gemv o");
      g = soc::GemvArgs{};
      g.x = w.x;
      g.gain = L.post_norm;
      g.eps = c.rms_norm_eps;
      g.w = L.wgate;
      g.w2 = L.wup;
      g.y = w.h;
      g.N = c.intermediate_size;
      g.K = c.hidden_size;
      if ((e = soc::launch_gemv(g, soc::EPI_SWIGLU, s)) != hipSuccess) return hip_fail(e, "gemv gate/up");
      g = soc::GemvArgs{};
      g.x = w.h;
      g.w = L.wdown;
      g.y = w.x;
      g.N = c.hidden_size;
      g.K = c.intermediate_size;
      if ((e = soc::launch_gemv(g, soc::EPI_RESIDUAL, s)) != hipSuccess) return hip_fail(e, "gemv down");
    }
  }
  soc::LmHeadArgs h{};
  h.x = w.x;
  h.gain = m->final_norm;
  h.eps = c.rms_norm_eps;
  h.w = m->lm_head;
  h.logits = w.logits;
  h.part_val = w.lm_val;
  h.part_idx = w.lm_idx;
  h.counter = w.lm_counter;
  h.state = w.state;
  h.ring = w.ring;
  h.ring_pos = w.ring_pos;
  h.N = c.vocab_size;
  h.K = c.hidden_size;
  if ((e = soc::launch_lm_head_argmax(h, s)) != hipSuccess) return hip_fail(e, "lm head");
  return SOC_OK;
}

int get_decode_graph(soc_model* m, soc_kv* kv, int slot, hipGraphExec_t* out) {
  auto it = kv->graphs.find(slot);
  if (it != kv->graphs.end()) {
    if (it->second.first == m->dws_gen) {
      *out = it->second.second;
      return SOC_OK;
    }
    (void)hipGraphExecDestroy(it->second.second);
    kv->graphs.erase(it);
  }
  hipStream_t s = m->ctx->stream;
  hipGraph_t graph;
  hipError_t e = hipStreamBeginCapture(s, hipStreamCaptureModeThreadLocal);
  if (e != hipSuccess) return hip_fail(e, "hipStreamBeginCapture");
  int rc = enqueue_decode(m, kv, slot, nullptr);
  e = hipStreamEndCapture(s, &graph);
  if (rc != SOC_OK) return rc;
  if (e != hipSuccess) return hip_fail(e, "hipStreamEndCapture");
  hipGraphExec_t exec;
  e = hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0);
  (void)hipGraphDestroy(graph);
  if (e != hipSuccess) return hip_fail(e, "hipGraphInstantiate");
  kv->graphs[slot] = std::make_pair(m->dws_gen, exec);
  *out = exec;
  return SOC_OK;
}

// Decode implementation for batch 1: the XCD-partitioned one-launch step when the model has one KV head per XCD and
// fits its tiling (2), else the one-launch step with attention blocks (1), else the per-op kernels replayed from a
// HIP graph (0). SOC_DECODE=xcd / persistent / graph restricts the choice (an unsupported choice falls back).
bool use_xcd(soc_model* m) {
  const char* mode = std::getenv("SOC_DECODE");
  if (mode != nullptr && std::strcmp(mode, "xcd") != 0) return false;
  if (env_flag("SOC_EAGER") || m->xcd_off || m->qbits != 0) return false;
  const soc_qwen_config& c = m->cfg;
  if (!soc::xcd_supported(c.hidden_size, c.intermediate_size, c.num_attention_heads, c.num_key_value_heads,
                          c.head_dim, m->ctx->num_cus))
    return false;
  int per_cu = 0;
  if (soc::xcd_blocks_per_cu(c.num_attention_heads / c.num_key_value_heads, &per_cu) != hipSuccess) return false;
  return per_cu >= 1;
}

bool use_persistent(soc_model* m) {
  const char* mode = std::getenv("SOC_DECODE");
  if (mode != nullptr && std::strcmp(mode, "persistent") != 0 && std::strcmp(mode, "xcd") != 0) return false;
  if (env_flag("SOC_EAGER") || m->qbits != 0) return false;
  const soc_qwen_config& c = m->cfg;
  const int nb = m->ctx->num_cus;
  if (!soc::persistent_supported(c.hidden_size, m->qd, c.intermediate_size, m->qkv_rows, c.num_attention_heads,
                                 c.num_key_value_heads, nb))
    return false;
  int per_cu = 0;
  if (soc::persistent_blocks_per_cu(c.num_attention_heads / c.num_key_value_heads, &per_cu) != hipSuccess) return false;
  return per_cu * m->ctx->num_cus >= nb;
}

soc::PersistArgs persist_args(soc_model* m, soc_kv* kv, int slot, const DecodeWs& w) {
  const soc_qwen_config& c = m->cfg;
  soc::PersistArgs p{};
  p.layer_w = m->d_layer_w;
  p.embed = m->embed;
  p.final_norm = m->final_norm;
  p.lm_head = m->lm_head;
  p.rope_cos = m->rope_cos;
  p.rope_sin = m->rope_sin;
  p.kcache = kv->k + static_cast<size_t>(slot) * kv->slot_stride;
  p.vcache = kv->v + static_cast<size_t>(slot) * kv->slot_stride;
  p.layer_stride = kv->layer_stride;
  p.cap = kv->cap;
  p.L = c.num_hidden_layers;
  p.H = c.hidden_size;
  p.I = c.intermediate_size;
  p.V = c.vocab_size;
  p.nq = c.num_attention_heads;
  p.nkv = c.num_key_value_heads;
  p.qkv_rows = m->qkv_rows;
  p.qd = m->qd;
  p.xs_cap = std::max(std::max(c.hidden_size, m->qd), c.intermediate_size);
  p.eps = c.rms_norm_eps;
  p.scale = 1.0f / std::sqrt(static_cast<float>(c.head_dim));
  p.xa = w.xa;
  p.xb = w.xb;
  p.qkv = w.qkv_x;
  p.attn = w.attn_x;
  p.h = w.h_x;
  p.logits = w.logits;
  p.part_val = w.pv;
  p.part_idx = w.pi;
  p.counter = w.lm_counter;
  p.state = w.state;
  p.ring = w.ring;
  p.ring_pos = w.ring_pos;
  p.err = w.err;
  p.xo = w.xo;
  p.xd = w.xd;
  p.xp = w.xp;
  p.loc = w.loc;
  p.loc_stride = w.loc_stride;
  p.xcd_ctr = w.xcd_ctr;
  p.steps = 1;
  if (const char* sl = std::getenv("SOC_SPIN_SLEEP")) p.spin_sleep = std::max(0, std::atoi(sl));
  // SOC_WAIT_TICKS=<n>: bound of the cross-block waits (tests force the time-out path with a tiny bound; every
  // block still exits normally, the waits only give up sooner)
  p.spin_ticks = soc::kSpinTicks;
  const char* coop = std::getenv("SOC_COOP_LAUNCH");
  p.cooperative = coop != nullptr && coop[0] == '1';
  if (const char* wt = std::getenv("SOC_WAIT_TICKS")) p.spin_ticks = std::strtoull(wt, nullptr, 10);
  return p;
}

// The status of a one-launch decode whose error word read `err` (0: none).
int one_launch_status(soc_model* m, bool xcd, int32_t err) {
  if (err == 0) return SOC_OK;
  // a bounded wait expired: drop the exchange state so the next call starts clean
  m->dws.ready = false;
  if (xcd && err == 2) {
    m->xcd_off = true;
    return soc::fail(SOC_ERR_HIP, "XCD decode: the launch did not place 32 blocks on each of the 8 XCDs");
  }
  return soc::fail(SOC_ERR_HIP, "one-launch decode: a cross-block wait timed out (grid not co-resident?)");
}

// `steps` decode steps of one slot from token `last` (host value) or, with dev_last, the id in device memory (staged
// and checked on the device). With err_out set (and no SOC_TRACE_FILE), the one-launch paths neither read their error
// word nor synchronise: the caller reads dws.err with its results and checks it with one_launch_status. logits_out
// (device memory of vocab floats, one-launch paths only) receives the logits in place of dws.logits.
int run_decode_steps(soc_model* m, soc_kv* kv, int slot, int32_t last, int steps, const int32_t* dev_last = nullptr,
                     int32_t* err_out = nullptr, float* logits_out = nullptr) {
  DecodeWs& w = m->dws;
  hipStream_t s = m->ctx->stream;
  hipError_t e;
  if ((e = soc::launch_decode_prologue(dev_last, last, kv->len[slot], m->cfg.vocab_size, w.state, w.ring_pos,
                                       m->ctx->id_err, s)) != hipSuccess)
    return hip_fail(e, "decode prologue");
  const bool xcd = use_xcd(m);
  if (xcd || use_persistent(m)) {
    soc::PersistArgs p = persist_args(m, kv, slot, w);
    if (logits_out != nullptr) p.logits = logits_out;
    if (env_flag("SOC_FORCE_WAIT_ERROR")) {
      // failure-path tests: the error flag as a timed-out wait leaves it, raised before the launches (each block of
      // each launch then leaves at entry)
      const int32_t one = 1;
      if ((e = hipMemcpyAsync(w.err, &one, sizeof(one), hipMemcpyHostToDevice, s)) != hipSuccess)
        return hip_fail(e, "hipMemcpyAsync err");
    }
    // SOC_TRACE_FILE=<path>: append the last step's per-phase timestamps (diagnostics)
    const char* trace_path = std::getenv("SOC_TRACE_FILE");
    const size_t trace_roles = 2 * (4 + 8 * static_cast<size_t>(m->cfg.num_hidden_layers));
    const size_t xcd_nb = static_cast<size_t>(soc::kXcdGroups) * soc::kXcdBlocks;
    const size_t trace_n = xcd ? static_cast<size_t>(soc::kTraceTotal)
                               : trace_roles + static_cast<size_t>(w.nblocks) * 8;
    if (trace_path != nullptr) {
      if ((e = hipMalloc(&p.trace, trace_n * sizeof(uint64_t))) != hipSuccess) return hip_fail(e, "hipMalloc trace");
      // on the decode stream: a null-stream memset is not ordered with the launches below and could clear the
      // timestamps after a long launch has written them (diagnostics only; this path is never captured)
      if ((e = hipMemsetAsync(p.trace, 0, trace_n * sizeof(uint64_t), s)) != hipSuccess) return hip_fail(e, "hipMemset");
    }
    if (xcd) {  // k_decode_xcd runs up to kXcdStepsPerLaunch steps per launch, releasing each token on the device
      for (int i = 0; i < steps; i += kXcdStepsPerLaunch) {
        p.steps = std::min(kXcdStepsPerLaunch, steps - i);
        if ((e = soc::launch_decode_xcd(p, s)) != hipSuccess) return hip_fail(e, "one-launch decode");
      }
    } else {
      for (int i = 0; i < steps; ++i)
        if ((e = soc::launch_decode_persistent(p, w.nblocks, s)) != hipSuccess)
          return hip_fail(e, "persistent decode launch");
    }
    if (err_out != nullptr && trace_path == nullptr) return SOC_OK;  // the caller reads the flag and synchronises
    int32_t err_local = 0;
    int32_t& err = err_out != nullptr ? *err_out : err_local;
    if ((e = hipMemcpyAsync(&err, w.err, 4, hipMemcpyDeviceToHost, s)) != hipSuccess)
      return hip_fail(e, "hipMemcpyAsync err");
    record_timer_stop(m->ctx);
    if ((e = hipStreamSynchronize(s)) != hipSuccess) return hip_fail(e, "persistent decode");
    if (p.trace != nullptr) {
      std::vector<uint64_t> t(trace_n);
      e = hipMemcpy(t.data(), p.trace, trace_n * sizeof(uint64_t), hipMemcpyDeviceToHost);
      (void)hipFree(p.trace);
      if (e != hipSuccess) return hip_fail(e, "hipMemcpy trace");
      if (xcd) {  // the raw timestamps of the last call, for offline analysis
        FILE* fb = std::fopen((std::string(trace_path) + ".bin").c_str(), "wb");
        if (fb != nullptr) {
          (void)std::fwrite(t.data(), sizeof(uint64_t), t.size(), fb);
          std::fclose(fb);
        }
      }
      FILE* f = std::fopen(trace_path, "a");
      if (f != nullptr && xcd) {
        // block (0, 0): layer durations, LM head; then the middle layer's phase points over all blocks
        const int L = m->cfg.num_hidden_layers;
        const uint64_t* t0p = t.data() + xcd_nb * soc::kTracePts;
        std::fprintf(f, "xcd block(0,0) layer us:");
        for (int l = 1; l <= L; ++l) std::fprintf(f, " %.2f", (static_cast<double>(t0p[l]) - t0p[l - 1]) * 0.01);
        std::fprintf(f, " | lm head %.2f\n", (static_cast<double>(t0p[L + 1]) - t0p[L]) * 0.01);
        // the per-block points are wave 0's
        for (size_t b = 0; b < xcd_nb; ++b)
          for (int pnt = 0; pnt < soc::kTracePts; ++pnt)
            t[b * soc::kTracePts + pnt] = t[soc::kTraceWaveBase + (b * 8) * soc::kTracePts + pnt];
        uint64_t tmin = ~0ull;
        for (size_t b = 0; b < xcd_nb; ++b)
          if (t[b * soc::kTracePts] != 0) tmin = std::min(tmin, t[b * soc::kTracePts]);
        std::fprintf(f, "xcd middle layer (us from earliest start):");
        for (int pnt = 0; pnt < soc::kTracePts; ++pnt) {
          std::vector<double> v;
          for (size_t b = 0; b < xcd_nb; ++b)
            if (t[b * soc::kTracePts + pnt] != 0) v.push_back((static_cast<double>(t[b * soc::kTracePts + pnt]) - tmin) * 0.01);
          std::sort(v.begin(), v.end());
          if (!v.empty()) std::fprintf(f, " %c[%.2f %.2f %.2f]", "0ABCDEFGHIJkbegaLMNOPQRSTUVWXYZ."[pnt], v.front(), v[v.size() / 2], v.back());
        }
        std::fprintf(f, "\n");
        // per block rank j (max over the XCDs) of point D and the first blocks with the latest D
        std::fprintf(f, "D by rank:");
        for (int j = 0; j < soc::kXcdBlocks; ++j) {
          double dmax = -1;
          for (int g = 0; g < soc::kXcdGroups; ++g) {
            const size_t b = static_cast<size_t>(g) * soc::kXcdBlocks + j;
            if (t[b * soc::kTracePts + 4] != 0) dmax = std::max(dmax, (static_cast<double>(t[b * soc::kTracePts + 4]) - tmin) * 0.01);
          }
          if (dmax >= 0) std::fprintf(f, " j%d:%.2f", j, dmax);
        }
        std::fprintf(f, "\n");
        std::fclose(f);
        f = nullptr;
      }
      if (f != nullptr) {
        const size_t per = trace_roles / 2;
        for (int which = 0; which < 2; ++which) {
          std::fprintf(f, "%s:", which == 0 ? "block0" : "blockN");
          for (size_t i = 1; i < per; ++i) {
            const uint64_t x = t[which * per + i], y = t[which * per + i - 1];
            if (x == 0 || y == 0) std::fprintf(f, " -");
            else std::fprintf(f, " %.2f", (static_cast<double>(x) - static_cast<double>(y)) * 0.01);  // us (100 MHz)
          }
          std::fprintf(f, "\n");
        }
        // middle layer, every projection block: per point, min / median / max relative to the earliest point-0
        const int ng = w.nblocks - m->cfg.num_key_value_heads;
        uint64_t t0 = ~0ull;
        for (int b = 0; b < ng; ++b)
          if (t[trace_roles + b * 8] != 0) t0 = std::min(t0, t[trace_roles + b * 8]);
        std::fprintf(f, "middle layer (us from earliest P1-input):");
        for (int pnt = 0; pnt < 8; ++pnt) {
          std::vector<double> v;
          for (int b = 0; b < ng; ++b)
            if (t[trace_roles + b * 8 + pnt] != 0) v.push_back((static_cast<double>(t[trace_roles + b * 8 + pnt]) - t0) * 0.01);
          std::sort(v.begin(), v.end());
          if (!v.empty()) std::fprintf(f, " p%d[%.2f %.2f %.2f]", pnt, v.front(), v[v.size() / 2], v.back());
        }
        std::fprintf(f, "\n");
        std::fclose(f);
      }
    }
    if (err != 0) {
      const int rc = one_launch_status(m, xcd, err);
      err = 0;  // reported here: the caller does not report it again
      return rc;
    }
  } else if (env_flag("SOC_EAGER")) {
    for (int i = 0; i < steps; ++i) SOC_TRY(enqueue_decode(m, kv, slot, nullptr));
  } else {
    hipGraphExec_t g;
    SOC_TRY(get_decode_graph(m, kv, slot, &g));
    for (int i = 0; i < steps; ++i)
      if ((e = hipGraphLaunch(g, s)) != hipSuccess) return hip_fail(e, "hipGraphLaunch");
  }
  return SOC_OK;
}

// Which prefill projections see their activations as hi/lo fp16 pairs (22 significant bits, close to the
// reference's fp32 activations) rather than as one fp16 value (half the MFMA work, less precision margin): a mask of
// kSplitQkv | kSplitO | kSplitGateUp | kSplitDown. Default: the QKV projection only — measured on the Qwen3-0.6B
// fixtures, the pairs on QKV keep most of the precision the pairs on all four give (largest logit error 9.6e-3 vs
// 6.6e-3 on the N(0, 0.05) model, 1.2e-3 vs 7.7e-4 at 2048 tokens; none: 1.43e-2 / 1.6e-3; tolerance 2e-2) at 84 %
// of the time (2048 tokens: 6.74 vs 8.06 ms). SOC_PREFILL_SPLIT: "1" / "all" = all four, "0" = none, otherwise a
// comma list of qkv, o, gateup, down.
enum { kSplitQkv = 1, kSplitO = 2, kSplitGateUp = 4, kSplitDown = 8, kSplitAll = 15 };
int prefill_split_mask() {
  const char* sp = std::getenv("SOC_PREFILL_SPLIT");
  if (sp == nullptr) return kSplitQkv;
  if (sp[0] == '0') return 0;
  const std::string v(sp);
  int mask = 0;
  size_t b = 0;
  while (b <= v.size()) {
    const size_t e = std::min(v.find(',', b), v.size());
    const std::string t = v.substr(b, e - b);
    if (t == "qkv") mask |= kSplitQkv;
    if (t == "o") mask |= kSplitO;
    if (t == "gateup") mask |= kSplitGateUp;
    if (t == "down") mask |= kSplitDown;
    if (t == "1" || t == "all") mask |= kSplitAll;
    b = e + 1;
  }
  return mask;
}

// Prefill projections on fp32 activations, on MFMA (every K the model config admits is a multiple of 32), the
// activations as fp16 or as hi/lo pairs (hi/lo when prefill_split_mask() has any of the bits `which`).
hipError_t prefill_gemm(const soc::GemmArgs& g, int epi, hipStream_t s, int which = kSplitAll) {
  return soc::launch_gemm_mfma(g, epi, (prefill_split_mask() & which) != 0, s);
}

// The prefill layers use the GEMM on fp16 activations written by their producers (direct-to-LDS pipeline);
// SOC_PREFILL_GEMM=staged keeps the register-staged MFMA kernel on fp32 activations (same products: the parity
// tests compare the two).
bool prefill_split_path(const soc_model* m) {
  (void)m;
  const char* mode = std::getenv("SOC_PREFILL_GEMM");
  return !(mode != nullptr && std::strcmp(mode, "staged") == 0);
}


hipError_t split_gemm(const soc::f16* ah, const soc::f16* al, int lda, const soc::f16* w, const soc::f16* w2,
                      float* c, soc::f16* ch, soc::f16* cl, int ldc, int M, int N, int K, int epi, hipStream_t s) {
  soc::GemmSplitArgs g{};
  g.ah = ah;
  g.al = al;
  g.lda = lda;
  g.w = w;
  g.w2 = w2;
  g.c = c;
  g.ch = ch;
  g.cl = cl;
  g.ldc = ldc;
  g.M = M;
  g.N = N;
  g.K = K;
  return soc::launch_gemm_split(g, epi, s);
}

// A ragged-batch projection on the skinny kernel, in chunks of 16 rows: `proto` carries the weights, the input
// RMSNorm gain (or none) and the epilogue's own arguments; rows m0.. of x, c, q_out, pos and slots per chunk.
hipError_t batch_skinny(const soc::SkinnyArgs& proto, int n, int epi, hipStream_t s) {
  for (int m0 = 0; m0 < n; m0 += 16) {
    soc::SkinnyArgs a = proto;
    a.x = proto.x + static_cast<size_t>(m0) * proto.ldx;
    a.M = std::min(16, n - m0);
    if (proto.c != nullptr) a.c = proto.c + static_cast<size_t>(m0) * proto.ldc;
    if (epi == soc::EPI_QKV) {
      a.q_out = proto.q_out + static_cast<size_t>(m0) * proto.nq * 128;
      a.pos = proto.pos + m0;
      a.slots = proto.slots + m0;
    }
    const hipError_t e = soc::launch_skinny(a, epi, s);
    if (e != hipSuccess) return e;
  }
  return hipSuccess;
}

// Largest split-K scratch any projection of the model needs in the skinny kernel (floats).
size_t skinny_scratch_floats(const soc_model* m) {
  const soc_qwen_config& c = m->cfg;
  const int H = c.hidden_size, I = c.intermediate_size;
  if (H % 256 != 0 || I % 256 != 0 || m->qd % 256 != 0) return 0;
  size_t need = 0;
  need = std::max(need, soc::skinny_part_floats(m->qkv_rows, H));
  need = std::max(need, soc::skinny_part_floats(H, m->qd));
  need = std::max(need, soc::skinny_part_floats(2 * I, H));
  need = std::max(need, soc::skinny_part_floats(H, I));
  need = std::max(need, soc::skinny_part_floats(c.vocab_size, H));
  return need;
}

// Prefill attention runs the load-balanced MFMA flash kernel (query-tile pairs) where the head grouping allows,
// else the per-tile MFMA flash kernel (SOC_PREFILL_ATTN=tiles forces the latter, SOC_PREFILL_ATTN=rows the per-row
// split-key kernel that decode also uses). With a.out_hi / a.out_lo set, the row kernel writes fp32 into `scratch`
// and a split pass produces the hi/lo pair.
hipError_t prefill_attention(const soc::AttnArgs& a, float* scratch, hipStream_t s) {
  const char* mode = std::getenv("SOC_PREFILL_ATTN");
  const bool rows = mode != nullptr && std::strcmp(mode, "rows") == 0;
  const bool tiles = mode != nullptr && std::strcmp(mode, "tiles") == 0;
  if (!rows && !tiles && soc::attention_prefill_pairs_supported(a.nq, a.nkv))
    return soc::launch_attention_prefill_pairs(a, s);
  if (!rows && soc::attention_prefill_mfma_supported(a.nq, a.nkv)) return soc::launch_attention_prefill_mfma(a, s);
  if (a.out_hi == nullptr) return soc::launch_attention(a, 0, s);
  soc::AttnArgs b = a;
  b.out = scratch;
  b.out_hi = b.out_lo = nullptr;
  const hipError_t e = soc::launch_attention(b, 0, s);
  if (e != hipSuccess) return e;
  return soc::launch_split_f16(scratch, static_cast<size_t>(a.B) * a.ld_out, a.out_hi, a.out_lo, s);
}

int validate_ids(const soc_model* m, const int32_t* ids, int n) {
  for (int i = 0; i < n; ++i)
    if (ids[i] < 0 || ids[i] >= m->cfg.vocab_size)
      return soc::fail(SOC_ERR_INVALID, "token id out of range");  // embedding.cpp:66-68
  return SOC_OK;
}


int ensure_batch_ws(soc_model* m, int n) {
  BatchWs& b = m->bws;
  if (b.cap >= n) return SOC_OK;
  hipError_t e = hipStreamSynchronize(m->ctx->stream);
  if (e != hipSuccess) return hip_fail(e, "hipStreamSynchronize");
  free_all(b.allocs);
  (void)hipFree(b.ring);
  ++m->bws_gen;
  b = BatchWs();
  SOC_TRY(dev_alloc_t(b.allocs, n, &b.ids));
  SOC_TRY(dev_alloc_t(b.allocs, n, &b.pos));
  SOC_TRY(dev_alloc_t(b.allocs, n, &b.start));
  SOC_TRY(dev_alloc_t(b.allocs, n, &b.slots));
  SOC_TRY(dev_alloc_t(b.allocs, n, &b.ring1));
  SOC_TRY(dev_alloc_t(b.allocs, static_cast<size_t>(n) * soc::kArgmaxMaxChunks, &b.am_val));
  SOC_TRY(dev_alloc_t(b.allocs, static_cast<size_t>(n) * soc::kArgmaxMaxChunks, &b.am_idx));
  SOC_TRY(dev_alloc_t(b.allocs, n, &b.am_cnt));
  if ((e = hipMemset(b.am_cnt, 0, static_cast<size_t>(n) * sizeof(int32_t))) != hipSuccess)
    return hip_fail(e, "hipMemset");
  b.cap = n;
  return SOC_OK;
}

// Checks a ragged batch: 1 <= n <= kMaxBatchRows, distinct slots in range, valid token ids, room for `steps` more
// positions in every slot. Returns the largest final length in *max_len.
int validate_batch(soc_model* m, soc_kv* kv, int n, const int32_t* slots, const int32_t* tokens, int steps,
                   int* max_len) {
  if (m == nullptr || kv == nullptr || slots == nullptr || tokens == nullptr)
    return soc::fail(SOC_ERR_INVALID, "null argument");
  SOC_TRY(bind_kv(kv, m));
  if (!m->finalized) return soc::fail(SOC_ERR_STATE, "model is not finalized");
  if (n <= 0 || n > kMaxBatchRows) return soc::fail(SOC_ERR_INVALID, "batch size must be in [1, 1024]");
  std::vector<char> seen(kv->slots, 0);
  int ml = 0;
  for (int i = 0; i < n; ++i) {
    const int sl = slots[i];
    if (sl < 0 || sl >= kv->slots) return soc::fail(SOC_ERR_INVALID, "slot out of range");
    if (seen[sl]) return soc::fail(SOC_ERR_INVALID, "a slot appears twice in the batch");
    seen[sl] = 1;
    if (kv->len[sl] + steps > kv->cap) return soc::fail(SOC_ERR_CAPACITY, "decode exceeds KV capacity");
    ml = std::max(ml, kv->len[sl] + steps);
  }
  SOC_TRY(validate_ids(m, tokens, n));
  *max_len = ml;
  return SOC_OK;
}

// Queues one decode step of the n rows in m->bws: row i runs token ids[i] at position pos[i] of KV slot slots[i].
// Its greedy token is written back to ids[i], recorded in ring[i * ring_stride + pos[i] - start[i]], and pos[i]
// advances. Used eagerly and under graph capture (every per-step quantity lives in device memory).
int enqueue_batch_step(soc_model* m, soc_kv* kv, int n, int max_split, int32_t* ring, int ring_stride) {
  const soc_qwen_config& c = m->cfg;
  PrefillWs& w = m->pws;
  BatchWs& b = m->bws;
  hipStream_t s = m->ctx->stream;
  const int H = c.hidden_size, I = c.intermediate_size;
  hipError_t e;
  // up to 64 rows: the skinny kernels per projection and 16 rows (input RMSNorm and the q/k norm, RoPE and KV append
  // folded into them); beyond, the tile GEMMs with separate normalisation and q/k kernels
  const bool fused = w.skpart != nullptr && n <= 64;
  soc::SkinnyArgs sk{};
  sk.part = w.skpart;
  sk.eps = c.rms_norm_eps;
  if ((e = soc::launch_embed(b.ids, n, m->embed, H, w.x, s)) != hipSuccess) return hip_fail(e, "embed");
  for (int l = 0; l < c.num_hidden_layers; ++l) {
    const DevLayer& L = m->layers[l];
    if (fused) {
      soc::SkinnyArgs a = sk;
      a.x = w.x;
      a.ldx = H;
      a.w = L.wqkv;
      a.N0 = a.Ntot = m->qkv_rows;
      a.K = H;
      a.gain = L.in_norm;
      a.q_out = w.q;
      a.kcache = kv->k;
      a.vcache = kv->v;
      a.q_gain = L.q_norm;
      a.k_gain = L.k_norm;
      a.rope_cos = m->rope_cos;
      a.rope_sin = m->rope_sin;
      a.pos = b.pos;
      a.slots = b.slots;
      a.slot_stride = kv->slot_stride;
      a.layer_stride = kv->layer_stride;
      a.layer = l;
      a.cap = kv->cap;
      a.nq = c.num_attention_heads;
      a.nkv = c.num_key_value_heads;
      if ((e = batch_skinny(a, n, soc::EPI_QKV, s)) != hipSuccess) return hip_fail(e, "skinny qkv");
    } else {
      if ((e = soc::launch_rmsnorm_rows(w.x, n, H, L.in_norm, c.rms_norm_eps, w.xn, nullptr, nullptr, s)) !=
          hipSuccess)
        return hip_fail(e, "rmsnorm");
      soc::GemmArgs g{};
      g.a = w.xn;
      g.lda = H;
      g.w = L.wqkv;
      g.c = w.qkv;
      g.ldc = m->qkv_rows;
      g.M = n;
      g.N = m->qkv_rows;
      g.K = H;
      if ((e = prefill_gemm(g, soc::EPI_STORE, s)) != hipSuccess) return hip_fail(e, "gemm qkv");
      soc::QkNormRopeArgs q{};
      q.qkv = w.qkv;
      q.ld_qkv = m->qkv_rows;
      q.q_gain = L.q_norm;
      q.k_gain = L.k_norm;
      q.eps = c.rms_norm_eps;
      q.rope_cos = m->rope_cos;
      q.rope_sin = m->rope_sin;
      q.q_out = w.q;
      q.kcache = kv->k;
      q.vcache = kv->v;
      q.slot_stride = kv->slot_stride;
      q.layer_stride = kv->layer_stride;
      q.layer = l;
      q.cap = kv->cap;
      q.T = n;
      q.nq = c.num_attention_heads;
      q.nkv = c.num_key_value_heads;
      q.pos = b.pos;
      q.slots = b.slots;
      if ((e = soc::launch_qk_norm_rope_append(q, s)) != hipSuccess) return hip_fail(e, "qk norm rope");
    }
    soc::AttnArgs at = attn_args(m, kv, l);
    at.qkv = w.q;
    at.ld_qkv = m->qd;
    at.pos = b.pos;
    at.slot = b.slots;
    at.out = w.attn;
    at.ld_out = m->qd;
    at.part = w.part;
    at.counters = w.attn_counters;
    at.B = n;
    at.max_split = max_split;
    if ((e = soc::launch_attention(at, 0, s)) != hipSuccess) return hip_fail(e, "attention");
    if (fused) {
      soc::SkinnyArgs a = sk;  // o: x += attn . Wo^T
      a.x = w.attn;
      a.ldx = m->qd;
      a.w = L.wo;
      a.N0 = a.Ntot = H;
      a.K = m->qd;
      a.c = w.x;
      a.ldc = H;
      if ((e = batch_skinny(a, n, soc::EPI_RESIDUAL, s)) != hipSuccess) return hip_fail(e, "skinny o");
      a = sk;  // gate/up of RMSNorm(x) + SwiGLU
      a.x = w.x;
      a.ldx = H;
      a.w = L.wgate;
      a.w2 = L.wup;
      a.N0 = I;
      a.Ntot = 2 * I;
      a.K = H;
      a.gain = L.post_norm;
      a.c = w.h;
      a.ldc = I;
      if ((e = batch_skinny(a, n, soc::EPI_SWIGLU, s)) != hipSuccess) return hip_fail(e, "skinny gate/up");
      a = sk;  // down: x += h . Wd^T
      a.x = w.h;
      a.ldx = I;
      a.w = L.wdown;
      a.N0 = a.Ntot = H;
      a.K = I;
      a.c = w.x;
      a.ldc = H;
      if ((e = batch_skinny(a, n, soc::EPI_RESIDUAL, s)) != hipSuccess) return hip_fail(e, "skinny down");
      continue;
    }
    soc::GemmArgs g{};
    g.a = w.attn;
    g.lda = m->qd;
    g.w = L.wo;
    g.c = w.x;
    g.ldc = H;
    g.M = n;
    g.N = H;
    g.K = m->qd;
    if ((e = prefill_gemm(g, soc::EPI_RESIDUAL, s)) != hipSuccess) return hip_fail(e, "gemm o");
    if ((e = soc::launch_rmsnorm_rows(w.x, n, H, L.post_norm, c.rms_norm_eps, w.xn, nullptr, nullptr, s)) != hipSuccess)
      return hip_fail(e, "rmsnorm");
    g = soc::GemmArgs{};
    g.a = w.xn;
    g.lda = H;
    g.w = L.wgate;
    g.w2 = L.wup;
    g.c = w.h;
    g.ldc = I;
    g.M = n;
    g.N = I;
    g.K = H;
    if ((e = prefill_gemm(g, soc::EPI_SWIGLU, s)) != hipSuccess) return hip_fail(e, "gemm gate/up");
    g = soc::GemmArgs{};
    g.a = w.h;
    g.lda = I;
    g.w = L.wdown;
    g.c = w.x;
    g.ldc = H;
    g.M = n;
    g.N = H;
    g.K = I;
    if ((e = prefill_gemm(g, soc::EPI_RESIDUAL, s)) != hipSuccess) return hip_fail(e, "gemm down");
  }
  if (fused) {
    soc::SkinnyArgs a = sk;  // LM head of RMSNorm(x) with the final gain
    a.x = w.x;
    a.ldx = H;
    a.w = m->lm_head;
    a.N0 = a.Ntot = c.vocab_size;
    a.K = H;
    a.gain = m->final_norm;
    a.c = w.logits;
    a.ldc = c.vocab_size;
    if ((e = batch_skinny(a, n, soc::EPI_STORE, s)) != hipSuccess) return hip_fail(e, "skinny lm head");
  } else {
    if ((e = soc::launch_rmsnorm_rows(w.x, n, H, m->final_norm, c.rms_norm_eps, w.xn, nullptr, nullptr, s)) !=
        hipSuccess)
      return hip_fail(e, "rmsnorm");
    soc::GemmArgs g{};
    g.a = w.xn;
    g.lda = H;
    g.w = m->lm_head;
    g.c = w.logits;
    g.ldc = c.vocab_size;
    g.M = n;
    g.N = c.vocab_size;
    g.K = H;
    if ((e = prefill_gemm(g, soc::EPI_STORE, s)) != hipSuccess) return hip_fail(e, "gemm lm head");
  }
  if ((e = soc::launch_argmax_rows(w.logits, c.vocab_size, n, b.ids, b.pos, b.start, ring, ring_stride, b.am_val,
                                   b.am_idx, b.am_cnt, s)) != hipSuccess)
    return hip_fail(e, "argmax");
  return SOC_OK;
}

// Uploads the batch's rows (ids, positions = current lengths, slots) into m->bws.
int upload_batch(soc_model* m, soc_kv* kv, int n, const int32_t* slots, const int32_t* tokens,
                 std::vector<int32_t>* pos_host) {
  hipStream_t s = m->ctx->stream;
  BatchWs& b = m->bws;
  pos_host->resize(n);
  for (int i = 0; i < n; ++i) (*pos_host)[i] = kv->len[slots[i]];
  hipError_t e;
  if ((e = hipMemcpyAsync(b.ids, tokens, static_cast<size_t>(n) * 4, hipMemcpyHostToDevice, s)) != hipSuccess ||
      (e = hipMemcpyAsync(b.slots, slots, static_cast<size_t>(n) * 4, hipMemcpyHostToDevice, s)) != hipSuccess ||
      (e = hipMemcpyAsync(b.pos, pos_host->data(), static_cast<size_t>(n) * 4, hipMemcpyHostToDevice, s)) !=
          hipSuccess ||
      (e = hipMemcpyAsync(b.start, pos_host->data(), static_cast<size_t>(n) * 4, hipMemcpyHostToDevice, s)) !=
          hipSuccess)
    return hip_fail(e, "hipMemcpyAsync batch");
  return SOC_OK;
}

}  // namespace

// ------------------------------------------------------------------------------------------------------------
// C ABI
// ------------------------------------------------------------------------------------------------------------
extern "C" {


int soc_ctx_create(int device, soc_ctx** out) {
  SOC_API_BEGIN
  if (out == nullptr) return soc::fail(SOC_ERR_INVALID, "soc_ctx_create: null output");
  *out = nullptr;
  int count = 0;
  hipError_t e = hipGetDeviceCount(&count);
  if (e != hipSuccess) return hip_fail(e, "hipGetDeviceCount");
  if (device < 0 || device >= count) return soc::fail(SOC_ERR_INVALID, "soc_ctx_create: no such device");
  if ((e = hipSetDevice(device)) != hipSuccess) return hip_fail(e, "hipSetDevice");
  std::unique_ptr<soc_ctx> c(new soc_ctx());
  c->device = device;
  // this device's copy of the no-allocation scratch array (the device is current)
  void* sp = nullptr;
  if ((e = hipGetSymbolAddress(&sp, HIP_SYMBOL(scratch))) != hipSuccess) return hip_fail(e, "hipGetSymbolAddress");
  c->scratch = static_cast<uint32_t*>(sp);
  if ((e = hipDeviceGetAttribute(&c->num_cus, hipDeviceAttributeMultiprocessorCount, device)) != hipSuccess)
    return hip_fail(e, "hipDeviceGetAttribute");
  if ((e = hipStreamCreateWithFlags(&c->stream, hipStreamNonBlocking)) != hipSuccess)
    return hip_fail(e, "hipStreamCreate");
  if ((e = hipEventCreate(&c->ev0)) != hipSuccess) return hip_fail(e, "hipEventCreate");
  if ((e = hipEventCreate(&c->ev1)) != hipSuccess) return hip_fail(e, "hipEventCreate");
  *out = c.release();
  return SOC_OK;
  SOC_API_END
}

int soc_ctx_destroy(soc_ctx* ctx) {
  if (ctx == nullptr) return SOC_OK;
  (void)hipStreamSynchronize(ctx->stream);
  (void)hipEventDestroy(ctx->ev0);
  (void)hipEventDestroy(ctx->ev1);
  (void)hipStreamDestroy(ctx->stream);
  (void)hipFree(ctx->sample_ws);
  (void)hipFree(ctx->sample_out);
  (void)hipHostFree(ctx->sample_host);
  (void)hipHostFree(ctx->readback);
  (void)hipFree(ctx->op_part);
  (void)hipFree(ctx->op_counters);
  (void)hipFree(ctx->id_err);
  delete ctx;
  return SOC_OK;
}

int soc_ctx_synchronize(soc_ctx* ctx) {
  if (ctx == nullptr) return soc::fail(SOC_ERR_INVALID, "null context");
  hipError_t e = hipStreamSynchronize(ctx->stream);
  return e == hipSuccess ? SOC_OK : hip_fail(e, "hipStreamSynchronize");
}

int soc_ctx_timer_start(soc_ctx* ctx) {
  if (ctx == nullptr) return soc::fail(SOC_ERR_INVALID, "null context");
  hipError_t e = hipEventRecord(ctx->ev0, ctx->stream);
  if (e != hipSuccess) return hip_fail(e, "hipEventRecord");
  ctx->timing = true;
  ctx->stop_recorded = false;
  return SOC_OK;
}

int soc_ctx_timer_stop(soc_ctx* ctx, float* ms) {
  if (ctx == nullptr || ms == nullptr) return soc::fail(SOC_ERR_INVALID, "null argument");
  if (!ctx->timing) return soc::fail(SOC_ERR_STATE, "soc_ctx_timer_stop without soc_ctx_timer_start");
  // a forward that ran since the start recorded the stop event before its own synchronisation: then the event has
  // completed and reading it costs no GPU round trip
  hipError_t e = ctx->stop_recorded ? hipSuccess : hipEventRecord(ctx->ev1, ctx->stream);
  if (e != hipSuccess) return hip_fail(e, "hipEventRecord");
  if ((e = hipEventSynchronize(ctx->ev1)) != hipSuccess) return hip_fail(e, "hipEventSynchronize");
  if ((e = hipEventElapsedTime(ms, ctx->ev0, ctx->ev1)) != hipSuccess) return hip_fail(e, "hipEventElapsedTime");
  ctx->timing = false;
  ctx->stop_recorded = false;
  return SOC_OK;
}

int soc_buffer_alloc(soc_ctx* ctx, size_t bytes, void** p) {
  if (ctx == nullptr || p == nullptr) return soc::fail(SOC_ERR_INVALID, "null argument");
  hipError_t e = hipMalloc(p, bytes == 0 ? 256 : bytes);
  if (e != hipSuccess) {
    (void)hipGetLastError();
    return soc::fail(SOC_ERR_NOMEM, "hipMalloc failed");
  }
  return SOC_OK;
}

int soc_buffer_free(soc_ctx* ctx, void* p) {
  if (ctx == nullptr) return soc::fail(SOC_ERR_INVALID, "null context");
  hipError_t e = hipStreamSynchronize(ctx->stream);
  if (e != hipSuccess) return hip_fail(e, "hipStreamSynchronize");
  if ((e = hipFree(p)) != hipSuccess) return hip_fail(e, "hipFree");
  return SOC_OK;
}

int soc_buffer_write(soc_ctx* ctx, void* dst, const void* src, size_t bytes) {
  if (ctx == nullptr || (bytes && (dst == nullptr || src == nullptr))) return soc::fail(SOC_ERR_INVALID, "null argument");
  hipError_t e = hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, ctx->stream);
  if (e == hipSuccess) e = hipStreamSynchronize(ctx->stream);
  return e == hipSuccess ? SOC_OK : hip_fail(e, "soc_buffer_write");
}

int soc_buffer_write_async(soc_ctx* ctx, void* dst, const void* src, size_t bytes) {
  if (ctx == nullptr || (bytes && (dst == nullptr || src == nullptr))) return soc::fail(SOC_ERR_INVALID, "null argument");
  hipError_t e;
  // a few aligned words into device memory travel in a kernel's arguments: no host staging copy, nothing to wait for
  if (bytes > 0 && bytes <= 64 && bytes % 4 == 0 && reinterpret_cast<uintptr_t>(dst) % 4 == 0 &&
      reinterpret_cast<uintptr_t>(src) % 4 == 0 && soc::classify_range(dst, bytes) == soc::MemRange::kDeviceRange)
    e = soc::launch_write_words(static_cast<int32_t*>(dst), static_cast<const int32_t*>(src),
                                static_cast<int>(bytes / 4), ctx->stream);
  else
    e = hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, ctx->stream);
  return e == hipSuccess ? SOC_OK : hip_fail(e, "soc_buffer_write_async");
}

int soc_buffer_read(soc_ctx* ctx, void* dst, const void* src, size_t bytes) {
  if (ctx == nullptr || (bytes && (dst == nullptr || src == nullptr))) return soc::fail(SOC_ERR_INVALID, "null argument");
  hipError_t e = hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, ctx->stream);
  if (e == hipSuccess) e = hipStreamSynchronize(ctx->stream);
  return e == hipSuccess ? SOC_OK : hip_fail(e, "soc_buffer_read");
}

int soc_model_create(soc_ctx* ctx, const soc_qwen_config* cfg, soc_model** out) {
  SOC_API_BEGIN
  if (ctx == nullptr || cfg == nullptr || out == nullptr) return soc::fail(SOC_ERR_INVALID, "null argument");
  *out = nullptr;
  SOC_TRY(check_config(*cfg));
  std::unique_ptr<soc_model> m(new soc_model());
  m->ctx = ctx;
  m->cfg = *cfg;
  const soc_qwen_config& c = m->cfg;
  m->qd = c.num_attention_heads * c.head_dim;
  m->kvd = c.num_key_value_heads * c.head_dim;
  m->qkv_rows = m->qd + 2 * m->kvd;
  const int64_t H = c.hidden_size, I = c.intermediate_size, V = c.vocab_size;
  // placement: every tensor 256-byte aligned inside one allocation
  struct Item {
    std::string name;
    int64_t numel;
    f16** dst;
    int64_t row_offset;  // for q/k/v inside the fused qkv matrix
  };
  std::vector<std::pair<std::string, int64_t>> order;
  size_t off = 0;
  std::map<std::string, size_t> offsets;
  auto place = [&](const std::string& name, int64_t numel) {
    offsets[name] = off;
    off += (static_cast<size_t>(numel) * 2 + 255) / 256 * 256;
  };
  place("model.embed_tokens.weight", V * H);
  place("model.norm.weight", H);
  if (!c.tie_word_embeddings) place("lm_head.weight", V * H);
  for (int l = 0; l < c.num_hidden_layers; ++l) {
    const std::string p = "model.layers." + std::to_string(l) + ".";
    place(p + "input_layernorm.weight", H);
    place(p + "post_attention_layernorm.weight", H);
    place(p + "self_attn.q_norm.weight", c.head_dim);
    place(p + "self_attn.k_norm.weight", c.head_dim);
    place(p + "@qkv", static_cast<int64_t>(m->qkv_rows) * H);
    place(p + "self_attn.o_proj.weight", H * m->qd);
    place(p + "mlp.gate_proj.weight", I * H);
    place(p + "mlp.up_proj.weight", I * H);
    place(p + "mlp.down_proj.weight", H * I);
  }
  m->wbytes = off;
  hipError_t e = hipMalloc(&m->wbuf, m->wbytes);
  if (e != hipSuccess) {
    (void)hipGetLastError();
    return soc::fail(SOC_ERR_NOMEM, "weight allocation of " + std::to_string(m->wbytes) + " bytes failed");
  }
  auto at = [&](const std::string& name) { return reinterpret_cast<f16*>(m->wbuf + offsets.at(name)); };
  m->embed = at("model.embed_tokens.weight");
  m->final_norm = at("model.norm.weight");
  m->lm_head = c.tie_word_embeddings ? m->embed : at("lm_head.weight");
  m->tensors["model.embed_tokens.weight"] = {m->embed, V * H, false};
  m->tensors["model.norm.weight"] = {m->final_norm, H, false};
  if (!c.tie_word_embeddings) m->tensors["lm_head.weight"] = {m->lm_head, V * H, false};
  m->layers.resize(c.num_hidden_layers);
  for (int l = 0; l < c.num_hidden_layers; ++l) {
    const std::string p = "model.layers." + std::to_string(l) + ".";
    DevLayer& L = m->layers[l];
    L.in_norm = at(p + "input_layernorm.weight");
    L.post_norm = at(p + "post_attention_layernorm.weight");
    L.q_norm = at(p + "self_attn.q_norm.weight");
    L.k_norm = at(p + "self_attn.k_norm.weight");
    L.wqkv = at(p + "@qkv");
    L.wo = at(p + "self_attn.o_proj.weight");
    L.wgate = at(p + "mlp.gate_proj.weight");
    L.wup = at(p + "mlp.up_proj.weight");
    L.wdown = at(p + "mlp.down_proj.weight");
    m->tensors[p + "input_layernorm.weight"] = {L.in_norm, H, false};
    m->tensors[p + "post_attention_layernorm.weight"] = {L.post_norm, H, false};
    m->tensors[p + "self_attn.q_norm.weight"] = {L.q_norm, c.head_dim, false};
    m->tensors[p + "self_attn.k_norm.weight"] = {L.k_norm, c.head_dim, false};
    m->tensors[p + "self_attn.q_proj.weight"] = {L.wqkv, static_cast<int64_t>(m->qd) * H, false};
    m->tensors[p + "self_attn.k_proj.weight"] = {L.wqkv + static_cast<size_t>(m->qd) * H,
                                                  static_cast<int64_t>(m->kvd) * H, false};
    m->tensors[p + "self_attn.v_proj.weight"] = {L.wqkv + static_cast<size_t>(m->qd + m->kvd) * H,
                                                  static_cast<int64_t>(m->kvd) * H, false};
    m->tensors[p + "self_attn.o_proj.weight"] = {L.wo, H * m->qd, false};
    m->tensors[p + "mlp.gate_proj.weight"] = {L.wgate, I * H, false};
    m->tensors[p + "mlp.up_proj.weight"] = {L.wup, I * H, false};
    m->tensors[p + "mlp.down_proj.weight"] = {L.wdown, H * I, false};
  }
  SOC_TRY(build_rope_table(m.get(), c.max_position_embeddings));
  {
    std::vector<const f16*> ptrs;
    for (const DevLayer& L : m->layers)
      for (const f16* p : {L.in_norm, L.post_norm, L.q_norm, L.k_norm, L.wqkv, L.wo, L.wgate, L.wup, L.wdown})
        ptrs.push_back(p);
    if ((e = hipMalloc(&m->d_layer_w, ptrs.size() * sizeof(f16*))) != hipSuccess) return hip_fail(e, "hipMalloc");
    if ((e = hipMemcpy(m->d_layer_w, ptrs.data(), ptrs.size() * sizeof(f16*), hipMemcpyHostToDevice)) != hipSuccess)
      return hip_fail(e, "hipMemcpy");
  }
  *out = m.release();
  return SOC_OK;
  SOC_API_END
}

int soc_model_destroy(soc_model* m) {
  if (m == nullptr) return SOC_OK;
  (void)hipStreamSynchronize(m->ctx->stream);
  free_all(m->dws.allocs);
  free_all(m->pws.allocs);
  free_all(m->bws.allocs);
  (void)hipFree(m->bws.ring);
  (void)hipFree(m->wbuf);
  (void)hipFree(m->rope_cos);
  (void)hipFree(m->rope_sin);
  (void)hipFree(m->d_layer_w);
  free_all(m->qallocs);
  (void)hipFree(m->qdeq);
  if (m->ukv != nullptr) soc_kv_destroy(m->ukv);
  delete m;
  return SOC_OK;
}

int soc_model_load_tensor(soc_model* m, const char* name, const uint16_t* host, int64_t numel) {
  SOC_API_BEGIN
  if (m == nullptr || name == nullptr || host == nullptr) return soc::fail(SOC_ERR_INVALID, "null argument");
  auto it = m->tensors.find(name);
  if (it == m->tensors.end()) return soc::fail(SOC_ERR_INVALID, std::string("unknown tensor name: ") + name);
  if (it->second.numel != numel)
    return soc::fail(SOC_ERR_INVALID, std::string("tensor ") + name + " has " + std::to_string(numel) +
                                          " elements, expected " + std::to_string(it->second.numel));
  hipError_t e = hipMemcpy(it->second.ptr, host, static_cast<size_t>(numel) * 2, hipMemcpyHostToDevice);
  if (e != hipSuccess) return hip_fail(e, "hipMemcpy weight");
  it->second.loaded = true;
  m->finalized = false;
  return SOC_OK;
  SOC_API_END
}

int soc_model_tensor(const soc_model* m, const char* name, void** device_ptr, int64_t* numel) {
  SOC_API_BEGIN
  if (m == nullptr || name == nullptr) return soc::fail(SOC_ERR_INVALID, "null argument");
  auto it = m->tensors.find(name);
  if (it == m->tensors.end()) return soc::fail(SOC_ERR_INVALID, std::string("unknown tensor name: ") + name);
  if (device_ptr != nullptr) *device_ptr = it->second.ptr;
  if (numel != nullptr) *numel = it->second.numel;
  return SOC_OK;
  SOC_API_END
}

int soc_model_synthesize(soc_model* m, uint64_t seed, float sigma) {
  SOC_API_BEGIN
  if (m == nullptr) return soc::fail(SOC_ERR_INVALID, "null model");
  std::vector<uint16_t> buf;
  for (auto& kv : m->tensors) {
    const std::string& name = kv.first;
    buf.resize(static_cast<size_t>(kv.second.numel));
    const bool gain = name.find("norm.weight") != std::string::npos;
    if (gain) {
      std::fill(buf.begin(), buf.end(), static_cast<uint16_t>(0x3c00));  // 1.0
    } else {
      SOC_TRY(soc_synth_normal_f16(seed, name.c_str(), sigma, 0, kv.second.numel, buf.data()));
    }
    hipError_t e = hipMemcpy(kv.second.ptr, buf.data(), buf.size() * 2, hipMemcpyHostToDevice);
    if (e != hipSuccess) return hip_fail(e, "hipMemcpy weight");
    kv.second.loaded = true;
  }
  m->finalized = false;
  return SOC_OK;
  SOC_API_END
}

int soc_model_finalize(soc_model* m) {
  if (m == nullptr) return soc::fail(SOC_ERR_INVALID, "null model");
  for (auto& kv : m->tensors)
    if (!kv.second.loaded) return soc::fail(SOC_ERR_INVALID, "missing tensor: " + kv.first);
  m->finalized = true;
  return SOC_OK;
}

int soc_model_quantize(soc_model* m, int32_t bits) {
  SOC_API_BEGIN
  if (m == nullptr) return soc::fail(SOC_ERR_INVALID, "null model");
  if (!m->finalized) return soc::fail(SOC_ERR_STATE, "model is not finalized");
  if (m->qbits != 0) return soc::fail(SOC_ERR_STATE, "model is already quantized");
  if (bits != 8 && bits != 4) return soc::fail(SOC_ERR_INVALID, "soc_model_quantize: bits must be 8 or 4");
  const soc_qwen_config& c = m->cfg;
  const int H = c.hidden_size, I = c.intermediate_size, qd = m->qd;
  for (int k : {H, qd, I})
    if (k % 64 != 0 || static_cast<size_t>(kQChunk) * k * 2 > 160 * 1024)
      return soc::fail(SOC_ERR_INVALID, "soc_model_quantize: hidden, q and intermediate sizes must be multiples of 64 "
                                        "and at most 10240");
  hipError_t e = hipStreamSynchronize(m->ctx->stream);
  if (e != hipSuccess) return hip_fail(e, "hipStreamSynchronize");
  std::vector<QLayer> ql(c.num_hidden_layers);
  std::vector<void*> allocs;
  auto fail_free = [&](int rc) {
    free_all(allocs);
    return rc;
  };
  std::vector<uint16_t> wbuf;
  std::vector<uint8_t> cbuf;
  std::vector<uint16_t> sbuf;
  // reads rows [N][K] of fp16 weights from one or two device tensors, quantizes them, uploads codes and scales
  auto pack = [&](std::initializer_list<std::pair<const f16*, int>> parts, int K, uint8_t** codes, f16** scales) {
    int N = 0;
    for (const auto& p : parts) N += p.second;
    wbuf.resize(static_cast<size_t>(N) * K);
    size_t off = 0;
    for (const auto& p : parts) {
      const hipError_t ee = hipMemcpy(wbuf.data() + off, p.first, static_cast<size_t>(p.second) * K * 2,
                                      hipMemcpyDeviceToHost);
      if (ee != hipSuccess) return hip_fail(ee, "hipMemcpy weights");
      off += static_cast<size_t>(p.second) * K;
    }
    const size_t ncode = static_cast<size_t>(N) * K / (bits == 8 ? 1 : 2), nscale = static_cast<size_t>(N) * K / 64;
    cbuf.resize(ncode);
    sbuf.resize(nscale);
    SOC_TRY(soc_quantize_group(wbuf.data(), N, K, bits, cbuf.data(), sbuf.data()));
    SOC_TRY(dev_alloc_t(allocs, ncode, codes));
    SOC_TRY(dev_alloc_t(allocs, nscale, scales));
    hipError_t ee = hipMemcpy(*codes, cbuf.data(), ncode, hipMemcpyHostToDevice);
    if (ee == hipSuccess) ee = hipMemcpy(*scales, sbuf.data(), nscale * 2, hipMemcpyHostToDevice);
    return ee == hipSuccess ? SOC_OK : hip_fail(ee, "hipMemcpy codes");
  };
  for (int l = 0; l < c.num_hidden_layers; ++l) {
    const DevLayer& L = m->layers[l];
    QLayer& q = ql[l];
    int rc;
    if ((rc = pack({{L.wqkv, m->qkv_rows}}, H, &q.qkv, &q.qkv_s)) != SOC_OK) return fail_free(rc);
    if ((rc = pack({{L.wo, H}}, qd, &q.o, &q.o_s)) != SOC_OK) return fail_free(rc);
    if ((rc = pack({{L.wgate, I}, {L.wup, I}}, H, &q.gu, &q.gu_s)) != SOC_OK) return fail_free(rc);
    if ((rc = pack({{L.wdown, H}}, I, &q.down, &q.down_s)) != SOC_OK) return fail_free(rc);
  }
  m->qlayers = std::move(ql);
  m->qallocs = std::move(allocs);
  m->qbits = bits;
  ++m->dws_gen;  // captured decode graphs hold the fp16 path: capture again
  return SOC_OK;
  SOC_API_END
}

int soc_model_weight_bytes(const soc_model* m, int64_t* bytes) {
  if (m == nullptr || bytes == nullptr) return soc::fail(SOC_ERR_INVALID, "null argument");
  int64_t total = 0;
  for (const auto& kv : m->tensors) total += kv.second.numel * 2;
  *bytes = total;
  return SOC_OK;
}

int soc_model_decode_path(soc_model* m, int32_t* path) {
  SOC_API_BEGIN
  if (m == nullptr || path == nullptr) return soc::fail(SOC_ERR_INVALID, "null argument");
  if (!m->finalized) return soc::fail(SOC_ERR_STATE, "model is not finalized");
  *path = use_xcd(m) ? 2 : (use_persistent(m) ? 1 : 0);
  return SOC_OK;
  SOC_API_END
}

namespace {
int kv_create(soc_ctx* ctx, soc_model* m, int layers, int nkv, int hd, int32_t slots, int32_t cap, soc_kv** out) {
  *out = nullptr;
  if (slots <= 0 || cap <= 0) return soc::fail(SOC_ERR_INVALID, "soc_kv_create: slots and capacity must be positive");
  std::unique_ptr<soc_kv> kv(new soc_kv());
  kv->ctx = ctx;
  kv->model = m;
  kv->layers = layers;
  kv->nkv = nkv;
  kv->hd = hd;
  kv->slots = slots;
  kv->cap = cap;
  kv->layer_stride = static_cast<long long>(nkv) * cap * hd;
  kv->slot_stride = kv->layer_stride * layers;
  const size_t bytes = static_cast<size_t>(kv->slot_stride) * slots * 2;
  hipError_t e = hipMalloc(&kv->k, bytes);
  if (e == hipSuccess) e = hipMalloc(&kv->v, bytes);
  if (e != hipSuccess) {
    (void)hipGetLastError();
    (void)hipFree(kv->k);
    return soc::fail(SOC_ERR_NOMEM, "KV cache allocation of " + std::to_string(2 * bytes) + " bytes failed");
  }
  kv->len.assign(slots, 0);
  *out = kv.release();
  return SOC_OK;
}
}  // namespace

int soc_kv_create(soc_model* m, int32_t slots, int32_t cap, soc_kv** out) {
  SOC_API_BEGIN
  if (m == nullptr || out == nullptr) return soc::fail(SOC_ERR_INVALID, "null argument");
  *out = nullptr;
  if (cap > m->rope_len)
    return soc::fail(SOC_ERR_CAPACITY, "soc_kv_create: capacity exceeds max_position_embeddings");
  const soc_qwen_config& c = m->cfg;
  return kv_create(m->ctx, m, c.num_hidden_layers, c.num_key_value_heads, c.head_dim, slots, cap, out);
  SOC_API_END
}

int soc_kv_create_dims(soc_ctx* ctx, int32_t layers, int32_t kv_heads, int32_t head_dim, int32_t slots, int32_t cap,
                       soc_kv** out) {
  SOC_API_BEGIN
  if (ctx == nullptr || out == nullptr) return soc::fail(SOC_ERR_INVALID, "null argument");
  *out = nullptr;
  if (layers <= 0 || kv_heads <= 0 || head_dim <= 0)
    return soc::fail(SOC_ERR_INVALID, "KVCache dimensions must be non-zero");  // kv_cache.mm:40-45
  if (head_dim != 128) return soc::fail(SOC_ERR_INVALID, "soc_kv_create_dims: head_dim must be 128");
  return kv_create(ctx, nullptr, layers, kv_heads, head_dim, slots, cap, out);
  SOC_API_END
}

int soc_kv_destroy(soc_kv* kv) {
  if (kv == nullptr) return SOC_OK;
  (void)hipStreamSynchronize(kv->ctx->stream);
  for (auto& g : kv->graphs) (void)hipGraphExecDestroy(g.second.second);
  for (auto& g : kv->batch_graphs) (void)hipGraphExecDestroy(g.second.second);
  (void)hipFree(kv->k);
  (void)hipFree(kv->v);
  delete kv;
  return SOC_OK;
}

int soc_kv_length(const soc_kv* kv, int32_t slot, int32_t* length) {
  if (kv == nullptr || length == nullptr) return soc::fail(SOC_ERR_INVALID, "null argument");
  if (slot < 0 || slot >= kv->slots) return soc::fail(SOC_ERR_INVALID, "slot out of range");
  *length = kv->len[slot];
  return SOC_OK;
}

int soc_kv_reset(soc_kv* kv, int32_t slot) {
  if (kv == nullptr) return soc::fail(SOC_ERR_INVALID, "null kv");
  if (slot < 0 || slot >= kv->slots) return soc::fail(SOC_ERR_INVALID, "slot out of range");
  kv->len[slot] = 0;
  return SOC_OK;
}

int soc_kv_write(soc_kv* kv, int32_t slot, int32_t layer, int32_t pos, const float* key, const float* value) {
  SOC_API_BEGIN
  if (kv == nullptr || key == nullptr || value == nullptr) return soc::fail(SOC_ERR_INVALID, "null argument");
  if (slot < 0 || slot >= kv->slots || layer < 0 || layer >= kv->layers || pos < 0 || pos >= kv->cap)
    return soc::fail(SOC_ERR_INVALID, "soc_kv_write: index out of range");  // kv_cache.cpp:51-53
  const int d = kv->hd;
  std::vector<_Float16> kh(d), vh(d);
  for (int h = 0; h < kv->nkv; ++h) {
    for (int i = 0; i < d; ++i) {
      kh[i] = static_cast<_Float16>(key[h * d + i]);
      vh[i] = static_cast<_Float16>(value[h * d + i]);
    }
    const size_t off = static_cast<size_t>(slot) * kv->slot_stride + static_cast<size_t>(layer) * kv->layer_stride +
                       (static_cast<size_t>(h) * kv->cap + pos) * d;
    hipError_t e = hipMemcpy(kv->k + off, kh.data(), d * 2, hipMemcpyHostToDevice);
    if (e == hipSuccess) e = hipMemcpy(kv->v + off, vh.data(), d * 2, hipMemcpyHostToDevice);
    if (e != hipSuccess) return hip_fail(e, "hipMemcpy kv");
  }
  if (pos + 1 > kv->len[slot]) kv->len[slot] = pos + 1;
  return SOC_OK;
  SOC_API_END
}

int soc_kv_fill_synthetic(soc_kv* kv, int32_t slot, int32_t length, uint64_t seed) {
  SOC_API_BEGIN
  if (kv == nullptr) return soc::fail(SOC_ERR_INVALID, "null kv");
  if (slot < 0 || slot >= kv->slots || length < 0 || length > kv->cap)
    return soc::fail(SOC_ERR_INVALID, "soc_kv_fill_synthetic: bad slot or length");
  const int d = kv->hd, L = kv->layers, nkv = kv->nkv;
  const size_t per_head = static_cast<size_t>(length) * d;
  // host image [layer][k|v][head][length][d], generated per (layer, k|v, head) stream on up to 16 threads
  std::vector<uint16_t> buf(static_cast<size_t>(L) * 2 * nkv * per_head);
  const int jobs = L * 2 * nkv;
  std::vector<int> rcs(jobs, SOC_OK);
  auto work = [&](int t, int nt) {
    for (int j = t; j < jobs; j += nt) {
      const int l = j / (2 * nkv), which = (j / nkv) % 2, h = j % nkv;
      const std::string name = "kv." + std::to_string(slot) + "." + std::to_string(l) + "." + std::to_string(h) +
                               (which ? ".v" : ".k");
      rcs[j] = soc_synth_normal_f16(seed, name.c_str(), 1.0f, 0, static_cast<int64_t>(per_head),
                                    buf.data() + static_cast<size_t>(j) * per_head);
    }
  };
  const unsigned hw = std::thread::hardware_concurrency();
  const int nt = std::max(1, std::min<int>(16, hw == 0 ? 1 : static_cast<int>(hw)));
  std::vector<std::thread> th;
  for (int t = 0; t < nt; ++t) th.emplace_back(work, t, nt);
  for (auto& t : th) t.join();
  for (int rc : rcs)
    if (rc != SOC_OK) return rc;
  if (length > 0) {
    for (int l = 0; l < L; ++l)
      for (int which = 0; which < 2; ++which) {
        const size_t off = static_cast<size_t>(slot) * kv->slot_stride + static_cast<size_t>(l) * kv->layer_stride;
        const uint16_t* src = buf.data() + static_cast<size_t>((l * 2 + which) * nkv) * per_head;
        hipError_t e = hipMemcpy2D((which ? kv->v : kv->k) + off, static_cast<size_t>(kv->cap) * d * 2, src,
                                   per_head * 2, per_head * 2, nkv, hipMemcpyHostToDevice);
        if (e != hipSuccess) return hip_fail(e, "hipMemcpy2D kv");
      }
  }
  kv->len[slot] = length;
  return SOC_OK;
  SOC_API_END
}

int soc_kv_read(const soc_kv* kv, int32_t slot, int32_t layer, uint16_t* keys, uint16_t* values) {
  SOC_API_BEGIN
  if (kv == nullptr) return soc::fail(SOC_ERR_INVALID, "null kv");
  if (slot < 0 || slot >= kv->slots || layer < 0 || layer >= kv->layers)
    return soc::fail(SOC_ERR_INVALID, "soc_kv_read: index out of range");
  hipError_t e = hipStreamSynchronize(kv->ctx->stream);
  if (e != hipSuccess) return hip_fail(e, "hipStreamSynchronize");
  const int d = kv->hd, n = kv->len[slot];
  for (int h = 0; h < kv->nkv; ++h) {
    const size_t off = static_cast<size_t>(slot) * kv->slot_stride + static_cast<size_t>(layer) * kv->layer_stride +
                       static_cast<size_t>(h) * kv->cap * d;
    if (keys && (e = hipMemcpy(keys + static_cast<size_t>(h) * n * d, kv->k + off, static_cast<size_t>(n) * d * 2,
                               hipMemcpyDeviceToHost)) != hipSuccess)
      return hip_fail(e, "hipMemcpy kv");
    if (values && (e = hipMemcpy(values + static_cast<size_t>(h) * n * d, kv->v + off,
                                 static_cast<size_t>(n) * d * 2, hipMemcpyDeviceToHost)) != hipSuccess)
      return hip_fail(e, "hipMemcpy kv");
  }
  return SOC_OK;
  SOC_API_END
}

int soc_kv_append(soc_kv* kv, int32_t slot, int32_t layer, int32_t pos, int32_t rows, const void* keys,
                  const void* values, int32_t dtype) {
  SOC_API_BEGIN
  if (kv == nullptr || (rows > 0 && (keys == nullptr || values == nullptr)))
    return soc::fail(SOC_ERR_INVALID, "null argument");
  if (slot < 0 || slot >= kv->slots) return soc::fail(SOC_ERR_INVALID, "slot out of range");
  if (layer < 0 || layer >= kv->layers) return soc::fail(SOC_ERR_INVALID, "KVCache layer index is out of range");
  if (dtype != SOC_DTYPE_F32 && dtype != SOC_DTYPE_F16) return soc::fail(SOC_ERR_INVALID, "dtype must be f32 or f16");
  if (rows < 0 || pos < 0) return soc::fail(SOC_ERR_INVALID, "rows and pos must be >= 0");
  if (pos + rows > kv->cap) return soc::fail(SOC_ERR_CAPACITY, "KVCache append would exceed max_sequence_length");
  if (rows == 0) return SOC_OK;
  const size_t off = static_cast<size_t>(slot) * kv->slot_stride + static_cast<size_t>(layer) * kv->layer_stride;
  hipStream_t s = kv->ctx->stream;
  hipError_t e = soc::launch_kv_append_rows(keys, values, dtype == SOC_DTYPE_F16, rows, kv->nkv, kv->hd, kv->cap, pos,
                                            kv->k + off, kv->v + off, s);
  if (e == hipSuccess) e = hipStreamSynchronize(s);  // the source rows may be released when this returns
  return e == hipSuccess ? SOC_OK : hip_fail(e, "kv append");
  SOC_API_END
}

int soc_kv_set_length(soc_kv* kv, int32_t slot, int32_t length) {
  if (kv == nullptr) return soc::fail(SOC_ERR_INVALID, "null kv");
  if (slot < 0 || slot >= kv->slots) return soc::fail(SOC_ERR_INVALID, "slot out of range");
  if (length < 0 || length > kv->cap) return soc::fail(SOC_ERR_CAPACITY, "length exceeds the KV capacity");
  kv->len[slot] = length;
  return SOC_OK;
}

int soc_kv_layer_planes(const soc_kv* kv, int32_t slot, int32_t layer, void** keys, void** values) {
  if (kv == nullptr) return soc::fail(SOC_ERR_INVALID, "null kv");
  if (slot < 0 || slot >= kv->slots || layer < 0 || layer >= kv->layers)
    return soc::fail(SOC_ERR_INVALID, "soc_kv_layer_planes: index out of range");
  const size_t off = static_cast<size_t>(slot) * kv->slot_stride + static_cast<size_t>(layer) * kv->layer_stride;
  if (keys) *keys = kv->k + off;
  if (values) *values = kv->v + off;
  return SOC_OK;
}

namespace {
// The layers of a quantized model's prefill over the n embedded rows in m->pws.x, kQChunk rows at a time (each chunk
// through every layer, so a chunk's attention sees the keys the earlier chunks appended): group-quantized
// projections, the prefill q/k-norm + RoPE + append kernel and the split-key attention over the slot's cache.
// Layer l of a quantized model with its projections dequantized to fp16 (rounded to nearest) in m->qdeq, for the
// prefill GEMMs of more than kQChunk rows: the norms are the model's own, the weight pointers the scratch's. The
// scratch holds one layer; stream order keeps a layer's GEMMs ahead of the next layer's dequantization.
int dequant_layer(soc_model* m, int l, DevLayer* out) {
  const soc_qwen_config& c = m->cfg;
  const size_t H = c.hidden_size, I = c.intermediate_size, qd = m->qd, qkv = m->qkv_rows;
  const size_t n_qkv = qkv * H, n_o = H * qd, n_gu = 2 * I * H, n_down = H * I;
  hipError_t e;
  if (m->qdeq == nullptr &&
      (e = hipMalloc(&m->qdeq, (n_qkv + n_o + n_gu + n_down) * sizeof(f16))) != hipSuccess)
    return hip_fail(e, "hipMalloc dequantized layer");
  const QLayer& q = m->qlayers[l];
  f16* const wqkv = m->qdeq;
  f16* const wo = wqkv + n_qkv;
  f16* const wgu = wo + n_o;
  f16* const wdown = wgu + n_gu;
  hipStream_t s = m->ctx->stream;
  const int b = m->qbits;
  if ((e = soc::launch_dequant_f16(q.qkv, b, q.qkv_s, static_cast<int>(qkv), static_cast<int>(H), wqkv, s)) !=
          hipSuccess ||
      (e = soc::launch_dequant_f16(q.o, b, q.o_s, static_cast<int>(H), static_cast<int>(qd), wo, s)) != hipSuccess ||
      (e = soc::launch_dequant_f16(q.gu, b, q.gu_s, static_cast<int>(2 * I), static_cast<int>(H), wgu, s)) !=
          hipSuccess ||
      (e = soc::launch_dequant_f16(q.down, b, q.down_s, static_cast<int>(H), static_cast<int>(I), wdown, s)) !=
          hipSuccess)
    return hip_fail(e, "dequantize layer");
  *out = m->layers[l];
  out->wqkv = wqkv;
  out->wo = wo;
  out->wgate = wgu;
  out->wup = wgu + I * H;
  out->wdown = wdown;
  return SOC_OK;
}

int prefill_layers_q(soc_model* m, soc_kv* kv, int slot, int n, int pos_off, const float* rope_cos,
                     const float* rope_sin) {
  const soc_qwen_config& c = m->cfg;
  PrefillWs& w = m->pws;
  hipStream_t s = m->ctx->stream;
  const int H = c.hidden_size;
  for (int c0 = 0; c0 < n; c0 += kQChunk) {
    const int T = std::min(kQChunk, n - c0);
    const int M = T <= 1 ? 1 : T <= 2 ? 2 : T <= 4 ? 4 : 8;  // the projection's row count (rows past T unused)
    float* xr = w.x + static_cast<size_t>(c0) * H;
    float* qrow = w.q + static_cast<size_t>(c0) * m->qd;
    float* arow = w.attn + static_cast<size_t>(c0) * m->qd;
    for (int l = 0; l < c.num_hidden_layers; ++l) {
      auto attend = [&]() -> int {
        const DevLayer& L = m->layers[l];
        soc::QkNormRopeArgs q{};
        q.qkv = w.qy;
        q.ld_qkv = m->qkv_rows;
        q.q_gain = L.q_norm;
        q.k_gain = L.k_norm;
        q.eps = c.rms_norm_eps;
        q.rope_cos = rope_cos;
        q.rope_sin = rope_sin;
        q.q_out = qrow;
        q.kcache = kv->k;
        q.vcache = kv->v;
        q.slot_stride = kv->slot_stride;
        q.layer_stride = kv->layer_stride;
        q.slot = slot;
        q.layer = l;
        q.cap = kv->cap;
        q.pos_base = pos_off + c0;
        q.T = T;
        q.nq = c.num_attention_heads;
        q.nkv = c.num_key_value_heads;
        hipError_t e = soc::launch_qk_norm_rope_append(q, s);
        if (e != hipSuccess) return hip_fail(e, "qk norm rope");
        soc::AttnArgs a = attn_args(m, kv, l);
        a.qkv = qrow;
        a.ld_qkv = m->qd;
        a.slot_base = slot;
        a.pos_base = pos_off + c0;
        a.out = arow;
        a.ld_out = m->qd;
        a.part = w.part;
        a.counters = w.attn_counters;
        a.B = T;
        a.max_split = (pos_off + n + kAttnChunk - 1) / kAttnChunk;
        e = soc::launch_attention(a, 0, s);
        return e == hipSuccess ? SOC_OK : hip_fail(e, "attention");
      };
      SOC_TRY(enqueue_layer_q(m, l, xr, T, M, w.qx, w.qy, w.qy, arow, attend, s));
    }
  }
  return SOC_OK;
}

// The forward of n tokens of one slot at positions [pos_off, pos_off + n) (QwenCausalLM::ForwardHiddenCached /
// ForwardLogitsCached, qwen_causal_lm.cpp:130-268): appends their K/V, writes the final-RMSNorm rows (hidden, [n][H],
// nullable), the logits of the last logit_rows rows and the greedy token of the last row. ids are host ids already
// validated, or, with ids_dev, device ids that are staged on the device (an id outside the vocabulary fails the call
// after the work ran). RoPE uses table rows rope_shift + position: rope_shift = 0 for a cached forward, and the
// reference's position_offset for an uncached one (run on a private cache from position 0). Nothing past the
// caller's inputs is changed on failure; on success the caller updates the slot length.
int run_prefill(soc_model* m, soc_kv* kv, int32_t slot, const int32_t* ids, bool ids_dev, int32_t n, int32_t pos_off,
                int32_t rope_shift, float* hidden, int32_t logit_rows, float* logits, int32_t* next_token) {
  SOC_TRY(ensure_prefill_ws(m, n, pos_off + n, logit_rows));
  const soc_qwen_config& c = m->cfg;
  PrefillWs& w = m->pws;
  hipStream_t s = m->ctx->stream;
  hipError_t e;
  if (ids_dev) {
    if ((e = soc::launch_stage_ids(ids, n, c.vocab_size, w.ids, m->ctx->id_err, s)) != hipSuccess)
      return hip_fail(e, "token id staging");
  } else if ((e = hipMemcpyAsync(w.ids, ids, static_cast<size_t>(n) * 4, hipMemcpyHostToDevice, s)) != hipSuccess) {
    return hip_fail(e, "hipMemcpyAsync ids");
  }
  if ((e = soc::launch_embed(w.ids, n, m->embed, c.hidden_size, w.x, s)) != hipSuccess) return hip_fail(e, "embed");
  const float* const rope_cos = m->rope_cos + static_cast<size_t>(rope_shift) * (c.head_dim / 2);
  const float* const rope_sin = m->rope_sin + static_cast<size_t>(rope_shift) * (c.head_dim / 2);
  const int H = c.hidden_size;
  // a quantized model's prompt of up to kQChunk rows streams the codes once through the group-quantized kernels;
  // longer prompts run the fp16 layers on each layer's projections dequantized to fp16
  const bool qchunks = m->qbits != 0 && n <= kQChunk;
  if (qchunks) SOC_TRY(prefill_layers_q(m, kv, slot, n, pos_off, rope_cos, rope_sin));
  const bool split = prefill_split_path(m);
  // lo parts of each projection's activations, or none (prefill_split_mask)
  const int smask = prefill_split_mask();
  f16* const pl_qkv = (smask & kSplitQkv) ? w.pl : nullptr;
  f16* const pl_o = (smask & kSplitO) ? w.pl : nullptr;
  f16* const pl_gu = (smask & kSplitGateUp) ? w.pl : nullptr;
  f16* const ql = (smask & kSplitDown) ? w.ql : nullptr;
  for (int l = 0; !qchunks && l < c.num_hidden_layers; ++l) {
    DevLayer deq;
    if (m->qbits != 0) SOC_TRY(dequant_layer(m, l, &deq));
    const DevLayer& L = m->qbits != 0 ? deq : m->layers[l];
    soc::GemmArgs g{};
    const bool qkv_fused = split;  // the staged kernel's QKV is followed by the separate q/k-norm kernel
    if (split) {
      if ((e = soc::launch_rmsnorm_rows(w.x, n, H, L.in_norm, c.rms_norm_eps, nullptr, w.ph, pl_qkv, s)) !=
          hipSuccess)
        return hip_fail(e, "rmsnorm");
      // QKV projection with the per-head q/k RMSNorm + RoPE, q output and K/V cache append in its epilogue
      soc::GemmSplitArgs g3{};
      g3.ah = w.ph;
      g3.al = pl_qkv;
      g3.lda = H;
      g3.w = L.wqkv;
      g3.c = w.qkv;
      g3.ldc = m->qkv_rows;
      g3.M = n;
      g3.N = m->qkv_rows;
      g3.K = H;
      {
        g3.qkv.q_out = w.q;
        g3.qkv.kcache = kv->k;
        g3.qkv.vcache = kv->v;
        g3.qkv.q_gain = L.q_norm;
        g3.qkv.k_gain = L.k_norm;
        g3.qkv.rope_cos = rope_cos;
        g3.qkv.rope_sin = rope_sin;
        g3.qkv.slot_stride = kv->slot_stride;
        g3.qkv.layer_stride = kv->layer_stride;
        g3.qkv.slot = slot;
        g3.qkv.layer = l;
        g3.qkv.cap = kv->cap;
        g3.qkv.pos_base = pos_off;
        g3.qkv.nq = c.num_attention_heads;
        g3.qkv.nkv = c.num_key_value_heads;
        g3.qkv.eps = c.rms_norm_eps;
      }
      if ((e = soc::launch_gemm_split(g3, soc::EPI_QKV, s)) != hipSuccess) return hip_fail(e, "gemm qkv");
    } else {
      if ((e = soc::launch_rmsnorm_rows(w.x, n, H, L.in_norm, c.rms_norm_eps, w.xn, nullptr, nullptr, s)) != hipSuccess)
        return hip_fail(e, "rmsnorm");
      g.a = w.xn;
      g.lda = H;
      g.w = L.wqkv;
      g.c = w.qkv;
      g.ldc = m->qkv_rows;
      g.M = n;
      g.N = m->qkv_rows;
      g.K = H;
      if ((e = prefill_gemm(g, soc::EPI_STORE, s, kSplitQkv)) != hipSuccess) return hip_fail(e, "gemm qkv");
    }
    soc::QkNormRopeArgs q{};
    q.qkv = w.qkv;
    q.ld_qkv = m->qkv_rows;
    q.q_gain = L.q_norm;
    q.k_gain = L.k_norm;
    q.eps = c.rms_norm_eps;
    q.rope_cos = rope_cos;
    q.rope_sin = rope_sin;
    q.q_out = w.q;
    q.kcache = kv->k;
    q.vcache = kv->v;
    q.slot_stride = kv->slot_stride;
    q.layer_stride = kv->layer_stride;
    q.slot = slot;
    q.layer = l;
    q.cap = kv->cap;
    q.pos_base = pos_off;
    q.T = n;
    q.nq = c.num_attention_heads;
    q.nkv = c.num_key_value_heads;
    if (!qkv_fused && (e = soc::launch_qk_norm_rope_append(q, s)) != hipSuccess) return hip_fail(e, "qk norm rope");
    soc::AttnArgs a = attn_args(m, kv, l);
    a.qkv = w.q;
    a.ld_qkv = m->qd;
    a.pos = nullptr;
    a.slot = nullptr;
    a.slot_base = slot;
    a.pos_base = pos_off;
    a.out = split ? nullptr : w.attn;
    a.out_hi = split ? w.ph : nullptr;
    a.out_lo = split ? pl_o : nullptr;
    a.ld_out = m->qd;
    a.part = w.part;
    a.counters = w.attn_counters;
    a.B = n;
    a.max_split = (pos_off + n + kAttnChunk - 1) / kAttnChunk;
    if ((e = prefill_attention(a, w.attn, s)) != hipSuccess) return hip_fail(e, "attention prefill");
    const int I = c.intermediate_size;
    if (split) {
      if ((e = split_gemm(w.ph, pl_o, m->qd, L.wo, nullptr, w.x, nullptr, nullptr, H, n, H, m->qd,
                          soc::EPI_RESIDUAL, s)) != hipSuccess)
        return hip_fail(e, "gemm o");
      if ((e = soc::launch_rmsnorm_rows(w.x, n, H, L.post_norm, c.rms_norm_eps, nullptr, w.ph, pl_gu, s)) !=
          hipSuccess)
        return hip_fail(e, "rmsnorm");
      if ((e = split_gemm(w.ph, pl_gu, H, L.wgate, L.wup, nullptr, w.qh, ql, I, n, I, H, soc::EPI_SWIGLU, s)) !=
          hipSuccess)
        return hip_fail(e, "gemm gate/up");
      if ((e = split_gemm(w.qh, ql, I, L.wdown, nullptr, w.x, nullptr, nullptr, H, n, H, I, soc::EPI_RESIDUAL, s)) !=
          hipSuccess)
        return hip_fail(e, "gemm down");
      continue;
    }
    g = soc::GemmArgs{};
    g.a = w.attn;
    g.lda = m->qd;
    g.w = L.wo;
    g.c = w.x;
    g.ldc = H;
    g.M = n;
    g.N = H;
    g.K = m->qd;
    if ((e = prefill_gemm(g, soc::EPI_RESIDUAL, s, kSplitO)) != hipSuccess) return hip_fail(e, "gemm o");
    if ((e = soc::launch_rmsnorm_rows(w.x, n, H, L.post_norm, c.rms_norm_eps, w.xn, nullptr, nullptr, s)) != hipSuccess)
      return hip_fail(e, "rmsnorm");
    g = soc::GemmArgs{};
    g.a = w.xn;
    g.lda = H;
    g.w = L.wgate;
    g.w2 = L.wup;
    g.c = w.h;
    g.ldc = I;
    g.M = n;
    g.N = I;
    g.K = H;
    if ((e = prefill_gemm(g, soc::EPI_SWIGLU, s, kSplitGateUp)) != hipSuccess) return hip_fail(e, "gemm gate/up");
    g = soc::GemmArgs{};
    g.a = w.h;
    g.lda = I;
    g.w = L.wdown;
    g.c = w.x;
    g.ldc = H;
    g.M = n;
    g.N = H;
    g.K = I;
    if ((e = prefill_gemm(g, soc::EPI_RESIDUAL, s, kSplitDown)) != hipSuccess) return hip_fail(e, "gemm down");
  }
  // logits of the last row (with the greedy token), then of the other requested rows
  soc::LmHeadArgs h{};
  h.x = w.x + static_cast<size_t>(n - 1) * H;
  h.gain = m->final_norm;
  h.eps = c.rms_norm_eps;
  h.w = m->lm_head;
  h.logits = w.logits + static_cast<size_t>(std::max(logit_rows, 1) - 1) * c.vocab_size;
  h.part_val = w.lm_val;
  h.part_idx = w.lm_idx;
  h.counter = w.lm_counter;
  h.token_out = w.token;
  h.N = c.vocab_size;
  h.K = H;
  if ((e = soc::launch_lm_head_argmax(h, s)) != hipSuccess) return hip_fail(e, "lm head");
  if (logit_rows > 1) {
    const int rows = logit_rows - 1;
    const float* xr = w.x + static_cast<size_t>(n - logit_rows) * H;
    if ((e = soc::launch_rmsnorm_rows(xr, rows, H, m->final_norm, c.rms_norm_eps, w.xn, nullptr, nullptr, s)) != hipSuccess)
      return hip_fail(e, "rmsnorm");
    soc::GemmArgs g{};
    g.a = w.xn;
    g.lda = H;
    g.w = m->lm_head;
    g.c = w.logits;
    g.ldc = c.vocab_size;
    g.M = rows;
    g.N = c.vocab_size;
    g.K = H;
    if ((e = prefill_gemm(g,soc::EPI_STORE, s)) != hipSuccess) return hip_fail(e, "gemm lm head");
  }
  if (logits != nullptr && logit_rows > 0) {
    if ((e = hipMemcpyAsync(logits, w.logits, static_cast<size_t>(logit_rows) * c.vocab_size * 4, hipMemcpyDefault,
                            s)) != hipSuccess)
      return hip_fail(e, "hipMemcpyAsync logits");
  }
  if (hidden != nullptr) {  // the final RMSNorm of every row (qwen_causal_lm.cpp:117-128)
    if ((e = soc::launch_rmsnorm_rows(w.x, n, H, m->final_norm, c.rms_norm_eps, w.xn, nullptr, nullptr, s)) !=
        hipSuccess)
      return hip_fail(e, "final rmsnorm");
    if ((e = hipMemcpyAsync(hidden, w.xn, static_cast<size_t>(n) * H * 4, hipMemcpyDefault, s)) != hipSuccess)
      return hip_fail(e, "hipMemcpyAsync hidden");
  }
  int32_t tok = 0, id_err = 0;
  if ((e = hipMemcpyAsync(&tok, w.token, 4, hipMemcpyDeviceToHost, s)) != hipSuccess)
    return hip_fail(e, "hipMemcpyAsync token");
  if (ids_dev && (e = hipMemcpyAsync(&id_err, m->ctx->id_err, 4, hipMemcpyDeviceToHost, s)) != hipSuccess)
    return hip_fail(e, "hipMemcpyAsync id flag");
  record_timer_stop(m->ctx);
  if ((e = hipStreamSynchronize(s)) != hipSuccess) return hip_fail(e, "prefill");
  if (id_err != 0) {
    if ((e = hipMemset(m->ctx->id_err, 0, 4)) != hipSuccess) return hip_fail(e, "hipMemset");
    return soc::fail(SOC_ERR_INVALID, "token id out of range");
  }
  if (next_token) *next_token = tok;
  return SOC_OK;
}

// The context's id-error flag (device words written by the id staging kernel), allocated on first use.
int ensure_id_flag(soc_ctx* ctx) {
  if (ctx->id_err != nullptr) return SOC_OK;
  hipError_t e = hipMalloc(&ctx->id_err, 64);
  if (e != hipSuccess) return hip_fail(e, "hipMalloc id flag");
  if ((e = hipMemset(ctx->id_err, 0, 64)) != hipSuccess) return hip_fail(e, "hipMemset");
  return SOC_OK;
}
}  // namespace

int soc_prefill(soc_model* m, soc_kv* kv, int32_t slot, const int32_t* ids, int32_t n, int32_t pos_off,
                int32_t logit_rows, float* logits, int32_t* next_token) {
  SOC_API_BEGIN
  if (m == nullptr || kv == nullptr || ids == nullptr) return soc::fail(SOC_ERR_INVALID, "null argument");
  SOC_TRY(bind_kv(kv, m));
  if (!m->finalized) return soc::fail(SOC_ERR_STATE, "model is not finalized");
  if (n <= 0) return soc::fail(SOC_ERR_INVALID, "prefill requires at least one token");  // generation_context.cpp:22-27
  if (slot < 0 || slot >= kv->slots) return soc::fail(SOC_ERR_INVALID, "slot out of range");
  if (pos_off != kv->len[slot])
    return soc::fail(SOC_ERR_STATE, "position_offset must equal the cached length of the slot");
  if (pos_off + n > kv->cap) return soc::fail(SOC_ERR_CAPACITY, "prefill exceeds KV capacity");
  if (logit_rows < 0 || logit_rows > n) return soc::fail(SOC_ERR_INVALID, "logit_rows out of range");
  SOC_TRY(validate_ids(m, ids, n));
  SOC_TRY(run_prefill(m, kv, slot, ids, false, n, pos_off, 0, nullptr, logit_rows, logits, next_token));
  kv->len[slot] = pos_off + n;
  return SOC_OK;
  SOC_API_END
}

namespace {
// One decode step of one slot (the checks done by the caller): token `last`, or the id at dev_last in device memory;
// logits [V] nullable (host or device), one synchronisation.
int ensure_readback(soc_ctx* ctx) {
  if (ctx->readback != nullptr) return SOC_OK;
  hipError_t e = hipHostMalloc(reinterpret_cast<void**>(&ctx->readback), 64);
  if (e != hipSuccess) return hip_fail(e, "hipHostMalloc readback words");
  if ((e = hipHostGetDevicePointer(reinterpret_cast<void**>(&ctx->readback_dev), ctx->readback, 0)) != hipSuccess) {
    (void)hipHostFree(ctx->readback);
    ctx->readback = nullptr;
    return hip_fail(e, "hipHostGetDevicePointer");
  }
  return SOC_OK;
}

int decode_one(soc_model* m, soc_kv* kv, int32_t slot, int32_t last, const int32_t* dev_last, float* logits,
               int32_t* next_token) {
  SOC_TRY(ensure_decode_ws(m, kv->cap));
  SOC_TRY(ensure_readback(m->ctx));
  const bool xcd = use_xcd(m);
  int32_t err = 0;
  const char* trace_path = std::getenv("SOC_TRACE_FILE");
  const size_t logit_bytes = static_cast<size_t>(m->cfg.vocab_size) * 4;
  // device logits are written where the caller wants them by the one-launch kernel itself
  const bool direct = logits != nullptr && (xcd || use_persistent(m)) &&
                      soc::classify_range(logits, logit_bytes) == soc::MemRange::kDeviceRange;
  SOC_TRY(run_decode_steps(m, kv, slot, last, 1, dev_last, &err, direct ? logits : nullptr));
  hipStream_t s = m->ctx->stream;
  hipError_t e;
  if (logits != nullptr && !direct &&
      (e = hipMemcpyAsync(logits, m->dws.logits, logit_bytes, hipMemcpyDefault, s)) != hipSuccess)
    return hip_fail(e, "hipMemcpyAsync logits");
  // next token and both error flags in one launch, written straight into pinned host words
  if ((e = soc::launch_decode_readback(m->dws.state, m->dws.err, dev_last != nullptr ? m->ctx->id_err : nullptr,
                                       m->ctx->readback_dev, s)) != hipSuccess)
    return hip_fail(e, "decode readback");
  record_timer_stop(m->ctx);
  if ((e = hipStreamSynchronize(s)) != hipSuccess) return hip_fail(e, "decode");
  const volatile int32_t* rb = m->ctx->readback;
  const int32_t tok = rb[0], id_err = rb[2];
  if (trace_path == nullptr) err = rb[1];  // with a trace, run_decode_steps has read the flag itself
  SOC_TRY(one_launch_status(m, xcd, err));
  if (id_err != 0) {
    if ((e = hipMemset(m->ctx->id_err, 0, 4)) != hipSuccess) return hip_fail(e, "hipMemset");
    return soc::fail(SOC_ERR_INVALID, "token id out of range");
  }
  kv->len[slot] += 1;
  if (next_token) *next_token = tok;
  return SOC_OK;
}

// An output of `bytes` bytes that the library copies into with hipMemcpyDefault: host memory, or device memory that
// holds the whole range.
int check_output(const char* what, const void* p, size_t bytes) {
  if (p == nullptr || soc::classify_range(p, bytes) != soc::MemRange::kOutside) return SOC_OK;
  return soc::fail(SOC_ERR_INVALID, std::string(what) + " extends past the end of its device allocation");
}
}  // namespace

int soc_decode(soc_model* m, soc_kv* kv, int32_t slot, int32_t last, float* logits, int32_t* next_token) {
  SOC_API_BEGIN
  if (m == nullptr || kv == nullptr) return soc::fail(SOC_ERR_INVALID, "null argument");
  SOC_TRY(bind_kv(kv, m));
  if (!m->finalized) return soc::fail(SOC_ERR_STATE, "model is not finalized");
  if (slot < 0 || slot >= kv->slots) return soc::fail(SOC_ERR_INVALID, "slot out of range");
  if (kv->len[slot] + 1 > kv->cap) return soc::fail(SOC_ERR_CAPACITY, "decode exceeds KV capacity");
  SOC_TRY(validate_ids(m, &last, 1));
  SOC_TRY(check_output("decode logits", logits, static_cast<size_t>(m->cfg.vocab_size) * 4));
  return decode_one(m, kv, slot, last, nullptr, logits, next_token);
  SOC_API_END
}

int soc_forward(soc_model* m, soc_kv* kv, int32_t slot, const int32_t* ids, int32_t n, int32_t pos_off, float* hidden,
                int32_t logit_rows, float* logits, int32_t* next_token) {
  SOC_API_BEGIN
  if (m == nullptr || ids == nullptr) return soc::fail(SOC_ERR_INVALID, "null argument");
  if (!m->finalized) return soc::fail(SOC_ERR_STATE, "model is not finalized");
  if (n <= 0) return soc::fail(SOC_ERR_INVALID, "forward requires at least one token");
  if (pos_off < 0) return soc::fail(SOC_ERR_INVALID, "position_offset must be >= 0");
  if (logit_rows < 0 || logit_rows > n) return soc::fail(SOC_ERR_INVALID, "logit_rows out of range");
  const soc_qwen_config& c = m->cfg;
  const soc::MemRange where = soc::classify_range(ids, static_cast<size_t>(n) * 4);
  if (where == soc::MemRange::kOutside)
    return soc::fail(SOC_ERR_INVALID, "token ids extend past the end of their device allocation");
  const bool ids_dev = where == soc::MemRange::kDeviceRange;
  if (ids_dev)
    SOC_TRY(ensure_id_flag(m->ctx));
  else
    SOC_TRY(validate_ids(m, ids, n));
  SOC_TRY(check_output("hidden output", hidden, static_cast<size_t>(n) * c.hidden_size * 4));
  SOC_TRY(check_output("logits output", logits, static_cast<size_t>(logit_rows) * c.vocab_size * 4));
  if (kv == nullptr) {
    // uncached (qwen_causal_lm.cpp:37-129, 231-248): causal attention over the n tokens alone, RoPE at
    // position_offset + i; the private cache starts empty and is left empty
    if (pos_off + n > m->rope_len)
      return soc::fail(SOC_ERR_CAPACITY, "position_offset + token count exceeds max_position_embeddings");
    if (m->ukv == nullptr || m->ukv->cap < n) {
      if (m->ukv != nullptr) {
        soc_kv_destroy(m->ukv);
        m->ukv = nullptr;
      }
      SOC_TRY(kv_create(m->ctx, m, c.num_hidden_layers, c.num_key_value_heads, c.head_dim, 1, std::max(n, 64),
                        &m->ukv));
    }
    m->ukv->len[0] = 0;
    return run_prefill(m, m->ukv, 0, ids, ids_dev, n, 0, pos_off, hidden, logit_rows, logits, next_token);
  }
  SOC_TRY(bind_kv(kv, m));
  if (slot < 0 || slot >= kv->slots) return soc::fail(SOC_ERR_INVALID, "slot out of range");
  if (pos_off != kv->len[slot])
    return soc::fail(SOC_ERR_STATE, "position_offset must equal the cached length of the slot");
  if (pos_off + n > kv->cap) return soc::fail(SOC_ERR_CAPACITY, "forward exceeds KV capacity");
  if (n == 1 && hidden == nullptr)
    return decode_one(m, kv, slot, ids_dev ? 0 : ids[0], ids_dev ? ids : nullptr, logit_rows > 0 ? logits : nullptr,
                      next_token);
  SOC_TRY(run_prefill(m, kv, slot, ids, ids_dev, n, pos_off, 0, hidden, logit_rows, logits, next_token));
  kv->len[slot] = pos_off + n;
  return SOC_OK;
  SOC_API_END
}

int soc_model_load_tensor_device(soc_model* m, const char* name, const void* src, int32_t dtype, int64_t numel) {
  SOC_API_BEGIN
  if (m == nullptr || name == nullptr || src == nullptr) return soc::fail(SOC_ERR_INVALID, "null argument");
  if (dtype != SOC_DTYPE_F32 && dtype != SOC_DTYPE_F16)
    return soc::fail(SOC_ERR_INVALID, "weights must be float32 or float16");
  auto it = m->tensors.find(name);
  if (it == m->tensors.end()) return soc::fail(SOC_ERR_INVALID, std::string("unknown tensor name: ") + name);
  if (it->second.numel != numel)
    return soc::fail(SOC_ERR_INVALID, std::string("tensor ") + name + " has " + std::to_string(numel) +
                                          " elements, expected " + std::to_string(it->second.numel));
  SOC_TRY(soc::check_device_operand(name, src, static_cast<size_t>(numel) * (dtype == SOC_DTYPE_F32 ? 4 : 2)));
  hipStream_t s = m->ctx->stream;
  hipError_t e = dtype == SOC_DTYPE_F16
                     ? hipMemcpyAsync(it->second.ptr, src, static_cast<size_t>(numel) * 2, hipMemcpyDeviceToDevice, s)
                     : soc::launch_f32_to_f16(static_cast<const float*>(src), static_cast<size_t>(numel),
                                              it->second.ptr, s);
  if (e == hipSuccess) e = hipStreamSynchronize(s);
  if (e != hipSuccess) return hip_fail(e, "weight copy");
  it->second.loaded = true;
  m->finalized = false;
  return SOC_OK;
  SOC_API_END
}

int soc_decode_steps(soc_model* m, soc_kv* kv, int32_t slot, int32_t last, int32_t steps, int32_t* tokens_out) {
  SOC_API_BEGIN
  if (m == nullptr || kv == nullptr || (steps > 0 && tokens_out == nullptr))
    return soc::fail(SOC_ERR_INVALID, "null argument");
  SOC_TRY(bind_kv(kv, m));
  if (!m->finalized) return soc::fail(SOC_ERR_STATE, "model is not finalized");
  if (slot < 0 || slot >= kv->slots) return soc::fail(SOC_ERR_INVALID, "slot out of range");
  if (steps < 0) return soc::fail(SOC_ERR_INVALID, "steps must be >= 0");
  if (kv->len[slot] + steps > kv->cap) return soc::fail(SOC_ERR_CAPACITY, "decode exceeds KV capacity");
  if (steps == 0) return SOC_OK;
  SOC_TRY(validate_ids(m, &last, 1));
  SOC_TRY(ensure_decode_ws(m, kv->cap));
  SOC_TRY(run_decode_steps(m, kv, slot, last, steps));
  hipStream_t s = m->ctx->stream;
  hipError_t e = hipMemcpyAsync(tokens_out, m->dws.ring, static_cast<size_t>(steps) * 4, hipMemcpyDeviceToHost, s);
  if (e != hipSuccess) return hip_fail(e, "hipMemcpyAsync tokens");
  if ((e = hipStreamSynchronize(s)) != hipSuccess) return hip_fail(e, "decode steps");
  kv->len[slot] += steps;
  return SOC_OK;
  SOC_API_END
}

int soc_decode_steps_noalloc(soc_model* m, soc_kv* kv, int32_t slot, int32_t last, int32_t steps,
                             int32_t* tokens_out) {
  SOC_API_BEGIN
  if (m == nullptr || kv == nullptr || (steps > 0 && tokens_out == nullptr))
    return soc::fail(SOC_ERR_INVALID, "null argument");
  SOC_TRY(bind_kv(kv, m));
  if (!m->finalized) return soc::fail(SOC_ERR_STATE, "model is not finalized");
  if (slot < 0 || slot >= kv->slots) return soc::fail(SOC_ERR_INVALID, "slot out of range");
  if (steps < 0) return soc::fail(SOC_ERR_INVALID, "steps must be >= 0");
  if (m->ctx->scratch == nullptr) return soc::fail(SOC_ERR_STATE, "no scratch address for this device");
  const soc_qwen_config& c = m->cfg;
  // word layout of the scratch array, regions rounded to 256 bytes: counters and flags, argmax partials (zeroed),
  // exchange vectors (0xff), token ring
  auto up = [](size_t n) { return (n + 63) & ~size_t{63}; };
  const size_t nb = static_cast<size_t>(std::max(m->ctx->num_cus, soc::kXcdGroups * soc::kXcdBlocks));
  const int G = c.num_attention_heads / c.num_key_value_heads;
  const size_t H = static_cast<size_t>(c.hidden_size), loc_stride = up(soc::xcd_loc_stride(G, c.intermediate_size));
  const size_t o_err = 0, o_state = 64, o_ring_pos = 128, o_counter = 192, o_xcd_ctr = 256, o_pv = 320,
               o_pi = o_pv + up(nb), n_zero = o_pi + up(nb);
  const size_t o_xa = n_zero, o_xb = o_xa + up(H), o_qkv = o_xb + up(H), o_attn = o_qkv + up(m->qkv_rows),
               o_h = o_attn + up(m->qd), o_xo = o_h + up(c.intermediate_size), o_xd = o_xo + soc::kXcdGroups * up(H),
               o_xp = o_xd + soc::kXcdGroups * up(H), o_loc = o_xp + up(H), o_ring = o_loc + soc::kXcdGroups * loc_stride;
  const size_t need = (o_ring + up(static_cast<size_t>(steps))) * 4;
  if (need > kNoAllocScratchBytes)
    return soc::fail(SOC_ERR_CAPACITY, "soc_decode_steps_noalloc: " + std::to_string(steps) + " steps need " +
                                           std::to_string(need) + " bytes of scratch; the maximum is " +
                                           std::to_string(kNoAllocScratchBytes) + " (4 bytes per step)");
  if (kv->len[slot] + steps > kv->cap) return soc::fail(SOC_ERR_CAPACITY, "decode exceeds KV capacity");
  if (steps == 0) return SOC_OK;
  SOC_TRY(validate_ids(m, &last, 1));
  const bool xcd = use_xcd(m);
  if (!xcd && !use_persistent(m))
    return soc::fail(SOC_ERR_INVALID, "soc_decode_steps_noalloc: this model has no one-launch decode kernel");
  const int dev = m->ctx->device;
  if (dev < 0 || dev >= kNoAllocMaxDevices)
    return soc::fail(SOC_ERR_INVALID, "soc_decode_steps_noalloc: device index beyond the supported 64");
  bool idle = false;
  if (!g_noalloc_busy[dev].compare_exchange_strong(idle, true))
    return soc::fail(SOC_ERR_STATE, "soc_decode_steps_noalloc: another call is using this device's scratch array");
  struct Release {
    std::atomic<bool>* f;
    ~Release() { f->store(false); }
  } release{&g_noalloc_busy[dev]};
  uint32_t* base = m->ctx->scratch;
  DecodeWs w;
  w.err = reinterpret_cast<int*>(base + o_err);
  w.state = reinterpret_cast<int*>(base + o_state);
  w.ring_pos = reinterpret_cast<int*>(base + o_ring_pos);
  w.lm_counter = reinterpret_cast<int*>(base + o_counter);
  w.xcd_ctr = reinterpret_cast<int*>(base + o_xcd_ctr);
  w.pv = reinterpret_cast<float*>(base + o_pv);
  w.pi = reinterpret_cast<int*>(base + o_pi);
  w.xa = base + o_xa;
  w.xb = base + o_xb;
  w.qkv_x = base + o_qkv;
  w.attn_x = base + o_attn;
  w.h_x = base + o_h;
  w.xo = base + o_xo;
  w.xd = base + o_xd;
  w.xp = base + o_xp;
  w.loc = base + o_loc;
  w.loc_stride = static_cast<int>(loc_stride);
  w.ring = reinterpret_cast<int*>(base + o_ring);
  w.nblocks = m->ctx->num_cus;
  hipStream_t s = m->ctx->stream;
  // the previous call's contents are stale (any model may have used the array): counters, flags and the decode
  // state restart, every exchange word carries tag 3; a kernel, not hipMemsetAsync, so a captured call replays it
  hipLaunchKernelGGL(k_noalloc_init, dim3(64), dim3(256), 0, s, base, static_cast<int>(n_zero),
                     static_cast<int>(o_state), static_cast<int>(o_xa), static_cast<int>(o_ring - o_xa), last,
                     kv->len[slot]);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return hip_fail(e, "scratch init launch");
  const soc::PersistArgs p = persist_args(m, kv, slot, w);
  for (int i = 0; i < steps; ++i)
    if ((e = xcd ? soc::launch_decode_xcd(p, s) : soc::launch_decode_persistent(p, w.nblocks, s)) != hipSuccess)
      return hip_fail(e, "one-launch decode launch");
  int32_t err = 0;
  if ((e = hipMemcpyAsync(tokens_out, w.ring, static_cast<size_t>(steps) * 4, hipMemcpyDeviceToHost, s)) !=
      hipSuccess)
    return hip_fail(e, "hipMemcpyAsync tokens");
  if ((e = hipMemcpyAsync(&err, w.err, 4, hipMemcpyDeviceToHost, s)) != hipSuccess)
    return hip_fail(e, "hipMemcpyAsync err");
  if ((e = hipStreamSynchronize(s)) != hipSuccess) return hip_fail(e, "decode steps (no allocation)");
  if (err != 0) {
    if (xcd && err == 2) {
      m->xcd_off = true;
      return soc::fail(SOC_ERR_HIP, "XCD decode: the launch did not place 32 blocks on each of the 8 XCDs");
    }
    return soc::fail(SOC_ERR_HIP, "one-launch decode: a cross-block wait timed out (grid not co-resident?)");
  }
  kv->len[slot] += steps;
  return SOC_OK;
  SOC_API_END
}

int soc_decode_batch(soc_model* m, soc_kv* kv, int32_t n, const int32_t* slots, const int32_t* tokens, float* logits,
                     int32_t* next_tokens) {
  SOC_API_BEGIN
  if (m != nullptr && m->qbits != 0)
    return soc::fail(SOC_ERR_INVALID, "ragged batch decode of a group-quantized model is not supported");
  if (next_tokens == nullptr) return soc::fail(SOC_ERR_INVALID, "null argument");
  int max_len = 0;
  SOC_TRY(validate_batch(m, kv, n, slots, tokens, 1, &max_len));
  SOC_TRY(ensure_prefill_ws(m, n, max_len, n));
  SOC_TRY(ensure_batch_ws(m, n));
  std::vector<int32_t> pos;
  SOC_TRY(upload_batch(m, kv, n, slots, tokens, &pos));
  SOC_TRY(enqueue_batch_step(m, kv, n, (max_len + kAttnChunk - 1) / kAttnChunk, m->bws.ring1, 1));
  hipStream_t s = m->ctx->stream;
  hipError_t e;
  if (logits != nullptr &&
      (e = hipMemcpyAsync(logits, m->pws.logits, static_cast<size_t>(n) * m->cfg.vocab_size * 4, hipMemcpyDefault,
                          s)) != hipSuccess)
    return hip_fail(e, "hipMemcpyAsync logits");
  if ((e = hipMemcpyAsync(next_tokens, m->bws.ids, static_cast<size_t>(n) * 4, hipMemcpyDeviceToHost, s)) !=
      hipSuccess)
    return hip_fail(e, "hipMemcpyAsync tokens");
  if ((e = hipStreamSynchronize(s)) != hipSuccess) return hip_fail(e, "decode batch");
  for (int i = 0; i < n; ++i) kv->len[slots[i]] += 1;
  return SOC_OK;
  SOC_API_END
}

int soc_decode_batch_steps(soc_model* m, soc_kv* kv, int32_t n, const int32_t* slots, const int32_t* tokens,
                           int32_t steps, int32_t* tokens_out) {
  SOC_API_BEGIN
  if (m != nullptr && m->qbits != 0)
    return soc::fail(SOC_ERR_INVALID, "ragged batch decode of a group-quantized model is not supported");
  if (steps < 0) return soc::fail(SOC_ERR_INVALID, "steps must be >= 0");
  if (steps > 0 && tokens_out == nullptr) return soc::fail(SOC_ERR_INVALID, "null argument");
  int max_len = 0;
  SOC_TRY(validate_batch(m, kv, n, slots, tokens, steps, &max_len));
  if (steps == 0) return SOC_OK;
  SOC_TRY(ensure_prefill_ws(m, n, kv->cap, n));
  SOC_TRY(ensure_batch_ws(m, n));
  std::vector<int32_t> pos;
  SOC_TRY(upload_batch(m, kv, n, slots, tokens, &pos));
  hipStream_t s = m->ctx->stream;
  BatchWs& b = m->bws;
  hipError_t e;
  const size_t ring_need = static_cast<size_t>(n) * steps;
  if (b.ring_cap < ring_need) {
    if ((e = hipStreamSynchronize(s)) != hipSuccess) return hip_fail(e, "hipStreamSynchronize");
    (void)hipFree(b.ring);
    b.ring = nullptr;
    b.ring_cap = 0;
    ++m->bws_gen;
    if ((e = hipMalloc(&b.ring, ring_need * 4)) != hipSuccess) return hip_fail(e, "hipMalloc ring");
    b.ring_cap = ring_need;
  }
  // the attention grid covers the whole capacity (rows past their own length exit at once), so one captured step
  // serves every call with the same (rows, steps)
  const int max_split = (kv->cap + kAttnChunk - 1) / kAttnChunk;
  if (env_flag("SOC_EAGER")) {
    for (int i = 0; i < steps; ++i) SOC_TRY(enqueue_batch_step(m, kv, n, max_split, b.ring, steps));
  } else {
    const std::pair<int, int> key(n, steps);
    hipGraphExec_t exec = nullptr;
    auto it = kv->batch_graphs.find(key);
    if (it != kv->batch_graphs.end() && it->second.first == m->bws_gen) {
      exec = it->second.second;
    } else {
      if (it != kv->batch_graphs.end()) {
        (void)hipGraphExecDestroy(it->second.second);
        kv->batch_graphs.erase(it);
      }
      hipGraph_t graph;
      if ((e = hipStreamBeginCapture(s, hipStreamCaptureModeThreadLocal)) != hipSuccess)
        return hip_fail(e, "hipStreamBeginCapture");
      const int rc = enqueue_batch_step(m, kv, n, max_split, b.ring, steps);
      e = hipStreamEndCapture(s, &graph);
      if (rc != SOC_OK) return rc;
      if (e != hipSuccess) return hip_fail(e, "hipStreamEndCapture");
      e = hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0);
      (void)hipGraphDestroy(graph);
      if (e != hipSuccess) return hip_fail(e, "hipGraphInstantiate");
      kv->batch_graphs[key] = std::make_pair(m->bws_gen, exec);
    }
    for (int i = 0; i < steps; ++i)
      if ((e = hipGraphLaunch(exec, s)) != hipSuccess) return hip_fail(e, "hipGraphLaunch");
  }
  int32_t* ring = b.ring;
  std::vector<int32_t> host(static_cast<size_t>(n) * steps);
  if ((e = hipMemcpyAsync(host.data(), ring, host.size() * 4, hipMemcpyDeviceToHost, s)) != hipSuccess)
    return hip_fail(e, "hipMemcpyAsync tokens");
  if ((e = hipStreamSynchronize(s)) != hipSuccess) return hip_fail(e, "decode batch steps");
  for (int t = 0; t < steps; ++t)
    for (int i = 0; i < n; ++i) tokens_out[static_cast<size_t>(t) * n + i] = host[static_cast<size_t>(i) * steps + t];
  for (int i = 0; i < n; ++i) kv->len[slots[i]] += steps;
  return SOC_OK;
  SOC_API_END
}

// ---- op-level ----
int soc_gemm_f16(soc_ctx* ctx, const void* x, const void* w, float* y, int32_t m, int32_t n, int32_t k) {
  SOC_API_BEGIN
  if (ctx == nullptr) return soc::fail(SOC_ERR_INVALID, "null context");
  if (m <= 0 || n <= 0 || k <= 0 || k % 32 != 0)
    return soc::fail(SOC_ERR_INVALID, "soc_gemm_f16: need m, n > 0 and k a positive multiple of 32");
  const size_t M = static_cast<size_t>(m), N = static_cast<size_t>(n), K = static_cast<size_t>(k);
  SOC_TRY(soc::check_device_operand("GEMM activations", x, M * K * 2));
  SOC_TRY(soc::check_device_operand("GEMM weights", w, N * K * 2));
  SOC_TRY(soc::check_device_operand("GEMM output", y, M * N * 4));
  if ((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(w)) % 16 != 0)
    return soc::fail(SOC_ERR_INVALID, "soc_gemm_f16: activations and weights must be 16-byte aligned");
  soc::GemmSplitArgs g{};
  g.ah = static_cast<const f16*>(x);
  g.lda = k;
  g.w = static_cast<const f16*>(w);
  g.c = y;
  g.ldc = n;
  g.M = m;
  g.N = n;
  g.K = k;
  hipError_t e = soc::launch_gemm_split(g, soc::EPI_STORE, ctx->stream);
  if (e == hipSuccess) e = hipStreamSynchronize(ctx->stream);
  return e == hipSuccess ? SOC_OK : hip_fail(e, "gemm");
  SOC_API_END
}

namespace {
// Grows the context's split-key attention scratch to `floats` partial words and `ints` zeroed arrival counters.
int ensure_op_attention_ws(soc_ctx* ctx, size_t floats, size_t ints) {
  hipError_t e;
  if (ctx->op_part_floats < floats) {
    if ((e = hipStreamSynchronize(ctx->stream)) != hipSuccess) return hip_fail(e, "hipStreamSynchronize");
    (void)hipFree(ctx->op_part);
    ctx->op_part = nullptr;
    ctx->op_part_floats = 0;
    if ((e = hipMalloc(&ctx->op_part, floats * 4)) != hipSuccess) return hip_fail(e, "hipMalloc attention scratch");
    ctx->op_part_floats = floats;
  }
  if (ctx->op_counter_ints < ints) {
    if ((e = hipStreamSynchronize(ctx->stream)) != hipSuccess) return hip_fail(e, "hipStreamSynchronize");
    (void)hipFree(ctx->op_counters);
    ctx->op_counters = nullptr;
    ctx->op_counter_ints = 0;
    if ((e = hipMalloc(&ctx->op_counters, ints * 4)) != hipSuccess) return hip_fail(e, "hipMalloc attention counters");
    // the combining block of each row resets its counter, so the zeros hold from one call to the next
    if ((e = hipMemset(ctx->op_counters, 0, ints * 4)) != hipSuccess) return hip_fail(e, "hipMemset");
    ctx->op_counter_ints = ints;
  }
  return SOC_OK;
}

int check_attention_shape(int32_t nq, int32_t nkv, int32_t head_dim, int32_t cap) {
  if (head_dim != 128) return soc::fail(SOC_ERR_INVALID, "attention: head_dim must be 128");
  if (nkv <= 0 || nq <= 0 || nq % nkv != 0 || (nq / nkv != 1 && nq / nkv != 2 && nq / nkv != 4 && nq / nkv != 8))
    return soc::fail(SOC_ERR_INVALID, "attention: query heads per KV head must be 1, 2, 4 or 8");
  if (cap <= 0) return soc::fail(SOC_ERR_INVALID, "attention: capacity must be positive");
  return SOC_OK;
}
}  // namespace

int soc_attention_prefill(soc_ctx* ctx, const float* q, const void* keys, const void* values, float* out, int32_t rows,
                          int32_t pos_base, int32_t nq, int32_t nkv, int32_t head_dim, int32_t cap) {
  SOC_API_BEGIN
  if (ctx == nullptr) return soc::fail(SOC_ERR_INVALID, "null context");
  SOC_TRY(check_attention_shape(nq, nkv, head_dim, cap));
  if (rows <= 0 || pos_base < 0 || pos_base + rows > cap)
    return soc::fail(SOC_ERR_INVALID, "attention: need rows > 0 and pos_base + rows <= capacity");
  const size_t qbytes = static_cast<size_t>(rows) * nq * 128 * 4, kvbytes = static_cast<size_t>(nkv) * cap * 128 * 2;
  SOC_TRY(soc::check_device_operand("attention queries", q, qbytes));
  SOC_TRY(soc::check_device_operand("attention keys", keys, kvbytes));
  SOC_TRY(soc::check_device_operand("attention values", values, kvbytes));
  SOC_TRY(soc::check_device_operand("attention output", out, qbytes));
  soc::AttnArgs a{};
  a.qkv = q;
  a.ld_qkv = nq * 128;
  a.kcache = static_cast<f16*>(const_cast<void*>(keys));
  a.vcache = static_cast<f16*>(const_cast<void*>(values));
  a.cap = cap;
  a.pos_base = pos_base;
  a.out = out;
  a.ld_out = nq * 128;
  a.B = rows;
  a.nq = nq;
  a.nkv = nkv;
  a.chunk = kAttnChunk;
  a.max_split = (pos_base + rows + kAttnChunk - 1) / kAttnChunk;
  a.scale = 1.0f / std::sqrt(128.0f);  // grouped_query_attention.cpp:81
  hipError_t e;
  if (soc::attention_prefill_pairs_supported(nq, nkv)) {
    e = soc::launch_attention_prefill_pairs(a, ctx->stream);
  } else if (soc::attention_prefill_mfma_supported(nq, nkv)) {
    e = soc::launch_attention_prefill_mfma(a, ctx->stream);
  } else {  // 8 query heads per KV head: the split-key row kernel
    if (a.max_split > 160) return soc::fail(SOC_ERR_INVALID, "attention: more than 40960 keys");
    SOC_TRY(ensure_op_attention_ws(ctx, static_cast<size_t>(rows) * nq * a.max_split * 130,
                                   static_cast<size_t>(rows) * nkv));
    a.part = ctx->op_part;
    a.counters = ctx->op_counters;
    e = soc::launch_attention(a, 0, ctx->stream);
  }
  if (e == hipSuccess) e = hipStreamSynchronize(ctx->stream);
  return e == hipSuccess ? SOC_OK : hip_fail(e, "attention prefill");
  SOC_API_END
}

int soc_attention_decode(soc_ctx* ctx, const float* q, const void* keys, const void* values, float* out,
                         int32_t kv_len, int32_t nq, int32_t nkv, int32_t head_dim, int32_t cap) {
  SOC_API_BEGIN
  if (ctx == nullptr) return soc::fail(SOC_ERR_INVALID, "null context");
  SOC_TRY(check_attention_shape(nq, nkv, head_dim, cap));
  if (kv_len <= 0 || kv_len > cap) return soc::fail(SOC_ERR_INVALID, "attention: need 0 < kv_len <= capacity");
  const size_t qbytes = static_cast<size_t>(nq) * 128 * 4, kvbytes = static_cast<size_t>(nkv) * cap * 128 * 2;
  SOC_TRY(soc::check_device_operand("attention queries", q, qbytes));
  SOC_TRY(soc::check_device_operand("attention keys", keys, kvbytes));
  SOC_TRY(soc::check_device_operand("attention values", values, kvbytes));
  SOC_TRY(soc::check_device_operand("attention output", out, qbytes));
  soc::AttnArgs a{};
  a.qkv = q;
  a.ld_qkv = nq * 128;
  a.kcache = static_cast<f16*>(const_cast<void*>(keys));
  a.vcache = static_cast<f16*>(const_cast<void*>(values));
  a.cap = cap;
  a.pos_base = kv_len - 1;  // the query sits at the last cached position and sees keys 0 .. kv_len - 1
  a.out = out;
  a.ld_out = nq * 128;
  a.B = 1;
  a.nq = nq;
  a.nkv = nkv;
  a.chunk = decode_attn_chunk(cap);
  a.max_split = (kv_len + a.chunk - 1) / a.chunk;
  a.scale = 1.0f / std::sqrt(128.0f);
  if (a.max_split > 160) return soc::fail(SOC_ERR_INVALID, "attention: too many keys for the capacity's chunk size");
  SOC_TRY(ensure_op_attention_ws(ctx, static_cast<size_t>(nq) * a.max_split * 130, static_cast<size_t>(nkv)));
  a.part = ctx->op_part;
  a.counters = ctx->op_counters;
  hipError_t e = soc::launch_attention(a, 0, ctx->stream);
  if (e == hipSuccess) e = hipStreamSynchronize(ctx->stream);
  return e == hipSuccess ? SOC_OK : hip_fail(e, "attention decode");
  SOC_API_END
}

int soc_gemv_f16(soc_ctx* ctx, const void* w, const void* x, float* y, int32_t n, int32_t k) {
  if (ctx == nullptr || w == nullptr || x == nullptr || y == nullptr) return soc::fail(SOC_ERR_INVALID, "null argument");
  if (n <= 0 || k <= 0 || k % 8 != 0 || k > 16384) return soc::fail(SOC_ERR_INVALID, "soc_gemv_f16: need n > 0, 0 < k <= 16384, k % 8 == 0");
  soc::GemvArgs g{};
  g.xh = static_cast<const f16*>(x);
  g.w = static_cast<const f16*>(w);
  g.y = y;
  g.N = n;
  g.K = k;
  hipError_t e = soc::launch_gemv(g, soc::EPI_STORE, ctx->stream);
  return e == hipSuccess ? SOC_OK : hip_fail(e, "gemv");
}

int soc_qmm(soc_ctx* ctx, const void* x, const void* codes, int32_t bits, const void* scales, float* y, int32_t mm,
            int32_t n, int32_t k) {
  if (ctx == nullptr || x == nullptr || codes == nullptr || scales == nullptr || y == nullptr)
    return soc::fail(SOC_ERR_INVALID, "null argument");
  if (bits != 8 && bits != 4) return soc::fail(SOC_ERR_INVALID, "soc_qmm: bits must be 8 or 4");
  if (!(mm == 1 || mm == 2 || mm == 4 || mm == 8)) return soc::fail(SOC_ERR_INVALID, "soc_qmm: m must be 1, 2, 4 or 8");
  if (n <= 0 || k <= 0 || k % 64 != 0) return soc::fail(SOC_ERR_INVALID, "soc_qmm: k must be a positive multiple of 64");
  if (static_cast<size_t>(mm) * k * 4 > 160 * 1024) return soc::fail(SOC_ERR_INVALID, "soc_qmm: m*k too large");
  soc::QmmArgs a{};
  a.x = static_cast<const f16*>(x);
  a.codes = codes;
  a.scales = static_cast<const f16*>(scales);
  a.y = y;
  a.M = mm;
  a.N = n;
  a.K = k;
  hipError_t e = soc::launch_qmm(a, bits, ctx->stream);
  return e == hipSuccess ? SOC_OK : hip_fail(e, "qmm");
}

int soc_dequant(soc_ctx* ctx, const void* codes, int32_t bits, const void* scales, float* w, int32_t n, int32_t k) {
  if (ctx == nullptr || codes == nullptr || scales == nullptr || w == nullptr)
    return soc::fail(SOC_ERR_INVALID, "null argument");
  if ((bits != 8 && bits != 4) || n <= 0 || k <= 0 || k % 64 != 0)
    return soc::fail(SOC_ERR_INVALID, "soc_dequant: bad shape or bits");
  hipError_t e = soc::launch_dequant(codes, bits, static_cast<const f16*>(scales), n, k, w, ctx->stream);
  return e == hipSuccess ? SOC_OK : hip_fail(e, "dequant");
}

}  // extern "C"

// ---- sampler (Mac/gpu/src/runtime/sampler.cpp:14-71) ----
int soc_sample_topk(soc_ctx* ctx, const float* row, int32_t vocab, int32_t top_k, float temperature,
                    int32_t* token_id, int32_t* top_ids, float* top_logits) {
  SOC_API_BEGIN
  if (ctx == nullptr || row == nullptr) return soc::fail(SOC_ERR_INVALID, "null argument");
  if (token_id == nullptr) return soc::fail(SOC_ERR_INVALID, "Sampler requires a non-null token_id output");
  if (vocab <= 0) return soc::fail(SOC_ERR_INVALID, "Sampler expects a non-empty logits row");
  // sampler.cpp:47-48: top_k clamped to [1, vocab]; a non-positive temperature means 1
  const int k = std::max(1, std::min(top_k, vocab));
  const float t = temperature <= 0.0f ? 1.0f : temperature;
  constexpr int kMaxOut = 4096;
  hipStream_t s = ctx->stream;
  hipError_t e;
  std::vector<int32_t> idx;
  std::vector<float> vals;
  // a row in pageable host memory is never handed to a kernel: it is sorted where it lies, as the reference does
  const soc::MemRange where = soc::classify_range(row, static_cast<size_t>(vocab) * 4);
  if (where == soc::MemRange::kOutside)
    return soc::fail(SOC_ERR_INVALID, "Sampler logits row extends past the end of its device allocation");
  bool whole_row = !soc::sample_device_fits(vocab, k) || where == soc::MemRange::kPageable;
  if (!whole_row) {
    const size_t need = soc::sample_ws_bytes(vocab);
    if (ctx->sample_ws_bytes < need) {
      if ((e = hipStreamSynchronize(s)) != hipSuccess) return hip_fail(e, "hipStreamSynchronize");
      (void)hipFree(ctx->sample_ws);
      ctx->sample_ws = nullptr;
      ctx->sample_ws_bytes = 0;
      if ((e = hipMalloc(&ctx->sample_ws, need)) != hipSuccess) return hip_fail(e, "hipMalloc sampler workspace");
      if ((e = hipMemset(ctx->sample_ws, 0, need)) != hipSuccess) {
        (void)hipFree(ctx->sample_ws);
        ctx->sample_ws = nullptr;
        return hip_fail(e, "hipMemset sampler workspace");
      }
      ctx->sample_ws_bytes = need;
    }
    constexpr size_t kOutInts = 2 + 2 * static_cast<size_t>(kMaxOut);
    if (ctx->sample_out == nullptr && (e = hipMalloc(&ctx->sample_out, kOutInts * sizeof(int))) != hipSuccess)
      return hip_fail(e, "hipMalloc sampler output");
    if (ctx->sample_host == nullptr &&
        (e = hipHostMalloc(reinterpret_cast<void**>(&ctx->sample_host), kOutInts * sizeof(int))) != hipSuccess)
      return hip_fail(e, "hipHostMalloc sampler output");
    if ((e = soc::launch_sample_topk(row, vocab, t, k, ctx->sample_ws, ctx->sample_out, kMaxOut, s)) != hipSuccess)
      return hip_fail(e, "sampler launch");
    // the head of the block first (it holds every candidate of a typical row), the rest only when needed
    constexpr int kHead = 512;
    const int* out = ctx->sample_host;
    if ((e = hipMemcpyAsync(ctx->sample_host, ctx->sample_out, (2 + 2 * kHead) * sizeof(int), hipMemcpyDeviceToHost,
                            s)) != hipSuccess)
      return hip_fail(e, "hipMemcpyAsync sampler");
    if ((e = hipStreamSynchronize(s)) != hipSuccess) return hip_fail(e, "sampler");
    const int n = out[0];
    if (out[1] != 0 || n > kMaxOut || n < k) {
      whole_row = true;  // NaN logits, or more candidates than the output block holds: the reference's full sort
    } else {
      if (n > kHead) {
        if ((e = hipMemcpyAsync(ctx->sample_host + 2 + 2 * kHead, ctx->sample_out + 2 + 2 * kHead,
                                static_cast<size_t>(n - kHead) * 2 * sizeof(int), hipMemcpyDeviceToHost, s)) !=
            hipSuccess)
          return hip_fail(e, "hipMemcpyAsync sampler");
        if ((e = hipStreamSynchronize(s)) != hipSuccess) return hip_fail(e, "sampler");
      }
      idx.resize(n);
      vals.resize(n);
      for (int j = 0; j < n; ++j) {
        idx[j] = out[2 + 2 * j];
        std::memcpy(&vals[j], &out[3 + 2 * j], 4);
      }
    }
  }
  if (whole_row) {
    vals.resize(vocab);
    if ((e = hipMemcpyAsync(vals.data(), row, static_cast<size_t>(vocab) * 4, hipMemcpyDefault, s)) != hipSuccess)
      return hip_fail(e, "hipMemcpyAsync logits row");
    if ((e = hipStreamSynchronize(s)) != hipSuccess) return hip_fail(e, "sampler");
    idx.resize(vocab);
    std::iota(idx.begin(), idx.end(), 0);
  }
  // the reference's partial sort, over the candidates in index order (the same comparisons on the same heap)
  std::vector<int32_t> order(idx.size());
  std::iota(order.begin(), order.end(), 0);
  std::partial_sort(order.begin(), order.begin() + k, order.end(),
                    [&vals, t](int32_t l, int32_t r) { return vals[l] / t > vals[r] / t; });
  *token_id = idx[order[0]];
  for (int r = 0; r < k; ++r) {
    if (top_ids) top_ids[r] = idx[order[r]];
    if (top_logits) top_logits[r] = vals[order[r]];
  }
  return SOC_OK;
  SOC_API_END
}
