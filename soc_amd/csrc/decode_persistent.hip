// decode_persistent.hip - one-launch decode step for batch 1: all layers, the LM head and the greedy argmax in a
// single persistent kernel with one 512-thread block per CU.
//
// Per layer the step has five dependent phases (reference: QwenBlock::ForwardCached, Mac/cpu/src/qwen_block.cpp:
// 63-73, with QwenAttention::ForwardCached and QwenMLP::Forward):
//   P1 RMSNorm(x) . Wqkv^T                                   every projection block, 1/NB of the rows
//   P2 q/k RMSNorm + RoPE + KV append + GQA attention        one block per KV head
//   P3 x' = x + Wo . attn                                    every projection block
//   P4 h = silu(RMSNorm(x') . Wg^T) * (RMSNorm(x') . Wu^T)   every projection block
//   P5 x'' = x' + Wd . h                                     every projection block
// Activations move between phases through small exchange vectors of 32-bit tagged words: the fp32 value rounded
// to 21 mantissa bits with a 2-bit phase tag in the two low bits (phase = (step - 1) * L + layer, mod 4). A reader
// spins until every element carries the expected tag. An aligned 4-byte store is single-copy atomic, so a value is
// never seen without its tag, and no barrier or cache flush is needed. Two bits are enough because every element is
// written once per phase and a producer can only reach phase p + 1 after every reader has consumed phase p (each
// phase needs all outputs of the one before it), so a reader waiting for phase p can find only phase p - 1 or p.
// Loads and stores of the exchange vectors are relaxed device-scope accesses (coherent across XCDs).
//
// Each block splits into seven compute waves and one receiver wave (wave 7). For the inputs that are RMSNorm-ed
// (P1, P4, the LM head) the receiver alone waits, applies the norm in its registers (or, in attention blocks, the
// per-head QK-RMSNorm + RoPE and the KV-cache append) and writes one of two LDS buffers; one block barrier then
// hands the buffer to the compute waves. The long inputs of P3 (q_dim elements) and P5 (I elements) are polled by
// all eight waves, each owning a share, which sees the last element sooner. Measured on MI355X: the receiver alone
// is faster for 1024 normed elements (one barrier instead of two), all waves for 2048 and more. The compute waves
// issue a layer's weight loads right after P1, in the order the phases consume them, so each phase waits only for
// its own rows. Every wait is bounded: on timeout the block raises an error flag and the whole grid drains.
#include <algorithm>

#include "exchange.h"
#include "kernels.h"

namespace soc {

namespace {

constexpr int NT = 512;          // threads per block
constexpr int NC = 448;          // compute threads: waves 0..6
constexpr int RECV = 7;          // receiver wave
constexpr int HD = 128;

// Receiver wave: elements i = lane + 64 e (e < MAXE) of a tagged vector, re-read until every one carries `tag`.
// `addr(i)` gives the source of element i < n. Returns false (wave-uniform) on timeout or a raised error flag.
template <int MAXE, typename Addr>
__device__ __forceinline__ bool recv_wait(uint32_t (&v)[MAXE], int n, uint32_t tag, Addr addr, int* err, int pause,
                                          uint64_t limit) {
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int e = 0; e < MAXE; ++e) {
    const int i = lane + 64 * e;
    v[e] = i < n ? ll_peek(addr(i)) : tag;
  }
  const uint64_t t0 = now_ticks();
  uint32_t spins = 0;
  while (true) {
    bool all = true;
#pragma unroll
    for (int e = 0; e < MAXE; ++e) all = all && tw_tag(v[e]) == tag;
    if (__all(all)) return true;
    if ((++spins & 63) == 0 && (now_ticks() - t0 > limit || err_raised(err))) {
      __hip_atomic_store(err, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      return false;
    }
    poll_pause(pause);
#pragma unroll
    for (int e = 0; e < MAXE; ++e) {
      const int i = lane + 64 * e;
      if (i < n && tw_tag(v[e]) != tag) v[e] = ll_peek(addr(i));
    }
  }
}

// Receiver: the tagged vector src[0..n) into dst; with NORM, RMSNorm-ed with `gain`
// (Mac/cpu/src/rms_norm_module.cpp:56-64: ms = sum x^2 / n; y = x * (1 / sqrt(ms + eps)) * g).
// Lane l polls the quads q = l + 64 e (elements 4q..4q+3) with one 16-byte load each; n is a multiple of 4.
template <int MAXQ, bool NORM>
__device__ __forceinline__ bool recv_vec(const uint32_t* src, int n, uint32_t tag, float* dst, const f16* gain,
                                         float eps, int* err, int pause, uint64_t limit) {
  const int lane = threadIdx.x & 63;
  const int nq = n / 4;
  f16x4 g[NORM ? MAXQ : 1];
  if constexpr (NORM) {
#pragma unroll
    for (int e = 0; e < MAXQ; ++e) {
      const int q = lane + 64 * e;
      g[e] = q < nq ? ld_global(reinterpret_cast<const f16x4*>(gain), q) : f16x4{0, 0, 0, 0};
    }
  }
  const __amdgpu_buffer_rsrc_t rsrc =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<uint32_t*>(src), 0, n * 4, 0x00020000);
  const u32x4 filler = {tag, tag, tag, tag};
  u32x4 v[MAXQ];
#pragma unroll
  for (int e = 0; e < MAXQ; ++e) v[e] = lane + 64 * e < nq ? ll_peek_buf4(rsrc, lane * 16 + 1024 * e) : filler;
  const uint64_t t0 = now_ticks();
  uint32_t spins = 0;
  bool ok = true;
  while (true) {
    bool all = true;
#pragma unroll
    for (int e = 0; e < MAXQ; ++e) all = all && tw_quad_ok(v[e], tag);
    if (__all(all)) break;
    if ((++spins & 63) == 0 && (now_ticks() - t0 > limit || err_raised(err))) {
      __hip_atomic_store(err, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      ok = false;
      break;
    }
    poll_pause(pause);
#pragma unroll
    for (int e = 0; e < MAXQ; ++e)
      if (lane + 64 * e < nq && !tw_quad_ok(v[e], tag)) v[e] = ll_peek_buf4(rsrc, lane * 16 + 1024 * e);
  }
  if (!ok) return false;
  float x[MAXQ][4];
#pragma unroll
  for (int e = 0; e < MAXQ; ++e) {
    x[e][0] = tw_val(v[e].x);
    x[e][1] = tw_val(v[e].y);
    x[e][2] = tw_val(v[e].z);
    x[e][3] = tw_val(v[e].w);
  }
  if constexpr (!NORM) {
#pragma unroll
    for (int e = 0; e < MAXQ; ++e) {
      const int q = lane + 64 * e;
      if (q < nq) *reinterpret_cast<f32x4*>(dst + 4 * q) = f32x4{x[e][0], x[e][1], x[e][2], x[e][3]};
    }
  } else {
    float ss = 0.0f;
#pragma unroll
    for (int e = 0; e < MAXQ; ++e)
      if (lane + 64 * e < nq) ss += x[e][0] * x[e][0] + x[e][1] * x[e][1] + x[e][2] * x[e][2] + x[e][3] * x[e][3];
    ss = wave_sum(ss);
    const float scale = 1.0f / sqrtf(ss / static_cast<float>(n) + eps);
#pragma unroll
    for (int e = 0; e < MAXQ; ++e) {
      const int q = lane + 64 * e;
      if (q < nq) {
        f32x4 y;
#pragma unroll
        for (int j = 0; j < 4; ++j) y[j] = x[e][j] * scale * static_cast<float>(g[e][j]);
        *reinterpret_cast<f32x4*>(dst + 4 * q) = y;
      }
    }
  }
  return true;
}

// Receiver, layer 0: the embedding row (embedding.cpp:51-77) RMSNorm-ed with the layer-0 input gain.
template <int MAXE>
__device__ __forceinline__ void recv_embed(const f16* row, int n, float* dst, const f16* gain, float eps) {
  const int lane = threadIdx.x & 63;
  float x[MAXE];
  float ss = 0.0f;
#pragma unroll
  for (int e = 0; e < MAXE; ++e) {
    const int i = lane + 64 * e;
    x[e] = i < n ? static_cast<float>(row[i]) : 0.0f;
    ss += x[e] * x[e];
  }
  ss = wave_sum(ss);
  const float scale = 1.0f / sqrtf(ss / static_cast<float>(n) + eps);
#pragma unroll
  for (int e = 0; e < MAXE; ++e) {
    const int i = lane + 64 * e;
    if (i < n) dst[i] = x[e] * scale * static_cast<float>(ld_global(gain, i));
  }
}

// A block's share of one weight matrix held in registers: slot s = threadIdx.x / TPR (threads < NC) owns row
// r0 + s; thread t of the slot holds the 8-half chunks at k = 8 (t + TPR c), c < CPT.
template <int TPR, int CPT>
struct Slice {
  u32x4 w[CPT];
};

template <int TPR, int CPT>
__device__ __forceinline__ void slice_load(Slice<TPR, CPT>& s, const f16* __restrict__ W, int K, int r0, int r1) {
  const int row = r0 + static_cast<int>(threadIdx.x) / TPR, t = threadIdx.x % TPR;
#pragma unroll
  for (int c = 0; c < CPT; ++c) {
    const int k = (t + TPR * c) * 8;
    s.w[c] = (row < r1 && k < K) ? load_stream16(W + static_cast<size_t>(row) * K + k) : u32x4{0, 0, 0, 0};
  }
}

// Row sum of the slot's row with xs[0..K) (TPR <= 64: the slot lives in one wave); every thread of the slot gets it.
template <int TPR, int CPT>
__device__ __forceinline__ float slice_dot(const Slice<TPR, CPT>& s, const float* xs, int K) {
  static_assert(TPR <= 64, "a slot must not span waves");
  const int t = threadIdx.x % TPR;
  float acc = 0.0f;
#pragma unroll
  for (int c = 0; c < CPT; ++c) {
    const int k = (t + TPR * c) * 8;
    if (k < K) {
      float wf[8], xv[8];
      f16x8_to_f32(s.w[c], wf);
      *reinterpret_cast<f32x4*>(xv) = *reinterpret_cast<const f32x4*>(xs + k);
      *reinterpret_cast<f32x4*>(xv + 4) = *reinterpret_cast<const f32x4*>(xs + k + 4);
#pragma unroll
      for (int i = 0; i < 8; ++i) acc += xv[i] * wf[i];
    }
  }
  return group_sum<TPR>(acc);
}

// Thread-per-row widths and chunk counts of each projection, sized for Qwen3-0.6B (H 1024, q_dim 2048, I 3072)
// over 248 projection blocks of 448 compute threads: up to 28 QKV rows, 7 hidden rows and 14 gate/up pairs per block.
constexpr int TPR_QKV = 16, CPT_QKV = 8;   // K = H
constexpr int TPR_O = 64, CPT_O = 4;       // K = q_dim
constexpr int TPR_GU = 32, CPT_GU = 4;     // K = H
constexpr int TPR_D = 64, CPT_D = 6;       // K = I
constexpr int TPR_LM = 32, CPT_LM = 4;     // LM head, NC / 32 = 14 rows per fragment
constexpr int MAXQ_H = 4;                 // receiver quads per lane: H <= 256 x MAXQ_H
constexpr int KCH = 224;                   // attention keys per chunk: 28 groups of 16 lanes x 8 keys

}  // namespace

// Optional phase timestamps (diagnostics): thread 0 of the first projection block and of the first attention block
// write the real-time counter at each phase boundary into trace[which][idx], idx < 4 + 8 L.
#define SOC_TRACE(idx)                                                                                   \
  do {                                                                                                   \
    if (c.a.trace != nullptr && threadIdx.x == 0) {                                                      \
      const uint64_t t_ = now_ticks();                                                                   \
      if (c.b == 0 || c.b == c.ng) c.a.trace[(c.b == 0 ? 0 : 1) * (4 + 8 * c.a.L) + (idx)] = t_;         \
      /* every block: the 8 points of the middle layer, after the two per-role rows */                   \
      if ((idx) >= 1 && ((idx) - 1) / 8 == c.a.L / 2)                                                    \
        c.a.trace[2 * (4 + 8 * c.a.L) + c.b * 8 + ((idx) - 1) % 8] = t_;                                 \
    }                                                                                                    \
  } while (0)

// Block barrier; afterwards every wave leaves if the receiver reported a failed wait (flag[0] != 0).
#define SOC_SYNC()                      \
  do {                                  \
    __syncthreads();                    \
    if (c.flag[0] != 0) return false;   \
  } while (0)

namespace {

// What every role of a block shares: the arguments, the step state and the LDS carve-up.
struct Ctx {
  const PersistArgs& a;
  int b, ng, token, pos;
  uint32_t phase0;  // (step - 1) * L: the tag of layer l is (phase0 + l) & 3
  float* xs0;   // [xs_cap] phase inputs, double buffered
  float* xs1;
  int* flag;    // [2] block-uniform status
  float* bv;    // [16] argmax values per slot
  int* bi;      // [16] argmax indices
  float* att;   // attention scratch
};

// Receiver wave reports a failed wait; the barrier that follows publishes it.
__device__ __forceinline__ void report(const Ctx& c, bool ok) {
  if (!ok && (threadIdx.x & 63) == 0) c.flag[0] = 1;
}

// ---------------- attention block (one KV head g): receiver wave ----------------
template <int G>
__device__ __forceinline__ bool attn_receiver(const Ctx& c, int g, float* qs, float* kn, float* vn) {
  const PersistArgs& a = c.a;
  const int lane = threadIdx.x & 63;
  for (int layer = 0; layer < a.L; ++layer) {
    const f16* W[9];  // in_norm, post_norm, q_norm, k_norm, wqkv, wo, wgate, wup, wdown
#pragma unroll
    for (int i = 0; i < 9; ++i) W[i] = ld_global(a.layer_w, static_cast<size_t>(layer) * 9 + i);
    const uint32_t tag = (c.phase0 + static_cast<uint32_t>(layer)) & 3u;
    f16* kb = a.kcache + static_cast<size_t>(layer) * a.layer_stride + static_cast<size_t>(g) * a.cap * HD;
    f16* vb = a.vcache + static_cast<size_t>(layer) * a.layer_stride + static_cast<size_t>(g) * a.cap * HD;
    // q heads, key and value of KV head g: (G + 2) x 128 tagged elements, two per lane per head
    constexpr int E = 2 * (G + 2);
    uint32_t v[E];
    const uint32_t* q_src = a.qkv + g * G * HD;
    const uint32_t* k_src = a.qkv + a.qd + g * HD;
    const uint32_t* v_src = a.qkv + a.qd + a.nkv * HD + g * HD;
    const float qg0 = static_cast<float>(ld_global(W[2], lane)), qg1 = static_cast<float>(ld_global(W[2], lane + 64));
    const float kg0 = static_cast<float>(ld_global(W[3], lane)), kg1 = static_cast<float>(ld_global(W[3], lane + 64));
    const float rc = a.rope_cos[static_cast<size_t>(c.pos) * (HD / 2) + lane];
    const float rs = a.rope_sin[static_cast<size_t>(c.pos) * (HD / 2) + lane];
    const bool ok = recv_wait<E>(v, E * 64, tag,
                                 [&](int i) {
                                   const int hidx = i / HD, d = i % HD;
                                   return hidx < G ? q_src + hidx * HD + d : (hidx == G ? k_src + d : v_src + d);
                                 },
                                 a.err, a.spin_sleep, a.spin_ticks);
    if (ok) {
      // per-head RMSNorm + rotate-half RoPE (qwen_attention.cpp:168-171; rope.cpp:81-84): lane holds dims
      // (lane, lane + 64) of each head; the key and value are rounded to fp16 and appended at `pos`
#pragma unroll
      for (int hh = 0; hh <= G; ++hh) {
        const float x0 = tw_val(v[2 * hh]), x1 = tw_val(v[2 * hh + 1]);
        const float ssum = wave_sum(x0 * x0 + x1 * x1);
        const float sc = 1.0f / sqrtf(ssum / static_cast<float>(HD) + a.eps);
        const float y0 = x0 * sc * (hh < G ? qg0 : kg0);
        const float y1 = x1 * sc * (hh < G ? qg1 : kg1);
        const float r0 = y0 * rc - y1 * rs;
        const float r1 = y0 * rs + y1 * rc;
        if (hh < G) {
          qs[hh * HD + lane] = r0;
          qs[hh * HD + lane + 64] = r1;
        } else {
          const f16 h0v = static_cast<f16>(r0), h1v = static_cast<f16>(r1);
          kb[static_cast<size_t>(c.pos) * HD + lane] = h0v;
          kb[static_cast<size_t>(c.pos) * HD + lane + 64] = h1v;
          kn[lane] = static_cast<float>(h0v);
          kn[lane + 64] = static_cast<float>(h1v);
        }
      }
      const f16 v0h = static_cast<f16>(tw_val(v[2 * G + 2])), v1h = static_cast<f16>(tw_val(v[2 * G + 3]));
      vb[static_cast<size_t>(c.pos) * HD + lane] = v0h;
      vb[static_cast<size_t>(c.pos) * HD + lane + 64] = v1h;
      vn[lane] = static_cast<float>(v0h);
      vn[lane + 64] = static_cast<float>(v1h);
    }
    report(c, ok);
    SOC_SYNC();                                    // inputs ready
    SOC_SYNC();                                    // partials
    SOC_SYNC();                                    // outputs stored; LDS free for the next layer
  }
  return true;
}

// ---------------- attention block: compute waves (28 groups of 16 lanes, 8 dims per lane) ----------------
// Flash-decoding inside the block (the online form of grouped_query_attention.cpp:105-136): every wave keeps its
// own running max, sum and weighted values over the keys its 4 groups own (key p of a chunk: group p % 28), in
// registers across all chunks; one barrier then merges the 7 waves: out = sum_w o_w e^(m_w - M) / sum_w l_w e^(m_w - M).
template <int G>
__device__ __forceinline__ bool attn_compute(const Ctx& c, int g, const float* qs, const float* kn, const float* vn) {
  const PersistArgs& a = c.a;
  const int tid = threadIdx.x, wid = tid >> 6, lane = tid & 63;
  const int sub = tid & 15, grp = tid >> 4;
  float* pred = c.att + G * HD + 2 * HD;   // [28][G][HD] group partial sums (scaled by the wave's max)
  float* wst = pred + (NC / 16) * G * HD;  // [7][G][2] wave max, wave sum
  const int pos = c.pos, S = pos + 1;
  u32x4 kreg[8], vreg[8];
  for (int layer = 0; layer < a.L; ++layer) {
    const uint32_t tag = (c.phase0 + static_cast<uint32_t>(layer)) & 3u;
    const f16* kb = a.kcache + static_cast<size_t>(layer) * a.layer_stride + static_cast<size_t>(g) * a.cap * HD;
    const f16* vb = a.vcache + static_cast<size_t>(layer) * a.layer_stride + static_cast<size_t>(g) * a.cap * HD;
    auto kv_fetch = [&](int c0) {
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        const int ap = c0 + grp + 28 * u;
        const bool ok = ap < pos;
        kreg[u] = ok ? load16(kb + static_cast<size_t>(ap) * HD + sub * 8) : u32x4{0, 0, 0, 0};
        vreg[u] = ok ? load16(vb + static_cast<size_t>(ap) * HD + sub * 8) : u32x4{0, 0, 0, 0};
      }
    };
    // cached keys/values of the first chunk do not depend on this layer's q/k/v: in flight before the wait
    kv_fetch(0);
    SOC_TRACE(1 + 8 * layer);
    SOC_SYNC();                                    // inputs ready
    SOC_TRACE(2 + 8 * layer);
    float qreg[G][8], acc[G][8], mw[G], lw[G];
#pragma unroll
    for (int j = 0; j < G; ++j) {
      mw[j] = -INFINITY;
      lw[j] = 0.0f;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        qreg[j][i] = qs[j * HD + sub * 8 + i];
        acc[j][i] = 0.0f;
      }
    }
    for (int c0 = 0; c0 < S; c0 += KCH) {
      const int n = min(KCH, S - c0);
      float sc[8][G];
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        const int p = grp + 28 * u;
        if (p < n) {
          float kf[8];
          if (c0 + p == pos) {
#pragma unroll
            for (int i = 0; i < 8; ++i) kf[i] = kn[sub * 8 + i];
          } else {
            f16x8_to_f32(kreg[u], kf);
          }
#pragma unroll
          for (int j = 0; j < G; ++j) {
            float d = 0.0f;
#pragma unroll
            for (int i = 0; i < 8; ++i) d += qreg[j][i] * kf[i];
            sc[u][j] = group_sum<16>(d) * a.scale;   // every lane of the group holds the key's score
          }
        } else {
#pragma unroll
          for (int j = 0; j < G; ++j) sc[u][j] = -INFINITY;
        }
      }
#pragma unroll
      for (int j = 0; j < G; ++j) {
        float mx = sc[0][j];
#pragma unroll
        for (int u = 1; u < 8; ++u) mx = fmaxf(mx, sc[u][j]);
        mx = wave_max(mx);
        const float mn = fmaxf(mw[j], mx);
        const float corr = mn == -INFINITY ? 1.0f : expf(mw[j] - mn);
        float ls = 0.0f;
#pragma unroll
        for (int u = 0; u < 8; ++u) {
          const float pw = sc[u][j] == -INFINITY ? 0.0f : expf(sc[u][j] - mn);
          sc[u][j] = pw;
          ls += pw;
        }
        // the 16 lanes of a group hold the same keys: the wave sum over 64 lanes counts each group 16 times
        lw[j] = lw[j] * corr + wave_sum(ls) * (1.0f / 16.0f);
        mw[j] = mn;
#pragma unroll
        for (int i = 0; i < 8; ++i) acc[j][i] *= corr;
      }
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        const int p = grp + 28 * u;
        if (p < n) {
          float vf[8];
          if (c0 + p == pos) {
#pragma unroll
            for (int i = 0; i < 8; ++i) vf[i] = vn[sub * 8 + i];
          } else {
            f16x8_to_f32(vreg[u], vf);
          }
#pragma unroll
          for (int j = 0; j < G; ++j)
#pragma unroll
            for (int i = 0; i < 8; ++i) acc[j][i] += sc[u][j] * vf[i];
        }
      }
      if (c0 + KCH < S) kv_fetch(c0 + KCH);
    }
    // group partials and the wave statistics, then one merge
#pragma unroll
    for (int j = 0; j < G; ++j)
#pragma unroll
      for (int i = 0; i < 8; ++i) pred[(grp * G + j) * HD + sub * 8 + i] = acc[j][i];
    if (lane == 0) {
#pragma unroll
      for (int j = 0; j < G; ++j) {
        wst[(wid * G + j) * 2] = mw[j];
        wst[(wid * G + j) * 2 + 1] = lw[j];
      }
    }
    SOC_SYNC();                                    // partials
    for (int idx = tid; idx < G * HD; idx += NC) {
      const int j = idx / HD, d = idx % HD;
      float M = -INFINITY;
#pragma unroll
      for (int w = 0; w < NC / 64; ++w) M = fmaxf(M, wst[(w * G + j) * 2]);
      float L = 0.0f, O = 0.0f;
#pragma unroll
      for (int w = 0; w < NC / 64; ++w) {
        const float m_w = wst[(w * G + j) * 2];
        if (m_w == -INFINITY) continue;          // a wave that owned no visible key
        const float e = expf(m_w - M);
        L += wst[(w * G + j) * 2 + 1] * e;
        float o = 0.0f;
#pragma unroll
        for (int q = 0; q < 4; ++q) o += pred[((w * 4 + q) * G + j) * HD + d];
        O += o * e;
      }
      ll_store(a.attn + (g * G + j) * HD + d, O / L, tag);
    }
    SOC_TRACE(3 + 8 * layer);
    SOC_SYNC();                                    // outputs stored; LDS free for the next layer
  }
  return true;
}

// ---------------- multi-wave receive (all eight waves; used where no wave has loads or stores in flight) -----
// Quads of the tagged vector src[0..n) are spread over the block's threads and go to dst; one block barrier
// follows. (A single polling wave sees the first data sooner, but more polling threads see the last element sooner
// when the vector is long; which wins is a per-phase measurement.)
__device__ __forceinline__ bool block_recv(const Ctx& c, const uint32_t* src, int n, uint32_t tag, float* dst) {
  constexpr int MQ = 2;  // quads per thread: n <= 4 x MQ x NT
  const int tid = threadIdx.x;
  const int nq = n / 4;
  const __amdgpu_buffer_rsrc_t rsrc =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<uint32_t*>(src), 0, n * 4, 0x00020000);
  const u32x4 filler = {tag, tag, tag, tag};
  u32x4 v[MQ];
#pragma unroll
  for (int e = 0; e < MQ; ++e) v[e] = tid + NT * e < nq ? ll_peek_buf4(rsrc, tid * 16 + NT * 16 * e) : filler;
  const uint64_t t0 = now_ticks();
  uint32_t spins = 0;
  bool ok = true;
  while (true) {
    bool all = true;
#pragma unroll
    for (int e = 0; e < MQ; ++e) all = all && tw_quad_ok(v[e], tag);
    if (__all(all)) break;
    if ((++spins & 63) == 0 && (now_ticks() - t0 > c.a.spin_ticks || err_raised(c.a.err))) {
      __hip_atomic_store(c.a.err, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      ok = false;
      break;
    }
    poll_pause(c.a.spin_sleep);
#pragma unroll
    for (int e = 0; e < MQ; ++e)
      if (tid + NT * e < nq && !tw_quad_ok(v[e], tag)) v[e] = ll_peek_buf4(rsrc, tid * 16 + NT * 16 * e);
  }
  if (!ok && (tid & 63) == 0) c.flag[0] = 1;
#pragma unroll
  for (int e = 0; e < MQ; ++e) {
    const int q = tid + NT * e;
    if (ok && q < nq)
      *reinterpret_cast<f32x4*>(dst + 4 * q) = f32x4{tw_val(v[e].x), tw_val(v[e].y), tw_val(v[e].z), tw_val(v[e].w)};
  }
  SOC_SYNC();
  return true;
}

// ---------------- projection block: receiver wave ----------------
__device__ __forceinline__ bool proj_receiver(const Ctx& c) {
  const PersistArgs& a = c.a;
  const int H = a.H;
  for (int layer = 0; layer < a.L; ++layer) {
    const f16* W[9];  // in_norm, post_norm, q_norm, k_norm, wqkv, wo, wgate, wup, wdown
#pragma unroll
    for (int i = 0; i < 9; ++i) W[i] = ld_global(a.layer_w, static_cast<size_t>(layer) * 9 + i);
    const uint32_t tag = (c.phase0 + static_cast<uint32_t>(layer)) & 3u;
    if (layer == 0) recv_embed<4 * MAXQ_H>(a.embed + static_cast<size_t>(c.token) * H, H, c.xs0, W[0], a.eps);
    else report(c, recv_vec<MAXQ_H, true>(a.xb, H, (tag - 1u) & 3u, c.xs0, W[0], a.eps, a.err, a.spin_sleep, a.spin_ticks));
    SOC_SYNC();                                    // P1 input
    if (!block_recv(c, a.attn, a.qd, tag, c.xs1)) return false;  // P3 input
    report(c, recv_vec<MAXQ_H, true>(a.xa, H, tag, c.xs0, W[1], a.eps, a.err, a.spin_sleep, a.spin_ticks));
    SOC_SYNC();                                    // P4 input (receiver alone: its first sight of the data is earliest)
    if (!block_recv(c, a.h, a.I, tag, c.xs1)) return false;      // P5 input
  }
  return true;
}

// ---------------- projection block: compute waves ----------------
__device__ __forceinline__ bool proj_compute(const Ctx& c) {
  const PersistArgs& a = c.a;
  const int tid = threadIdx.x;
  const int H = a.H, I = a.I, qd = a.qd, ng = c.ng, b = c.b;
  const int rq = (a.qkv_rows + ng - 1) / ng, q0 = b * rq, q1 = min(a.qkv_rows, q0 + rq);
  const int rh = (H + ng - 1) / ng, h0 = b * rh, h1 = min(H, h0 + rh);
  const int ri = (I + ng - 1) / ng, i0 = b * ri, i1 = min(I, i0 + ri);
  const int slot_q = tid / TPR_QKV, slot_h = tid / TPR_O, slot_i = tid / TPR_GU;
  const bool lead_q = (tid % TPR_QKV) == 0, lead_h = (tid % TPR_O) == 0, lead_i = (tid % TPR_GU) == 0;
  Slice<TPR_QKV, CPT_QKV> sq;
  Slice<TPR_O, CPT_O> so;
  Slice<TPR_GU, CPT_GU> sg, su;
  Slice<TPR_D, CPT_D> sd;
  // residual stream value of this slot's H-row; layer 0 starts from the embedding row (embedding.cpp:51-77)
  const int hrow = h0 + slot_h;
  float xres = hrow < h1 ? static_cast<float>(a.embed[static_cast<size_t>(c.token) * H + hrow]) : 0.0f;
  slice_load(sq, ld_global(a.layer_w, 4), H, q0, q1);
  SOC_TRACE(0);
  for (int layer = 0; layer < a.L; ++layer) {
    const f16* W[9];  // in_norm, post_norm, q_norm, k_norm, wqkv, wo, wgate, wup, wdown
#pragma unroll
    for (int i = 0; i < 9; ++i) W[i] = ld_global(a.layer_w, static_cast<size_t>(layer) * 9 + i);  // in_norm, post_norm, q_norm, k_norm, wqkv, wo, wgate, wup, wdown
    const uint32_t tag = (c.phase0 + static_cast<uint32_t>(layer)) & 3u;
    // ---- P1: RMSNorm + QKV projection ----
    SOC_SYNC();
    SOC_TRACE(1 + 8 * layer);
    {
      const float out = slice_dot(sq, c.xs0, H);
      const int row = q0 + slot_q;
      if (lead_q && row < q1) ll_store(a.qkv + row, out, tag);
    }
    // the layer's other weight rows, in the order the phases use them, then the next layer's QKV rows: they stream
    // while the attention blocks work
    slice_load(so, W[5], qd, h0, h1);
    slice_load(sg, W[6], H, i0, i1);
    slice_load(su, W[7], H, i0, i1);
    slice_load(sd, W[8], I, h0, h1);
    if (layer + 1 < a.L) slice_load(sq, ld_global(a.layer_w, static_cast<size_t>(layer + 1) * 9 + 4), H, q0, q1);
    if (a.trace != nullptr) __builtin_amdgcn_s_waitcnt(0);  // diagnostics: point 2 = the weight stream has landed
    SOC_TRACE(2 + 8 * layer);
    // ---- P3: o_proj + residual (the attention output is 2048 elements: every wave polls a share) ----
    if (!block_recv(c, a.attn, qd, tag, c.xs1)) return false;
    SOC_TRACE(3 + 8 * layer);
    {
      const float out = slice_dot(so, c.xs1, qd);
      xres = xres + out;
      if (lead_h && hrow < h1) ll_store(a.xa + hrow, xres, tag);
    }
    SOC_TRACE(4 + 8 * layer);
    // ---- P4: RMSNorm + gate/up + SwiGLU ----
    SOC_SYNC();
    SOC_TRACE(5 + 8 * layer);
    {
      const float og = slice_dot(sg, c.xs0, H);
      const float ou = slice_dot(su, c.xs0, H);
      const int row = i0 + slot_i;
      if (lead_i && row < i1) ll_store(a.h + row, silu_ref(og) * ou, tag);
    }
    SOC_TRACE(6 + 8 * layer);
    // ---- P5: down + residual ----
    if (!block_recv(c, a.h, I, tag, c.xs1)) return false;
    SOC_TRACE(7 + 8 * layer);
    {
      const float out = slice_dot(sd, c.xs1, I);
      xres = xres + out;
      if (lead_h && hrow < h1) ll_store(a.xb + hrow, xres, tag);
    }
    SOC_TRACE(8 + 8 * layer);
  }
  return true;
}

// ---------------- LM head: receiver wave gets the final hidden state ----------------
__device__ __forceinline__ bool lm_receiver(const Ctx& c) {
  const PersistArgs& a = c.a;
  const uint32_t last_tag = (c.phase0 + static_cast<uint32_t>(a.L) - 1u) & 3u;
  report(c, recv_vec<MAXQ_H, true>(a.xb, a.H, last_tag, c.xs0, a.final_norm, a.eps, a.err, a.spin_sleep, a.spin_ticks));
  SOC_SYNC();
  return true;
}

// ---------------- LM head: compute waves, this block's rows, best (value, index) per 32-lane slot ----------------
__device__ __forceinline__ bool lm_compute(const Ctx& c) {
  const PersistArgs& a = c.a;
  const int tid = threadIdx.x;
  const int slot32 = tid / 32;
  const bool lead32 = (tid % 32) == 0;
  const int rv = (a.V + static_cast<int>(gridDim.x) - 1) / static_cast<int>(gridDim.x);
  const int v0 = c.b * rv, v1 = min(a.V, v0 + rv);
  constexpr int STEP = NC / TPR_LM;  // rows per fragment
  Slice<TPR_LM, CPT_LM> f0, f1;
  slice_load(f0, a.lm_head, a.H, v0, v1);  // does not depend on the hidden state: in flight before the wait
  SOC_SYNC();
  SOC_TRACE(1 + 8 * a.L);
  float best = -INFINITY;
  int best_i = 0x7fffffff;
  auto consume = [&](const Slice<TPR_LM, CPT_LM>& f, int r0) {
    const float out = slice_dot(f, c.xs0, a.H);
    const int row = r0 + slot32;
    if (row < v1) {
      if (lead32 && a.logits != nullptr) a.logits[row] = out;
      if (out > best) {  // a slot's rows ascend: strict > keeps the lowest index
        best = out;
        best_i = row;
      }
    }
  };
  for (int r0 = v0; r0 < v1; r0 += 2 * STEP) {
    slice_load(f1, a.lm_head, a.H, r0 + STEP, v1);
    consume(f0, r0);
    slice_load(f0, a.lm_head, a.H, r0 + 2 * STEP, v1);
    consume(f1, r0 + STEP);
  }
  if (lead32) {
    c.bv[slot32] = best;
    c.bi[slot32] = best_i;
  }
  SOC_TRACE(2 + 8 * a.L);
  return true;
}

}  // namespace

// Block roles: blocks [0, ng) hold weight rows and run the projections (P1, P3, P4, P5); the last nkv blocks hold no
// weights and run attention for one KV head each (P2), prefetching the next layer's cached keys/values while the
// projections run. All blocks share the LM head. In every block wave 7 is the receiver, waves 0..6 compute; the two
// run separate loops with the same sequence of block barriers.
template <int G>
__global__ __launch_bounds__(NT) void k_decode_persistent(PersistArgs a) {
  extern __shared__ __attribute__((aligned(16))) float lds[];
  float* red = lds + 2 * a.xs_cap;
  const int tid = threadIdx.x, wid = tid >> 6, lane = tid & 63;
  const int ng = static_cast<int>(gridDim.x) - a.nkv;
  Ctx c{a, static_cast<int>(blockIdx.x), ng, a.state[0], a.state[1],
        (static_cast<uint32_t>(a.state[2]) - 1u) * static_cast<uint32_t>(a.L),
        lds, lds + a.xs_cap, reinterpret_cast<int*>(red + 16), red + 32, reinterpret_cast<int*>(red + 48), red + 96};
  // a launch queued behind a failed one leaves at once (the failed step did not advance the step count)
  if (tid == 0) c.flag[0] = err_raised(a.err) ? 1 : 0;
  __syncthreads();
  if (c.flag[0] != 0) return;
  const bool recv = wid == RECV;
  bool ok;
  if (c.b >= ng) {
    const int g = c.b - ng;
    float* qs = c.att;
    float* kn = qs + G * HD;
    float* vn = kn + HD;
    ok = recv ? attn_receiver<G>(c, g, qs, kn, vn) : attn_compute<G>(c, g, qs, kn, vn);
  } else {
    ok = recv ? proj_receiver(c) : proj_compute(c);
  }
  if (!ok) return;
  ok = recv ? lm_receiver(c) : lm_compute(c);
  if (!ok) return;

  // ---- greedy argmax over the blocks' candidates (sampler.cpp:26-61 with top_k = 1) ----
  __syncthreads();
  if (tid == 0) {
    float v = c.bv[0];
    int i = c.bi[0];
    for (int w = 1; w < NC / 32; ++w)
      if (c.bv[w] > v || (c.bv[w] == v && c.bi[w] < i)) {
        v = c.bv[w];
        i = c.bi[w];
      }
    st_dev(a.part_val + c.b, v);
    st_dev(a.part_idx + c.b, i);
    wait_mem();  // the block's candidate is visible device-wide before it is counted
    const int done = __hip_atomic_fetch_add(a.counter, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    c.flag[1] = (done == static_cast<int>(gridDim.x) - 1);
  }
  __syncthreads();
  if (c.flag[1] == 0) return;
  float v = -INFINITY;
  int i = 0x7fffffff;
  for (int q = tid; q < static_cast<int>(gridDim.x); q += NT) {
    const float pv = ld_dev(a.part_val + q);
    const int pi = ld_dev(a.part_idx + q);
    if (pv > v || (pv == v && pi < i)) {
      v = pv;
      i = pi;
    }
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    const float ov = __shfl_xor(v, off, kWave);
    const int oi = __shfl_xor(i, off, kWave);
    if (ov > v || (ov == v && oi < i)) {
      v = ov;
      i = oi;
    }
  }
  __syncthreads();
  if (lane == 0) {
    c.bv[wid] = v;
    c.bi[wid] = i;
  }
  __syncthreads();
  if (tid == 0) {
    for (int w = 1; w < NT / 64; ++w)
      if (c.bv[w] > c.bv[0] || (c.bv[w] == c.bv[0] && c.bi[w] < c.bi[0])) {
        c.bv[0] = c.bv[w];
        c.bi[0] = c.bi[w];
      }
    const int tok = c.bi[0] == 0x7fffffff ? 0 : c.bi[0];
    a.state[0] = tok;
    a.state[1] = c.pos + 1;
    a.state[2] += 1;
    if (a.ring != nullptr) {
      a.ring[*a.ring_pos] = tok;
      *a.ring_pos += 1;
    }
    __hip_atomic_store(a.counter, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
}
#undef SOC_SYNC
#undef SOC_TRACE

size_t persistent_lds_bytes(const PersistArgs& a, int G) {
  const size_t att = static_cast<size_t>(G) * HD + 2 * HD + (NC / 16) * G * HD + (NC / 64) * G * 2;
  return (2 * static_cast<size_t>(a.xs_cap) + 96 + att) * sizeof(float);
}

namespace {
template <int G>
hipError_t launch_g(const PersistArgs& a, int nblocks, size_t lds, hipStream_t s) {
  static size_t attr_lds = 0;
  if (attr_lds < lds) {
    hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(k_decode_persistent<G>),
                                       hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(lds));
    if (e != hipSuccess) return e;
    attr_lds = lds;
  }
  if (a.cooperative) {
    void* args[] = {const_cast<PersistArgs*>(&a)};
    return hipLaunchCooperativeKernel(reinterpret_cast<const void*>(k_decode_persistent<G>), dim3(nblocks), dim3(NT),
                                      args, static_cast<unsigned>(lds), s);
  }
  hipLaunchKernelGGL(k_decode_persistent<G>, dim3(nblocks), dim3(NT), lds, s, a);
  return hipGetLastError();
}
}  // namespace

hipError_t launch_decode_persistent(const PersistArgs& a, int nblocks, hipStream_t s) {
  const int G = a.nq / a.nkv;
  const size_t lds = std::max<size_t>(persistent_lds_bytes(a, G), 96 * 1024);  // >80 KB: one block per CU
  if (G == 1) return launch_g<1>(a, nblocks, lds, s);
  if (G == 2) return launch_g<2>(a, nblocks, lds, s);
  if (G == 4) return launch_g<4>(a, nblocks, lds, s);
  return hipErrorInvalidValue;
}

hipError_t persistent_blocks_per_cu(int G, int* blocks) {
  *blocks = 0;
  const size_t lds = 96 * 1024;
  if (G == 1) return hipOccupancyMaxActiveBlocksPerMultiprocessor(blocks, k_decode_persistent<1>, NT, lds);
  if (G == 2) return hipOccupancyMaxActiveBlocksPerMultiprocessor(blocks, k_decode_persistent<2>, NT, lds);
  if (G == 4) return hipOccupancyMaxActiveBlocksPerMultiprocessor(blocks, k_decode_persistent<4>, NT, lds);
  return hipErrorInvalidValue;
}

// Shapes the register tiling covers: K = hidden <= 1024, q_dim <= 2048, intermediate <= 3072; over the projection
// blocks (all but nkv) at most 28 QKV rows, 7 hidden rows and 14 gate/up pairs per block.
bool persistent_supported(int H, int qd, int I, int qkv_rows, int nq, int nkv, int nblocks) {
  const int G = nq / nkv;
  if (G != 1 && G != 2 && G != 4) return false;
  if (H > CPT_QKV * TPR_QKV * 8 || H > CPT_GU * TPR_GU * 8 || qd > CPT_O * TPR_O * 8 || I > CPT_D * TPR_D * 8)
    return false;
  if (H > 256 * MAXQ_H || qd > 8 * NT || I > 8 * NT) return false;
  if (H % 8 || qd % 8 || I % 8) return false;
  const int ng = nblocks - nkv;
  if (ng < 1) return false;
  auto rpb = [ng](int n) { return (n + ng - 1) / ng; };
  if (rpb(qkv_rows) > NC / TPR_QKV || rpb(I) > NC / TPR_GU || rpb(H) > NC / TPR_O) return false;
  return true;
}

}  // namespace soc
