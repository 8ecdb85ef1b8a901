// decode_persistent.hip - one-launch decode step for batch 1: all layers, the LM head and the greedy argmax in a
// single persistent kernel with one 512-thread block per CU.
//
// Per layer the step has five dependent phases (reference: QwenBlock::ForwardCached, Mac/cpu/src/qwen_block.cpp:
// 63-73, with QwenAttention::ForwardCached and QwenMLP::Forward):
//   P1 RMSNorm(x) . Wqkv^T                                   every block, 1/NB of the rows
//   P2 q/k RMSNorm + RoPE + KV append + GQA attention        one block per KV head
//   P3 x' = x + Wo . attn                                    every block
//   P4 h = silu(RMSNorm(x') . Wg^T) * (RMSNorm(x') . Wu^T)   every block
//   P5 x'' = x' + Wd . h                                     every block
// Activations move between phases through small exchange vectors written with 8-byte stores that carry the value
// and a tag unique to (step, layer): a reader spins until every element carries the expected tag. An aligned 8-byte
// store is single-copy atomic, so a value is never seen without its tag, and no barrier or cache flush is needed.
// Loads and stores of the exchange vectors are relaxed device-scope atomics (coherent across XCDs). Before waiting
// for a phase's input, a block issues the loads of everything that phase needs and that does not depend on the
// input (its weight rows, norm gains, RoPE factors, cached keys/values), so HBM streaming overlaps the hand-off.
// A block's rows are spread over all 512 threads (TPR threads per row). Every wait is bounded: on timeout the block
// raises an error flag and the whole grid drains.
#include "kernels.h"

namespace soc {

namespace {

constexpr int NT = 512;  // threads per block
constexpr int HD = 128;
constexpr uint64_t kSpinTicks = 20000000ull;  // 200 ms of the 100 MHz real-time counter per wait
constexpr int MAXG = 2;                       // norm-gain values held per thread (H <= 1024)

__device__ __forceinline__ uint64_t now_ticks() { return __builtin_amdgcn_s_memrealtime(); }

__device__ __forceinline__ void ll_store(uint64_t* p, float v, uint32_t tag) {
  const uint64_t u = (static_cast<uint64_t>(tag) << 32) | __float_as_uint(v);
  __hip_atomic_store(p, u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ uint64_t ll_peek(const uint64_t* p) {
  return __hip_atomic_load(const_cast<uint64_t*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ bool err_raised(int* err) {
  return __hip_atomic_load(err, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != 0;
}

// Up to three tagged ranges read into LDS in one polling loop: range r copies src[r][0..n[r]) to dst[r].
// Returns false (block-uniform) when the wait timed out or an error was raised somewhere in the grid.
struct LLRanges {
  const uint64_t* src[3];
  float* dst[3];
  int n[3];
  int count;
};

__device__ bool ll_read(const LLRanges& rg, uint32_t tag, int* err, int* flag) {
  constexpr int MAXE = 8;  // elements per thread per round
  int total = 0;
  for (int r = 0; r < rg.count; ++r) total += rg.n[r];
  bool ok = true;
  for (int base = 0; base < total && ok; base += NT * MAXE) {
    uint64_t v[MAXE];
    const uint64_t* sp[MAXE];
    float* dp[MAXE];
    bool done[MAXE];
    const int n0 = rg.n[0], n01 = rg.n[0] + (rg.count > 1 ? rg.n[1] : 0);
#pragma unroll
    for (int e = 0; e < MAXE; ++e) {
      const int i = base + e * NT + static_cast<int>(threadIdx.x);
      done[e] = i >= total;
      if (i < n0) {
        sp[e] = rg.src[0] + i;
        dp[e] = rg.dst[0] + i;
      } else if (i < n01) {
        sp[e] = rg.src[1] + (i - n0);
        dp[e] = rg.dst[1] + (i - n0);
      } else {
        sp[e] = rg.src[2] + (i - n01);
        dp[e] = rg.dst[2] + (i - n01);
      }
      v[e] = done[e] ? 0 : ll_peek(sp[e]);
    }
    const uint64_t t0 = now_ticks();
    uint32_t spins = 0;
    while (true) {
      bool all = true;
#pragma unroll
      for (int e = 0; e < MAXE; ++e) {
        if (!done[e]) {
          if (static_cast<uint32_t>(v[e] >> 32) == tag) {
            *dp[e] = __uint_as_float(static_cast<uint32_t>(v[e]));
            done[e] = true;
          } else {
            all = false;
          }
        }
      }
      if (all) break;
      if ((++spins & 63) == 0 && (now_ticks() - t0 > kSpinTicks || err_raised(err))) {
        __hip_atomic_store(err, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        ok = false;
        break;
      }
#pragma unroll
      for (int e = 0; e < MAXE; ++e)
        if (!done[e]) v[e] = ll_peek(sp[e]);
    }
  }
  if (threadIdx.x == 0) *flag = 0;
  __syncthreads();
  if (!ok) *flag = 1;
  __syncthreads();
  return *flag == 0;
}

__device__ __forceinline__ bool ll_read1(const uint64_t* src, int n, float* dst, uint32_t tag, int* err, int* flag) {
  LLRanges rg{};
  rg.src[0] = src;
  rg.dst[0] = dst;
  rg.n[0] = n;
  rg.count = 1;
  return ll_read(rg, tag, err, flag);
}

// A block's share of one weight matrix held in registers: slot s = threadIdx.x / TPR owns row r0 + s; thread t of the
// slot holds the 8-half chunks at k = 8 (t + TPR c), c < CPT.
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

// Row sum of the slot's row with xs[0..K); every thread of the slot gets it. TPR > 64 reduces through LDS
// (`part` holds NT / 64 floats) and synchronises the block.
template <int TPR, int CPT>
__device__ __forceinline__ float slice_dot(const Slice<TPR, CPT>& s, const float* xs, int K, float* part) {
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
  if constexpr (TPR <= 64) {
    return group_sum<TPR>(acc);
  } else {
    acc = wave_sum(acc);
    const int w = threadIdx.x >> 6, slot = threadIdx.x / TPR;
    if ((threadIdx.x & 63) == 0) part[w] = acc;
    __syncthreads();
    float sum = 0.0f;
#pragma unroll
    for (int i = 0; i < TPR / 64; ++i) sum += part[slot * (TPR / 64) + i];
    __syncthreads();
    return sum;
  }
}

// Norm gain values used by this thread (elements threadIdx.x + NT j).
struct Gains {
  float g[MAXG];
};

__device__ __forceinline__ void gains_load(Gains& gs, const f16* gain, int n) {
#pragma unroll
  for (int j = 0; j < MAXG; ++j) {
    const int i = threadIdx.x + NT * j;
    gs.g[j] = i < n ? static_cast<float>(gain[i]) : 0.0f;
  }
}

// RMSNorm of xs[0..n) in place (Mac/cpu/src/rms_norm_module.cpp:56-64): ms = sum x^2 / n; y = x * (1/sqrt(ms+eps)) * g.
__device__ __forceinline__ void rmsnorm_lds(float* xs, int n, const Gains& gs, float eps, float* red) {
  float ss = 0.0f;
#pragma unroll
  for (int j = 0; j < MAXG; ++j) {
    const int i = threadIdx.x + NT * j;
    if (i < n) ss += xs[i] * xs[i];
  }
  ss = block_sum<NT>(ss, red);
  const float scale = 1.0f / sqrtf(ss / static_cast<float>(n) + eps);
#pragma unroll
  for (int j = 0; j < MAXG; ++j) {
    const int i = threadIdx.x + NT * j;
    if (i < n) xs[i] = xs[i] * scale * gs.g[j];
  }
  __syncthreads();
}

__device__ __forceinline__ int rows_per_block(int n) { return (n + static_cast<int>(gridDim.x) - 1) / gridDim.x; }

// Thread-per-row widths and chunk counts of each projection, sized for Qwen3-0.6B (H 1024, q_dim 2048, I 3072)
// over 248 GEMV blocks: up to 32 QKV rows, 8 hidden rows and 16 gate/up pairs per block.
constexpr int TPR_QKV = 16, CPT_QKV = 8;   // K = H
constexpr int TPR_O = 64, CPT_O = 4;       // K = q_dim
constexpr int TPR_GU = 32, CPT_GU = 4;     // K = H
constexpr int TPR_D = 64, CPT_D = 6;       // K = I
constexpr int TPR_LM = 32, CPT_LM = 4;     // LM head, 16 rows per fragment

}  // namespace

// Optional phase timestamps (diagnostics): thread 0 of the first GEMV block and of the first attention block write
// the real-time counter at each phase boundary into trace[which][idx], idx < 3 + 5 L.
#define SOC_TRACE(idx)                                                                                   \
  do {                                                                                                   \
    if (a.trace != nullptr && threadIdx.x == 0 && (b == 0 || b == ng))                                   \
      a.trace[(b == 0 ? 0 : 1) * (3 + 5 * a.L) + (idx)] = now_ticks();                                   \
  } while (0)

// Block roles: blocks [0, ng) hold weight rows and run the projections (P1, P3, P4, P5); the last nkv blocks hold no
// weights and run attention for one KV head each (P2), prefetching the next layer's cached keys/values while the
// projections run. All blocks share the LM head.
template <int G>
__global__ __launch_bounds__(NT) void k_decode_persistent(PersistArgs a) {
  extern __shared__ float lds[];
  float* xs = lds;                                   // [max(H, qd, I)] staged input vector
  float* red = lds + a.xs_cap;                       // [16] block reductions
  int* flag = reinterpret_cast<int*>(red + 16);      // [1]  block-uniform status
  float* bv = red + 32;                              // [16] argmax values per slot
  int* bi = reinterpret_cast<int*>(red + 48);        // [16] argmax indices
  float* part = red + 64;                            // [16] cross-wave row sums
  float* att = red + 96;                             // attention scratch

  const int b = blockIdx.x;
  const int tid = threadIdx.x;
  const int token = a.state[0], pos = a.state[1];
  const uint32_t step = static_cast<uint32_t>(a.state[2]);
  const int H = a.H, I = a.I, qd = a.qd, qkv_rows = a.qkv_rows;
  const int ng = static_cast<int>(gridDim.x) - a.nkv;

  if (b >= ng) {
    // ================================ attention block ================================
    const int g = b - ng;
    float* qs = att;                       // [G][HD]
    float* kn = qs + G * HD;               // [HD]
    float* vn = kn + HD;                   // [HD]
    float* sc = vn + HD;                   // [G][256]
    float* pred = sc + G * 256;            // [8][G][HD] wave partials
    float* stat = pred + 8 * G * HD;       // [G] running max, [G] running sum, [G] correction
    const int wid = tid >> 6, lane = tid & 63;
    const int sub = tid & 15, grp = tid >> 4;  // 32 groups of 16 lanes, 8 dims per lane
    const bool normer = wid <= G;              // waves 0..G-1 normalise q heads, wave G the key
    const int S = pos + 1;
    u32x4 kreg[8], vreg[8];
    for (int layer = 0; layer < a.L; ++layer) {
      const f16* const* W = a.layer_w + layer * 9;
      const uint32_t tag = step * 64u + static_cast<uint32_t>(layer) + 1u;
      f16* kb = a.kcache + static_cast<size_t>(layer) * a.layer_stride + static_cast<size_t>(g) * a.cap * HD;
      f16* vb = a.vcache + static_cast<size_t>(layer) * a.layer_stride + static_cast<size_t>(g) * a.cap * HD;
      // everything that does not depend on this layer's q/k/v is loaded before waiting for them: the first 256-key
      // chunk of cached keys/values, the q/k norm gains and the RoPE factors of this position
      auto kv_fetch = [&](int c0) {
#pragma unroll
        for (int u = 0; u < 8; ++u) {
          const int ap = c0 + grp + 32 * u;
          const bool ok = ap < pos;
          kreg[u] = ok ? load16(kb + static_cast<size_t>(ap) * HD + sub * 8) : u32x4{0, 0, 0, 0};
          vreg[u] = ok ? load16(vb + static_cast<size_t>(ap) * HD + sub * 8) : u32x4{0, 0, 0, 0};
        }
      };
      kv_fetch(0);
      const f16* ngain = wid < G ? W[2] : W[3];
      float gn0 = 0.f, gn1 = 0.f, rc = 0.f, rs = 0.f;
      if (normer) {
        gn0 = static_cast<float>(ngain[lane]);
        gn1 = static_cast<float>(ngain[lane + 64]);
        rc = a.rope_cos[static_cast<size_t>(pos) * (HD / 2) + lane];
        rs = a.rope_sin[static_cast<size_t>(pos) * (HD / 2) + lane];
      }
      LLRanges rg{};
      rg.src[0] = a.qkv + g * G * HD;
      rg.dst[0] = qs;
      rg.n[0] = G * HD;
      rg.src[1] = a.qkv + qd + g * HD;
      rg.dst[1] = kn;
      rg.n[1] = HD;
      rg.src[2] = a.qkv + qd + a.nkv * HD + g * HD;
      rg.dst[2] = vn;
      rg.n[2] = HD;
      rg.count = 3;
      SOC_TRACE(1 + 5 * layer);
      if (!ll_read(rg, tag, a.err, flag)) return;
      SOC_TRACE(2 + 5 * layer);
      // per-head RMSNorm + RoPE (lane l holds dims l and l+64); the new key/value are rounded to fp16 and appended
      if (normer) {
        float* v = wid < G ? qs + wid * HD : kn;
        float x0 = v[lane], x1 = v[lane + 64];
        const float ss = wave_sum(x0 * x0 + x1 * x1);
        const float s = 1.0f / sqrtf(ss / static_cast<float>(HD) + a.eps);
        const float y0 = x0 * s * gn0;
        const float y1 = x1 * s * gn1;
        x0 = y0 * rc - y1 * rs;
        x1 = y0 * rs + y1 * rc;
        if (wid == G) {
          const f16 h0v = static_cast<f16>(x0), h1v = static_cast<f16>(x1);
          kb[static_cast<size_t>(pos) * HD + lane] = h0v;
          kb[static_cast<size_t>(pos) * HD + lane + 64] = h1v;
          x0 = static_cast<float>(h0v);
          x1 = static_cast<float>(h1v);
        }
        v[lane] = x0;
        v[lane + 64] = x1;
      } else if (wid == G + 1) {
        const f16 h0v = static_cast<f16>(vn[lane]), h1v = static_cast<f16>(vn[lane + 64]);
        vb[static_cast<size_t>(pos) * HD + lane] = h0v;
        vb[static_cast<size_t>(pos) * HD + lane + 64] = h1v;
        vn[lane] = static_cast<float>(h0v);
        vn[lane + 64] = static_cast<float>(h1v);
      }
      if (tid < G) {
        stat[tid] = -INFINITY;
        stat[G + tid] = 0.0f;
      }
      __syncthreads();
      float qreg[G][8];
#pragma unroll
      for (int j = 0; j < G; ++j)
#pragma unroll
        for (int i = 0; i < 8; ++i) qreg[j][i] = qs[j * HD + sub * 8 + i];
      float acc[G][8];
#pragma unroll
      for (int j = 0; j < G; ++j)
#pragma unroll
        for (int i = 0; i < 8; ++i) acc[j][i] = 0.0f;
      for (int c0 = 0; c0 < S; c0 += 256) {
        const int n = min(256, S - c0);
        // scores (grouped_query_attention.cpp:105-116); key p of the chunk lives in group p % 32, slot p / 32
#pragma unroll
        for (int u = 0; u < 8; ++u) {
          const int p = grp + 32 * u;
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
              d = group_sum<16>(d);
              if (sub == 0) sc[j * 256 + p] = d * a.scale;
            }
          }
        }
        __syncthreads();
        // running max / sum (online form of :113-122)
        if (wid < G) {
          const int j = wid;
          float m = -INFINITY;
          for (int p = lane; p < n; p += 64) m = fmaxf(m, sc[j * 256 + p]);
          m = wave_max(m);
          const float m_old = stat[j];
          const float m_new = fmaxf(m_old, m);
          float ssum = 0.0f;
          for (int p = lane; p < n; p += 64) {
            const float w = expf(sc[j * 256 + p] - m_new);
            sc[j * 256 + p] = w;
            ssum += w;
          }
          ssum = wave_sum(ssum);
          if (lane == 0) {
            const float corr = expf(m_old - m_new);
            stat[2 * G + j] = corr;
            stat[G + j] = stat[G + j] * corr + ssum;
            stat[j] = m_new;
          }
        }
        __syncthreads();
#pragma unroll
        for (int j = 0; j < G; ++j) {
          const float corr = stat[2 * G + j];
#pragma unroll
          for (int i = 0; i < 8; ++i) acc[j][i] *= corr;
        }
        // weighted values (:130-136)
#pragma unroll
        for (int u = 0; u < 8; ++u) {
          const int p = grp + 32 * u;
          if (p < n) {
            float vf[8];
            if (c0 + p == pos) {
#pragma unroll
              for (int i = 0; i < 8; ++i) vf[i] = vn[sub * 8 + i];
            } else {
              f16x8_to_f32(vreg[u], vf);
            }
#pragma unroll
            for (int j = 0; j < G; ++j) {
              const float w = sc[j * 256 + p];
#pragma unroll
              for (int i = 0; i < 8; ++i) acc[j][i] += w * vf[i];
            }
          }
        }
        if (c0 + 256 < S) kv_fetch(c0 + 256);
        __syncthreads();
      }
      // reduce the 4 key groups of a wave, then the 8 waves
#pragma unroll
      for (int j = 0; j < G; ++j)
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          float v = acc[j][i];
          v += __shfl_xor(v, 16, kWave);
          v += __shfl_xor(v, 32, kWave);
          acc[j][i] = v;
        }
      if ((lane >> 4) == 0) {
#pragma unroll
        for (int j = 0; j < G; ++j)
#pragma unroll
          for (int i = 0; i < 8; ++i) pred[(wid * G + j) * HD + sub * 8 + i] = acc[j][i];
      }
      __syncthreads();
      for (int idx = tid; idx < G * HD; idx += NT) {
        const int j = idx / HD, i = idx % HD;
        float o = 0.0f;
#pragma unroll
        for (int w = 0; w < NT / 64; ++w) o += pred[(w * G + j) * HD + i];
        ll_store(a.attn + (g * G + j) * HD + i, o / stat[G + j], tag);
      }
      SOC_TRACE(3 + 5 * layer);
      __syncthreads();
    }
  } else {
    // ================================ projection block ================================
    const int rq = (qkv_rows + ng - 1) / ng, q0 = b * rq, q1 = min(qkv_rows, q0 + rq);
    const int rh = (H + ng - 1) / ng, h0 = b * rh, h1 = min(H, h0 + rh);
    const int ri = (I + ng - 1) / ng, i0 = b * ri, i1 = min(I, i0 + ri);
    const int slot_q = tid / TPR_QKV, slot_h = tid / TPR_O, slot_i = tid / TPR_GU;
    const bool lead_q = (tid % TPR_QKV) == 0, lead_h = (tid % TPR_O) == 0, lead_i = (tid % TPR_GU) == 0;
    Slice<TPR_QKV, CPT_QKV> sq;
    Slice<TPR_O, CPT_O> so;
    Slice<TPR_GU, CPT_GU> sg, su;
    Slice<TPR_D, CPT_D> sd;
    Gains gin, gpost;
    // residual stream value of this slot's H-row; layer 0 starts from the embedding row (embedding.cpp:51-77)
    const int hrow = h0 + slot_h;
    float xres = hrow < h1 ? static_cast<float>(a.embed[static_cast<size_t>(token) * H + hrow]) : 0.0f;
    slice_load(sq, a.layer_w[4], H, q0, q1);
    gains_load(gin, a.layer_w[0], H);
    SOC_TRACE(0);

    for (int layer = 0; layer < a.L; ++layer) {
      const f16* const* W = a.layer_w + layer * 9;  // in_norm, post_norm, q_norm, k_norm, wqkv, wo, wgate, wup, wdown
      const uint32_t tag = step * 64u + static_cast<uint32_t>(layer) + 1u;

      // ---- P1: RMSNorm + QKV projection ----
      if (layer == 0) {
        for (int i = tid; i < H; i += NT) xs[i] = static_cast<float>(a.embed[static_cast<size_t>(token) * H + i]);
        __syncthreads();
      } else if (!ll_read1(a.xb, H, xs, tag - 1, a.err, flag)) {
        return;
      }
      rmsnorm_lds(xs, H, gin, a.eps, red);
      {
        const float out = slice_dot(sq, xs, H, part);
        const int row = q0 + slot_q;
        if (lead_q && row < q1) ll_store(a.qkv + row, out, tag);
      }
      // every remaining weight row of this layer and the next layer's QKV rows: the stream drains while the
      // attention blocks work, so the later polls of this layer wait behind nothing
      slice_load(so, W[5], qd, h0, h1);
      slice_load(sg, W[6], H, i0, i1);
      slice_load(su, W[7], H, i0, i1);
      slice_load(sd, W[8], I, h0, h1);
      gains_load(gpost, W[1], H);
      if (layer + 1 < a.L) {
        slice_load(sq, a.layer_w[(layer + 1) * 9 + 4], H, q0, q1);
        gains_load(gin, a.layer_w[(layer + 1) * 9 + 0], H);
      }
      SOC_TRACE(1 + 5 * layer);

      // ---- P3: o_proj + residual ----
      if (!ll_read1(a.attn, qd, xs, tag, a.err, flag)) return;
      SOC_TRACE(2 + 5 * layer);
      {
        const float out = slice_dot(so, xs, qd, part);
        xres = xres + out;
        if (lead_h && hrow < h1) ll_store(a.xa + hrow, xres, tag);
      }
      SOC_TRACE(3 + 5 * layer);

      // ---- P4: RMSNorm + gate/up + SwiGLU ----
      if (!ll_read1(a.xa, H, xs, tag, a.err, flag)) return;
      rmsnorm_lds(xs, H, gpost, a.eps, red);
      {
        const float og = slice_dot(sg, xs, H, part);
        const float ou = slice_dot(su, xs, H, part);
        const int row = i0 + slot_i;
        if (lead_i && row < i1) ll_store(a.h + row, silu_ref(og) * ou, tag);
      }
      SOC_TRACE(4 + 5 * layer);

      // ---- P5: down + residual ----
      if (!ll_read1(a.h, I, xs, tag, a.err, flag)) return;
      {
        const float out = slice_dot(sd, xs, I, part);
        xres = xres + out;
        if (lead_h && hrow < h1) ll_store(a.xb + hrow, xres, tag);
      }
      SOC_TRACE(5 + 5 * layer);
    }
  }

  // ---- final RMSNorm + LM head + greedy argmax (sampler.cpp:26-61 with top_k = 1), all blocks ----
  const int slot32 = tid / 32;
  const bool lead32 = (tid % 32) == 0;
  const uint32_t last_tag = step * 64u + static_cast<uint32_t>(a.L);
  const int rv = rows_per_block(a.V), v0 = b * rv, v1 = min(a.V, v0 + rv);
  constexpr int STEP = NT / TPR_LM;  // rows per fragment
  Slice<TPR_LM, CPT_LM> f0, f1;
  Gains gfin;
  slice_load(f0, a.lm_head, H, v0, v1);  // does not depend on the hidden state: issue before waiting for it
  gains_load(gfin, a.final_norm, H);
  if (!ll_read1(a.xb, H, xs, last_tag, a.err, flag)) return;
  SOC_TRACE(1 + 5 * a.L);
  rmsnorm_lds(xs, H, gfin, a.eps, red);
  float best = -INFINITY;
  int best_i = 0x7fffffff;
  auto consume = [&](const Slice<TPR_LM, CPT_LM>& f, int r0) {
    const float out = slice_dot(f, xs, H, part);
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
    slice_load(f1, a.lm_head, H, r0 + STEP, v1);
    consume(f0, r0);
    slice_load(f0, a.lm_head, H, r0 + 2 * STEP, v1);
    consume(f1, r0 + STEP);
  }
  SOC_TRACE(2 + 5 * a.L);
  __syncthreads();
  if (lead32) {
    bv[slot32] = best;
    bi[slot32] = best_i;
  }
  __syncthreads();
  if (tid == 0) {
    float v = bv[0];
    int i = bi[0];
    for (int w = 1; w < NT / 32; ++w)
      if (bv[w] > v || (bv[w] == v && bi[w] < i)) {
        v = bv[w];
        i = bi[w];
      }
    st_dev(a.part_val + b, v);
    st_dev(a.part_idx + b, i);
    __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): the partial is in memory before the arrival is counted
    const int done = __hip_atomic_fetch_add(a.counter, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    *flag = (done == static_cast<int>(gridDim.x) - 1);
  }
  __syncthreads();
  if (*flag == 0) return;
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
  if ((tid & 63) == 0) {
    bv[tid >> 6] = v;
    bi[tid >> 6] = i;
  }
  __syncthreads();
  if (tid == 0) {
    for (int w = 1; w < NT / 64; ++w)
      if (bv[w] > bv[0] || (bv[w] == bv[0] && bi[w] < bi[0])) {
        bv[0] = bv[w];
        bi[0] = bi[w];
      }
    const int tok = bi[0] == 0x7fffffff ? 0 : bi[0];
    a.state[0] = tok;
    a.state[1] = pos + 1;
    a.state[2] = static_cast<int>(step + 1);
    if (a.ring != nullptr) {
      a.ring[*a.ring_pos] = tok;
      *a.ring_pos += 1;
    }
    __hip_atomic_store(a.counter, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
}

size_t persistent_lds_bytes(const PersistArgs& a, int G) {
  const size_t att = static_cast<size_t>(G) * HD + 2 * HD + static_cast<size_t>(G) * 256 + 8 * G * HD + 3 * G;
  return (static_cast<size_t>(a.xs_cap) + 96 + att) * sizeof(float);
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
// blocks (all but nkv) at most 32 QKV rows, 8 hidden rows and 16 gate/up pairs per block.
bool persistent_supported(int H, int qd, int I, int qkv_rows, int nq, int nkv, int nblocks) {
  const int G = nq / nkv;
  if (G != 1 && G != 2 && G != 4) return false;
  if (H > CPT_QKV * TPR_QKV * 8 || H > CPT_GU * TPR_GU * 8 || qd > CPT_O * TPR_O * 8 || I > CPT_D * TPR_D * 8)
    return false;
  if (H > MAXG * NT) return false;
  if (H % 8 || qd % 8 || I % 8) return false;
  const int ng = nblocks - nkv;
  if (ng < 1) return false;
  auto rpb = [ng](int n) { return (n + ng - 1) / ng; };
  if (rpb(qkv_rows) > NT / TPR_QKV || rpb(I) > NT / TPR_GU || rpb(H) > NT / TPR_O) return false;
  return true;
}

}  // namespace soc
