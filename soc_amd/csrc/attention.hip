// attention.hip - per-head QK-RMSNorm + RoPE + KV-cache append, GQA causal attention over the fp16 KV cache in
// HBM (split over the key axis with a log-sum-exp combine), and the prefill row helpers (embedding, RMSNorm rows).
//
// Reference computation (batch 1, fp32): QwenAttention::ForwardCached (Mac/cpu/src/qwen_attention.cpp:142-205):
//   q,k,v projections -> q_norm/k_norm over each head's d features (:168-169) -> RoPE at the absolute position
//   (:170-171; rope.cpp:70-88) -> cache write (:180-193) -> GroupedQueryAttention with prefix = position offset
//   (grouped_query_attention.cpp:91-139): kv head = h / (nq/nkv), score = (q.k) * (1/sqrt(d)), softmax by
//   max-subtract and divide-by-sum, output = sum_j w_j v_j over the visible keys j <= position.
// Here the cache holds fp16 K/V in [slot][layer][kv_head][pos][d]; a new token's key and value are rounded to
// fp16 before use so that decode and prefill see identical keys.
#include "kernels.h"

#include <algorithm>
#include <cstdlib>

namespace soc {

namespace {

constexpr int HD = 128;  // head_dim handled by these kernels
constexpr int kMaxCombine = 160;  // key chunks one attention row may be split into (160 x 256 = 40960 keys)

}  // namespace

// grid = (nkv, max_split, B), block = 256 (4 waves). Each block: one KV head g, its G query heads, one batch row,
// one chunk of keys. The KV head is the fastest grid index: consecutive blocks go to consecutive XCDs (and
// alternate chunks to alternate shader engines), so with 8 KV heads XCD g serves head g and every XCD gets the same
// number of chunks however ragged the rows are. (With the chunk index fastest, rows of few chunks would load only
// the XCDs and shader engines that low chunk indices map to.)
template <int G, bool FUSED, int KH>
__global__ __launch_bounds__(256) void k_attention(AttnArgs a) {
  __shared__ float qs[G][HD];
  __shared__ float kn[HD], vn[HD];
  __shared__ float sc[G][256];
  __shared__ float red[4][G][HD];
  __shared__ float mstat[G], lstat[G];
  __shared__ float cm[G][kMaxCombine], cl[G][kMaxCombine];  // split combine: chunk maxima / weights, sums
  __shared__ int last;

  const int b = blockIdx.z, g = blockIdx.x, s = blockIdx.y;
  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
  const int qpos = (a.pos != nullptr ? a.pos[b] : b) + a.pos_base;
  const int S = qpos + 1;
  // up to 256 keys one block per (row, KV head) takes them all (no partials and no combine); longer rows use the
  // caller's chunk (single-sequence decode splits them finer than 256 for more blocks)
  const int chunk = S <= 256 ? 256 : a.chunk;
  const int nact = (S + chunk - 1) / chunk;
  if (s >= nact) return;
  const int slot = a.slot != nullptr ? a.slot[b] : a.slot_base;
  const size_t head_base = static_cast<size_t>(slot) * a.slot_stride + static_cast<size_t>(a.layer) * a.layer_stride +
                           static_cast<size_t>(g) * a.cap * HD;
  f16* kb = a.kcache + head_base;
  f16* vb = a.vcache + head_base;
  const float* row = a.qkv + static_cast<size_t>(b) * a.ld_qkv;
  const int c0 = s * chunk;
  const int n = min(chunk, S - c0);

  // The chunk's keys, as MFMA B operands: the wave's keys are 64 w .. 64 w + 63 of the chunk; lane (key kl, group kg)
  // = (lane % 16, lane / 16) holds the 16 bytes of dims 32 t + 8 kg of its key for t = 0..3, as stored (fp16 keys are
  // exact). Keys past the chunk's end load the last key (their scores are never stored), so the loads need no
  // branch. They are issued right after the query's own loads; loads complete in issue order, so the staging waits
  // for the query only and the keys stay in flight.
  const int kl = lane & 15, kg = lane >> 4;
  // KH = 2: the keys and the values in two halves each (half the registers, so more blocks per CU; a second round
  // trip for each)
  constexpr int T4H = 4 / KH, UH = 16 / KH;
  u32x4 raw[16 / KH];  // keys: [tile t4][dim step t] -> raw[4 (t4 % T4H) + t]; values: the row layout below
  // keys and values stream past the caches (each is read once per step: 4.05 -> 4.02 ms per Qwen3-4B x 16 ragged
  // step, 1.99 -> 1.98 ms per Qwen3-4B batch-1 token)
  auto kv_load = [](const f16* p) { return load_stream16(p); };
  auto load_keys = [&](int h) {
#pragma unroll
    for (int t4 = h * T4H; t4 < (h + 1) * T4H; ++t4) {
      const int p = min(64 * wid + 16 * t4 + kl, n - 1);
#pragma unroll
      for (int t = 0; t < 4; ++t)
        raw[4 * (t4 - h * T4H) + t] = kv_load(kb + static_cast<size_t>(c0 + p) * HD + 32 * t + 8 * kg);
    }
  };

  if constexpr (FUSED) {
    // The wave's rows vi = wid, wid + 4, ... of the G query heads, the key head and the value head (rows past G + 1
    // load row G + 1 again, unused), the q/k gains and the RoPE table row: all requested before the keys, and the
    // norms computed while the keys are in flight.
    constexpr int NV = (G + 2 + 3) / 4;
    float x0v[NV], x1v[NV];
#pragma unroll
    for (int t = 0; t < NV; ++t) {
      const int vi = min(wid + 4 * t, G + 1);
      const float* src = vi < G ? row + (g * G + vi) * HD : row + (vi == G ? a.nq : a.nq + a.nkv) * HD + g * HD;
      x0v[t] = src[lane];
      x1v[t] = src[lane + 64];
    }
    const float qg0 = static_cast<float>(a.q_gain[lane]), qg1 = static_cast<float>(a.q_gain[lane + 64]);
    const float kg0 = static_cast<float>(a.k_gain[lane]), kg1 = static_cast<float>(a.k_gain[lane + 64]);
    const float rc = a.rope_cos[static_cast<size_t>(qpos) * (HD / 2) + lane];
    const float rs = a.rope_sin[static_cast<size_t>(qpos) * (HD / 2) + lane];
    __builtin_amdgcn_sched_barrier(0);
    load_keys(0);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int t = 0; t < NV; ++t) {
      const int vi = wid + 4 * t;
      if (vi >= G + 2) break;  // wave-uniform
      float x0 = x0v[t], x1 = x1v[t];
      if (vi < G) {
        norm_rope_pair(x0, x1, qg0, qg1, a.eps, rc, rs);
        qs[vi][lane] = x0;
        qs[vi][lane + 64] = x1;
      } else if (vi == G) {
        norm_rope_pair(x0, x1, kg0, kg1, a.eps, rc, rs);
        const f16 h0 = static_cast<f16>(x0), h1 = static_cast<f16>(x1);
        kn[lane] = static_cast<float>(h0);
        kn[lane + 64] = static_cast<float>(h1);
        if (s == nact - 1) {
          kb[static_cast<size_t>(qpos) * HD + lane] = h0;
          kb[static_cast<size_t>(qpos) * HD + lane + 64] = h1;
        }
      } else {
        const f16 h0 = static_cast<f16>(x0), h1 = static_cast<f16>(x1);
        vn[lane] = static_cast<float>(h0);
        vn[lane + 64] = static_cast<float>(h1);
        if (s == nact - 1) {
          vb[static_cast<size_t>(qpos) * HD + lane] = h0;
          vb[static_cast<size_t>(qpos) * HD + lane + 64] = h1;
        }
      }
    }
  } else {
    constexpr int QN = (G * HD + 255) / 256;
    float qv[QN];
#pragma unroll
    for (int u = 0; u < QN; ++u) qv[u] = row[(g * G) * HD + min(tid + 256 * u, G * HD - 1)];
    __builtin_amdgcn_sched_barrier(0);
    load_keys(0);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int u = 0; u < QN; ++u) {
      const int i = tid + 256 * u;
      if (i < G * HD) qs[i / HD][i % HD] = qv[u];
    }
  }
  __syncthreads();

  const int sub = lane & 15, r = lane >> 4;

  // scores on matrix cores: D[row][key] = Q . K^T with v_mfma_f32_16x16x32_f16 over 16-key tiles, the keys loaded
  // above as B. The A operand rows are the G query heads as fp16 hi = f16(q) and, in rows G..2G-1,
  // lo = f16((q - hi) 2^11) (rows 2G..15 zero), so hi + lo 2^-11 carries about 22 bits of each fp32 query and the
  // score loses nothing a fp32 dot product would keep beyond the order of its sums.
  static_assert(2 * G <= 16, "hi and lo rows of the query heads fit one 16-row tile");
  f16x8 qa[4];  // A operand: row kl = query head kl (hi) or kl - G (lo), dims 32 t + 8 kg .. + 7
#pragma unroll
  for (int t = 0; t < 4; ++t) {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int d = 32 * t + 8 * kg + i;
      float v = 0.0f;
      if (kl < G) {
        v = qs[kl][d];
      } else if (kl < 2 * G) {
        const float x = qs[kl - G][d];
        v = (x - static_cast<float>(static_cast<f16>(x))) * 2048.0f;
      }
      qa[t][i] = static_cast<f16>(v);
    }
  }
#pragma unroll
  for (int t4 = 0; t4 < 4; ++t4) {
    if (64 * wid + 16 * t4 >= n) break;  // wave-uniform: no key of this tile is in the chunk
    if (KH == 2 && t4 == T4H) load_keys(1);
    const int ri = 4 * (t4 % T4H);
    const int p = 64 * wid + 16 * t4 + kl;
    if (FUSED && c0 + p == qpos) {  // the new key: from this kernel's own normed and roped copy
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        f16x8 kv;
#pragma unroll
        for (int i = 0; i < 8; ++i) kv[i] = static_cast<f16>(kn[32 * t + 8 * kg + i]);
        raw[ri + t] = __builtin_bit_cast(u32x4, kv);
      }
    }
    f32x4 d = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int t = 0; t < 4; ++t)
      d = __builtin_amdgcn_mfma_f32_16x16x32_f16(qa[t], __builtin_bit_cast(f16x8, raw[ri + t]), d, 0, 0, 0);
    // lane holds D rows 4 kg + i of key p: head j's score is row j + row (G + j) 2^-11
    if constexpr (G == 8) {
      f32x4 lo;
#pragma unroll
      for (int i = 0; i < 4; ++i) lo[i] = __shfl_xor(d[i], 32, kWave);
      if (kg < 2 && p < n)
#pragma unroll
        for (int i = 0; i < 4; ++i) sc[4 * kg + i][p] = (d[i] + lo[i] * (1.0f / 2048.0f)) * a.scale;
    } else if constexpr (G == 4) {
      f32x4 lo;
#pragma unroll
      for (int i = 0; i < 4; ++i) lo[i] = __shfl_xor(d[i], 16, kWave);
      if (kg == 0 && p < n)
#pragma unroll
        for (int i = 0; i < 4; ++i) sc[i][p] = (d[i] + lo[i] * (1.0f / 2048.0f)) * a.scale;
    } else {
      if (kg == 0 && p < n)
#pragma unroll
        for (int j = 0; j < G; ++j) sc[j][p] = (d[j] + d[G + j] * (1.0f / 2048.0f)) * a.scale;
    }
  }
  auto load_values = [&](int h) {  // (keys past the chunk's end load the last one, never used)
#pragma unroll
    for (int u = h * UH; u < (h + 1) * UH; ++u) {
      const int p = min(u * 16 + wid * 4 + r, n - 1);
      raw[u - h * UH] = kv_load(vb + static_cast<size_t>(c0 + p) * HD + sub * 8);
    }
  };
  load_values(0);
  __syncthreads();

  // softmax statistics per query head
  for (int j = wid; j < G; j += 4) {
    float m = -INFINITY;
    for (int p = lane; p < n; p += 64) m = fmaxf(m, sc[j][p]);
    m = wave_max(m);
    float l = 0.0f;
    for (int p = lane; p < n; p += 64) {
      const float w = expf(sc[j][p] - m);
      sc[j][p] = w;
      l += w;
    }
    l = wave_sum(l);
    if (lane == 0) {
      mstat[j] = m;
      lstat[j] = l;
    }
  }
  __syncthreads();

  // weighted sum of values
  float acc[G][8];
#pragma unroll
  for (int j = 0; j < G; ++j)
#pragma unroll
    for (int i = 0; i < 8; ++i) acc[j][i] = 0.0f;
#pragma unroll
  for (int u = 0; u < 16; ++u) {
    const int p = u * 16 + wid * 4 + r;
    if (u * 16 >= n) break;
    if (KH == 2 && u == UH) load_values(1);
    if (p < n) {
      float vf[8];
      if (FUSED && c0 + p == qpos) {
#pragma unroll
        for (int i = 0; i < 8; ++i) vf[i] = vn[sub * 8 + i];
      } else {
        f16x8_to_f32(raw[u % UH], vf);
      }
#pragma unroll
      for (int j = 0; j < G; ++j) {
        const float w = sc[j][p];
#pragma unroll
        for (int i = 0; i < 8; ++i) acc[j][i] += w * vf[i];
      }
    }
  }
#pragma unroll
  for (int j = 0; j < G; ++j)
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      float v = acc[j][i];
      v += __shfl_xor(v, 16, kWave);
      v += __shfl_xor(v, 32, kWave);
      acc[j][i] = v;
    }
  if (r == 0) {
#pragma unroll
    for (int j = 0; j < G; ++j)
#pragma unroll
      for (int i = 0; i < 8; ++i) red[wid][j][sub * 8 + i] = acc[j][i];
  }
  __syncthreads();

  if (nact == 1) {
    for (int idx = tid; idx < G * HD; idx += 256) {
      const int j = idx / HD, i = idx % HD;
      const float o = red[0][j][i] + red[1][j][i] + red[2][j][i] + red[3][j][i];
      a.out[static_cast<size_t>(b) * a.ld_out + (g * G + j) * HD + i] = o / lstat[j];
    }
    return;
  }
  // several chunks: write (o, m, l) partials; the last chunk block to arrive combines them
  const int stride = HD + 2;
  for (int idx = tid; idx < G * HD; idx += 256) {
    const int j = idx / HD, i = idx % HD;
    const float o = red[0][j][i] + red[1][j][i] + red[2][j][i] + red[3][j][i];
    float* p = a.part + ((static_cast<size_t>(b) * a.nq + g * G + j) * a.max_split + s) * stride;
    st_dev(p + i, o);
    if (i == 0) {
      st_dev(p + HD, mstat[j]);
      st_dev(p + HD + 1, lstat[j]);
    }
  }
  wait_mem();  // partials (device-scope stores) complete before this block is counted
  __syncthreads();
  if (tid == 0) {
    const int done = atomicAdd(a.counters + b * a.nkv + g, 1);
    last = (done == nact - 1);
  }
  __syncthreads();
  if (!last) return;  // the last block reads every partial with device-scope loads
  // combine: the first sixteen chunks' partial outputs of the thread's outputs and every chunk's (m, l) are
  // requested together (one memory round trip for up to 16 chunks); then the chunk weights, and the weighted sums
  // over chunks in chunk order (further chunks fetched sixteen at a time, no branch between the loads)
  constexpr int OPT = (G * HD + 255) / 256;  // outputs per thread
  float v0[OPT][16];
#pragma unroll
  for (int q = 0; q < OPT; ++q) {
    const int idx = min(tid + 256 * q, G * HD - 1);
    const float* p0 = a.part + (static_cast<size_t>(b) * a.nq + g * G + idx / HD) * a.max_split * stride + idx % HD;
#pragma unroll
    for (int u = 0; u < 16; ++u) v0[q][u] = ld_dev(p0 + min(u, nact - 1) * stride);
  }
  for (int idx = tid; idx < G * nact; idx += 256) {
    const int j = idx / nact, t = idx % nact;
    const float* pj = a.part + ((static_cast<size_t>(b) * a.nq + g * G + j) * a.max_split + t) * stride;
    cm[j][t] = ld_dev(pj + HD);
    cl[j][t] = ld_dev(pj + HD + 1);
  }
  __syncthreads();
  if (tid < G) {
    float M = -INFINITY;
    for (int t = 0; t < nact; ++t) M = fmaxf(M, cm[tid][t]);
    float L = 0.0f;
    for (int t = 0; t < nact; ++t) {
      const float e = expf(cm[tid][t] - M);
      cm[tid][t] = e;
      L += cl[tid][t] * e;
    }
    lstat[tid] = L;
  }
  __syncthreads();
#pragma unroll
  for (int q = 0; q < OPT; ++q) {
    const int idx = tid + 256 * q;
    if (idx >= G * HD) break;
    const int j = idx / HD, i = idx % HD;
    const float* p0 = a.part + (static_cast<size_t>(b) * a.nq + g * G + j) * a.max_split * stride + i;
    const float* ej = cm[j];
    float O = 0.0f;
#pragma unroll
    for (int u = 0; u < 16; ++u)
      if (u < nact) O += v0[q][u] * ej[u];
    for (int t = 16; t < nact; t += 16) {
      float v[16];
#pragma unroll
      for (int u = 0; u < 16; ++u) v[u] = ld_dev(p0 + min(t + u, nact - 1) * stride);
#pragma unroll
      for (int u = 0; u < 16; ++u)
        if (t + u < nact) O += v[u] * ej[t + u];
    }
    a.out[static_cast<size_t>(b) * a.ld_out + (g * G + j) * HD + i] = O / lstat[j];
  }
  if (tid == 0) st_dev(a.counters + b * a.nkv + g, 0);
}

// grid = (T, nq + nkv), block = 64: one wave per (row, head). q heads -> q_out; k heads -> cache (and v copy).
__global__ __launch_bounds__(64) void k_qk_norm_rope_append(QkNormRopeArgs a) {
  const int t = blockIdx.x, h = blockIdx.y, lane = threadIdx.x;
  const int pos = a.pos != nullptr ? a.pos[t] : a.pos_base + t;
  const int slot = a.slots != nullptr ? a.slots[t] : a.slot;
  const float* row = a.qkv + static_cast<size_t>(t) * a.ld_qkv;
  const float* cr = a.rope_cos + static_cast<size_t>(pos) * (HD / 2);
  const float* sr = a.rope_sin + static_cast<size_t>(pos) * (HD / 2);
  if (h < a.nq) {
    float x0 = row[h * HD + lane], x1 = row[h * HD + lane + 64];
    norm_rope_pair(x0, x1, a.q_gain, a.eps, cr, sr, lane);
    float* dst = a.q_out + static_cast<size_t>(t) * a.nq * HD + h * HD;
    dst[lane] = x0;
    dst[lane + 64] = x1;
  } else {
    const int g = h - a.nq;
    const float* ks = row + a.nq * HD + g * HD;
    const float* vs = row + (a.nq + a.nkv) * HD + g * HD;
    float x0 = ks[lane], x1 = ks[lane + 64];
    norm_rope_pair(x0, x1, a.k_gain, a.eps, cr, sr, lane);
    const size_t base = static_cast<size_t>(slot) * a.slot_stride + static_cast<size_t>(a.layer) * a.layer_stride +
                        static_cast<size_t>(g) * a.cap * HD + static_cast<size_t>(pos) * HD;
    a.kcache[base + lane] = static_cast<f16>(x0);
    a.kcache[base + lane + 64] = static_cast<f16>(x1);
    a.vcache[base + lane] = static_cast<f16>(vs[lane]);
    a.vcache[base + lane + 64] = static_cast<f16>(vs[lane + 64]);
  }
}

__global__ __launch_bounds__(256) void k_embed(const int32_t* ids, const f16* table, int H, float* x) {
  const int t = blockIdx.x;
  const f16* src = table + static_cast<size_t>(ids[t]) * H;
  for (int i = threadIdx.x; i < H; i += 256) x[static_cast<size_t>(t) * H + i] = static_cast<float>(src[i]);
}

// yh = f16(y); with ylo also set, ylo = f16((y - yh) * 2^11): the hi/lo activation pair of the MFMA GEMMs.
__global__ __launch_bounds__(256) void k_rmsnorm_rows(const float* x, int H, const f16* gain, float eps, float* yf,
                                                      f16* yh, f16* ylo) {
  __shared__ float red[4];
  const float* xr = x + static_cast<size_t>(blockIdx.x) * H;
  float ss = 0.0f;
  for (int i = threadIdx.x; i < H; i += 256) ss += xr[i] * xr[i];
  ss = block_sum<256>(ss, red);
  const float scale = 1.0f / sqrtf(ss / static_cast<float>(H) + eps);
  for (int i = threadIdx.x; i < H; i += 256) {
    const float y = xr[i] * scale * static_cast<float>(gain[i]);
    const size_t o = static_cast<size_t>(blockIdx.x) * H + i;
    if (yf) yf[o] = y;
    if (yh) {
      const f16 hi = static_cast<f16>(y);
      yh[o] = hi;
      if (ylo) ylo[o] = static_cast<f16>((y - static_cast<float>(hi)) * 2048.0f);
    }
  }
}

// One wave per row for H % 4 == 0 (4 rows per block): the row's 16-byte pieces i = lane + 64 e (e < MAXV) are all
// loaded before the sum of squares (per lane in e order, then across the wave); otherwise as k_rmsnorm_rows.
template <int MAXV>
__global__ __launch_bounds__(256) void k_rmsnorm_rows_v(const float* x, int T, int H, const f16* gain, float eps,
                                                        float* yf, f16* yh, f16* ylo) {
  const int t = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
  if (t >= T) return;
  const int nv = H / 4;
  const float* xr = x + static_cast<size_t>(t) * H;
  f32x4 v[MAXV];
  f16x4 gv[MAXV];  // the gains, requested with the row (no second round trip after the reduction)
  float ss = 0.0f;
#pragma unroll
  for (int e = 0; e < MAXV; ++e) {
    const int i = min(lane + 64 * e, nv - 1);
    v[e] = *reinterpret_cast<const f32x4*>(xr + 4 * i);  // pieces past the row reload its last one: zeroed below
    gv[e] = *reinterpret_cast<const f16x4*>(gain + 4 * i);
  }
#pragma unroll
  for (int e = 0; e < MAXV; ++e)
    if (lane + 64 * e >= nv) v[e] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
  for (int e = 0; e < MAXV; ++e)
#pragma unroll
    for (int c = 0; c < 4; ++c) ss += v[e][c] * v[e][c];
  ss = wave_sum(ss);
  const float scale = 1.0f / sqrtf(ss / static_cast<float>(H) + eps);
#pragma unroll
  for (int e = 0; e < MAXV; ++e) {
    const int i = lane + 64 * e;
    if (i >= nv) break;
    f32x4 y;
#pragma unroll
    for (int c = 0; c < 4; ++c) y[c] = v[e][c] * scale * static_cast<float>(gv[e][c]);
    const size_t o = static_cast<size_t>(t) * H + 4 * i;
    if (yf) *reinterpret_cast<f32x4*>(yf + o) = y;
    if (yh) {
      f16x4 hi, lo;
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        hi[c] = static_cast<f16>(y[c]);
        lo[c] = static_cast<f16>((y[c] - static_cast<float>(hi[c])) * 2048.0f);
      }
      *reinterpret_cast<f16x4*>(yh + o) = hi;
      if (ylo) *reinterpret_cast<f16x4*>(ylo + o) = lo;
    }
  }
}

__global__ __launch_bounds__(256) void k_split_f16(const float* x, size_t n, f16* hi, f16* lo) {
  for (size_t i = static_cast<size_t>(blockIdx.x) * 256 + threadIdx.x; i < n; i += static_cast<size_t>(gridDim.x) * 256) {
    const float v = x[i];
    const f16 h = static_cast<f16>(v);
    hi[i] = h;
    if (lo != nullptr) lo[i] = static_cast<f16>((v - static_cast<float>(h)) * 2048.0f);
  }
}

// ------------------------------------------------------------------------------------------------------------
// Causal GQA attention for a prefill chunk on MFMA (v_mfma_f32_32x32x16_f16), flash-style: one pass over the
// visible keys in tiles of 32 with an online softmax, K/V tiles staged through LDS (double buffered) and shared by
// the G query heads of a KV head.
//
// Each wave owns 32 query rows of one head. Scores are computed transposed, S^T[key][query] = K . Q^T, so that in
// the MFMA result layout (lane l holds rows (r/4)*8 + (l/32)*4 + r%4, r = 0..15, of column l%32) a lane owns one
// query's scores: the running max and sum stay in the lane, and only the lane pair (l, l^32) that splits a query's
// 32 keys exchanges its max. The same register file then feeds P^T as the B operand of O^T = V^T . P^T: the k index
// 8*(l/32)+i of that MFMA meets key (i/4)*8 + (l/32)*4 + i%4 of the 16-key step, so V^T is stored in LDS with key
// bits 2 and 3 swapped, which makes each lane's 8 keys one contiguous 16-byte LDS read.
//
// Precision: K and V are exact fp16 (the cache format). q (fp32) is split as hi = f16(q), lo = f16((q - hi) 2^11)
// into two accumulators; p = exp(s - m) in [0, 1] is split as hi + f16(p - hi) into the same accumulator. Both keep
// about 22 bits of the fp32 operand, so scores and weighted sums track the fp32 reference
// (grouped_query_attention.cpp:96-137) to fp32 rounding, with the order of the sums changed.
// grid = (ceil(B / (32 * 4 / G)), nkv), block = 256 (4 waves: head g*G + w%G, rows 32*(w/G) of the block's tile).
// ------------------------------------------------------------------------------------------------------------
namespace {
constexpr int FA_KT = 32;           // keys per tile
constexpr int FA_KLD = HD + 8;      // K tile row stride in halves (272 B: 8 consecutive rows hit disjoint banks)
constexpr int FA_VLD = FA_KT + 8;   // V^T tile row stride in halves (80 B)
typedef _Float16 fa_h8 __attribute__((ext_vector_type(8)));
__device__ __forceinline__ int fa_swizzle(int k) { return (k & ~12) | ((k & 4) << 1) | ((k & 8) >> 1); }
}  // namespace

template <int G>
__global__ __launch_bounds__(256, 2) void k_attention_prefill_mfma(AttnArgs a) {
  constexpr int SUB = 4 / G;     // 32-row sub-tiles per block
  constexpr int BP = 32 * SUB;   // query rows per block
  __shared__ _Float16 Ks[2][FA_KT * FA_KLD];
  __shared__ _Float16 Vt[2][HD * FA_VLD];
  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
  const int g = blockIdx.y;
  const int qt = gridDim.x - 1 - blockIdx.x;  // the longest (last) query tiles start first
  const int head = g * G + wid % G;
  const int t0 = qt * BP + (wid / G) * 32;    // first query row of this wave
  const int ql = lane & 31, hb = lane >> 5;
  const int t = t0 + ql;
  const int tq = min(t, a.B - 1);             // rows past the chunk compute a copy of the last row, never stored
  const int qpos = a.pos_base + tq;           // keys 0..qpos are visible to this row
  const int blk_last = a.pos_base + min(qt * BP + BP, a.B) - 1;
  const int ntiles = blk_last / FA_KT + 1;
  const int wtiles = t0 < a.B ? (a.pos_base + min(t0 + 31, a.B - 1)) / FA_KT + 1 : 0;
  const int nkeys = blk_last + 1;             // keys written to the cache so far that this block reads
  const size_t head_base = static_cast<size_t>(a.slot_base) * a.slot_stride +
                           static_cast<size_t>(a.layer) * a.layer_stride + static_cast<size_t>(g) * a.cap * HD;
  const f16* kb = a.kcache + head_base;
  const f16* vb = a.vcache + head_base;

  // Q^T operand: lane holds q[t][16 ks + 8 hb + i]
  fa_h8 qh[8], qlo[8];
  {
    const float* qrow = a.qkv + static_cast<size_t>(tq) * a.ld_qkv + head * HD;
#pragma unroll
    for (int ks = 0; ks < 8; ++ks) {
      const f32x4 v0 = *reinterpret_cast<const f32x4*>(qrow + ks * 16 + hb * 8);
      const f32x4 v1 = *reinterpret_cast<const f32x4*>(qrow + ks * 16 + hb * 8 + 4);
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const float v = t < a.B ? (i < 4 ? v0[i] : v1[i - 4]) : 0.0f;
        const _Float16 h = static_cast<_Float16>(v);
        qh[ks][i] = h;
        qlo[ks][i] = static_cast<_Float16>((v - static_cast<float>(h)) * 2048.0f);
      }
    }
  }

  // tile staging: 2 x (32 keys x 16 chunks of 8 dims) per thread pair; chunk c: key c % 32, dims 8 (c / 32)
  u32x4 rk[2], rv[2];
  auto load_tile = [&](int kt) {
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int c = tid + u * 256;
      const int key = kt * FA_KT + (c & 31);
      const size_t off = static_cast<size_t>(key) * HD + (c >> 5) * 8;
      rk[u] = key < nkeys ? load16(kb + off) : u32x4{0, 0, 0, 0};
      rv[u] = key < nkeys ? load16(vb + off) : u32x4{0, 0, 0, 0};
    }
  };
  auto store_tile = [&](int buf) {
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int c = tid + u * 256;
      const int key = c & 31, d0 = (c >> 5) * 8;
      *reinterpret_cast<u32x4*>(&Ks[buf][key * FA_KLD + d0]) = rk[u];
      const fa_h8 v = __builtin_bit_cast(fa_h8, rv[u]);
      const int col = fa_swizzle(key);
#pragma unroll
      for (int i = 0; i < 8; ++i) Vt[buf][(d0 + i) * FA_VLD + col] = v[i];
    }
  };

  f32x16 o[4];
#pragma unroll
  for (int db = 0; db < 4; ++db)
#pragma unroll
    for (int r = 0; r < 16; ++r) o[db][r] = 0.0f;
  // the online softmax runs in base 2: scores carry log2(e), so exp(s - m) = 2^(s' - m') is one v_exp_f32
  const float scale2 = a.scale * 1.4426950408889634f;
  const int wave_min_pos = a.pos_base + min(t0, a.B - 1);  // smallest query position among the wave's rows
  float m = -INFINITY, l = 0.0f;

  load_tile(0);
  store_tile(0);
  __syncthreads();
  for (int kt = 0; kt < ntiles; ++kt) {
    const int buf = kt & 1;
    if (kt + 1 < ntiles) load_tile(kt + 1);
    if (kt < wtiles) {
      f32x16 sh, sl;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        sh[r] = 0.0f;
        sl[r] = 0.0f;
      }
#pragma unroll
      for (int ks = 0; ks < 8; ++ks) {
        const fa_h8 ka = *reinterpret_cast<const fa_h8*>(&Ks[buf][ql * FA_KLD + ks * 16 + hb * 8]);
        sh = __builtin_amdgcn_mfma_f32_32x32x16_f16(ka, qh[ks], sh, 0, 0, 0);
        sl = __builtin_amdgcn_mfma_f32_32x32x16_f16(ka, qlo[ks], sl, 0, 0, 0);
      }
      // this lane: keys kt*32 + (r/4)*8 + hb*4 + r%4 of query row t
      float s[16];
      float mt = -INFINITY;
      if (kt * FA_KT + FA_KT - 1 <= wave_min_pos) {  // every key of the tile is visible to every row of the wave
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          s[r] = (sh[r] + sl[r] * (1.0f / 2048.0f)) * scale2;
          mt = fmaxf(mt, s[r]);
        }
      } else {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int key = kt * FA_KT + (r >> 2) * 8 + hb * 4 + (r & 3);
          const float v = (sh[r] + sl[r] * (1.0f / 2048.0f)) * scale2;
          s[r] = key <= qpos ? v : -INFINITY;
          mt = fmaxf(mt, s[r]);
        }
      }
      mt = fmaxf(mt, __shfl_xor(mt, 32));
      const float mn = fmaxf(m, mt);  // finite: key 0 is visible to every row and tile 0 comes first
      const float corr = __builtin_amdgcn_exp2f(m - mn);
      m = mn;
      l *= corr;
      if (!__all(corr == 1.0f)) {  // no row's running max moved: nothing to rescale
#pragma unroll
        for (int db = 0; db < 4; ++db)
#pragma unroll
          for (int r = 0; r < 16; ++r) o[db][r] *= corr;
      }
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        s[r] = __builtin_amdgcn_exp2f(s[r] - mn);
        l += s[r];
      }
#pragma unroll
      for (int k2 = 0; k2 < 2; ++k2) {
        fa_h8 ph, pl;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          const float p = s[k2 * 8 + i];
          ph[i] = static_cast<_Float16>(p);
          pl[i] = static_cast<_Float16>(p - static_cast<float>(ph[i]));
        }
#pragma unroll
        for (int db = 0; db < 4; ++db) {
          const fa_h8 va = *reinterpret_cast<const fa_h8*>(&Vt[buf][(db * 32 + ql) * FA_VLD + k2 * 16 + hb * 8]);
          o[db] = __builtin_amdgcn_mfma_f32_32x32x16_f16(va, ph, o[db], 0, 0, 0);
          o[db] = __builtin_amdgcn_mfma_f32_32x32x16_f16(va, pl, o[db], 0, 0, 0);
        }
      }
    }
    if (kt + 1 < ntiles) store_tile(buf ^ 1);
    __syncthreads();
  }

  const float lt = l + __shfl_xor(l, 32);
  if (t < a.B) {
    const size_t row = static_cast<size_t>(t) * a.ld_out + head * HD;
#pragma unroll
    for (int db = 0; db < 4; ++db)
#pragma unroll
      for (int r4 = 0; r4 < 4; ++r4) {
        f32x4 v;
#pragma unroll
        for (int i = 0; i < 4; ++i) v[i] = o[db][r4 * 4 + i] / lt;
        const size_t off = row + db * 32 + r4 * 8 + hb * 4;
        if (a.out != nullptr) *reinterpret_cast<f32x4*>(a.out + off) = v;
        if (a.out_hi != nullptr) {  // the hi/lo activation pair of the o projection
          f16x4 hi, lo;
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            hi[i] = static_cast<f16>(v[i]);
            lo[i] = static_cast<f16>((v[i] - static_cast<float>(hi[i])) * 2048.0f);
          }
          *reinterpret_cast<f16x4*>(a.out_hi + off) = hi;
          if (a.out_lo != nullptr) *reinterpret_cast<f16x4*>(a.out_lo + off) = lo;
        }
      }
  }
}

// ------------------------------------------------------------------------------------------------------------
// Causal GQA attention for a prefill chunk, balanced: a block takes two 32-row query tiles of one KV head, tile j
// and tile nqt - 1 - j, one after the other, so every block sees about the same number of visible keys. Its 8 waves
// are HB query heads (the whole group of the KV head) x R = 8 / HB key residues: key tile kt goes to the waves of
// residue kt % R, and each step stages R tiles. At the end of a query tile the R partial (max, sum, weighted values)
// of each row are merged through LDS: every wave owns 4 / R of the four 32-dimension blocks of its head's output and
// combines them from the other residues' partials, in residue order.
// The query rows (fp32) go global -> LDS with global_load_lds_dwordx4 together with the first key tiles, and when the
// merge area fits in the key/value ring the rows of the block's second query tile are requested while the first
// tile's keys are processed, so neither waits on a load of its own.
// Per tile a wave does what k_attention_prefill_mfma does (S^T = K . Q^T on MFMA, one query per lane, P^T straight
// from registers into O^T = V^T . P^T with V^T stored key-swizzled), with three changes:
//  * q is pre-multiplied by scale * log2(e) before its hi/lo split (lo = f16(q - hi), not rescaled), and both parts
//    accumulate into the same scores;
//  * the running max is lazy: it moves only when a score exceeds it by more than 8 (log2 units), so p <= 2^8 and
//    the 64 accumulators are rescaled rarely; the result is the same softmax (every partial keeps its own max and
//    the merge rescales exactly);
//  * p = hi + lo with hi = p with its low 13 mantissa bits cleared (exact in fp16 for p >= 2^-14) and lo = p - hi.
// K and V tiles go global -> LDS row-major with buffer_load_dwordx4 ... lds (32 rows x 256 B; 16-byte chunk c of
// row r at slot c ^ (r & 15) for K, c ^ 2 (r & 7) for V) and V^T operands come out of LDS through the transposing
// read ds_read_b64_tr_b16 (in each 16-lane group, lane j names 8 bytes = 4 dims of one key, and lane i receives dim
// i of 4 consecutive keys), so no register staging or transposed stores are needed. Keys past the chunk's last row
// read as zero (the buffer range ends there) and are masked (p = 0).
// grid = ceil(ceil(B / 32) / 2) * nkv blocks (block b: KV head b % nkv, so with 8 KV heads each XCD's L2 holds one
// head), block = 512, dynamic LDS = [key/value ring | query rows], with the merge area over the ring (and past it
// when it does not fit, in which case the query rows are not prefetched).
// ------------------------------------------------------------------------------------------------------------
namespace {
constexpr int FP_KD = FA_KT * HD;     // K or V tile in halves (row-major, swizzled)
typedef __fp16 fp_hv4 __attribute__((__vector_size__(4 * sizeof(__fp16))));  // operand type of the transposing read
typedef __attribute__((address_space(3))) void pa_lds_void;
template <int HB, int R>
struct PairsLds {
  static constexpr size_t ring = static_cast<size_t>(2) * R * 2 * FP_KD * sizeof(_Float16);  // [2][R] K, [2][R] V
  static constexpr size_t qrows = static_cast<size_t>(HB) * 32 * HD * sizeof(float);     // [HB][32 rows][128]
  // per head: the o blocks a wave does not own ([4 blocks][R - 1 writers][16][64 lanes]), then (max, sum) per
  // residue ([R][2][64])
  static constexpr size_t merge = static_cast<size_t>(HB) * (4 * (R - 1) * 16 + 2 * R) * 64 * sizeof(float);
  static constexpr bool prefetch_q = merge <= ring;
  static constexpr size_t bytes = ring + qrows > merge ? ring + qrows : merge;
};
// a barrier with no fence: global loads and stores stay in flight across it; the signal fences keep the compiler
// from moving LDS accesses across it
__device__ __forceinline__ void block_barrier() {
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  __builtin_amdgcn_s_barrier();
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
}
}  // namespace

// LOQ / LOP = false: q / p enter as single fp16 values (round to nearest) instead of hi/lo pairs (one MFMA chain
// fewer each).
template <int HB, int R, bool LOQ, bool LOP>
__global__ __launch_bounds__(512, 1) void k_attention_prefill_pairs(AttnArgs a) {
  static_assert(HB * R == 8, "8 waves");
  extern __shared__ __attribute__((aligned(16))) _Float16 plds[];
  _Float16* Ksb = plds;                  // [2][R][FP_KD]
  _Float16* Vb = plds + 2 * R * FP_KD;   // [2][R][FP_KD]
  float* xs = reinterpret_cast<float*>(plds);  // merge area, after the key loop
  float* qs = reinterpret_cast<float*>(plds + 4 * R * FP_KD);  // query rows [HB][32][32 chunks of 4]
  using Lds = PairsLds<HB, R>;
  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
  const int hh = wid % HB, res = wid / HB;
  const int g = static_cast<int>(blockIdx.x % a.nkv);
  const int head = g * HB + hh;
  const int ql = lane & 31, hb = lane >> 5;
  const int nqt = (a.B + 31) / 32;
  const int j = static_cast<int>(blockIdx.x / a.nkv);
  const size_t head_base = static_cast<size_t>(a.slot_base) * a.slot_stride +
                           static_cast<size_t>(a.layer) * a.layer_stride + static_cast<size_t>(g) * a.cap * HD;
  const f16* kb = a.kcache + head_base;
  const f16* vb = a.vcache + head_base;
  const float scale2 = a.scale * 1.4426950408889634f;
  // byte offsets of this lane's 16-byte chunk in a K / V tile: row 4 w + lane / 16, chunk slot lane % 16 holding
  // chunk (lane % 16) ^ (row % 16) of K and (lane % 16) ^ 2 (row % 8) of V
  const int krow = 4 * wid + (lane >> 4);
  const int koff = (krow * HD + (((lane & 15) ^ (krow & 15)) * 8)) * 2;
  const int voff = (krow * HD + (((lane & 15) ^ (2 * (krow & 7))) * 8)) * 2;
  // the rows of query tile qt for the block's HB heads -> qs; 16-byte chunk c of row r at slot c ^ r (conflict-free
  // reads of one chunk index by 32 rows). Instruction n of wave w fills rows 2 (w NI + n) and 2 (w NI + n) + 1.
  auto load_q = [&](int qt) {
    constexpr int NI = HB * 32 / 2 / 8;
    int ln = lane;
    __asm__ volatile("" : "+v"(ln));  // addresses computed here, not kept in registers across the key loop
#pragma unroll
    for (int n = 0; n < NI; ++n) {
      const int rr = 2 * (wid * NI + n) + (ln >> 5);
      const int h = rr / 32, r = rr % 32;
      const int c = (ln & 31) ^ r;
      const int tq = min(qt * 32 + r, a.B - 1);
      __builtin_amdgcn_global_load_lds(a.qkv + static_cast<size_t>(tq) * a.ld_qkv + (g * HB + h) * HD + c * 4,
                                       qs + (wid * NI + n) * 256, 16, 0, 0);
    }
  };

  for (int ph = 0; ph < 2; ++ph) {
    if (ph == 1 && nqt - 1 - j == j) break;  // odd tile count: the middle tile has no partner
    const int qt = ph == 0 ? j : nqt - 1 - j;
    const int t0 = qt * 32;
    const int t = t0 + ql;
    const int tq = min(t, a.B - 1);  // rows past the chunk compute a copy of the last row, never stored
    const int qpos = a.pos_base + tq;
    const int last = a.pos_base + min(t0 + 31, a.B - 1);  // last key any row of the tile sees
    const int ntiles = last / FA_KT + 1;
    const int nsteps = (ntiles + R - 1) / R;
    const int wave_min_pos = a.pos_base + t0;

    // K and V tiles of a step: wave w writes rows 4w..4w+3 of tile p through a buffer resource that starts at the
    // tile's first key and ends after key `last`, so rows past it read as zero (masked: p = 0) and the lane's byte
    // offset is the same for every tile (no per-step address arithmetic on the vector ALUs)
    auto load_step = [&](int step, int buf) {
#pragma unroll
      for (int p = 0; p < R; ++p) {
        const int key0 = (R * step + p) * FA_KT;
        const int nrec = max(0, last + 1 - key0) * HD * 2;
        const __amdgpu_buffer_rsrc_t rk =
            __builtin_amdgcn_make_buffer_rsrc(const_cast<f16*>(kb) + static_cast<size_t>(key0) * HD, 0, nrec, 0x00020000);
        const __amdgpu_buffer_rsrc_t rv =
            __builtin_amdgcn_make_buffer_rsrc(const_cast<f16*>(vb) + static_cast<size_t>(key0) * HD, 0, nrec, 0x00020000);
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rk, (pa_lds_void*)(Ksb + (buf * R + p) * FP_KD + 4 * wid * HD), 16,
                                                 koff, 0, 0, 0);
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rv, (pa_lds_void*)(Vb + (buf * R + p) * FP_KD + 4 * wid * HD), 16,
                                                 voff, 0, 0, 0);
      }
    };
    if (ph == 0 || !Lds::prefetch_q) load_q(qt);
    load_step(0, 0);
    __syncthreads();  // also waits for the tiles and the query rows (vmcnt)

    // Q^T operand (lane holds q[t][16 ks + 8 hb + i]) of q * scale * log2(e)
    fa_h8 qh[8], qlo[8];
    {
      const float* qrow = qs + (hh * 32 + ql) * HD;
#pragma unroll
      for (int ks = 0; ks < 8; ++ks) {
        const int c0 = 4 * ks + 2 * hb;
        const f32x4 v0 = *reinterpret_cast<const f32x4*>(qrow + (c0 ^ ql) * 4);
        const f32x4 v1 = *reinterpret_cast<const f32x4*>(qrow + ((c0 + 1) ^ ql) * 4);
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          float v = (i < 4 ? v0[i] : v1[i - 4]) * scale2;
          // keep the rounded fp32 product in a register: otherwise the compiler may fold the product into the
          // fp16 conversion of hi (one rounding) but not into lo, and hi + lo would no longer equal v
          __asm__ volatile("" : "+v"(v));
          const _Float16 h = static_cast<_Float16>(v);
          qh[ks][i] = h;
          if constexpr (LOQ) qlo[ks][i] = static_cast<_Float16>(v - static_cast<float>(h));
        }
      }
    }
    if (Lds::prefetch_q && ph == 0 && nqt - 1 - j != j) {
      block_barrier();  // every wave has read its query rows: the partner tile's rows go to the same place
      load_q(nqt - 1 - j);
    }
    // A operand of O^T = V^T . P^T for dims db*32.. and the 16-key step k2: lane (dim l % 32, hb) needs keys
    // hb*4 + 0..3 and 8 + hb*4 + 0..3 of the step (the key order of the P^T operand); 16-lane group grp covers dims
    // (grp & 1) * 16.. and keys (grp >> 1) * 4..
    const int grp = lane >> 4, jj = lane & 15;
    auto read_vt = [&](const _Float16* Vt, int db, int k2) {
      fa_h8 out;
#pragma unroll
      for (int half = 0; half < 2; ++half) {
        const int row = k2 * 16 + half * 8 + (grp >> 1) * 4 + (jj >> 2);
        const int dim = db * 32 + (grp & 1) * 16 + 4 * (jj & 3);
        const int slot = (dim >> 3) ^ (2 * (row & 7));
        const _Float16* p = Vt + row * HD + slot * 8 + (dim & 4);
        const fp_hv4 v = __builtin_amdgcn_ds_read_tr16_b64_v4f16(
            (__attribute__((address_space(3))) fp_hv4*)((__attribute__((address_space(3))) _Float16*)(p)));
        const f16x4 w = __builtin_bit_cast(f16x4, v);
#pragma unroll
        for (int q = 0; q < 4; ++q) out[half * 4 + q] = w[q];
      }
      return out;
    };

    f32x16 o[4];
#pragma unroll
    for (int db = 0; db < 4; ++db)
#pragma unroll
      for (int r = 0; r < 16; ++r) o[db][r] = 0.0f;
    float m = -INFINITY, l = 0.0f;

    for (int step = 0; step < nsteps; ++step) {
      const int buf = step & 1;
      if (step + 1 < nsteps) load_step(step + 1, buf ^ 1);
      const int kt = R * step + res;
      if (kt < ntiles) {
        const _Float16* Ks = Ksb + (buf * R + res) * FP_KD;
        const _Float16* Vt = Vb + (buf * R + res) * FP_KD;
        f32x16 sh;
#pragma unroll
        for (int r = 0; r < 16; ++r) sh[r] = 0.0f;
        // a wave's MFMA runs at raised priority: on a SIMD whose other wave is in its softmax, the matrix core then
        // takes this wave's MFMAs as they come while the other wave's VALU work fills the issue slots between them
        __builtin_amdgcn_s_setprio(1);
#pragma unroll
        for (int ks = 0; ks < 8; ++ks) {
          const fa_h8 ka = *reinterpret_cast<const fa_h8*>(&Ks[ql * HD + ((2 * ks + hb) ^ (ql & 15)) * 8]);
          sh = __builtin_amdgcn_mfma_f32_32x32x16_f16(ka, qh[ks], sh, 0, 0, 0);
          if constexpr (LOQ) sh = __builtin_amdgcn_mfma_f32_32x32x16_f16(ka, qlo[ks], sh, 0, 0, 0);
        }
        __builtin_amdgcn_s_setprio(0);
        // this lane: keys kt*32 + (r/4)*8 + hb*4 + r%4 of query row t
        float sv[16];
        float mt = -INFINITY;
        if (kt * FA_KT + FA_KT - 1 <= wave_min_pos) {  // every key of the tile is visible to every row
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            sv[r] = sh[r];
            mt = fmaxf(mt, sv[r]);
          }
        } else {
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const int key = kt * FA_KT + (r >> 2) * 8 + hb * 4 + (r & 3);
            sv[r] = key <= qpos ? sh[r] : -INFINITY;
            mt = fmaxf(mt, sv[r]);
          }
        }
        mt = fmaxf(mt, __shfl_xor(mt, 32));
        const bool up = mt > m + 8.0f;  // rows with no visible key yet keep m = -inf (and p = 0)
        if (__any(up)) {
          const float corr = up ? __builtin_amdgcn_exp2f(m - mt) : 1.0f;
          if (up) m = mt;
          l *= corr;
#pragma unroll
          for (int db = 0; db < 4; ++db)
#pragma unroll
            for (int r = 0; r < 16; ++r) o[db][r] *= corr;
        }
        const float mref = m == -INFINITY ? 0.0f : m;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          sv[r] = __builtin_amdgcn_exp2f(sv[r] - mref);
          l += sv[r];
        }
#pragma unroll
        for (int k2 = 0; k2 < 2; ++k2) {
          fa_h8 ph8, pl8;
#pragma unroll
          for (int i = 0; i < 8; i += 2) {
            const float p0 = sv[k2 * 8 + i], p1 = sv[k2 * 8 + i + 1];
            if constexpr (LOP) {
              const float h0 = __uint_as_float(__float_as_uint(p0) & 0xFFFFE000u);
              const float h1 = __uint_as_float(__float_as_uint(p1) & 0xFFFFE000u);
              const auto hv = __builtin_amdgcn_cvt_pkrtz(h0, h1);
              const auto lv = __builtin_amdgcn_cvt_pkrtz(p0 - h0, p1 - h1);
              ph8[i] = hv[0];
              ph8[i + 1] = hv[1];
              pl8[i] = lv[0];
              pl8[i + 1] = lv[1];
            } else {
              ph8[i] = static_cast<_Float16>(p0);
              ph8[i + 1] = static_cast<_Float16>(p1);
            }
          }
          __builtin_amdgcn_s_setprio(1);
#pragma unroll
          for (int db = 0; db < 4; ++db) {
            const fa_h8 va = read_vt(Vt, db, k2);
            o[db] = __builtin_amdgcn_mfma_f32_32x32x16_f16(va, ph8, o[db], 0, 0, 0);
            if constexpr (LOP) o[db] = __builtin_amdgcn_mfma_f32_32x32x16_f16(va, pl8, o[db], 0, 0, 0);
          }
          __builtin_amdgcn_s_setprio(0);
        }
      }
      __syncthreads();
    }

    // merge the R residues of each (head, row): wave (hh, res) owns the output blocks db with db % R == res and
    // parks the other blocks and its (max, sum) for their owners; each owner adds the partials in residue order
    const float lt = l + __shfl_xor(l, 32);
    float* mls = xs + HB * 4 * (R - 1) * 16 * 64;  // [HB][R][max, sum][64]
    mls[(hh * R + res) * 2 * 64 + lane] = m;
    mls[((hh * R + res) * 2 + 1) * 64 + lane] = lt;
#pragma unroll
    for (int db = 0; db < 4; ++db) {
      const int own = db % R;
      if (own != res) {
        float* dst = xs + ((hh * 4 + db) * (R - 1) + (res < own ? res : res - 1)) * 16 * 64 + lane;
#pragma unroll
        for (int r = 0; r < 16; ++r) dst[r * 64] = o[db][r];
      }
    }
    __syncthreads();
    {
      float mr[R], lr[R];
#pragma unroll
      for (int q = 0; q < R; ++q) {
        mr[q] = q == res ? m : mls[(hh * R + q) * 2 * 64 + lane];
        lr[q] = q == res ? lt : mls[((hh * R + q) * 2 + 1) * 64 + lane];
      }
      float M = mr[0];
#pragma unroll
      for (int q = 1; q < R; ++q) M = fmaxf(M, mr[q]);
      float cq[R];
      cq[0] = __builtin_amdgcn_exp2f(mr[0] - M);  // residue 0's max is finite: key 0 is in its first tile
#pragma unroll
      for (int q = 1; q < R; ++q) cq[q] = mr[q] == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(mr[q] - M);
      float L = lr[0] * cq[0];
#pragma unroll
      for (int q = 1; q < R; ++q) L += lr[q] * cq[q];
#pragma unroll
      for (int db = 0; db < 4; ++db) {
        if (db % R != res || t >= a.B) continue;
        const size_t row = static_cast<size_t>(t) * a.ld_out + head * HD;
#pragma unroll
        for (int r4 = 0; r4 < 4; ++r4) {
          f32x4 v;
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const int r = r4 * 4 + i;
            float x[R];
#pragma unroll
            for (int q = 0; q < R; ++q)
              x[q] = q == res ? o[db][r] : xs[(((hh * 4 + db) * (R - 1) + (q < res ? q : q - 1)) * 16 + r) * 64 + lane];
            float acc = x[0] * cq[0];
#pragma unroll
            for (int q = 1; q < R; ++q) acc += x[q] * cq[q];
            v[i] = acc / L;
          }
          const size_t off = row + db * 32 + r4 * 8 + hb * 4;
          if (a.out != nullptr) *reinterpret_cast<f32x4*>(a.out + off) = v;
          if (a.out_hi != nullptr) {  // the hi/lo activation pair of the o projection
            f16x4 hi, lo;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
              hi[i] = static_cast<f16>(v[i]);
              lo[i] = static_cast<f16>((v[i] - static_cast<float>(hi[i])) * 2048.0f);
            }
            *reinterpret_cast<f16x4*>(a.out_hi + off) = hi;
            if (a.out_lo != nullptr) *reinterpret_cast<f16x4*>(a.out_lo + off) = lo;
          }
        }
      }
    }
    // the merge area is the next query tile's staging area: every wave's reads of it have returned (the output
    // stores may still be in flight)
    __builtin_amdgcn_s_waitcnt(0xC07F);
    block_barrier();
  }
}


namespace {
template <int HB, bool LOQ, bool LOP>
hipError_t launch_pairs_lo(const AttnArgs& a, hipStream_t s) {
  constexpr int R = 8 / HB;
  constexpr size_t lds = PairsLds<HB, R>::bytes;
  static const hipError_t attr = hipFuncSetAttribute(
      reinterpret_cast<const void*>(k_attention_prefill_pairs<HB, R, LOQ, LOP>), hipFuncAttributeMaxDynamicSharedMemorySize,
      static_cast<int>(lds));
  if (attr != hipSuccess) return attr;
  const int nqt = (a.B + 31) / 32;
  hipLaunchKernelGGL((k_attention_prefill_pairs<HB, R, LOQ, LOP>), dim3(((nqt + 1) / 2) * a.nkv), dim3(512), lds, s, a);
  return hipGetLastError();
}
// SOC_PREFILL_ATTN_SPLIT=0: q and p as single fp16 values; =q: hi/lo for q only; =p: for p only
template <int HB>
hipError_t launch_pairs(const AttnArgs& a, hipStream_t s) {
  const char* e = std::getenv("SOC_PREFILL_ATTN_SPLIT");
  if (e != nullptr && e[0] == '0') return launch_pairs_lo<HB, false, false>(a, s);
  if (e != nullptr && e[0] == 'q') return launch_pairs_lo<HB, true, false>(a, s);
  if (e != nullptr && e[0] == 'p') return launch_pairs_lo<HB, false, true>(a, s);
  return launch_pairs_lo<HB, true, true>(a, s);
}
}  // namespace

hipError_t launch_attention_prefill_pairs(const AttnArgs& a, hipStream_t s) {
  const int G = a.nq / a.nkv;
  if (a.pos != nullptr || a.slot != nullptr || a.B <= 0 || a.nkv <= 0 || a.nq % a.nkv != 0) return hipErrorInvalidValue;
  if (a.ld_qkv % 4 != 0 || a.ld_out % 4 != 0) return hipErrorInvalidValue;
  if ((a.out_lo != nullptr && a.out_hi == nullptr) || (a.out == nullptr && a.out_hi == nullptr))
    return hipErrorInvalidValue;
  if (G == 2) return launch_pairs<2>(a, s);
  if (G == 4) return launch_pairs<4>(a, s);
  return hipErrorInvalidValue;
}

bool attention_prefill_pairs_supported(int nq, int nkv) { return nkv > 0 && nq % nkv == 0 && (nq / nkv == 2 || nq / nkv == 4); }

hipError_t launch_attention_prefill_mfma(const AttnArgs& a, hipStream_t s) {
  const int G = a.nq / a.nkv;
  if (a.pos != nullptr || a.slot != nullptr || a.B <= 0 || a.nq % a.nkv != 0) return hipErrorInvalidValue;
  if (a.ld_qkv % 4 != 0 || a.ld_out % 4 != 0) return hipErrorInvalidValue;
  if ((a.out_lo != nullptr && a.out_hi == nullptr) || (a.out == nullptr && a.out_hi == nullptr))
    return hipErrorInvalidValue;
#define SOC_FA_CASE(GG)                                                                        \
  if (G == GG) {                                                                               \
    const dim3 grid((a.B + 32 * (4 / GG) - 1) / (32 * (4 / GG)), a.nkv);                       \
    hipLaunchKernelGGL((k_attention_prefill_mfma<GG>), grid, dim3(256), 0, s, a);              \
    return hipGetLastError();                                                                  \
  }
  SOC_FA_CASE(1)
  SOC_FA_CASE(2)
  SOC_FA_CASE(4)
#undef SOC_FA_CASE
  return hipErrorInvalidValue;
}

bool attention_prefill_mfma_supported(int nq, int nkv) {
  return nkv > 0 && nq % nkv == 0 && (nq / nkv == 1 || nq / nkv == 2 || nq / nkv == 4);
}

hipError_t launch_attention(const AttnArgs& a, int fused, hipStream_t s) {
  const int G = a.nq / a.nkv;
  if (a.chunk > 256 || a.chunk <= 0) return hipErrorInvalidValue;
  if (a.max_split > kMaxCombine) return hipErrorInvalidValue;
  const dim3 grid(a.nkv, a.max_split, a.B), block(256);
  // unfused rows (the ragged batch): keys and values in halves, 88 instead of 112 registers, five blocks per CU
  // instead of four (Qwen3-4B x 16 ragged step 4.07 -> 4.04 ms); the fused single-sequence decode runs few blocks and
  // keeps the one round trip per operand
#define SOC_ATTN_CASE(GG)                                                                  \
  if (G == GG) {                                                                          \
    if (fused) hipLaunchKernelGGL((k_attention<GG, true, 1>), grid, block, 0, s, a);       \
    else hipLaunchKernelGGL((k_attention<GG, false, 2>), grid, block, 0, s, a);            \
    return hipGetLastError();                                                             \
  }
  SOC_ATTN_CASE(1)
  SOC_ATTN_CASE(2)
  SOC_ATTN_CASE(4)
  SOC_ATTN_CASE(8)
#undef SOC_ATTN_CASE
  return hipErrorInvalidValue;
}

hipError_t launch_qk_norm_rope_append(const QkNormRopeArgs& a, hipStream_t s) {
  hipLaunchKernelGGL(k_qk_norm_rope_append, dim3(a.T, a.nq + a.nkv), dim3(64), 0, s, a);
  return hipGetLastError();
}

hipError_t launch_embed(const int32_t* ids, int T, const f16* table, int H, float* x, hipStream_t s) {
  hipLaunchKernelGGL(k_embed, dim3(T), dim3(256), 0, s, ids, table, H, x);
  return hipGetLastError();
}

hipError_t launch_rmsnorm_rows(const float* x, int T, int H, const f16* gain, float eps, float* yf, f16* yh,
                               f16* ylo, hipStream_t s) {
  if (ylo != nullptr && yh == nullptr) return hipErrorInvalidValue;
  const int nv = H / 4;
  const bool vec = H % 4 == 0 && nv <= 64 * 32 &&
                   (reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(gain) | reinterpret_cast<uintptr_t>(yf) |
                    reinterpret_cast<uintptr_t>(yh) | reinterpret_cast<uintptr_t>(ylo)) % 16 == 0;
  if (!vec) {
    hipLaunchKernelGGL(k_rmsnorm_rows, dim3(T), dim3(256), 0, s, x, H, gain, eps, yf, yh, ylo);
    return hipGetLastError();
  }
  const dim3 grid((T + 3) / 4);
  if (nv <= 64 * 4) hipLaunchKernelGGL(k_rmsnorm_rows_v<4>, grid, dim3(256), 0, s, x, T, H, gain, eps, yf, yh, ylo);
  else if (nv <= 64 * 8) hipLaunchKernelGGL(k_rmsnorm_rows_v<8>, grid, dim3(256), 0, s, x, T, H, gain, eps, yf, yh, ylo);
  else if (nv <= 64 * 16) hipLaunchKernelGGL(k_rmsnorm_rows_v<16>, grid, dim3(256), 0, s, x, T, H, gain, eps, yf, yh, ylo);
  else hipLaunchKernelGGL(k_rmsnorm_rows_v<32>, grid, dim3(256), 0, s, x, T, H, gain, eps, yf, yh, ylo);
  return hipGetLastError();
}

hipError_t launch_split_f16(const float* x, size_t n, f16* hi, f16* lo, hipStream_t s) {
  const size_t blocks = std::min<size_t>((n + 255) / 256, 4096);
  hipLaunchKernelGGL(k_split_f16, dim3(static_cast<unsigned>(std::max<size_t>(blocks, 1))), dim3(256), 0, s, x, n, hi,
                     lo);
  return hipGetLastError();
}

}  // namespace soc
