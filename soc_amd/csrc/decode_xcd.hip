// decode_xcd.hip - one-launch decode step for batch 1 with every layer partitioned over the eight XCDs of MI355X, the
// layers alternating between two groups of blocks.
//
// Block (g, j): XCD g, read from the XCC_ID hardware register, and rank j < 32 among the blocks of this launch that
// arrived on it. Group p = j / 16 computes the layers l with l % 2 == p while the other group streams the weight rows
// of its next layer into registers: a CU never waits on hand-offs while its own weight loads are in flight (its
// vector memory requests would queue behind them). XCD g owns KV head g (every Qwen3 model has 8 KV heads) with its
// G = nq / 8 query heads and 1/8 of every matrix: the q/k/v rows of its heads, the o_proj columns of its query heads,
// the gate/up rows and down_proj columns of its eighth of the intermediate dimension; the group's 16 blocks of the
// XCD split that share. Per layer (reference: QwenBlock::ForwardCached, Mac/cpu/src/qwen_block.cpp:63-73, with
// QwenAttention::ForwardCached and QwenMLP::Forward):
//   A  x = x' + sum_k D_k: the previous layer's residual and its eight XCDs' partial down outputs (cross-XCD), RMSNorm
//   B  the block's q/k/v rows of the XCD's heads                                   -> XCD-local exchange
//   C  the XCD's q/k/v; per-head QK-RMSNorm + RoPE; rank 0 appends k and v to the cache
//   D  causal attention over the block's share of the keys; the 32 lane groups' partials merged in LDS
//   E  the XCD's block partials (XCD-local), log-sum-exp merge
//   F  O_g = Wo[the block's rows][the XCD's query columns] . attn                  -> cross-XCD exchange
//   G  x' = x + sum_k O_k (cross-XCD), RMSNorm; the block publishes its rows of x' for the other group
//   H  h = silu(gate) * up on the block's share of the XCD's intermediate slice     -> XCD-local exchange
//   I  the XCD's h slice (XCD-local)
//   J  D_g = Wd[the block's rows][the slice's columns] . h                         -> cross-XCD exchange
// Cross-XCD words are written with device-scope stores; XCD-local ones with plain stores served by the XCD's own L2
// (see exchange.h). Every block of the computing group holds the whole residual stream in LDS, computed in the same
// order from the same words, so all blocks hold identical bits. All eight waves of a block poll, compute and hold
// weight rows. Every wait is bounded; a timeout raises the error flag and the grid drains.
#include <algorithm>

#include "exchange.h"
#include "kernels.h"

namespace soc {

namespace {

constexpr int NT = 512;   // threads per block
constexpr int HD = 128;   // head dim
constexpr int NX = kXcdGroups, NBX = kXcdBlocks;
constexpr int NBG = NBX / 2;      // blocks of one group on one XCD
constexpr int HMAX = 1024;        // hidden size covered by the register tiling
constexpr int IMAX = 3072;        // intermediate size covered: I / 128 <= 24 gate/up pairs per block
constexpr int PW = HD + 4;        // words per (block, query head) attention partial: 128 values, max, sum, 2 pad
constexpr int NGRP = NT / 16;     // attention lane groups per block (16 lanes, 8 dims each)
constexpr int KPG = 8;            // keys per lane group when every block takes all keys (S <= NGRP * KPG)
constexpr float kNoKeys = -1e30f; // running max of a group that owns no key (finite: a tag bit must not make a NaN)

// A block's rows of one weight matrix in registers: slot s = tid / TPR owns one row; thread t of the slot holds the
// 8-half chunks at k = 8 (t + TPR c), c < CPT.
template <int TPR, int CPT>
struct Slice {
  u32x4 w[CPT];
};

template <int TPR, int CPT>
__device__ __forceinline__ void slice_load(Slice<TPR, CPT>& s, const f16* row, int K) {
  const int t = threadIdx.x % TPR;
#pragma unroll
  for (int c = 0; c < CPT; ++c) {
    const int k = (t + TPR * c) * 8;
    s.w[c] = (row != nullptr && k < K) ? load_stream16(row + k) : u32x4{0, 0, 0, 0};
  }
}

// Row sum of the slot's row with xs[0..K); every thread of the slot gets it.
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

// A block of `rows` rows of `K` halves (row r at src + r * ld) straight to LDS (dst[r * K ..]) with 16-byte
// global -> LDS loads, one 1 KB wave instruction per 64 chunks; waves w < 8 take every eighth instruction.
__device__ __forceinline__ void rows_to_lds(const f16* src, size_t ld, int rows, int K, f16* dst) {
  const int wid = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int cpr = K / 8, nch = rows * cpr;
  for (int c0 = wid * 64; c0 < nch; c0 += 512) {
    const int ch = min(c0 + lane, nch - 1), row = ch / cpr, col = ch % cpr;
    __builtin_amdgcn_global_load_lds(src + static_cast<size_t>(row) * ld + col * 8,
                                     (__attribute__((address_space(3))) void*)(dst + c0 * 8), 16, 0, 0);
  }
}

// Row sum of an LDS row (K halves) with xs[0..K): TPR threads per row, thread t takes the chunks t + TPR c.
template <int TPR, int CPT>
__device__ __forceinline__ float lds_row_dot(const f16* rowp, const float* xs, int K) {
  const int t = threadIdx.x % TPR;
  float acc = 0.0f;
#pragma unroll
  for (int c = 0; c < CPT; ++c) {
    const int k = (t + TPR * c) * 8;
    if (k < K) {
      float wf[8];
      f16x8_to_f32(*reinterpret_cast<const u32x4*>(rowp + k), wf);
#pragma unroll
      for (int i = 0; i < 8; ++i) acc += xs[k + i] * wf[i];
    }
  }
  return group_sum<TPR>(acc);
}

// Register tiling of a block's share of one layer (512 threads). Rows per block: q/k/v (G + 2) * 8, o/down H / 16,
// gate/up pairs I / 128.
template <int G>
struct Tiling {
  static constexpr int RQ = (G + 2) * 8;
  static constexpr int TPR_Q = 16, CPT_Q = HMAX / (TPR_Q * 8);     // 32 slots, K = H
  static constexpr int TPR_O = 8, CPT_O = G * HD / (TPR_O * 8);    // 64 slots, K = G * 128 columns of o_proj (LDS)
  static constexpr int TPR_GU = 16, CPT_GU = HMAX / (TPR_GU * 8);  // 32 slots, K = H
  static constexpr int TPR_D = 8, CPT_D = IMAX / 8 / (TPR_D * 8);  // 64 slots, K = I / 8 columns of down_proj (LDS)
  static constexpr int TPR_LM = 32, CPT_LM = HMAX / (TPR_LM * 8);  // 16 rows per fragment
  static constexpr int MQ_E = (NBG * PW / 4 + 63) / 64;            // one head's partial quads per lane
  static_assert(RQ <= NT / TPR_Q && HMAX / NBG <= NT / TPR_O && IMAX / (NX * NBG) <= NT / TPR_GU, "slots");
  static_assert(TPR_D == TPR_O, "o_proj and down_proj rows share the slot mapping");
};

// LDS carve-up (floats).
template <int G>
struct Lds {
  static constexpr int XRES = 0;                     // [HMAX] residual stream x / x'
  static constexpr int XN = XRES + HMAX;             // [HMAX] x * gain of the next RMSNorm (the scale is applied later)
  static constexpr int RED = XN + HMAX;              // [8] the waves' partial sums of x^2
  static constexpr int HS = RED + 8;                 // [IMAX / 8] the XCD's h slice
  static constexpr int ATT = HS + IMAX / 8;          // [G][HD] merged attention output
  static constexpr int QS = ATT + G * HD;            // [G][HD] normed, rotated queries
  static constexpr int KN = QS + G * HD;             // [HD] new key (fp16-rounded)
  static constexpr int VN = KN + HD;                 // [HD] new value (fp16-rounded)
  static constexpr int RAW = VN + HD;                // [(G + 2) HD] the XCD's raw q/k/v
  static constexpr int GPART = RAW + (G + 2) * HD;   // [32][G][PW] lane-group partials, [8][G] maxima, [256][2] sums
  static constexpr int BPART = GPART + NGRP * G * PW + 8 * G + NT;  // [G][NBG PW] words: the XCD's block partials
  static constexpr int WD = BPART + G * NBG * PW;    // [HMAX / 16][IMAX / 8] halves: the block's down_proj rows
  static constexpr int WO = WD + HMAX / 16 * IMAX / 8 / 2;  // [HMAX / 16][G HD] halves: the block's o_proj rows
  static constexpr int FLAG = WO + HMAX / 16 * G * HD / 2;  // [8] ints: status, g, j, last block
  static constexpr int BV = FLAG + 8;                // [16] argmax values per slot
  static constexpr int BI = BV + 16;                 // [16] argmax indices
  static constexpr int TOTAL = BI + 16;
};

struct Ctx {
  const PersistArgs& a;
  int g, j, token, pos;
  uint32_t phase0;  // (step - 1) * L: the tag of layer l is (phase0 + l) & 3
  float* lds;
  int* flag;
};

// Attention blocks of the XCD's computing group for S keys (about 32 keys each, one per lane group, at most 16
// blocks) and keys per block; na is recomputed from the chunk so that every block jj < na owns at least one key.
__device__ __forceinline__ void attn_split(int S, int& na, int& chunk) {
  na = min(NBG, (S + NGRP - 1) / NGRP);
  chunk = (S + na - 1) / na;
  na = (S + chunk - 1) / chunk;
}

// RMSNorm scale 1 / sqrt(sum x^2 / n + eps) from the eight waves' partial sums, added in a fixed order.
__device__ __forceinline__ float rms_scale(const float* red, int n, float eps) {
  const float s = ((red[0] + red[1]) + (red[2] + red[3])) + ((red[4] + red[5]) + (red[6] + red[7]));
  return 1.0f / sqrtf(s / static_cast<float>(n) + eps);
}

// Optional phase timestamps (diagnostics): the middle layer's phase points of every block of its group go to
// trace[block * 16 + point]; block 0 of each group on XCD 0 also writes its layers' starts, the final norm and the
// step's end into trace[256 * 16 + i].
#define XTRACE(pt)                                                                                           \
  do {                                                                                                       \
    if (c.a.trace != nullptr && threadIdx.x == 0 && layer == c.a.L / 2)                                      \
      c.a.trace[(c.g * NBX + c.j) * 16 + (pt)] = now_ticks();                                                \
  } while (0)
#define XTRACE0(i)                                                                                           \
  do {                                                                                                       \
    if (c.a.trace != nullptr && threadIdx.x == 0 && c.g == 0 && c.j % NBG == 0)                              \
      c.a.trace[NX * NBX * 16 + (i)] = now_ticks();                                                          \
  } while (0)

// Block barrier; afterwards every thread leaves if a wave reported a failed wait (flag[0] != 0).
#define XSYNC()                       \
  do {                                \
    __syncthreads();                  \
    if (c.flag[0] != 0) return false; \
  } while (0)

// Wave: polls MQ quads per lane (byte offsets off[e] into r, or -1 for none) of a tagged vector until every
// one carries `tag`. Returns false (wave-uniform) on timeout or a raised error flag, after recording it in flag[0].
template <int MQ>
__device__ __forceinline__ bool poll_quads(const Ctx& c, __amdgpu_buffer_rsrc_t r, const int (&off)[MQ], uint32_t tag,
                                           u32x4 (&v)[MQ]) {
  const u32x4 filler = {tag, tag, tag, tag};
#pragma unroll
  for (int e = 0; e < MQ; ++e) v[e] = off[e] >= 0 ? ll_peek_buf4(r, off[e]) : filler;
  const uint64_t t0 = now_ticks();
  uint32_t spins = 0;
  while (true) {
    bool all = true;
#pragma unroll
    for (int e = 0; e < MQ; ++e) all = all && tw_quad_ok(v[e], tag);
    if (__all(all)) return true;
    if ((++spins & 63) == 0 && (now_ticks() - t0 > kSpinTicks || err_raised(c.a.err))) {
      __hip_atomic_fetch_max(c.a.err, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);  // keeps a placement error (2)
      c.flag[0] = 1;
      return false;
    }
#pragma unroll
    for (int e = 0; e < MQ; ++e)
      if (off[e] >= 0 && !tw_quad_ok(v[e], tag)) v[e] = ll_peek_buf4(r, off[e]);
  }
}

// Wave: the quads qi = lane + 64 e < nq of the XCD-local tagged words src[0 .. 4 nq) into dst[4 qi ..] (raw
// words: the tags are kept). Load e of a lane is at byte 16 lane + 1024 e: one register offset for all loads.
template <int MQ>
__device__ __forceinline__ bool recv_contig(const Ctx& c, const uint32_t* src, int nq, uint32_t tag, uint32_t* dst) {
  int lane = threadIdx.x & 63;
  __asm__ volatile("" : "+v"(lane));
  const __amdgpu_buffer_rsrc_t r = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint32_t*>(src), 0, nq * 16, 0x00020000);
  const u32x4 filler = {tag, tag, tag, tag};
  u32x4 v[MQ];
#pragma unroll
  for (int e = 0; e < MQ; ++e)
    v[e] = lane + 64 * e < nq ? __builtin_amdgcn_raw_buffer_load_b128(r, lane * 16, e * 1024, 16) : filler;
  const uint64_t t0 = now_ticks();
  uint32_t spins = 0;
  while (true) {
    bool all = true;
#pragma unroll
    for (int e = 0; e < MQ; ++e) all = all && tw_quad_ok(v[e], tag);
    if (__all(all)) break;
    if ((++spins & 63) == 0 && (now_ticks() - t0 > kSpinTicks || err_raised(c.a.err))) {
      __hip_atomic_fetch_max(c.a.err, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);  // keeps a placement error (2)
      c.flag[0] = 1;
      return false;
    }
#pragma unroll
    for (int e = 0; e < MQ; ++e)
      if (lane + 64 * e < nq && !tw_quad_ok(v[e], tag))
        v[e] = __builtin_amdgcn_raw_buffer_load_b128(r, lane * 16, e * 1024, 16);
  }
#pragma unroll
  for (int e = 0; e < MQ; ++e)
    if (lane + 64 * e < nq) *reinterpret_cast<u32x4*>(dst + 4 * (lane + 64 * e)) = v[e];
  return true;
}

// Sum over aligned groups of 8 lanes that is bit-identical in every lane of the group: each step adds two values
// that are equal in both partner lanes up to the order of one addition, and IEEE addition commutes exactly.
__device__ __forceinline__ float sum8(float v) {
  v += dpp_mov<0xB1>(v);   // lane ^ 1
  v += dpp_mov<0x4E>(v);   // lane ^ 2
  v += dpp_mov<0x141>(v);  // lane ^ 7 within 8: the other (now uniform) quad
  return v;
}

// Sum over the four 16-lane rows of a wave (lanes l, l ^ 16, l ^ 32, l ^ 48) with the gfx950 cross-row swaps: with
// both operands equal, the two results of v_permlane32_swap hold v[l] and v[l ^ 32] (in some order) in every lane,
// and likewise for v_permlane16_swap with l ^ 16; no LDS round trip.
__device__ __forceinline__ float sum_rows4(float v) {
  const auto r32 = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  v = __uint_as_float(r32[0]) + __uint_as_float(r32[1]);
  const auto r16 = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(r16[0]) + __uint_as_float(r16[1]);
}

// Wave w < 8 of the block: its eighth of x = base + sum_k partial_k over the eight XCDs, then x * gain into xn and its
// partial sum of x^2 into red[w] (the RMSNorm of rms_norm_module.cpp:56-64 is completed by rms_scale). The base is
// the tagged vector xbase (the previous layer's residual published by the other group) or, when xbase is null, the
// residual in LDS; for layer 0 the embedding row replaces it all. The wave owns the element quads w * H / 32 ..
// + H / 32; its load i brings 8 of them from all eight partials (lane l: quad i * 8 + l / 8 of partial l % 8) and
// the 8 lanes of a quad add their partials with sum8; lanes l % 8 == 0 also load the base quad.
__device__ __forceinline__ bool cross_reduce(const Ctx& c, int w, const uint32_t* src, const uint32_t* xbase,
                                             uint32_t tag, const f16* embed_row, const f16* gain, float* xres,
                                             float* xn, float* red) {
  constexpr int NI = HMAX / 256;
  int lane = threadIdx.x & 63;
  __asm__ volatile("" : "+v"(lane));  // per call: keeps the compiler from hoisting per-lane addresses out of the layers
  const int k = lane & 7;
  const int H = c.a.H, ni = H / 256, q0 = w * (H / 32);
  float ss = 0.0f;
  if (embed_row != nullptr) {
#pragma unroll
    for (int i = 0; i < NI; ++i) {
      const int q = q0 + i * 8 + (lane >> 3);
      if (i < ni && k == 0) {
        const f16x4 e4 = ld_global(reinterpret_cast<const f16x4*>(embed_row), q);
        const f16x4 g4 = ld_global(reinterpret_cast<const f16x4*>(gain), q);
        f32x4 x, y;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          x[e] = static_cast<float>(e4[e]);
          y[e] = x[e] * static_cast<float>(g4[e]);
          ss += x[e] * x[e];
        }
        *reinterpret_cast<f32x4*>(xres + 4 * q) = x;
        *reinterpret_cast<f32x4*>(xn + 4 * q) = y;
      }
    }
  } else {
    // one poll for the partials and, when given, the base quads (lanes l % 8 == 0): the base is published earlier,
    // so it costs no extra round trip
    const __amdgpu_buffer_rsrc_t r =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<uint32_t*>(src), 0, H * NX * 4, 0x00020000);
    const __amdgpu_buffer_rsrc_t rb = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint32_t*>(xbase != nullptr ? xbase : src), 0, H * 4, 0x00020000);
    const u32x4 filler = {tag, tag, tag, tag};
    u32x4 v[NI], bq[NI];
#pragma unroll
    for (int i = 0; i < NI; ++i) {
      const bool live = i < ni, blive = live && xbase != nullptr && k == 0;
      v[i] = live ? ll_peek_buf4(r, k * H * 4 + (q0 + i * 8 + (lane >> 3)) * 16) : filler;
      bq[i] = blive ? ll_peek_buf4(rb, (q0 + i * 8 + (lane >> 3)) * 16) : filler;
    }
    const uint64_t t0 = now_ticks();
    uint32_t spins = 0;
    while (true) {
      bool all = true;
#pragma unroll
      for (int i = 0; i < NI; ++i) all = all && tw_quad_ok(v[i], tag) && tw_quad_ok(bq[i], tag);
      if (__all(all)) break;
      if ((++spins & 63) == 0 && (now_ticks() - t0 > kSpinTicks || err_raised(c.a.err))) {
        __hip_atomic_fetch_max(c.a.err, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);  // keeps a placement error
        c.flag[0] = 1;
        return false;
      }
#pragma unroll
      for (int i = 0; i < NI; ++i) {
        const bool live = i < ni, blive = live && xbase != nullptr && k == 0;
        if (live && !tw_quad_ok(v[i], tag)) v[i] = ll_peek_buf4(r, k * H * 4 + (q0 + i * 8 + (lane >> 3)) * 16);
        if (blive && !tw_quad_ok(bq[i], tag)) bq[i] = ll_peek_buf4(rb, (q0 + i * 8 + (lane >> 3)) * 16);
      }
    }
#pragma unroll
    for (int i = 0; i < NI; ++i) {
      const int q = q0 + i * 8 + (lane >> 3);
      const float s0 = sum8(tw_val(v[i].x)), s1 = sum8(tw_val(v[i].y));
      const float s2 = sum8(tw_val(v[i].z)), s3 = sum8(tw_val(v[i].w));
      if (i < ni && k == 0) {
        f32x4 x = xbase != nullptr ? f32x4{tw_val(bq[i].x), tw_val(bq[i].y), tw_val(bq[i].z), tw_val(bq[i].w)}
                                   : *reinterpret_cast<const f32x4*>(xres + 4 * q);
        const f16x4 g4 = ld_global(reinterpret_cast<const f16x4*>(gain), q);
        x[0] += s0;
        x[1] += s1;
        x[2] += s2;
        x[3] += s3;
        f32x4 y;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          y[e] = x[e] * static_cast<float>(g4[e]);
          ss += x[e] * x[e];
        }
        *reinterpret_cast<f32x4*>(xres + 4 * q) = x;
        *reinterpret_cast<f32x4*>(xn + 4 * q) = y;
      }
    }
  }
  ss = wave_sum(ss);
  if (lane == 0) red[w] = ss;
  return true;
}

// Two-stage form of the same reduction, x = base + sum_k P_k over the eight XCDs' partials P_k (src, [8][H] words),
// that reads each remote partial once per XCD instead of once per block:
// stage 1 (wave 0 of a block with do1): the block's 1/16 of the elements, quads jj * H/64 ..; base from base_loc
//   (XCD-local words) or, if null, from xres; x goes to out[0, H) and the block's sum of squares of x to out[H + jj],
//   as XCD-local words with the same tag;
// stage 2 (every wave): all of x and the 16 sums from out; x into xres, x * gain into xn, red[0..7] = pair sums of the
//   16 sums (rms_scale adds them in a fixed order). Every block reads the same words, so x and the norm agree in every
//   block of every XCD. The caller's barrier publishes xres, xn and red.
__device__ __forceinline__ bool cross_reduce2(const Ctx& c, int w, int jj, bool do1, const uint32_t* src,
                                              const uint32_t* base_loc, uint32_t tag, uint32_t* out, const f16* gain,
                                              float* xres, float* xn, float* red, int trace_pt = -1) {
  int lane = threadIdx.x & 63;
  __asm__ volatile("" : "+v"(lane));  // per call: keeps the compiler from hoisting per-lane addresses out of the layers
  const int H = c.a.H;
  const u32x4 filler = {tag, tag, tag, tag};
  const uint64_t t0 = now_ticks();
  auto failed = [&]() {
    __hip_atomic_fetch_max(c.a.err, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    c.flag[0] = 1;
  };
  if (w == 0 && do1) {
    const int k = lane & 7, nq1 = H / 64, qb = jj * nq1;
    const __amdgpu_buffer_rsrc_t r =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<uint32_t*>(src), 0, H * NX * 4, 0x00020000);
    const __amdgpu_buffer_rsrc_t rb = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint32_t*>(base_loc != nullptr ? base_loc : src), 0, H * 4, 0x00020000);
    u32x4 v[2], bq[2];
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int qi = (lane >> 3) + 8 * i;
      const bool live = qi < nq1, blive = live && base_loc != nullptr && k == 0;
      v[i] = live ? ll_peek_buf4(r, (k * H + 4 * (qb + qi)) * 4) : filler;
      bq[i] = blive ? ll_peek_buf4(rb, (qb + qi) * 16) : filler;
    }
    uint32_t spins = 0;
    while (true) {
      bool all = true;
#pragma unroll
      for (int i = 0; i < 2; ++i) all = all && tw_quad_ok(v[i], tag) && tw_quad_ok(bq[i], tag);
      if (__all(all)) break;
      if ((++spins & 63) == 0 && (now_ticks() - t0 > kSpinTicks || err_raised(c.a.err))) {
        failed();
        return false;
      }
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        const int qi = (lane >> 3) + 8 * i;
        const bool live = qi < nq1, blive = live && base_loc != nullptr && k == 0;
        if (live && !tw_quad_ok(v[i], tag)) v[i] = ll_peek_buf4(r, (k * H + 4 * (qb + qi)) * 4);
        if (blive && !tw_quad_ok(bq[i], tag)) bq[i] = ll_peek_buf4(rb, (qb + qi) * 16);
      }
    }
    const __amdgpu_buffer_rsrc_t ro = __builtin_amdgcn_make_buffer_rsrc(out, 0, (H + NBG) * 4, 0x00020000);
    float ss = 0.0f;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int qi = (lane >> 3) + 8 * i, q = qb + qi;
      const float s0 = sum8(tw_val(v[i].x)), s1 = sum8(tw_val(v[i].y));
      const float s2 = sum8(tw_val(v[i].z)), s3 = sum8(tw_val(v[i].w));
      if (qi < nq1 && k == 0) {
        f32x4 x = base_loc != nullptr ? f32x4{tw_val(bq[i].x), tw_val(bq[i].y), tw_val(bq[i].z), tw_val(bq[i].w)}
                                      : *reinterpret_cast<const f32x4*>(xres + 4 * q);
        x[0] += s0;
        x[1] += s1;
        x[2] += s2;
        x[3] += s3;
        u32x4 wq;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          wq[e] = tw_pack(x[e], tag);
          const float xr = tw_val(wq[e]);
          ss += xr * xr;
        }
        __builtin_amdgcn_raw_buffer_store_b128(wq, ro, q * 16, 0, 0);
      }
    }
    ss = wave_sum(ss);
    if (lane == 0) ll_store_local(out, H + jj, ss, tag);
    if (trace_pt >= 0 && c.a.trace != nullptr && threadIdx.x == 0)
      c.a.trace[(c.g * NBX + c.j) * 16 + trace_pt] = now_ticks();  // stage 1 done (diagnostics)
  }
  // stage 2: waves 0..3 take quad w * H/16 + lane of x, wave 4's lanes 0..3 the 16 sums (fewer waves polling L2)
  const int per = H / 16;
  const bool xlive = w < 4 && lane < per, slive = w == 4 && lane < 4;
  const int off = xlive ? (w * per + lane) * 16 : (H + 4 * lane) * 4;
  const __amdgpu_buffer_rsrc_t ro = __builtin_amdgcn_make_buffer_rsrc(out, 0, (H + NBG) * 4, 0x00020000);
  u32x4 v = (xlive || slive) ? ll_peek_buf4(ro, off) : filler;
  uint32_t spins = 0;
  while (!__all(tw_quad_ok(v, tag))) {
    if ((++spins & 63) == 0 && (now_ticks() - t0 > kSpinTicks || err_raised(c.a.err))) {
      failed();
      return false;
    }
    if (!tw_quad_ok(v, tag)) v = ll_peek_buf4(ro, off);
  }
  if (xlive) {
    const int q = w * per + lane;
    const f32x4 x = {tw_val(v.x), tw_val(v.y), tw_val(v.z), tw_val(v.w)};
    const f16x4 g4 = ld_global(reinterpret_cast<const f16x4*>(gain), q);
    f32x4 y;
#pragma unroll
    for (int e = 0; e < 4; ++e) y[e] = x[e] * static_cast<float>(g4[e]);
    *reinterpret_cast<f32x4*>(xres + 4 * q) = x;
    *reinterpret_cast<f32x4*>(xn + 4 * q) = y;
  }
  if (slive) {
    const int m = lane;
    red[2 * m] = tw_val(v.x) + tw_val(v.y);
    red[2 * m + 1] = tw_val(v.z) + tw_val(v.w);
  }
  return true;
}

// The layers l % 2 == p of one decode step for a block of group p, then the final hidden state (all blocks).
template <int G>
__device__ __forceinline__ bool run_layers(const Ctx& c) {
  using T = Tiling<G>;
  using LD = Lds<G>;
  const PersistArgs& a = c.a;
  const int tid = threadIdx.x, wid = tid >> 6;
  const int g = c.g, pgrp = c.j / NBG, jj = c.j % NBG, pos = c.pos, S = pos + 1;
  const int H = a.H, I = a.I, qd = a.qd;
  const int RH = H / NBG;   // o/down rows per block
  const int IS = I / NX;    // intermediate slice of the XCD
  const int RI = IS / NBG;  // gate/up pairs per block
  float* lds = c.lds;
  float* xres = lds + LD::XRES;
  float* xn = lds + LD::XN;
  float* red = lds + LD::RED;
  float* hs = lds + LD::HS;
  float* att = lds + LD::ATT;
  float* qs = lds + LD::QS;
  float* kn = lds + LD::KN;
  float* vn = lds + LD::VN;
  uint32_t* raw = reinterpret_cast<uint32_t*>(lds + LD::RAW);
  float* gpart = lds + LD::GPART;
  uint32_t* bpart = reinterpret_cast<uint32_t*>(lds + LD::BPART);
  f16* wd = reinterpret_cast<f16*>(lds + LD::WD);
  f16* wo = reinterpret_cast<f16*>(lds + LD::WO);
  uint32_t* loc = a.loc + static_cast<size_t>(g) * a.loc_stride;
  uint32_t* loc_qkv = loc;                                  // [(G + 2) HD]
  uint32_t* loc_att = loc + (((G + 2) * HD + 63) & ~63);    // [G][NBX][PW]
  uint32_t* loc_h = loc_att + ((NBX * G * PW + 63) & ~63);  // [IS]
  uint32_t* loc_xa = loc_h + ((IS + 63) & ~63);               // [H + 16]: x after the attention-input reduction
  uint32_t* loc_xg = loc_xa + HMAX + 64;                      // [H + 16]: x' after the o_proj reduction
  // this block's q/k/v row: local row lr of the XCD's (G + 2) * 128 (q heads, key, value)
  const int q_slot = tid / T::TPR_Q;
  const int q_lr = jj * T::RQ + q_slot;
  const bool q_live = q_slot < T::RQ;
  const int q_row = q_lr < G * HD ? g * G * HD + q_lr
                                  : (q_lr < (G + 1) * HD ? qd + g * HD + (q_lr - G * HD)
                                                         : qd + a.nkv * HD + g * HD + (q_lr - (G + 1) * HD));
  const int o_slot = tid / T::TPR_O, gu_slot = tid / T::TPR_GU;
  const int hrow = jj * RH + o_slot;           // o/down output row
  const bool h_live = o_slot < RH;
  const int iidx = g * IS + jj * RI + gu_slot; // gate/up row
  const bool i_live = gu_slot < RI;
  // attention: up to NGRP * KPG keys every block takes all keys (lane group grp: keys grp + 32 u); beyond that block
  // jj < na takes keys [k0, k1) (lane group grp: keys k0 + grp + 32 u) and the blocks' partials are exchanged
  const bool allkeys = S <= NGRP * KPG;
  int na, chunk;
  attn_split(S, na, chunk);
  const int k0 = allkeys ? 0 : (jj < na ? min(S, jj * chunk) : S);
  const int k1 = allkeys ? S : (jj < na ? min(S, k0 + chunk) : S);
  int lane = tid & 63, grp = tid >> 4, sub = tid & 15;

  Slice<T::TPR_Q, T::CPT_Q> sq;
  Slice<T::TPR_GU, T::CPT_GU> sg, su;
  u32x4 kr = {0, 0, 0, 0}, vr = {0, 0, 0, 0};
  auto kv_fetch = [&](int layer, int p) {  // cached key/value p (< pos) of this layer, 8 dims per lane
    if (p < k1 && p < pos) {
      const size_t base = static_cast<size_t>(layer) * a.layer_stride + static_cast<size_t>(g) * a.cap * HD +
                          static_cast<size_t>(p) * HD + sub * 8;
      kr = load16(a.kcache + base);
      vr = load16(a.vcache + base);
    }
  };
  // the weight rows of layer `layer` and its first cached key/value of this lane group
  auto stream = [&](int layer) {
    // recomputed per call: keeps the 64-bit row offsets from staying live across the layer loop
    int qr = q_row, hr = jj * RH, ir = iidx;
    __asm__ volatile("" : "+v"(qr), "+v"(ir), "+s"(hr));
    const f16* W4 = ld_global(a.layer_w, static_cast<size_t>(layer) * 9 + 4);
    const f16* W5 = ld_global(a.layer_w, static_cast<size_t>(layer) * 9 + 5);
    const f16* W6 = ld_global(a.layer_w, static_cast<size_t>(layer) * 9 + 6);
    const f16* W7 = ld_global(a.layer_w, static_cast<size_t>(layer) * 9 + 7);
    const f16* W8 = ld_global(a.layer_w, static_cast<size_t>(layer) * 9 + 8);
    slice_load(sq, q_live ? W4 + static_cast<size_t>(qr) * H : nullptr, H);
    rows_to_lds(W5 + static_cast<size_t>(hr) * qd + g * G * HD, qd, RH, G * HD, wo);
    slice_load(sg, i_live ? W6 + static_cast<size_t>(ir) * H : nullptr, H);
    slice_load(su, i_live ? W7 + static_cast<size_t>(ir) * H : nullptr, H);
    rows_to_lds(W8 + static_cast<size_t>(hr) * I + g * IS, I, RH, IS, wd);
    kv_fetch(layer, k0 + grp);
    if (allkeys) {
      // this block's share of KV head g's cached keys and values into the XCD's L2 (keys jj + 16 m): every block
      // of the group then reads them from there
      const int p = jj + NBG * (tid >> 4);
      if (p < pos) {
        const size_t base = static_cast<size_t>(layer) * a.layer_stride + static_cast<size_t>(g) * a.cap * HD +
                            static_cast<size_t>(p) * HD + sub * 8;
        const u32x4 pfk = load16(a.kcache + base);
        const u32x4 pfv = load16(a.vcache + base);
        // the words are only kept alive (a compare that is practically never true, and harmless if it is); the
        // wait this implies is free: the group has nothing to do until the other group's layer is done
        if (pfk.x == 0x9e3779b9u && pfv.y == 0x7f7f7f7fu && pfk.z == pfv.w) c.flag[7] = 1;
      }
    }
  };
  if (pgrp < a.L) stream(pgrp);

  for (int layer = pgrp; layer < a.L; layer += 2) {
    const f16* W[4];  // in_norm, post_norm, q_norm, k_norm
#pragma unroll
    for (int i = 0; i < 4; ++i) W[i] = ld_global(a.layer_w, static_cast<size_t>(layer) * 9 + i);
    const uint32_t tag = (c.phase0 + static_cast<uint32_t>(layer)) & 3u;
    // per layer: keeps the compiler from hoisting per-lane addresses out of the loop (register pressure)
    __asm__ volatile("" : "+v"(lane), "+v"(grp), "+v"(sub));
    XTRACE0(layer);
    XTRACE(0);
    // ---- A: x = x' + sum_k D_k (layer 0: the embedding row, embedding.cpp:51-77), RMSNorm input ----
    wait_mem();  // this wave's rows of the layer have landed (its LDS rows are published by the barrier below)
    if (layer == 0)
      cross_reduce(c, wid, a.xd, nullptr, tag, a.embed + static_cast<size_t>(c.token) * H, W[0], xres, xn, red);
    else
      cross_reduce2(c, wid, jj, true, a.xd, loc_xg, (tag - 1u) & 3u, loc_xa, W[0], xres, xn, red,
                    layer == a.L / 2 ? 15 : -1);
    XTRACE(1);
    XSYNC();  // #1
    // ---- B: q/k/v rows of RMSNorm(x) ----
    {
      const float out = slice_dot(sq, xn, H) * rms_scale(red, H, a.eps);
      if (q_live && tid % T::TPR_Q == 0) ll_store_local(loc_qkv, q_lr, out, tag);
    }
    XTRACE(2);
    // ---- C: head wid of the XCD's q/k/v; QK-RMSNorm + rotate-half RoPE (qwen_attention.cpp:168-171,
    //      rope.cpp:81-84); rank 0 appends the key and value, rounded to the cache's fp16, at `pos` ----
    if (wid < G + 2) {
      const int hh = wid;
      if (recv_contig<1>(c, loc_qkv + hh * HD, HD / 4, tag, raw + hh * HD)) {
        float x0 = tw_val(raw[hh * HD + lane]), x1 = tw_val(raw[hh * HD + lane + 64]);
        if (hh <= G)
          norm_rope_pair(x0, x1, hh < G ? W[2] : W[3], a.eps, a.rope_cos + static_cast<size_t>(pos) * (HD / 2),
                         a.rope_sin + static_cast<size_t>(pos) * (HD / 2), lane);
        if (hh < G) {
          qs[hh * HD + lane] = x0;
          qs[hh * HD + lane + 64] = x1;
        } else {
          const f16 h0 = static_cast<f16>(x0), h1 = static_cast<f16>(x1);
          float* dst = hh == G ? kn : vn;
          dst[lane] = static_cast<float>(h0);
          dst[lane + 64] = static_cast<float>(h1);
          if (jj == 0) {
            f16* cache = (hh == G ? a.kcache : a.vcache) + static_cast<size_t>(layer) * a.layer_stride +
                         static_cast<size_t>(g) * a.cap * HD + static_cast<size_t>(pos) * HD;
            cache[lane] = h0;
            cache[lane + 64] = h1;
          }
        }
      }
    }
    XTRACE(3);
    XSYNC();  // #2: qs, kn, vn
    if (allkeys) {
      // NK keys per lane group (4 or 8): a straight-line body for each, chosen by the uniform S
      auto all_keys = [&](auto nk) {
        constexpr int NK = decltype(nk)::value;
        // ---- D, up to 256 keys: every block takes all S keys of KV head g (the softmax of
        //      grouped_query_attention.cpp:105-136): scores and the block max per head, then base-2 weights; the 4
        //      lane groups of a wave add with cross-row swaps, the 8 waves through LDS. No hand-off between blocks. ----
        const float qscale = a.scale * 1.44269504088896341f;
        // the head's cached keys/values through buffer resources (scalar base, 32-bit lane offsets; keys at or past
        // `pos` read as zero)
        const size_t kvb = static_cast<size_t>(layer) * a.layer_stride + static_cast<size_t>(g) * a.cap * HD;
        const __amdgpu_buffer_rsrc_t rk = __builtin_amdgcn_make_buffer_rsrc(a.kcache + kvb, 0, pos * HD * 2, 0x00020000);
        const __amdgpu_buffer_rsrc_t rv = __builtin_amdgcn_make_buffer_rsrc(a.vcache + kvb, 0, pos * HD * 2, 0x00020000);
        const int kvo = (grp * HD + sub * 8) * 2;
        float qreg[G][8], sc[NK][G], mloc[G];
#pragma unroll
        for (int h = 0; h < G; ++h) {
          mloc[h] = kNoKeys;
#pragma unroll
          for (int i = 0; i < 8; ++i) qreg[h][i] = qs[h * HD + sub * 8 + i] * qscale;
        }
        u32x4 vw0[4];
#pragma unroll
        for (int u0 = 0; u0 < NK; u0 += 4) {
          u32x4 kw[4];
#pragma unroll
          for (int v = 0; v < 4; ++v) {
            kw[v] = (u0 + v == 0) ? kr : __builtin_amdgcn_raw_buffer_load_b128(rk, kvo, NGRP * (u0 + v) * HD * 2, 0);
          }
          if constexpr (NK == 4) {  // one round: its values are requested with the keys
#pragma unroll
            for (int v = 0; v < 4; ++v)
              vw0[v] = v == 0 ? vr : __builtin_amdgcn_raw_buffer_load_b128(rv, kvo, NGRP * v * HD * 2, 0);
          }
#pragma unroll
          for (int v = 0; v < 4; ++v) {
            const int p = grp + NGRP * (u0 + v);
            float kf[8];
            if (p == pos) {
#pragma unroll
              for (int i = 0; i < 8; ++i) kf[i] = kn[sub * 8 + i];
            } else {
              f16x8_to_f32(kw[v], kf);
            }
#pragma unroll
            for (int h = 0; h < G; ++h) {
              float d = 0.0f;
#pragma unroll
              for (int i = 0; i < 8; ++i) d += qreg[h][i] * kf[i];
              const float sv = group_sum<16>(d);
              sc[u0 + v][h] = p < S ? sv : kNoKeys;
              mloc[h] = fmaxf(mloc[h], sc[u0 + v][h]);
            }
          }
        }
        // weights relative to the wave's max (no block barrier); the 8 waves' sums are rescaled when merged
        XTRACE(4);
        float mblk[G], o[G][8], l[G];
#pragma unroll
        for (int h = 0; h < G; ++h) {
          mblk[h] = wave_max(mloc[h]);
          l[h] = 0.0f;
#pragma unroll
          for (int i = 0; i < 8; ++i) o[h][i] = 0.0f;
        }
#pragma unroll
        for (int u0 = 0; u0 < NK; u0 += 4) {
          u32x4 vw[4];
#pragma unroll
          for (int v = 0; v < 4; ++v) {
            if constexpr (NK == 4)
              vw[v] = vw0[v];
            else
              vw[v] = (u0 + v == 0) ? vr : __builtin_amdgcn_raw_buffer_load_b128(rv, kvo, NGRP * (u0 + v) * HD * 2, 0);
          }
#pragma unroll
          for (int v = 0; v < 4; ++v) {
            const int p = grp + NGRP * (u0 + v);
            if (p < S) {
              float vf[8];
              if (p == pos) {
#pragma unroll
                for (int i = 0; i < 8; ++i) vf[i] = vn[sub * 8 + i];
              } else {
                f16x8_to_f32(vw[v], vf);
              }
#pragma unroll
              for (int h = 0; h < G; ++h) {
                const float pw = __builtin_amdgcn_exp2f(sc[u0 + v][h] - mblk[h]);
                l[h] += pw;
#pragma unroll
                for (int i = 0; i < 8; ++i) o[h][i] += pw * vf[i];
              }
            }
          }
        }
        // the wave's 4 lane groups added across rows; row 0 writes the wave's sums
#pragma unroll
        for (int h = 0; h < G; ++h) {
#pragma unroll
          for (int i = 0; i < 8; ++i) {
            const float ov = sum_rows4(o[h][i]);
            if (lane < 16) gpart[(wid * G + h) * PW + sub * 8 + i] = ov;
          }
          const float lv = sum_rows4(l[h]);
          if (lane == 0) {
            gpart[(wid * G + h) * PW + HD + 1] = lv;
            gpart[(wid * G + h) * PW + HD + 2] = mblk[h];
          }
        }
        XTRACE(11);
        XSYNC();  // #2b: the 8 waves' sums
        XTRACE(12);
        for (int t = tid; t < G * HD; t += NT) {
          const int h = t / HD, d = t % HD;
          float M = kNoKeys;
#pragma unroll
          for (int w = 0; w < NT / 64; ++w) M = fmaxf(M, gpart[(w * G + h) * PW + HD + 2]);
          float L = 0.0f, O = 0.0f;
#pragma unroll
          for (int w = 0; w < NT / 64; ++w) {
            const float f = __builtin_amdgcn_exp2f(gpart[(w * G + h) * PW + HD + 2] - M);  // 0 for a wave without keys
            L += gpart[(w * G + h) * PW + HD + 1] * f;
            O += gpart[(w * G + h) * PW + d] * f;
          }
          att[h * HD + d] = O / L;
        }
        XTRACE(13);
        return true;
      };
      if (!(S <= NGRP * 4 ? all_keys(std::integral_constant<int, 4>{}) : all_keys(std::integral_constant<int, KPG>{})))
        return false;
    } else {
    // ---- D: attention over keys [k0, k1) (the softmax of grouped_query_attention.cpp:105-136) in two passes over the
    //      block's keys: scores and the block's max per head, then base-2 weights relative to that max, so that the
    //      lane groups' partials merge by plain sums. q is prescaled by scale * log2(e). ----
    float qreg[G][8], mblk[G];
    {
      const float qscale = a.scale * 1.44269504088896341f;
      float mloc[G];
#pragma unroll
      for (int h = 0; h < G; ++h) {
        mloc[h] = kNoKeys;
#pragma unroll
        for (int i = 0; i < 8; ++i) qreg[h][i] = qs[h * HD + sub * 8 + i] * qscale;
      }
      // the score of key p for every head (every lane of the group gets it)
      auto scores = [&](int p, int u, float (&sc)[G]) {
        float kf[8];
        if (p == pos) {
#pragma unroll
          for (int i = 0; i < 8; ++i) kf[i] = kn[sub * 8 + i];
        } else {
          const u32x4 kw = u == 0 ? kr
                                  : load16(a.kcache + static_cast<size_t>(layer) * a.layer_stride +
                                           static_cast<size_t>(g) * a.cap * HD + static_cast<size_t>(p) * HD + sub * 8);
          f16x8_to_f32(kw, kf);
        }
#pragma unroll
        for (int h = 0; h < G; ++h) {
          float d = 0.0f;
#pragma unroll
          for (int i = 0; i < 8; ++i) d += qreg[h][i] * kf[i];
          sc[h] = group_sum<16>(d);
        }
      };
      if (jj < na)
        for (int p = k0 + grp, u = 0; p < k1; p += NGRP, ++u) {
          float sc[G];
          scores(p, u, sc);
#pragma unroll
          for (int h = 0; h < G; ++h) mloc[h] = fmaxf(mloc[h], sc[h]);
        }
      // the block's max per head: wave maxima, then the 8 waves' through LDS
#pragma unroll
      for (int h = 0; h < G; ++h) {
        const float mw = wave_max(mloc[h]);
        if (lane == 0) gpart[NGRP * G * PW + wid * G + h] = mw;
      }
      XSYNC();  // #2a: wave maxima
#pragma unroll
      for (int h = 0; h < G; ++h) {
        float M = kNoKeys;
#pragma unroll
        for (int w = 0; w < NT / 64; ++w) M = fmaxf(M, gpart[NGRP * G * PW + w * G + h]);
        mblk[h] = M == kNoKeys ? M : tw_val(tw_pack(M, 0u));  // as the exchange word will carry it
      }
      float o[G][8], l[G];
#pragma unroll
      for (int h = 0; h < G; ++h) {
        l[h] = 0.0f;
#pragma unroll
        for (int i = 0; i < 8; ++i) o[h][i] = 0.0f;
      }
      if (jj < na)
        for (int p = k0 + grp, u = 0; p < k1; p += NGRP, ++u) {
          float sc[G], vf[8];
          scores(p, u, sc);
          if (p == pos) {
#pragma unroll
            for (int i = 0; i < 8; ++i) vf[i] = vn[sub * 8 + i];
          } else {
            const u32x4 vw = u == 0 ? vr
                                    : load16(a.vcache + static_cast<size_t>(layer) * a.layer_stride +
                                             static_cast<size_t>(g) * a.cap * HD + static_cast<size_t>(p) * HD + sub * 8);
            f16x8_to_f32(vw, vf);
          }
#pragma unroll
          for (int h = 0; h < G; ++h) {
            const float pw = __builtin_amdgcn_exp2f(sc[h] - mblk[h]);
            l[h] += pw;
#pragma unroll
            for (int i = 0; i < 8; ++i) o[h][i] += pw * vf[i];
          }
        }
      // the group's partial sums (relative to the block max) to LDS
#pragma unroll
      for (int h = 0; h < G; ++h) {
#pragma unroll
        for (int i = 0; i < 8; ++i) gpart[(grp * G + h) * PW + sub * 8 + i] = o[h][i];
        if (sub == 0) gpart[(grp * G + h) * PW + HD + 1] = l[h];
      }
    }
    XTRACE(11);
    XSYNC();  // #2b: the block's lane-group partials
    XTRACE(12);
    if (jj < na) {
      // output t (head t / 128, dim t % 128) is the sum over the 32 groups in a fixed order: threads t and t + 256 of
      // the same lane add groups 0..15 and 16..31, and the lower half adds the upper half's sum through LDS
      static_assert(G * HD <= NT / 2, "two threads per output");
      const int t = tid & (NT / 2 - 1), half = tid / (NT / 2);
      const int h = t / HD, d = t % HD;
      float L = 0.0f, O = 0.0f;
      if (t < G * HD) {
#pragma unroll
        for (int q = 0; q < NGRP / 2; ++q) {
          const int qq = half * (NGRP / 2) + q;
          L += gpart[(qq * G + h) * PW + HD + 1];
          O += gpart[(qq * G + h) * PW + d];
        }
      }
      float* hsum = gpart + NGRP * G * PW + 8 * G;  // [NT / 2][2] the upper halves' sums (spare LDS after the maxima)
      if (half == 1 && t < G * HD) {
        hsum[2 * t] = O;
        hsum[2 * t + 1] = L;
      }
      __syncthreads();  // every thread of the block reaches this barrier (jj < na is block-uniform)
      if (half == 0 && t < G * HD) {
        O += hsum[2 * t];
        L += hsum[2 * t + 1];
        const int w0 = (h * NBX + jj) * PW;  // [head][block][PW]
        ll_store_local(loc_att, w0 + d, O, tag);
        if (d < 4) ll_store_local(loc_att, w0 + HD + d, d == 0 ? mblk[h] : (d == 1 ? L : 0.0f), tag);
      }
    }
    XTRACE(4);
    // ---- E: head wid's block partials of the XCD, merged in a fixed order ----
    if (wid < G) {
      const int h = wid;
      if (recv_contig<T::MQ_E>(c, loc_att + h * NBX * PW, na * (PW / 4), tag, bpart + h * (NBG * PW))) {
        XTRACE(13);
        const uint32_t* bp = bpart + h * (NBG * PW);
        // lane r < na holds block r's max and sum; the weights e_r are broadcast with readlane
        const float mr = lane < na ? tw_val(bp[lane * PW + HD]) : kNoKeys;
        const float lr = lane < na ? tw_val(bp[lane * PW + HD + 1]) : 0.0f;
        const float M = wave_max(mr);
        const float er = mr < 0.5f * kNoKeys ? 0.0f : __builtin_amdgcn_exp2f(mr - M);  // base 2; a keyless block adds 0
        const float L = wave_sum(lr * er);
#pragma unroll
        for (int dd = 0; dd < 2; ++dd) {
          const int d = lane + 64 * dd;
          float O = 0.0f;
#pragma unroll
          for (int r = 0; r < NBG; ++r)
            if (r < na) O += tw_val(bp[r * PW + d]) * __int_as_float(__builtin_amdgcn_readlane(__float_as_int(er), r));
          att[h * HD + d] = O / L;
        }
      }
    }
    XTRACE(5);
    }  // the split path
    XSYNC();  // #3: merged attention output
    // ---- F: partial o_proj over the XCD's query columns ----
    {
      const float out = lds_row_dot<T::TPR_O, T::CPT_O>(wo + (h_live ? o_slot : 0) * (G * HD), att, G * HD);
      if (h_live && tid % T::TPR_O == 0) ll_store_buf(a.xo, g * H + hrow, out, tag);
    }
    XTRACE(6);
    // ---- G: x' = x + sum_k O_k, RMSNorm input ----
    cross_reduce2(c, wid, jj, true, a.xo, nullptr, tag, loc_xg, W[1], xres, xn, red,  // x' also for the other group
                  layer == a.L / 2 ? 14 : -1);
    XTRACE(7);
    XSYNC();  // #4
    // ---- H: gate/up of RMSNorm(x') + SwiGLU (qwen_mlp.cpp:31) on the block's share of the XCD's slice ----
    {
      const float scale = rms_scale(red, H, a.eps);
      const float og = slice_dot(sg, xn, H) * scale;
      const float ou = slice_dot(su, xn, H) * scale;
      if (i_live && tid % T::TPR_GU == 0) ll_store_local(loc_h, jj * RI + gu_slot, silu_ref(og) * ou, tag);
    }
    XTRACE(8);
    // ---- I: the XCD's h slice ----
    if (wid * 64 < IS / 4 &&
        recv_contig<1>(c, loc_h + wid * 256, min(64, IS / 4 - wid * 64), tag, reinterpret_cast<uint32_t*>(hs) + wid * 256)) {
      const int q = wid * 64 + lane;  // the words this lane brought, as floats
      if (q < IS / 4) {
        const uint32_t* w4 = reinterpret_cast<const uint32_t*>(hs) + 4 * q;
        float f[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) f[e] = tw_val(w4[e]);
        *reinterpret_cast<f32x4*>(hs + 4 * q) = f32x4{f[0], f[1], f[2], f[3]};
      }
    }
    XTRACE(9);
    XSYNC();  // #5
    // ---- J: partial down_proj over the slice's columns ----
    {
      const float out = lds_row_dot<T::TPR_D, T::CPT_D>(wd + (h_live ? o_slot : 0) * IS, hs, IS);
      if (h_live && tid % T::TPR_D == 0) ll_store_buf(a.xd, g * H + hrow, out, tag);
    }
    XTRACE(10);
    // the group's next layer: its weight rows stream into registers and LDS while the other group computes (after a
    // barrier: no wave may still read this layer's rows in LDS)
    if (layer + 2 < a.L) {
      XSYNC();
      stream(layer + 2);
    }
  }
  // final hidden state x = x' + sum_k D_k of the last layer, RMSNorm input with the final gain (all blocks)
  cross_reduce2(c, wid, jj, pgrp == 0, a.xd, loc_xg, (c.phase0 + static_cast<uint32_t>(a.L) - 1u) & 3u, loc_xa,
                a.final_norm, xres, xn, red);
  XTRACE0(a.L);
  XSYNC();
  return true;
}

// LM head rows of block b = 32 g + j on all 512 threads, best (value, index) per 32-lane slot into bv/bi. The logits
// are RMSNorm(x) . W = (x * gain) . W * scale.
template <int G>
__device__ __forceinline__ void lm_head(const Ctx& c) {
  using T = Tiling<G>;
  const PersistArgs& a = c.a;
  const int tid = threadIdx.x, slot = tid / T::TPR_LM;
  const bool lead = (tid % T::TPR_LM) == 0;
  const float* xn = c.lds + Lds<G>::XN;
  const float scale = rms_scale(c.lds + Lds<G>::RED, a.H, a.eps);
  const int b = c.g * NBX + c.j;
  const int rv = (a.V + NX * NBX - 1) / (NX * NBX);
  const int v0 = b * rv, v1 = min(a.V, v0 + rv);
  constexpr int STEP = NT / T::TPR_LM;
  Slice<T::TPR_LM, T::CPT_LM> f0, f1;
  auto rowp = [&](int r) { return r < v1 ? a.lm_head + static_cast<size_t>(r) * a.H : nullptr; };
  slice_load(f0, rowp(v0 + slot), a.H);
  float best = -INFINITY;
  int best_i = 0x7fffffff;
  auto consume = [&](const Slice<T::TPR_LM, T::CPT_LM>& f, int r0) {
    const float out = slice_dot(f, xn, a.H) * scale;
    const int row = r0 + slot;
    if (row < v1) {
      if (lead && a.logits != nullptr) a.logits[row] = out;
      if (out > best) {  // a slot's rows ascend: strict > keeps the lowest index
        best = out;
        best_i = row;
      }
    }
  };
  for (int r0 = v0; r0 < v1; r0 += 2 * STEP) {
    slice_load(f1, rowp(r0 + STEP + slot), a.H);
    consume(f0, r0);
    slice_load(f0, rowp(r0 + 2 * STEP + slot), a.H);
    consume(f1, r0 + STEP);
  }
  float* bv = c.lds + Lds<G>::BV;
  int* bi = reinterpret_cast<int*>(c.lds + Lds<G>::BI);
  if (lead) {
    bv[slot] = best;
    bi[slot] = best_i;
  }
}

}  // namespace

template <int G>
__global__ __launch_bounds__(NT) void k_decode_xcd(PersistArgs a) {
  extern __shared__ float lds[];
  using LD = Lds<G>;
  int* flag = reinterpret_cast<int*>(lds + LD::FLAG);
  const int tid = threadIdx.x, wid = tid >> 6, lane = tid & 63;
  const uint32_t step = static_cast<uint32_t>(a.state[2]);
  if (tid == 0) {
    const int xcc = static_cast<int>(__builtin_amdgcn_s_getreg((3 << 11) | 20) & 15u);  // HW_REG_XCC_ID
    const int rank = xcc < NX ? atomicAdd(a.xcd_ctr + (step & 1u) * NX + xcc, 1) : NBX;
    flag[0] = 0;
    flag[1] = xcc;
    flag[2] = rank;
  }
  __syncthreads();
  const int g = flag[1], j = flag[2];
  if (j >= NBX) {  // not the expected 32 blocks per XCD: fail the step (every other block's wait then times out)
    if (tid == 0) __hip_atomic_store(a.err, 2, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    return;
  }
  Ctx c{a, g, j, a.state[0], a.state[1], (step - 1u) * static_cast<uint32_t>(a.L), lds, flag};
  if (!run_layers<G>(c)) return;
  lm_head<G>(c);
  XTRACE0(a.L + 1);

  // ---- greedy argmax over the blocks' candidates (sampler.cpp:26-61 with top_k = 1) ----
  float* bv = lds + LD::BV;
  int* bi = reinterpret_cast<int*>(lds + LD::BI);
  const int b = g * NBX + j, nb = NX * NBX;
  __syncthreads();
  if (tid == 0) {
    float v = bv[0];
    int i = bi[0];
    for (int w = 1; w < NT / Tiling<G>::TPR_LM; ++w)
      if (bv[w] > v || (bv[w] == v && bi[w] < i)) {
        v = bv[w];
        i = bi[w];
      }
    st_dev(a.part_val + b, v);
    st_dev(a.part_idx + b, i);
    wait_mem();  // the block's candidate is visible device-wide before it is counted
    const int done = __hip_atomic_fetch_add(a.counter, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    flag[3] = (done == nb - 1);
  }
  __syncthreads();
  if (flag[3] == 0) return;
  float v = -INFINITY;
  int i = 0x7fffffff;
  for (int q = tid; q < nb; q += NT) {
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
    bv[wid] = v;
    bi[wid] = i;
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
    a.state[1] = c.pos + 1;
    a.state[2] = static_cast<int>(step + 1u);
    if (a.ring != nullptr) {
      a.ring[*a.ring_pos] = tok;
      *a.ring_pos += 1;
    }
    for (int k = 0; k < NX; ++k) a.xcd_ctr[((step + 1u) & 1u) * NX + k] = 0;  // the next step's arrival counters
    __hip_atomic_store(a.counter, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
}
#undef XSYNC
#undef XTRACE
#undef XTRACE0

namespace {
template <int G>
hipError_t launch_g(const PersistArgs& a, hipStream_t s) {
  // more than 80 KB of LDS per block: one block per CU, so 32 blocks land on each XCD
  const size_t lds = std::max<size_t>(Lds<G>::TOTAL * sizeof(float), 96 * 1024);
  static size_t attr_lds = 0;
  if (attr_lds < lds) {
    hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(k_decode_xcd<G>),
                                       hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(lds));
    if (e != hipSuccess) return e;
    attr_lds = lds;
  }
  hipLaunchKernelGGL(k_decode_xcd<G>, dim3(NX * NBX), dim3(NT), lds, s, a);
  return hipGetLastError();
}
}  // namespace

hipError_t launch_decode_xcd(const PersistArgs& a, hipStream_t s) {
  const int G = a.nq / a.nkv;
  if (G == 1) return launch_g<1>(a, s);
  if (G == 2) return launch_g<2>(a, s);
  return hipErrorInvalidValue;
}

hipError_t xcd_blocks_per_cu(int G, int* blocks) {
  *blocks = 0;
  const size_t lds = std::max<size_t>((G == 1 ? Lds<1>::TOTAL : Lds<2>::TOTAL) * sizeof(float), 96 * 1024);
  if (G == 1) return hipOccupancyMaxActiveBlocksPerMultiprocessor(blocks, k_decode_xcd<1>, NT, lds);
  if (G == 2) return hipOccupancyMaxActiveBlocksPerMultiprocessor(blocks, k_decode_xcd<2>, NT, lds);
  return hipErrorInvalidValue;
}

int xcd_loc_stride(int G, int I) {
  return (((G + 2) * HD + 63) & ~63) + ((NBX * G * PW + 63) & ~63) + ((I / NX + 63) & ~63) + 2 * (HMAX + 64);
}

// Shapes the partition and the register tiling cover: 8 KV heads of 128 dims (one per XCD), G = 1 or 2 query heads
// per KV head, hidden size a multiple of 256 up to 1024, intermediate size a multiple of 256 up to 3072, and a device
// of 8 XCDs x 32 CUs.
bool xcd_supported(int H, int I, int nq, int nkv, int head_dim, int num_cus) {
  if (num_cus != NX * NBX || nkv != NX || head_dim != HD) return false;
  const int G = nq / nkv;
  if (nq % nkv != 0 || (G != 1 && G != 2)) return false;
  if (H % 256 != 0 || H > HMAX) return false;  // each of a block's 8 waves reduces whole 8-line loads
  if (I % (NX * NBX) != 0 || I > IMAX) return false;
  return true;
}

}  // namespace soc
