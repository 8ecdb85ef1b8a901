// decode_xcd.hip - one-launch decode for batch 1 with every layer partitioned over the eight XCDs of MI355X, the
// layers alternating between two groups of blocks, and every dot product of a layer on the matrix cores. One launch
// runs a.steps decode steps: the blocks stay resident from token to token, the last block to finish a step's LM head
// hands the greedy token to the next step through one device word, and with an even layer count group 0, which has
// nothing to compute during the last layer, streams the next step's first layer then (instead of every step starting
// with a whole layer's rows to load).
//
// Block (g, j): XCD g, read from the XCC_ID hardware register, and rank j < 32 among the blocks of this launch that
// arrived on it. Group p = j / 16 computes the layers l with l % 2 == p while the other group streams the weight rows
// of its next layer into registers and LDS: a CU never waits on hand-offs while its own weight loads are in flight
// (its vector memory requests would queue behind them). XCD g owns KV head g (every Qwen3 model has 8 KV heads) with
// its G = nq / 8 query heads and 1/8 of every matrix: the q/k/v rows of its heads, the o_proj columns of its query
// heads, the gate/up rows and down_proj columns of its eighth of the intermediate dimension; the group's 16 blocks of
// the XCD split that share. Per layer (reference: QwenBlock::ForwardCached, Mac/cpu/src/qwen_block.cpp:63-73, with
// QwenAttention::ForwardCached and QwenMLP::Forward):
//   A  x = x' + sum_k D_k: the previous layer's residual and its eight XCDs' partial down outputs (cross-XCD), RMSNorm
//   B  the block's q/k/v rows of the XCD's heads                                   -> XCD-local exchange
//   C  the XCD's q/k/v; per-head QK-RMSNorm + RoPE; rank 0 appends k and v to the cache
//   D  causal attention over the block's share of the keys, 32-key tiles per wave, the waves' partials merged in LDS
//   E  the XCD's block partials (XCD-local), log-sum-exp merge (more than 256 keys only)
//   F  O_g = Wo[the block's rows][the XCD's query columns] . attn                  -> cross-XCD exchange
//   G  x' = x + sum_k O_k (cross-XCD), RMSNorm; the block publishes its rows of x' for the other group
//   H  h = silu(gate) * up on the block's share of the XCD's intermediate slice     -> XCD-local exchange
//   I  the XCD's h slice (XCD-local)
//   J  D_g = Wd[the block's rows][the slice's columns] . h                         -> cross-XCD exchange
//
// Matrix cores (v_mfma_f32_16x16x32_f16) for a vector times a matrix: the fp32 vector enters as two fp16 rows of the
// A operand, hi = f16(v) and lo = f16((v - hi) 2^11) (about 22 bits of v; the weights are exact fp16, every product is
// exact in fp32 and the sums are fp32), 16 weight rows form the B operand, and lanes 0..15 receive row j's
// hi-sum and lo-sum, added as hi + lo 2^-11. The other 14 rows of A are zero: at batch 1 the matrix cores are idle
// most of the time anyway, and one MFMA replaces 512 FMAs and their fp16 conversions on the vector ALUs, which at
// one 512-thread block per CU were what bounded every compute phase. q/k/v and gate/up rows sit in registers (each
// wave holds 1/8 of K for all of the block's rows, and the eight partial sums meet in LDS); o_proj and down_proj rows
// sit in LDS with 16-byte chunks XOR-swizzled by row (conflict-free operand reads) and each wave takes 16 rows over
// the whole K. Attention: a wave takes 32-key tiles; S^T = q . K^T with q's hi/lo rows (prescaled by scale log2 e) as
// A and 16 keys straight from the cache as B, base-2 softmax with a running maximum per wave, then O = P . V with P's
// hi/lo rows as A and V^T from the transposing LDS read of the tile (brought global -> LDS by range-checked buffer
// loads, so keys at or past `pos` read as zero).
//
// Cross-XCD words are written with device-scope stores; XCD-local ones with plain stores served by the XCD's own L2
// (see exchange.h). Every block of the computing group holds the whole residual stream in LDS, computed in the same
// order from the same words, so all blocks hold identical bits. Every wait is bounded; a timeout raises the error flag
// and the grid drains.
#include <algorithm>

#include "exchange.h"
#include "kernels.h"

namespace soc {

namespace {

constexpr int NT = 512;           // threads per block
constexpr int NW = NT / 64;       // waves per block
constexpr int HD = 128;           // head dim
constexpr int NX = kXcdGroups, NBX = kXcdBlocks;
constexpr int NBG = NBX / 2;      // blocks of one group on one XCD
constexpr int HMAX = 1024;        // hidden size covered by the register tiling
constexpr int IMAX = 3072;        // intermediate size covered: I / 128 <= 24 gate/up pairs per block
constexpr int ISM = IMAX / NX;    // intermediate slice of an XCD at most
constexpr int PW = HD + 4;        // words per (block, query head) attention partial: 128 values, max, sum, 2 pad
constexpr int KT = 32;            // keys per attention tile (the K depth of one P . V MFMA)
constexpr int KALL = NW * KT;     // up to this many keys every block computes its KV head's whole attention
constexpr float kNoKeys = -1e30f; // running max of a wave or block that owns no key (finite: exp2 of it is 0)
constexpr float kLo = 1.0f / 2048.0f;

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef __fp16 hv4 __attribute__((__vector_size__(4 * sizeof(__fp16))));  // operand type of the transposing read
typedef __attribute__((address_space(3))) void lds_void;

__device__ __forceinline__ h8 as_h8(u32x4 v) { return __builtin_bit_cast(h8, v); }
__device__ __forceinline__ f32x4 mfma16(h8 a, h8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

// A block's LM-head rows in registers: slot s = tid / TPR owns one row; thread t of the slot holds the 8-half chunks
// at k = 8 (t + TPR c), c < CPT.
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

// XOR mask of the 16-byte chunk swizzle of an LDS row of `cpr` chunks: chunk c of row r is stored at c ^ (r & mask),
// with mask + 1 the largest power of two (at most 16) that divides cpr, so the swizzled chunk stays in the row.
__device__ __forceinline__ int swz_mask(int cpr) { return min(16, cpr & -cpr) - 1; }

// A block of `rows` rows of `K` halves (row r at src + r * ld) straight to LDS with 16-byte global -> LDS loads, one
// 1 KB wave instruction per 64 chunks, into rows of CPR >= K / 8 chunks: chunk c of row r is stored at slot
// c ^ (r & swz_mask(CPR)) of dst row r, and slots whose chunk lies past K hold a copy of the row's first chunk (finite
// values that meet zero operands), so the consumers run a fixed number of MFMA steps for every K.
template <int CPR>
__device__ __forceinline__ void rows_to_lds(const f16* src, size_t ld, int rows, int K, f16* dst) {
  const int wid = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int cpr = K / 8, nch = rows * CPR, msk = swz_mask(CPR);
  for (int c0 = wid * 64; c0 < nch; c0 += NT) {
    const int ch = min(c0 + lane, nch - 1), row = ch / CPR, slot = ch % CPR, col = slot ^ (row & msk);
    __builtin_amdgcn_global_load_lds(src + static_cast<size_t>(row) * ld + (col < cpr ? col : 0) * 8,
                                     (lds_void*)(dst + c0 * 8), 16, 0, 0);
  }
}

// hl[i .. i+3] = f16(y), hl[ld + i ..] = f16((y - hi) 2^11): the hi/lo rows of a vector operand.
__device__ __forceinline__ void store_hl4(f16* hl, int ld, int i, f32x4 y) {
  f16x4 hi, lo;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    float v = y[e];
    __asm__ volatile("" : "+v"(v));  // hi and lo come from the same rounded fp32 value
    hi[e] = static_cast<f16>(v);
    lo[e] = static_cast<f16>((v - static_cast<float>(hi[e])) * 2048.0f);
  }
  *reinterpret_cast<f16x4*>(hl + i) = hi;
  *reinterpret_cast<f16x4*>(hl + ld + i) = lo;
}

// Register tiling of a block's share of one layer. Each wave holds K slice [w H/8, (w+1) H/8) of all the block's
// q/k/v rows (QT tiles of 16) and gate/up rows (GT tiles: the gate rows, then the up rows) as MFMA B operands:
// lane (j, kq) of tile t, step s holds row 16 t + j, halves k0 + 32 s + 8 kq .. + 8.
template <int G>
struct Tiling {
  static constexpr int RQ = (G + 2) * 8;          // q/k/v rows per block
  static constexpr int QT = (RQ + 15) / 16;
  static constexpr int RIM = ISM / NBG;           // gate/up pairs per block at most
  static constexpr int GT = (2 * RIM + 15) / 16;
  static constexpr int SW = HMAX / NW / 32;       // MFMA steps of a wave's K slice at most
  static constexpr int RHM = HMAX / NBG;          // o/down rows per block at most (16 per wave: RHM / 16 waves)
  static constexpr int GHD = G * HD;              // o_proj columns of the XCD
  static constexpr int TPR_LM = 32, CPT_LM = HMAX / (TPR_LM * 8);  // LM head: 16 rows per fragment
  static constexpr int MQ_E = (NBG * PW / 4 + 63) / 64;            // one head's block-partial quads per lane
  static_assert(RHM / 16 <= NW, "o/down tiles");
};

// LDS carve-up, byte offsets.
template <int G>
struct Lds {
  static constexpr int XRES = 0;                               // fp32 [HMAX] residual stream x / x'
  static constexpr int XHL = XRES + HMAX * 4;                  // fp16 [2][HMAX] hi/lo of x * gain (next RMSNorm)
  static constexpr int HHL = XHL + 2 * HMAX * 2;               // fp16 [2][ISM] hi/lo of the XCD's h slice
  static constexpr int AHL = HHL + 2 * ISM * 2;                // fp16 [2][G HD] hi/lo of the attention output
  static constexpr int QHL = AHL + 2 * G * HD * 2;             // fp16 [2G][HD] hi/lo rows of q * scale * log2 e
  static constexpr int KN = QHL + 2 * G * HD * 2;              // fp16 [HD] new key
  static constexpr int VN = KN + HD * 2;                       // fp16 [HD] new value
  static constexpr int PT = VN + HD * 2;                       // fp16 [NW][2G][KT] the waves' softmax weights
  static constexpr int RED = PT + NW * 2 * G * KT * 2;         // fp32 [16] partial sums of squares
  static constexpr int FLAG = RED + 16 * 4;                    // int [8] status, g, j, last block
  static constexpr int BV = FLAG + 8 * 4;                      // fp32 [16] argmax values per slot
  static constexpr int BI = BV + 16 * 4;                       // int [16] argmax indices
  static constexpr int PART = BI + 16 * 4;                     // fp32 [NW][GT 16] the projections' partial sums
  // fp16 [NW][KT][HD] the waves' V tiles (a wave's first tile is requested at the start of its layer). Phases that
  // never overlap the attention tiles use the same bytes: the waves' attention partials, E's block partials, the
  // final x * gain of the LM head.
  static constexpr int VT = PART + NW * Tiling<G>::GT * 16 * 4;
  static constexpr int WD = VT + NW * KT * HD * 2;             // fp16 [HMAX / 16][ISM] down_proj rows (swizzled)
  static constexpr int WO = WD + (HMAX / NBG) * ISM * 2;       // fp16 [HMAX / 16][G HD] o_proj rows (swizzled)
  static constexpr int TOTAL = WO + (HMAX / NBG) * G * HD * 2;
  static_assert(VT % 16 == 0 && WD % 16 == 0 && WO % 16 == 0, "16-byte aligned operand rows");
  static_assert(TOTAL <= 160 * 1024, "LDS of one CU");
  static_assert(G * NBG * PW * 4 <= NW * KT * HD * 2 && HMAX * 4 <= NW * KT * HD * 2, "VT reuse");
};

// cross_reduce2's first stage runs on this many waves, wave w's first poll issued w * kStage1Stagger sleep units
// (64 clocks each) after wave 0's.
constexpr int kStage1Waves = 4, kStage1Stagger = 8;

struct Ctx {
  const PersistArgs& a;
  int g, j, token, pos;
  uint32_t phase0;  // (step - 1) * L: the tag of layer l is (phase0 + l) & 3
  uint32_t step;    // this step's number (state[3] when it started; steps count from 1)
  uint32_t step1;   // the launch's first step
  int ring1;        // ring slot of the launch's first token
  char* lds;
  int* flag;  // LDS: [0] a wait failed, [1] XCD, [2] rank, [3] last block, [4] cross_reduce2 stage-1 marker
};

// Attention blocks of the XCD's computing group for S keys (at most 16, whole 32-key tiles each) and keys per block;
// na is recomputed from the chunk so that every block jj < na owns at least one key.
__device__ __forceinline__ void attn_split(int S, int& na, int& chunk) {
  na = min(NBG, (S + KT - 1) / KT);
  chunk = ((S + na - 1) / na + KT - 1) / KT * KT;
  na = (S + chunk - 1) / chunk;
}

// RMSNorm scale 1 / sqrt(sum x^2 / n + eps) from the eight waves' partial sums, added in a fixed order.
__device__ __forceinline__ float rms_scale(const float* red, int n, float eps) {
  const float s = ((red[0] + red[1]) + (red[2] + red[3])) + ((red[4] + red[5]) + (red[6] + red[7]));
  return 1.0f / sqrtf(s / static_cast<float>(n) + eps);
}

// Optional phase timestamps (diagnostics): lane 0 of every wave of the middle layer's group writes its phase points to
// trace[kTraceWaveBase + (block * 8 + wave) * kTracePts + point]; block 0 of each group on XCD 0 also writes its
// layers' starts, the final norm and the step's end into trace[256 * kTracePts + i].
// (The wave's slot, trw, is a wave-uniform pointer computed once per step, nullptr without a trace.)
#define XTRACE(pt)                                                                                           \
  do {                                                                                                       \
    if (trw != nullptr && layer == c.a.L / 2 && (threadIdx.x & 63) == 0) trw[pt] = now_ticks();               \
  } while (0)
#define XTRACE0(i)                                                                                           \
  do {                                                                                                       \
    if (c.a.trace != nullptr && threadIdx.x == 0 && c.g == 0 && c.j % NBG == 0)                              \
      c.a.trace[NX * NBX * kTracePts + (i)] = now_ticks();                                                   \
  } while (0)

// Same, recorded by lane 0 of the wave that takes the first attention tile.
#define XTRACEW(pt) XTRACE(pt)

// Block barrier; afterwards every thread leaves if a wave reported a failed wait (flag[0] != 0).
#define XSYNC()                       \
  do {                                \
    __syncthreads();                  \
    if (c.flag[0] != 0) return false; \
  } while (0)

// A failed wait: the error flag keeps a placement error (2) over a timeout (1); the block leaves at its next barrier.
__device__ __forceinline__ void wait_failed(const Ctx& c) {
  __hip_atomic_fetch_max(c.a.err, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  c.flag[0] = 1;
}

__device__ __forceinline__ bool give_up(const Ctx& c, uint32_t& spins, uint64_t t0) {
  return (++spins & 63) == 0 && (now_ticks() - t0 > c.a.spin_ticks || err_raised(c.a.err));
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
    if (give_up(c, spins, t0)) {
      wait_failed(c);
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

// Wave: words lane and lane + 64 of a 128-word XCD-local tagged vector (one head of the XCD's q/k/v), into registers.
__device__ __forceinline__ bool recv_head(const Ctx& c, const uint32_t* src, uint32_t tag, float& x0, float& x1) {
  int lane = threadIdx.x & 63;
  __asm__ volatile("" : "+v"(lane));
  const __amdgpu_buffer_rsrc_t r = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint32_t*>(src), 0, HD * 4, 0x00020000);
  // two staggered reads in flight (kStaggerLocal); every re-read is unconditional so the in-flight count is fixed
  uint32_t w0 = __builtin_amdgcn_raw_buffer_load_b32(r, lane * 4, 0, 16);
  uint32_t w1 = __builtin_amdgcn_raw_buffer_load_b32(r, lane * 4 + 256, 0, 16);
  stagger<kStaggerLocal>();
  uint32_t u0 = __builtin_amdgcn_raw_buffer_load_b32(r, lane * 4, 0, 16);
  uint32_t u1 = __builtin_amdgcn_raw_buffer_load_b32(r, lane * 4 + 256, 0, 16);
  const uint64_t t0 = now_ticks();
  uint32_t spins = 0;
  while (true) {
    if (__all(tw_tag(w0) == tag && tw_tag(w1) == tag)) break;
    if (give_up(c, spins, t0)) {
      wait_failed(c);
      return false;
    }
    w0 = __builtin_amdgcn_raw_buffer_load_b32(r, lane * 4, 0, 16);
    w1 = __builtin_amdgcn_raw_buffer_load_b32(r, lane * 4 + 256, 0, 16);
    if (__all(tw_tag(u0) == tag && tw_tag(u1) == tag)) {
      w0 = u0;
      w1 = u1;
      break;
    }
    u0 = __builtin_amdgcn_raw_buffer_load_b32(r, lane * 4, 0, 16);
    u1 = __builtin_amdgcn_raw_buffer_load_b32(r, lane * 4 + 256, 0, 16);
  }
  x0 = tw_val(w0);
  x1 = tw_val(w1);
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

// Wave w < 8 of the block: its eighth of x = embedding row (layer 0, embedding.cpp:51-77), into xres, the hi/lo
// rows of x * gain into xhl and its partial sum of x^2 into red[w] (the RMSNorm of rms_norm_module.cpp:56-64 is
// completed by rms_scale). The wave owns the element quads w * H / 32 .. + H / 32. embed_fetch requests the quads and
// gains, embed_finish consumes them (the first layer's first key tile is requested in between).
struct EmbedFetch {
  f16x4 e[HMAX / 256], g[HMAX / 256];
};
__device__ __forceinline__ void embed_fetch(const Ctx& c, int w, const f16* embed_row, const f16* gain, EmbedFetch& f) {
  constexpr int NI = HMAX / 256;
  int lane = threadIdx.x & 63;
  __asm__ volatile("" : "+v"(lane));
  const int H = c.a.H, ni = H / 256, q0 = w * (H / 32);
#pragma unroll
  for (int i = 0; i < NI; ++i) {
    const int q = i < ni ? q0 + i * 8 + (lane >> 3) : q0;  // quads past the slice re-read its first (unused)
    f.e[i] = ld_global(reinterpret_cast<const f16x4*>(embed_row), q);
    f.g[i] = ld_global(reinterpret_cast<const f16x4*>(gain), q);
  }
}
__device__ __forceinline__ void embed_finish(const Ctx& c, int w, const EmbedFetch& f, float* xres, f16* xhl,
                                             float* red) {
  constexpr int NI = HMAX / 256;
  int lane = threadIdx.x & 63;
  __asm__ volatile("" : "+v"(lane));
  const int H = c.a.H, ni = H / 256, q0 = w * (H / 32);
  float ss = 0.0f;
#pragma unroll
  for (int i = 0; i < NI; ++i) {
    const int q = q0 + i * 8 + (lane >> 3);
    if (i < ni && (lane & 7) == 0) {
      f32x4 x, y;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        x[e] = static_cast<float>(f.e[i][e]);
        y[e] = x[e] * static_cast<float>(f.g[i][e]);
        ss += x[e] * x[e];
      }
      *reinterpret_cast<f32x4*>(xres + 4 * q) = x;
      store_hl4(xhl, HMAX, 4 * q, y);
    }
  }
  ss = wave_sum(ss);
  if (lane == 0) red[w] = ss;
}

// x = base + sum_k P_k over the eight XCDs' partials P_k (src, [8][H] words), reading each remote partial once per
// XCD instead of once per block:
// stage 1 (waves 0 .. kStage1Waves - 1 of a block with do1, staggered; the first to see the partials writes, and
//   marks the call done with `marker`, positive and unique among one launch's calls): the block's 1/16 of the
//   elements, quads jj * H/64 ..; base from base_loc (XCD-local words) or, if null, from xres; x goes to out[0, H)
//   and the block's sum of squares of x to out[H + jj], as XCD-local words with the same tag;
// stage 2 (every wave): all of x and the 16 sums from out; x into xres, the hi/lo rows of x * gain into xhl (or, with
//   xn32 set, x * gain in fp32 into xn32), red[0..7] = pair sums of the 16 sums (rms_scale adds them in a fixed
//   order). Every block reads the same words, so x and the norm agree in every block of every XCD. The caller's
//   barrier publishes xres, xhl / xn32 and red.
__device__ __forceinline__ bool cross_reduce2(const Ctx& c, int w, int jj, bool do1, const uint32_t* src,
                                              const uint32_t* base_loc, uint32_t tag, uint32_t* out, const f16* gain,
                                              float* xres, f16* xhl, float* xn32, float* red, int marker,
                                              int trace_pt = -1) {
  int lane = threadIdx.x & 63;
  __asm__ volatile("" : "+v"(lane));  // per call: keeps the compiler from hoisting per-lane addresses out of the layers
  const int H = c.a.H;
  const u32x4 filler = {tag, tag, tag, tag};
  const uint64_t t0 = now_ticks();
  // stage 1 on kStage1Waves waves, the first polls of wave w issued w * kStage1Stagger sleep units after wave 0's:
  // whichever wave sees the remote partials first writes the block's elements (every wave computes the same bits),
  // then marks the call done in flag[4] so the others stop polling
  if (w < kStage1Waves && do1) {
    const int k = lane & 7, nq1 = H / 64, qb = jj * nq1;
    const __amdgpu_buffer_rsrc_t r =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<uint32_t*>(src), 0, H * NX * 4, 0x00020000);
    const __amdgpu_buffer_rsrc_t rb = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint32_t*>(base_loc != nullptr ? base_loc : src), 0, H * 4, 0x00020000);
    uint32_t spins = 0;
    // the base first, into registers: from the XCD-local words (written a phase earlier: normally already there) or
    // from xres, which stage 2 of a faster wave may overwrite while this wave still polls
    f32x4 bx[2];
    if (base_loc != nullptr) {
      u32x4 bq[2];
      auto read_b = [&]() {
#pragma unroll
        for (int i = 0; i < 2; ++i) {
          const int qi = (lane >> 3) + 8 * i;
          const u32x4 tb = ll_peek_buf4(rb, (qb + min(qi, nq1 - 1)) * 16);
          bq[i] = qi < nq1 && k == 0 ? tb : filler;
        }
      };
      read_b();
      while (!__all(tw_quad_ok(bq[0], tag) && tw_quad_ok(bq[1], tag))) {
        if (give_up(c, spins, t0)) {
          wait_failed(c);
          return false;
        }
        read_b();
      }
#pragma unroll
      for (int i = 0; i < 2; ++i) bx[i] = f32x4{tw_val(bq[i].x), tw_val(bq[i].y), tw_val(bq[i].z), tw_val(bq[i].w)};
    } else {
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        const int qi = (lane >> 3) + 8 * i;
        bx[i] = *reinterpret_cast<const f32x4*>(xres + 4 * (qb + min(qi, nq1 - 1)));
      }
    }
    poll_pause(w * kStage1Stagger);
    // remote partials; reads unconditional (a dead lane's words are replaced by the filler after the load)
    u32x4 v[2];
    auto read_v = [&]() {
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        const int qi = (lane >> 3) + 8 * i;
        const u32x4 tv = ll_peek_buf4(r, (k * H + 4 * (qb + min(qi, nq1 - 1))) * 4);
        v[i] = qi < nq1 ? tv : filler;
      }
    };
    read_v();
    bool mine = true;
    while (!__all(tw_quad_ok(v[0], tag) && tw_quad_ok(v[1], tag))) {
      if (*reinterpret_cast<volatile int*>(&c.flag[4]) == marker) {  // another wave of the block was first
        mine = false;
        break;
      }
      if (give_up(c, spins, t0)) {
        wait_failed(c);
        return false;
      }
      read_v();
    }
    if (mine) {
      const __amdgpu_buffer_rsrc_t ro = __builtin_amdgcn_make_buffer_rsrc(out, 0, (H + NBG) * 4, 0x00020000);
      float ss = 0.0f;
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        const int qi = (lane >> 3) + 8 * i, q = qb + qi;
        const float s0 = sum8(tw_val(v[i].x)), s1 = sum8(tw_val(v[i].y));
        const float s2 = sum8(tw_val(v[i].z)), s3 = sum8(tw_val(v[i].w));
        if (qi < nq1 && k == 0) {
          f32x4 x = bx[i];
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
      if (lane == 0) {
        ll_store_local(out, H + jj, ss, tag);
        c.flag[4] = marker;
      }
      if (trace_pt >= 0 && c.a.trace != nullptr && lane == 0)
        c.a.trace[(c.g * NBX + c.j) * kTracePts + trace_pt] = now_ticks();  // stage 1 done (diagnostics)
    }
  }
  // stage 2: waves 0..3 take quad w * H/16 + lane of x, wave 4's lanes 0..3 the 16 sums (fewer waves polling L2)
  const int per = H / 16;
  const bool xlive = w < 4 && lane < per, slive = w == 4 && lane < 4;
  const int off = xlive ? (w * per + lane) * 16 : (H + 4 * lane) * 4;
  const __amdgpu_buffer_rsrc_t ro = __builtin_amdgcn_make_buffer_rsrc(out, 0, (H + NBG) * 4, 0x00020000);
  // the gains of the lane's quad are requested before the poll: they do not depend on the exchanged words
  const f16x4 g4 = xlive ? ld_global(reinterpret_cast<const f16x4*>(gain), w * per + lane) : f16x4{0, 0, 0, 0};
  // two staggered reads in flight (kStaggerLocal), unconditional (dead lanes read in range or past the resource's
  // end, which returns zeros, and take the filler)
  const bool live = xlive || slive;
  u32x4 t = ll_peek_buf4(ro, off);
  u32x4 v = live ? t : filler;
  stagger<kStaggerLocal>();
  t = ll_peek_buf4(ro, off);
  u32x4 v2 = live ? t : filler;
  uint32_t spins = 0;
  while (true) {
    if (__all(tw_quad_ok(v, tag))) break;
    if (give_up(c, spins, t0)) {
      wait_failed(c);
      return false;
    }
    t = ll_peek_buf4(ro, off);
    v = live ? t : filler;
    if (__all(tw_quad_ok(v2, tag))) {
      v = v2;
      break;
    }
    t = ll_peek_buf4(ro, off);
    v2 = live ? t : filler;
  }
  if (xlive) {
    const int q = w * per + lane;
    const f32x4 x = {tw_val(v.x), tw_val(v.y), tw_val(v.z), tw_val(v.w)};
    f32x4 y;
#pragma unroll
    for (int e = 0; e < 4; ++e) y[e] = x[e] * static_cast<float>(g4[e]);
    *reinterpret_cast<f32x4*>(xres + 4 * q) = x;
    if (xn32 != nullptr)
      *reinterpret_cast<f32x4*>(xn32 + 4 * q) = y;
    else
      store_hl4(xhl, HMAX, 4 * q, y);
  }
  if (slive) {
    const int m = lane;
    red[2 * m] = tw_val(v.x) + tw_val(v.y);
    red[2 * m + 1] = tw_val(v.z) + tw_val(v.w);
  }
  return true;
}

// LM head rows of block b = 32 g + j on all 512 threads, best (value, index) per 32-lane slot into bv/bi. The logits
// are RMSNorm(x) . W = (x * gain) . W * scale.
template <int G>
__device__ __forceinline__ void lm_head(const Ctx& c) {
  using T = Tiling<G>;
  using LD = Lds<G>;
  const PersistArgs& a = c.a;
  const int tid = threadIdx.x, slot = tid / T::TPR_LM;
  const bool lead = (tid % T::TPR_LM) == 0;
  const float* xn = reinterpret_cast<const float*>(c.lds + LD::VT);
  const float scale = rms_scale(reinterpret_cast<const float*>(c.lds + LD::RED), a.H, a.eps);
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
  float* bv = reinterpret_cast<float*>(c.lds + LD::BV);
  int* bi = reinterpret_cast<int*>(c.lds + LD::BI);
  if (lead) {
    bv[slot] = best;
    bi[slot] = best_i;
  }
}

// Greedy token of the step (sampler.cpp:26-61 with top_k = 1): every block's best (value, index) over its LM-head
// rows is published and counted; the last block to arrive picks the best (lowest index on ties) and writes it to the
// ring. Within a launch the next step learns its token from one 64-bit word {step, token} (state[8..9]), written and
// read with device scope and no fence: nothing else the last block writes is read before the launch ends. The
// arrival counter only grows during a launch (a step's last block sees a multiple of the block count); the launch's
// last step resets it and writes the state the next launch starts from.
template <int G>
__device__ __forceinline__ void finish_step(const Ctx& c) {
  using LD = Lds<G>;
  const PersistArgs& a = c.a;
  const int tid = threadIdx.x, wid = tid >> 6, lane = tid & 63;
  float* bv = reinterpret_cast<float*>(c.lds + LD::BV);
  int* bi = reinterpret_cast<int*>(c.lds + LD::BI);
  const int b = c.g * NBX + c.j, nb = NX * NBX;
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
    c.flag[3] = (done + 1) % nb == 0;
  }
  __syncthreads();
  if (c.flag[3] == 0) return;
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
    const int k = static_cast<int>(c.step - c.step1);  // the step's index in this launch
    if (a.ring != nullptr) __hip_atomic_store(a.ring + c.ring1 + k, tok, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (k + 1 < a.steps) {
      const uint64_t word = (static_cast<uint64_t>(c.step + 1u) << 32) | static_cast<uint32_t>(tok);
      __hip_atomic_store(reinterpret_cast<uint64_t*>(a.state + 8), word, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    } else {  // the launch's last step: the next launch's start
      a.state[0] = tok;
      a.state[1] = c.pos + 1;
      a.state[3] = static_cast<int>(c.step + 1u);
      if (a.ring != nullptr) *a.ring_pos = c.ring1 + a.steps;
      for (int x = 0; x < NX; ++x) a.xcd_ctr[((c.step + 1u) & 1u) * NX + x] = 0;  // the next launch's arrivals
      __hip_atomic_store(a.counter, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
}

// Start of the launch's next step: thread 0 waits (bounded) for the previous step's word {step, token}; every thread
// takes the token from LDS; the position advances by one.
template <int G>
__device__ __forceinline__ bool next_step(Ctx& c) {
  const PersistArgs& a = c.a;
  const uint32_t want = c.step + 1u;
  if (threadIdx.x == 0) {
    const uint64_t t0 = now_ticks();
    uint32_t spins = 0;
    uint64_t w;
    while (true) {
      w = __hip_atomic_load(reinterpret_cast<const uint64_t*>(a.state + 8), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      if (static_cast<uint32_t>(w >> 32) == want) break;
      if (give_up(c, spins, t0)) {
        wait_failed(c);
        break;
      }
      __builtin_amdgcn_s_sleep(1);
    }
    c.flag[5] = static_cast<int>(static_cast<uint32_t>(w));
    c.flag[4] = 0;  // cross_reduce2's stage-1 marker
  }
  __syncthreads();
  if (c.flag[0] != 0) return false;
  c.token = __builtin_amdgcn_readfirstlane(c.flag[5]);  // uniform: scalar registers
  c.pos += 1;
  c.step = want;
  c.phase0 += static_cast<uint32_t>(a.L);
  return true;
}

// The a.steps decode steps of one launch: per step, the layers l % 2 == p for a block of group p, the final hidden
// state (all blocks), the LM head and the greedy token.
template <int G>
__device__ __forceinline__ bool run_steps(Ctx& c) {
  using T = Tiling<G>;
  using LD = Lds<G>;
  const PersistArgs& a = c.a;
  const int tid = threadIdx.x, wid = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave index, kept in an SGPR
  const int g = c.g, pgrp = c.j / NBG, jj = c.j % NBG;
  uint64_t* const trw =
      a.trace != nullptr ? a.trace + kTraceWaveBase + ((g * NBX + c.j) * NW + wid) * kTracePts : nullptr;
  const int H = a.H, I = a.I, qd = a.qd;
  const int RH = H / NBG;          // o/down rows per block
  const int IS = I / NX;           // intermediate slice of the XCD
  const int RI = IS / NBG;         // gate/up pairs per block
  const int kw0 = wid * (H / NW);  // this wave's K slice of the projections from the hidden state
  const int sw = H / NW / 32;      // and its MFMA steps (the registers past them hold zeros)
  char* L = c.lds;
  float* xres = reinterpret_cast<float*>(L + LD::XRES);
  f16* xhl = reinterpret_cast<f16*>(L + LD::XHL);
  f16* hhl = reinterpret_cast<f16*>(L + LD::HHL);
  f16* ahl = reinterpret_cast<f16*>(L + LD::AHL);
  f16* qhl = reinterpret_cast<f16*>(L + LD::QHL);
  f16* kn = reinterpret_cast<f16*>(L + LD::KN);
  f16* vn = reinterpret_cast<f16*>(L + LD::VN);
  f16* pt = reinterpret_cast<f16*>(L + LD::PT) + wid * 2 * G * KT;  // this wave's [2G][KT] softmax weights
  float* red = reinterpret_cast<float*>(L + LD::RED);
  char* vtb = L + LD::VT;
  f16* vt = reinterpret_cast<f16*>(vtb + wid * KT * HD * 2);        // this wave's V tile [KT][HD] (swizzled)
  float* part = reinterpret_cast<float*>(L + LD::PART);              // [NW][GT 16] projection partial sums
  f16* wd = reinterpret_cast<f16*>(L + LD::WD);
  f16* wo = reinterpret_cast<f16*>(L + LD::WO);
  uint32_t* loc = a.loc + static_cast<size_t>(g) * a.loc_stride;
  uint32_t* loc_qkv = loc;                                  // [(G + 2) HD]
  uint32_t* loc_att = loc + (((G + 2) * HD + 63) & ~63);    // [G][NBX][PW]
  uint32_t* loc_h = loc_att + ((NBX * G * PW + 63) & ~63);  // [IS]
  uint32_t* loc_xa = loc_h + ((IS + 63) & ~63);               // [H + 16]: x after the attention-input reduction
  uint32_t* loc_xg = loc_xa + HMAX + 64;                      // [H + 16]: x' after the o_proj reduction
  constexpr int PST = T::GT * 16;                             // partial-sum row stride of a wave
  int lane = tid & 63, rl = lane & 15, kq = lane >> 4;
  // this block's local q/k/v row lr of the XCD's (G + 2) * 128 (q heads, key, value) as a row of the fused matrix
  auto qkv_row = [&](int lr) {
    return lr < G * HD ? g * G * HD + lr
                       : (lr < (G + 1) * HD ? qd + g * HD + (lr - G * HD) : qd + a.nkv * HD + g * HD + (lr - (G + 1) * HD));
  };
  // The block's slot of the XCD's attention partials when it owns no keys (every block in the short-context path,
  // blocks jj >= na in the split path): max kNoKeys, sum 0. Every slot is written in every layer, so every word of
  // the region carries the tag of one of the two latest layers and a later phase can never mistake a stale word for
  // a fresh one, whatever the layer count and however na changes from step to step.
  auto keyless_partial = [&](uint32_t tg) {
    for (int t = tid; t < G * PW; t += NT) {
      const int h = t / PW, d = t % PW;
      ll_store_local(loc_att, (h * NBX + jj) * PW + d, d == HD ? kNoKeys : 0.0f, tg);
    }
  };

  u32x4 wq[T::QT][T::SW], wg[T::GT][T::SW];
  // the weight rows of layer `layer`: q/k/v and gate/up slices into registers, o_proj and down_proj rows into LDS
  auto stream = [&](int layer) {
    int l16 = rl, k8 = kq * 8;
    __asm__ volatile("" : "+v"(l16), "+v"(k8));  // recomputed per call: no 64-bit row offsets live across layers
    const f16* W4 = ld_global(a.layer_w, static_cast<size_t>(layer) * 9 + 4);
    const f16* W5 = ld_global(a.layer_w, static_cast<size_t>(layer) * 9 + 5);
    const f16* W6 = ld_global(a.layer_w, static_cast<size_t>(layer) * 9 + 6);
    const f16* W7 = ld_global(a.layer_w, static_cast<size_t>(layer) * 9 + 7);
    const f16* W8 = ld_global(a.layer_w, static_cast<size_t>(layer) * 9 + 8);
#pragma unroll
    for (int t = 0; t < T::QT; ++t) {
      const int r = 16 * t + l16;
      const f16* row = r < T::RQ ? W4 + static_cast<size_t>(qkv_row(jj * T::RQ + r)) * H + kw0 + k8 : nullptr;
#pragma unroll
      for (int s = 0; s < T::SW; ++s) wq[t][s] = (row != nullptr && s < sw) ? load_stream16(row + 32 * s) : u32x4{0, 0, 0, 0};
    }
#pragma unroll
    for (int t = 0; t < T::GT; ++t) {
      const int r = 16 * t + l16;
      const int ir = g * IS + jj * RI + (r < RI ? r : r - RI);
      const f16* row = r < 2 * RI ? (r < RI ? W6 : W7) + static_cast<size_t>(ir) * H + kw0 + k8 : nullptr;
#pragma unroll
      for (int s = 0; s < T::SW; ++s) wg[t][s] = (row != nullptr && s < sw) ? load_stream16(row + 32 * s) : u32x4{0, 0, 0, 0};
    }
    rows_to_lds<T::GHD / 8>(W5 + static_cast<size_t>(jj * RH) * qd + g * G * HD, qd, RH, G * HD, wo);
    rows_to_lds<ISM / 8>(W8 + static_cast<size_t>(jj * RH) * I + g * IS, I, RH, IS, wd);
  };
  // vector A operand of one MFMA step over columns k .. k + 32: rows 0 and 1 = hi and lo rows of hl (row stride ld),
  // rows 2..15 zero
  auto vec_operand = [&](const f16* hl, int ld, int k) -> h8 {
    return rl < 2 ? *reinterpret_cast<const h8*>(hl + rl * ld + k + 8 * kq) : h8{0, 0, 0, 0, 0, 0, 0, 0};
  };
  // the hi/lo rows of x and h are zero past H and IS (the fixed-length MFMA steps read them)
  for (int i = tid; i < 2 * HMAX; i += NT) xhl[i] = static_cast<f16>(0.0f);
  for (int i = tid; i < 2 * ISM; i += NT) hhl[i] = static_cast<f16>(0.0f);
  // With an even layer count the last layer is group 1's, and group 0, idle during it, streams the next step's first
  // layer then; otherwise each group streams its first layer when the step starts.
  const bool pre0 = a.L % 2 == 0;
  if (pgrp < a.L) stream(pgrp);

  for (int k = 0; k < a.steps; ++k) {
  if (k > 0) {
    // the next token: the previous step's last block releases the step count after the token and the position
    if (!next_step<G>(c)) return false;
    if (pgrp < a.L && !(pre0 && pgrp == 0)) stream(pgrp);
  }
  const int pos = c.pos, S = pos + 1;
  // attention: up to KALL keys every block takes all keys; beyond that block jj < na takes keys [k0, k1) and the
  // blocks' partials are exchanged
  const bool allkeys = S <= KALL;
  int na, chunk;
  attn_split(S, na, chunk);
  const int k0 = allkeys ? 0 : (jj < na ? min(S, jj * chunk) : S);
  const int k1 = allkeys ? S : (jj < na ? min(S, k0 + chunk) : S);

  for (int layer = pgrp; layer < a.L; layer += 2) {
    const f16* W[4];  // in_norm, post_norm, q_norm, k_norm
#pragma unroll
    for (int i = 0; i < 4; ++i) W[i] = ld_global(a.layer_w, static_cast<size_t>(layer) * 9 + i);
    const uint32_t tag = (c.phase0 + static_cast<uint32_t>(layer)) & 3u;
    // per layer: keeps the compiler from hoisting per-lane addresses out of the loop (register pressure)
    __asm__ volatile("" : "+v"(lane), "+v"(rl), "+v"(kq));
    XTRACE0(layer);
    XTRACE(0);
    wait_mem();  // this wave's rows of the layer have landed (its LDS rows are published by the barrier below)
    // ---- D's key tiles: wave w takes tiles kb / 32 + (7 - w), + 8, ... The first is requested here, at the start
    //      of the layer: the group has nothing to do until the other group's layer ends, and the keys of cached
    //      positions do not depend on this layer (the first layer of a step has no such slack) ----
    const int kb = allkeys ? 0 : k0, ke = allkeys ? S : k1;
    const int wr = NW - 1 - wid;  // the wave's tile rank: tiles kb / KT + wr, + 8, ...
    const size_t kvb = static_cast<size_t>(layer) * a.layer_stride + static_cast<size_t>(g) * a.cap * HD;
    // keys at or past `pos` read as zero: their whole byte offset is in voffset, which the range check covers
    const __amdgpu_buffer_rsrc_t rk = __builtin_amdgcn_make_buffer_rsrc(a.kcache + kvb, 0, pos * HD * 2, 0x00020000);
    const __amdgpu_buffer_rsrc_t rv = __builtin_amdgcn_make_buffer_rsrc(a.vcache + kvb, 0, pos * HD * 2, 0x00020000);
    u32x4 kw[2][HD / 32];
    // K operands of tile t (lane: key 16 sb + rl, dims 32 s + 8 kq ..) into kw; then its V tile -> LDS (instruction n
    // brings rows 4n .. 4n+3, lane (slot rl, row 4n + kq), chunk rl ^ 2 (row & 7)): loads return in order, and the
    // scores need only the keys
    auto load_tile = [&](int t) {
      const int p0 = t * KT;
#pragma unroll
      for (int sb = 0; sb < 2; ++sb)
#pragma unroll
        for (int s = 0; s < HD / 32; ++s)
          kw[sb][s] = __builtin_amdgcn_raw_buffer_load_b128(rk, (p0 + 16 * sb + rl) * HD * 2 + (32 * s + 8 * kq) * 2, 0, 0);
#pragma unroll
      for (int n = 0; n < KT / 4; ++n) {
        const int row = 4 * n + kq;
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rv, (lds_void*)(vt + n * 4 * HD), 16,
                                                 (p0 + row) * HD * 2 + ((rl ^ (2 * (row & 7))) * 16), 0, 0, 0);
      }
    };
    const bool early = (kb / KT + wr) * KT < ke;
    // ---- A: x = x' + sum_k D_k (layer 0: the embedding row, embedding.cpp:51-77, requested before the key tile),
    //      RMSNorm input ----
    if (layer == 0) {
      EmbedFetch ef;
      embed_fetch(c, wid, a.embed + static_cast<size_t>(c.token) * H, W[0], ef);
      if (early) load_tile(kb / KT + wr);
      embed_finish(c, wid, ef, xres, xhl, red);
    } else {
      if (early) load_tile(kb / KT + wr);
      cross_reduce2(c, wid, jj, true, a.xd, loc_xg, (tag - 1u) & 3u, loc_xa, W[0], xres, xhl, nullptr, red, 2 * layer + 1,
                    layer == a.L / 2 ? 15 : -1);
    }
    XTRACE(1);
    XSYNC();  // #1
    // ---- B: q/k/v rows of RMSNorm(x): each wave its K slice of every row, the partial sums added in LDS ----
    {
      h8 xa[T::SW];
#pragma unroll
      for (int s = 0; s < T::SW; ++s) xa[s] = vec_operand(xhl, HMAX, kw0 + 32 * s);
      f32x4 acc[T::QT];
#pragma unroll
      for (int t = 0; t < T::QT; ++t) acc[t] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int s = 0; s < T::SW; ++s)  // the tiles' chains interleaved; steps past H meet zero weights
#pragma unroll
        for (int t = 0; t < T::QT; ++t) acc[t] = mfma16(xa[s], as_h8(wq[t][s]), acc[t]);
      if (kq == 0)
#pragma unroll
        for (int t = 0; t < T::QT; ++t) part[wid * PST + 16 * t + rl] = acc[t][0] + acc[t][1] * kLo;
    }
    XSYNC();  // #1b
    if (wid == 0 && lane < T::RQ) {
      float p[NW];
#pragma unroll
      for (int w = 0; w < NW; ++w) p[w] = part[w * PST + lane];
      float s = 0.0f;
#pragma unroll
      for (int w = 0; w < NW; ++w) s += p[w];
      ll_store_local(loc_qkv, jj * T::RQ + lane, s * rms_scale(red, H, a.eps), tag);
    }
    XTRACE(2);
    // ---- C: head wid of the XCD's q/k/v; QK-RMSNorm + rotate-half RoPE (qwen_attention.cpp:168-171,
    //      rope.cpp:81-84); q -> hi/lo rows prescaled by scale * log2(e); k and v rounded to the cache's fp16, and
    //      rank 0 appends them at `pos` ----
    if (wid < G + 2) {
      const int hh = wid;
      // the head's gains and the RoPE entries are requested before the poll: they do not depend on the exchange
      float g0 = 1.0f, g1 = 1.0f, rc = 0.0f, rs = 0.0f;
      if (hh <= G) {
        const f16* gn = hh < G ? W[2] : W[3];
        g0 = static_cast<float>(ld_global(gn, lane));
        g1 = static_cast<float>(ld_global(gn, lane + 64));
        rc = ld_global(a.rope_cos, static_cast<size_t>(pos) * (HD / 2) + lane);
        rs = ld_global(a.rope_sin, static_cast<size_t>(pos) * (HD / 2) + lane);
      }
      float x0, x1;
      if (recv_head(c, loc_qkv + hh * HD, tag, x0, x1)) {
        if (hh <= G) norm_rope_pair(x0, x1, g0, g1, a.eps, rc, rs);
        if (hh < G) {
          const float qscale = a.scale * 1.44269504088896341f;
#pragma unroll
          for (int half = 0; half < 2; ++half) {
            float v = (half == 0 ? x0 : x1) * qscale;
            __asm__ volatile("" : "+v"(v));
            const f16 hi = static_cast<f16>(v);
            qhl[(2 * hh) * HD + lane + 64 * half] = hi;
            qhl[(2 * hh + 1) * HD + lane + 64 * half] = static_cast<f16>((v - static_cast<float>(hi)) * 2048.0f);
          }
        } else {
          const f16 h0 = static_cast<f16>(x0), h1 = static_cast<f16>(x1);
          f16* dst = hh == G ? kn : vn;
          dst[lane] = h0;
          dst[lane + 64] = h1;
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
    XSYNC();  // #2: q rows, kn, vn; the projection partials are consumed
    XTRACE(17);
    // ---- D: attention over keys [kb, ke) (the softmax of grouped_query_attention.cpp:105-136). Wave w takes the
    //      32-key tiles kb / 32 + (7 - w), + 8, ...: scores S^T = q . K^T, a running base-2 softmax per wave,
    //      O += P . V ----
    {
      // A operand of step s: rows 2h, 2h + 1 = hi, lo of head h's q; rows >= 2G zero
      auto q_operand = [&](int s) -> h8 {
        return rl < 2 * G ? *reinterpret_cast<const h8*>(qhl + rl * HD + 32 * s + 8 * kq) : h8{0, 0, 0, 0, 0, 0, 0, 0};
      };
      float mrun[G], lsum[G];
      f32x4 o[HD / 16];
#pragma unroll
      for (int h = 0; h < G; ++h) {
        mrun[h] = -INFINITY;
        lsum[h] = 0.0f;
      }
#pragma unroll
      for (int dt = 0; dt < HD / 16; ++dt) o[dt] = f32x4{0.f, 0.f, 0.f, 0.f};
      for (int t = kb / KT + wr; t * KT < ke; t += NW) {
        const int p0 = t * KT;
        if (!(early && t == kb / KT + wr)) load_tile(t);
#pragma unroll
        for (int sb = 0; sb < 2; ++sb)
          if (p0 + 16 * sb + rl == pos)
#pragma unroll
            for (int s = 0; s < HD / 32; ++s) kw[sb][s] = *reinterpret_cast<const u32x4*>(kn + 32 * s + 8 * kq);
        f32x4 sc[2] = {f32x4{0.f, 0.f, 0.f, 0.f}, f32x4{0.f, 0.f, 0.f, 0.f}};
#pragma unroll
        for (int s = 0; s < HD / 32; ++s) {
          const h8 qa = q_operand(s);
#pragma unroll
          for (int sb = 0; sb < 2; ++sb) sc[sb] = mfma16(qa, as_h8(kw[sb][s]), sc[sb]);
        }
        if (t == kb / KT + wr) XTRACEW(19);
        // lanes 0..15 hold the scores of keys p0 + rl and p0 + 16 + rl for every head
        float pv[2][G];
#pragma unroll
        for (int h = 0; h < G; ++h) {
#pragma unroll
          for (int sb = 0; sb < 2; ++sb)
            pv[sb][h] = (kq == 0 && p0 + 16 * sb + rl < ke) ? sc[sb][2 * h] + sc[sb][2 * h + 1] * kLo : -INFINITY;
          const float mt = wave_max(fmaxf(pv[0][h], pv[1][h]));  // finite: key p0 < ke is in the tile
          const float mnew = fmaxf(mrun[h], mt);
          const float corr = __builtin_amdgcn_exp2f(mrun[h] - mnew);  // 0 on the first tile
          mrun[h] = mnew;
          lsum[h] *= corr;
#pragma unroll
          for (int dt = 0; dt < HD / 16; ++dt) {
            o[dt][2 * h] *= corr;
            o[dt][2 * h + 1] *= corr;
          }
#pragma unroll
          for (int sb = 0; sb < 2; ++sb) pv[sb][h] = __builtin_amdgcn_exp2f(pv[sb][h] - mnew);
          lsum[h] += pv[0][h] + pv[1][h];
        }
        if (t == kb / KT + wr) XTRACEW(18);
        // P rows 2h, 2h + 1 (hi, lo 2^11) of the tile's 32 keys -> the wave's LDS rows
        if (kq == 0) {
#pragma unroll
          for (int h = 0; h < G; ++h)
#pragma unroll
            for (int sb = 0; sb < 2; ++sb) {
              const float p = pv[sb][h];
              const f16 hi = static_cast<f16>(p);
              pt[(2 * h) * KT + 16 * sb + rl] = hi;
              pt[(2 * h + 1) * KT + 16 * sb + rl] = static_cast<f16>((p - static_cast<float>(hi)) * 2048.0f);
            }
        }
        wait_mem();  // the V tile has landed in LDS
        if (t == kb / KT + wr) XTRACEW(16);
        if (pos >= p0 && pos < p0 + KT && lane < 16) {  // the new value is not in the cache (read as zero): its row
          const int row = pos - p0;
          *reinterpret_cast<u32x4*>(vt + row * HD + ((lane ^ (2 * (row & 7))) * 8)) =
              *reinterpret_cast<const u32x4*>(vn + lane * 8);
        }
        const h8 pa = rl < 2 * G ? *reinterpret_cast<const h8*>(pt + rl * KT + 8 * kq) : h8{0, 0, 0, 0, 0, 0, 0, 0};
        // B operand V[8 kq + e][16 dt + rl]: two transposing reads of 4 keys each; in each 16-lane group lane rl names
        // 4 dims of one key and receives dim rl of the 4 keys. Read (dt, half) is at row 8 kq + 4 half + rl / 4,
        // dims 16 dt + 4 (rl & 3): chunk 2 dt + (rl & 3) / 2 stored at slot (2 dt + (rl & 3) / 2) ^ 2 (row & 7), i.e.
        // byte 32 ((dt ^ (rl / 4)) ^ 4 half) + 16 ((rl & 3) / 2) + 8 (rl & 1) of the row
        const int vbase = (8 * kq + (rl >> 2)) * HD * 2 + ((rl & 3) >> 1) * 16 + (rl & 1) * 8, vsw = (rl >> 2) * 32;
        // in two halves of the head's dims (fewer registers at the kernel's peak)
#pragma unroll
        for (int d0 = 0; d0 < HD / 16; d0 += HD / 32) {
          hv4 vr[HD / 32][2];
#pragma unroll
          for (int dt = 0; dt < HD / 32; ++dt)
#pragma unroll
            for (int half = 0; half < 2; ++half)
              vr[dt][half] = __builtin_amdgcn_ds_read_tr16_b64_v4f16((__attribute__((address_space(3))) hv4*)(
                  (__attribute__((address_space(3))) char*)(vt) + vbase + half * 4 * HD * 2 +
                  ((32 * (d0 + dt)) ^ vsw ^ (128 * half))));
#pragma unroll
          for (int dt = 0; dt < HD / 32; ++dt) {
            const f16x4 w0 = __builtin_bit_cast(f16x4, vr[dt][0]), w1 = __builtin_bit_cast(f16x4, vr[dt][1]);
            const h8 vb = {w0[0], w0[1], w0[2], w0[3], w1[0], w1[1], w1[2], w1[3]};
            o[d0 + dt] = mfma16(pa, vb, o[d0 + dt]);
          }
        }
        if (t == kb / KT + wr) XTRACEW(20);
      }
      XTRACE(4);
      // the wave's partial (its max, sum and weighted values per head) into the first bytes of its own V tile
      {
        float* gp = reinterpret_cast<float*>(vt);  // [G][HD] values, [G] maxima, [G] sums
        if (kq == 0) {
#pragma unroll
          for (int dt = 0; dt < HD / 16; ++dt)
#pragma unroll
            for (int h = 0; h < G; ++h) gp[h * HD + 16 * dt + rl] = o[dt][2 * h] + o[dt][2 * h + 1] * kLo;
        }
#pragma unroll
        for (int h = 0; h < G; ++h) {
          const float l = wave_sum(lsum[h]);
          if (lane == 0) {
            gp[G * HD + h] = mrun[h] == -INFINITY ? kNoKeys : mrun[h];
            gp[G * HD + G + h] = l;
          }
        }
      }
      XTRACE(11);
      XSYNC();  // #2b: the 8 waves' partials
      XTRACE(12);
      if (allkeys || jj < na) {
        // output t (head t / 128, dim t % 128): the waves' partials rescaled to the block max, in wave order
        for (int t = tid; t < G * HD; t += NT) {
          const int h = t / HD, d = t % HD;
          float M = kNoKeys, mw[NW];
#pragma unroll
          for (int w = 0; w < NW; ++w) {
            mw[w] = reinterpret_cast<const float*>(vtb + w * KT * HD * 2)[G * HD + h];
            M = fmaxf(M, mw[w]);
          }
          if (!allkeys) M = tw_val(tw_pack(M, 0u));  // as the exchange word will carry it
          // the weight of wave w's partial, exp2(max_w - M) (0 for a wave without keys), is the same for every dim
          // of the head: lane w computes it once and the wave reads it back per w (G * HD is a multiple of 64, so
          // every thread of a wave is here with the same head)
          float ml = mw[0];
#pragma unroll
          for (int w = 1; w < NW; ++w) ml = (lane & (NW - 1)) == w ? mw[w] : ml;
          const float fl = __builtin_amdgcn_exp2f(ml - M);
          float O = 0.0f, Lw = 0.0f;
#pragma unroll
          for (int w = 0; w < NW; ++w) {
            const float* gw = reinterpret_cast<const float*>(vtb + w * KT * HD * 2);
            const float f = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(fl), w));
            Lw += gw[G * HD + G + h] * f;
            O += gw[h * HD + d] * f;
          }
          if (allkeys) {
            float v = O / Lw;
            __asm__ volatile("" : "+v"(v));
            const f16 hi = static_cast<f16>(v);
            ahl[t] = hi;
            ahl[G * HD + t] = static_cast<f16>((v - static_cast<float>(hi)) * 2048.0f);
          } else {
            const int w0 = (h * NBX + jj) * PW;  // [head][block][PW]
            ll_store_local(loc_att, w0 + d, O, tag);
            if (d < 4) ll_store_local(loc_att, w0 + HD + d, d == 0 ? M : (d == 1 ? Lw : 0.0f), tag);
          }
        }
      }
      if (allkeys || jj >= na) keyless_partial(tag);
      XTRACE(13);
    }
    if (!allkeys) {
      XSYNC();  // the merge has read the waves' partials: E's block partials may overwrite them
      // ---- E: head wid's block partials of the XCD, merged in a fixed order ----
      if (wid < G) {
        const int h = wid;
        uint32_t* bpart = reinterpret_cast<uint32_t*>(vtb) + h * (NBG * PW);
        if (recv_contig<T::MQ_E>(c, loc_att + h * NBX * PW, na * (PW / 4), tag, bpart)) {
          // lane r < na holds block r's max and sum; the weights e_r are broadcast with readlane
          const float mr = lane < na ? tw_val(bpart[lane * PW + HD]) : kNoKeys;
          const float lr = lane < na ? tw_val(bpart[lane * PW + HD + 1]) : 0.0f;
          const float M = wave_max(mr);
          const float er = mr < 0.5f * kNoKeys ? 0.0f : __builtin_amdgcn_exp2f(mr - M);  // a keyless block adds 0
          const float Ls = wave_sum(lr * er);
#pragma unroll
          for (int dd = 0; dd < 2; ++dd) {
            const int d = lane + 64 * dd;
            float O = 0.0f;
#pragma unroll
            for (int r = 0; r < NBG; ++r)
              if (r < na) O += tw_val(bpart[r * PW + d]) * __int_as_float(__builtin_amdgcn_readlane(__float_as_int(er), r));
            float v = O / Ls;
            __asm__ volatile("" : "+v"(v));
            const f16 hi = static_cast<f16>(v);
            ahl[h * HD + d] = hi;
            ahl[G * HD + h * HD + d] = static_cast<f16>((v - static_cast<float>(hi)) * 2048.0f);
          }
        }
      }
    }
    XTRACE(5);
    XSYNC();  // #3: merged attention output
    // ---- F: partial o_proj over the XCD's query columns: wave w < RH / 16 takes rows 16 w .. over all G * 128 ----
    if (wid < RH / 16) {
      const int row = 16 * wid + rl;
      constexpr int msk = T::GHD / 8 >= 16 ? 15 : T::GHD / 8 - 1;
      constexpr int NS = T::GHD / 32, NH = (NS + 1) / 2;
      f32x4 acc[2] = {f32x4{0.f, 0.f, 0.f, 0.f}, f32x4{0.f, 0.f, 0.f, 0.f}};
#pragma unroll
      for (int s0 = 0; s0 < NS; s0 += NH) {  // the operands of half the steps requested before their MFMAs
        h8 av[NH], bv[NH];
#pragma unroll
        for (int s = s0; s < s0 + NH && s < NS; ++s) {
          av[s - s0] = vec_operand(ahl, T::GHD, 32 * s);
          bv[s - s0] = *reinterpret_cast<const h8*>(wo + row * T::GHD + (((4 * s + kq) ^ (row & msk)) * 8));
        }
#pragma unroll
        for (int s = s0; s < s0 + NH && s < NS; ++s) acc[s & 1] = mfma16(av[s - s0], bv[s - s0], acc[s & 1]);
      }
      const f32x4 r = acc[0] + acc[1];
      if (kq == 0) ll_store_buf(a.xo, g * H + jj * RH + row, r[0] + r[1] * kLo, tag);
    }
    XTRACE(6);
    // ---- G: x' = x + sum_k O_k, RMSNorm input ----
    cross_reduce2(c, wid, jj, true, a.xo, nullptr, tag, loc_xg, W[1], xres, xhl, nullptr, red, 2 * layer + 2,  // x' also for the other group
                  layer == a.L / 2 ? 14 : -1);
    XTRACE(7);
    XSYNC();  // #4
    // ---- H: gate/up of RMSNorm(x') + SwiGLU (qwen_mlp.cpp:31) on the block's share of the XCD's slice ----
    {
      h8 xa[T::SW];
#pragma unroll
      for (int s = 0; s < T::SW; ++s) xa[s] = vec_operand(xhl, HMAX, kw0 + 32 * s);
      f32x4 acc[T::GT];
#pragma unroll
      for (int t = 0; t < T::GT; ++t) acc[t] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int s = 0; s < T::SW; ++s)
#pragma unroll
        for (int t = 0; t < T::GT; ++t) acc[t] = mfma16(xa[s], as_h8(wg[t][s]), acc[t]);
      if (kq == 0)
#pragma unroll
        for (int t = 0; t < T::GT; ++t) part[wid * PST + 16 * t + rl] = acc[t][0] + acc[t][1] * kLo;
    }
    XSYNC();  // #4b
    if (wid == 0 && lane < RI) {
      const float scale = rms_scale(red, H, a.eps);
      float pg[NW], pu[NW];
#pragma unroll
      for (int w = 0; w < NW; ++w) {
        pg[w] = part[w * PST + lane];
        pu[w] = part[w * PST + RI + lane];
      }
      float gs = 0.0f, us = 0.0f;
#pragma unroll
      for (int w = 0; w < NW; ++w) {
        gs += pg[w];
        us += pu[w];
      }
      ll_store_local(loc_h, jj * RI + lane, silu_ref(gs * scale) * (us * scale), tag);
    }
    XTRACE(8);
    // ---- I: the XCD's h slice, as hi/lo rows ----
    if (wid * 64 < IS / 4) {
      int ln = lane;
      __asm__ volatile("" : "+v"(ln));
      const int nq = min(64, IS / 4 - wid * 64);
      const __amdgpu_buffer_rsrc_t r = __builtin_amdgcn_make_buffer_rsrc(loc_h + wid * 256, 0, nq * 16, 0x00020000);
      const u32x4 filler = {tag, tag, tag, tag};
      // two staggered reads in flight (kStaggerLocal), unconditional (lanes past nq read past the resource's end,
      // which returns zeros, and take the filler)
      u32x4 t = ll_peek_buf4(r, ln * 16);
      u32x4 v = ln < nq ? t : filler;
      stagger<kStaggerLocal>();
      t = ll_peek_buf4(r, ln * 16);
      u32x4 v2 = ln < nq ? t : filler;
      const uint64_t t0 = now_ticks();
      uint32_t spins = 0;
      bool ok = true;
      while (true) {
        if (__all(tw_quad_ok(v, tag))) break;
        if (give_up(c, spins, t0)) {
          wait_failed(c);
          ok = false;
          break;
        }
        t = ll_peek_buf4(r, ln * 16);
        v = ln < nq ? t : filler;
        if (__all(tw_quad_ok(v2, tag))) {
          v = v2;
          break;
        }
        t = ll_peek_buf4(r, ln * 16);
        v2 = ln < nq ? t : filler;
      }
      if (ok && ln < nq)
        store_hl4(hhl, ISM, 4 * (wid * 64 + ln), f32x4{tw_val(v.x), tw_val(v.y), tw_val(v.z), tw_val(v.w)});
    }
    XTRACE(9);
    XSYNC();  // #5
    // ---- J: partial down_proj over the slice's columns: wave w < RH / 16 takes rows 16 w .. over all IS ----
    if (wid < RH / 16) {
      const int row = 16 * wid + rl;
      constexpr int msk = ISM / 8 >= 16 ? 15 : ISM / 8 - 1;
      constexpr int NS = ISM / 32, NH = (NS + 1) / 2;  // steps past IS meet zero operands
      f32x4 acc[3] = {f32x4{0.f, 0.f, 0.f, 0.f}, f32x4{0.f, 0.f, 0.f, 0.f}, f32x4{0.f, 0.f, 0.f, 0.f}};
#pragma unroll
      for (int s0 = 0; s0 < NS; s0 += NH) {  // the operands of half the steps requested before their MFMAs
        h8 av[NH], bv[NH];
#pragma unroll
        for (int s = s0; s < s0 + NH && s < NS; ++s) {
          av[s - s0] = vec_operand(hhl, ISM, 32 * s);
          bv[s - s0] = *reinterpret_cast<const h8*>(wd + row * ISM + (((4 * s + kq) ^ (row & msk)) * 8));
        }
#pragma unroll
        for (int s = s0; s < s0 + NH && s < NS; ++s) acc[s % 3] = mfma16(av[s - s0], bv[s - s0], acc[s % 3]);
      }
      const f32x4 r = (acc[0] + acc[1]) + acc[2];
      if (kq == 0) ll_store_buf(a.xd, g * H + jj * RH + row, r[0] + r[1] * kLo, tag);
    }
    XTRACE(10);
    // the group's next layer: its weight rows stream into registers and LDS while the other group computes (after a
    // barrier: no wave may still read this layer's rows in LDS)
    if (layer + 2 < a.L) {
      XSYNC();
      stream(layer + 2);
    } else if (pre0 && pgrp == 0 && k + 1 < a.steps) {
      XSYNC();
      stream(0);  // the next step's first layer, while group 1 computes the last one
    }
  }
  // final hidden state x = x' + sum_k D_k of the last layer, RMSNorm input with the final gain (all blocks), in fp32
  // for the LM head
  cross_reduce2(c, wid, jj, pgrp == 0, a.xd, loc_xg, (c.phase0 + static_cast<uint32_t>(a.L) - 1u) & 3u, loc_xa,
                a.final_norm, xres, xhl, reinterpret_cast<float*>(vtb), red, 2 * a.L + 3);
  XTRACE0(a.L);
  XSYNC();
  lm_head<G>(c);
  XTRACE0(a.L + 1);
  finish_step<G>(c);
  }
  return true;
}

}  // namespace

template <int G>
__global__ __launch_bounds__(NT) void k_decode_xcd(PersistArgs a) {
  extern __shared__ __attribute__((aligned(16))) char lds[];
  using LD = Lds<G>;
  int* flag = reinterpret_cast<int*>(lds + LD::FLAG);
  const int tid = threadIdx.x, wid = tid >> 6, lane = tid & 63;
  const uint32_t step = static_cast<uint32_t>(a.state[3]);  // this kernel's own step count (the legacy one-launch
                                                             // kernel counts its steps in state[2])
  if (tid == 0) {
    // a launch queued behind a failed one leaves at once: the failed step did not advance the step count or reset
    // the arrival counters, so a rank taken now would be meaningless, and the first failure's cause is kept
    const bool failed = err_raised(a.err);
    const int xcc = static_cast<int>(__builtin_amdgcn_s_getreg((3 << 11) | 20) & 15u);  // HW_REG_XCC_ID
    const int rank = failed ? -1 : (xcc < NX ? atomicAdd(a.xcd_ctr + (step & 1u) * NX + xcc, 1) : NBX);
    flag[0] = 0;
    flag[1] = xcc;
    flag[2] = rank;
    flag[4] = 0;  // cross_reduce2's stage-1 marker (its markers are positive)
  }
  __syncthreads();
  const int g = flag[1], j = flag[2];
  if (j < 0) return;
  if (j >= NBX) {  // not the expected 32 blocks per XCD: fail the step (every other block's wait then times out)
    if (tid == 0) __hip_atomic_store(a.err, 2, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    return;
  }
  Ctx c{a, g, j, a.state[0], a.state[1], (step - 1u) * static_cast<uint32_t>(a.L), step, step,
        a.ring != nullptr ? *a.ring_pos : 0, lds, flag};
  run_steps<G>(c);
}

#undef XSYNC
#undef XTRACE
#undef XTRACE0
#undef XTRACEW

namespace {
template <int G>
hipError_t launch_g(const PersistArgs& a, hipStream_t s) {
  // more than 80 KB of LDS per block: one block per CU, so 32 blocks land on each XCD
  const size_t lds = std::max<size_t>(Lds<G>::TOTAL, 96 * 1024);
  static size_t attr_lds = 0;
  if (attr_lds < lds) {
    hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(k_decode_xcd<G>),
                                       hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(lds));
    if (e != hipSuccess) return e;
    attr_lds = lds;
  }
  if (a.cooperative) {
    void* args[] = {const_cast<PersistArgs*>(&a)};
    return hipLaunchCooperativeKernel(reinterpret_cast<const void*>(k_decode_xcd<G>), dim3(NX * NBX), dim3(NT), args,
                                      static_cast<unsigned>(lds), s);
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
  const size_t lds = std::max<size_t>(G == 1 ? Lds<1>::TOTAL : Lds<2>::TOTAL, 96 * 1024);
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
  if (H % 256 != 0 || H > HMAX) return false;  // each of a block's 8 waves takes whole 32-deep MFMA steps
  if (I % (NX * NBX) != 0 || I > IMAX) return false;
  return true;
}

}  // namespace soc
