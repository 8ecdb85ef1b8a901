// gemv.hip - decode-time weight GEMVs (batch 1) with fused RMSNorm prologue and epilogues, the LM head with a
// fused greedy argmax, and the group-quantized (int8 / int4, fp16 scale per 64 inputs) GEMV.
//
// Reference computation: Linear::Forward (Mac/cpu/src/linear.cpp:51-84): y[o] = sum_i x[i] * float(W[o][i]),
// accumulated in fp32. Weights stay fp16 in HBM (row-major [out][in], the Hugging Face layout) and are streamed
// with 16-byte nontemporal loads; each wave owns R output rows and reduces its 64 partial sums with shuffles.
#include "kernels.h"

#include <algorithm>
#include <cstdlib>
#include <cstring>

namespace soc {

namespace {

// Loads x (fp32 [K]) into LDS, optionally applying RMSNorm with an fp16 gain exactly in the reference's order:
// ms = sum(x^2) / K; scale = 1 / sqrt(ms + eps); y = x * scale * gain (Mac/cpu/src/rms_norm_module.cpp:56-64).
template <int NT>
__device__ __forceinline__ void stage_x(const float* __restrict__ x, const f16* __restrict__ xh,
                                        const f16* __restrict__ gain, float eps, int K, float* xs, float* red) {
  float ss = 0.0f;
  for (int i = threadIdx.x * 4; i < K; i += NT * 4) {
    f32x4 v;
    if (xh != nullptr) {
      const f16x4 h = *reinterpret_cast<const f16x4*>(xh + i);
      v = f32x4{static_cast<float>(h.x), static_cast<float>(h.y), static_cast<float>(h.z), static_cast<float>(h.w)};
    } else {
      v = *reinterpret_cast<const f32x4*>(x + i);
    }
    *reinterpret_cast<f32x4*>(xs + i) = v;
    ss += v.x * v.x + v.y * v.y + v.z * v.z + v.w * v.w;
  }
  if (gain != nullptr) {
    ss = block_sum<NT>(ss, red);
    const float scale = 1.0f / sqrtf(ss / static_cast<float>(K) + eps);
    for (int i = threadIdx.x; i < K; i += NT) xs[i] = xs[i] * scale * static_cast<float>(gain[i]);
  }
  __syncthreads();
}

// Dot products of R consecutive rows (starting at row0) with xs over the 512-wide chunks of K starting at kbase,
// kbase + cs, kbase + 2 cs, ... (cs = 512: all of K from kbase = 0); U chunks are loaded per iteration.
template <int R, int U>
__device__ __forceinline__ void rows_dot(const f16* __restrict__ W, int row0, int N, int K, const float* xs, float* acc,
                                         int kbase = 0, int cs = 512) {
  const int lane = threadIdx.x & (kWave - 1);
#pragma unroll
  for (int r = 0; r < R; ++r) acc[r] = 0.0f;
  for (int k0 = kbase + lane * 8; k0 < K; k0 += cs * U) {
    u32x4 w[U][R];
#pragma unroll
    for (int u = 0; u < U; ++u)
#pragma unroll
      for (int r = 0; r < R; ++r) {
        const int row = min(row0 + r, N - 1);
        const int k = k0 + u * cs;
        w[u][r] = k < K ? load_stream16(W + static_cast<size_t>(row) * K + k) : u32x4{0, 0, 0, 0};
      }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int k = k0 + u * cs;
      if (k < K) {
        float xv[8];
        *reinterpret_cast<f32x4*>(xv) = *reinterpret_cast<const f32x4*>(xs + k);
        *reinterpret_cast<f32x4*>(xv + 4) = *reinterpret_cast<const f32x4*>(xs + k + 4);
#pragma unroll
        for (int r = 0; r < R; ++r) {
          float wf[8];
          f16x8_to_f32(w[u][r], wf);
          float a = acc[r];
#pragma unroll
          for (int i = 0; i < 8; ++i) a += xv[i] * wf[i];
          acc[r] = a;
        }
      }
    }
  }
#pragma unroll
  for (int r = 0; r < R; ++r) acc[r] = wave_sum(acc[r]);
}

}  // namespace

// y = epilogue(W . norm(x)). EPI_STORE: y[n] = acc. EPI_RESIDUAL: y[n] = y[n] + acc (in place on the residual
// stream, Mac/cpu/src/qwen_block.cpp:70-72). EPI_SWIGLU: y[n] = silu(W.x) * (W2.x) (qwen_mlp.cpp:69-72).
template <int R, int U, int EPI>
__global__ __launch_bounds__(256) void k_gemv(GemvArgs a) {
  extern __shared__ __attribute__((aligned(16))) float xs[];
  __shared__ float red[4];
  stage_x<256>(a.x, a.xh, a.gain, a.eps, a.K, xs, red);
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = blockIdx.x * 4 + (threadIdx.x >> 6);
  const int nwaves = gridDim.x * 4;
  for (int row0 = wave * R; row0 < a.N; row0 += nwaves * R) {
    float acc[R];
    rows_dot<R, U>(a.w, row0, a.N, a.K, xs, acc);
    if constexpr (EPI == EPI_SWIGLU) {
      float acc2[R];
      rows_dot<R, U>(a.w2, row0, a.N, a.K, xs, acc2);
#pragma unroll
      for (int r = 0; r < R; ++r) acc[r] = silu_ref(acc[r]) * acc2[r];
    }
    if (lane < R && row0 + lane < a.N) {
      float v = acc[0];
#pragma unroll
      for (int r = 1; r < R; ++r)
        if (lane == r) v = acc[r];
      float* dst = a.y + row0 + lane;
      if constexpr (EPI == EPI_RESIDUAL) v = *dst + v;
      *dst = v;
    }
  }
}

// The same for matrices with few rows (where a wave per R rows would leave most of the chip idle): block b owns
// rows R b .. R b + R - 1 and its four waves split K (wave w takes the 512-wide chunks w, w + 4, ...). Nothing is
// staged: a lane loads its own 8 activations (and gains) with the weights, in one round trip, and the RMSNorm scale
// 1 / rms, which is the same for every product, multiplies the finished sums (the gain multiplies x before the
// products); the sums of squares and the four partial dot products of a row are added in wave order.
template <int R, int U, int EPI>
__global__ __launch_bounds__(256) void k_gemv_ks(GemvArgs a) {
  __shared__ float part[2][4][R];
  __shared__ float ssw[4];
  const int lane = threadIdx.x & (kWave - 1), wid = threadIdx.x >> 6;
  const int row0 = blockIdx.x * R, K = a.K;
  const bool norm = a.gain != nullptr;
  float acc[R], acc2[R], ss = 0.0f;
#pragma unroll
  for (int r = 0; r < R; ++r) acc[r] = acc2[r] = 0.0f;
  for (int kw = wid * 512; kw < K; kw += 2048 * U) {  // the wave's first chunk of this iteration
    u32x4 w[U][R], w2[U][R];
    f32x4 xa[U], xb[U];
    u32x4 gv[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int k = min(kw + 2048 * u + lane * 8, K - 8);  // in range; runs past K are loaded and not used
#pragma unroll
      for (int r = 0; r < R; ++r) {
        const size_t off = static_cast<size_t>(min(row0 + r, a.N - 1)) * K + k;
        w[u][r] = load_stream16(a.w + off);
        if constexpr (EPI == EPI_SWIGLU) w2[u][r] = load_stream16(a.w2 + off);
      }
      if (a.xh != nullptr) {
        const u32x4 h = load16(a.xh + k);
        float f[8];
        f16x8_to_f32(h, f);
        xa[u] = f32x4{f[0], f[1], f[2], f[3]};
        xb[u] = f32x4{f[4], f[5], f[6], f[7]};
      } else {
        xa[u] = *reinterpret_cast<const f32x4*>(a.x + k);
        xb[u] = *reinterpret_cast<const f32x4*>(a.x + k + 4);
      }
      gv[u] = norm ? load16(a.gain + k) : u32x4{0, 0, 0, 0};
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      if (kw + 2048 * u + lane * 8 >= K) continue;
      float xv[8] = {xa[u][0], xa[u][1], xa[u][2], xa[u][3], xb[u][0], xb[u][1], xb[u][2], xb[u][3]};
      if (norm) {
        float g[8];
        f16x8_to_f32(gv[u], g);
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          ss = fmaf(xv[i], xv[i], ss);
          xv[i] *= g[i];
        }
      }
#pragma unroll
      for (int r = 0; r < R; ++r) {
        float wf[8];
        f16x8_to_f32(w[u][r], wf);
#pragma unroll
        for (int i = 0; i < 8; ++i) acc[r] += xv[i] * wf[i];
        if constexpr (EPI == EPI_SWIGLU) {
          f16x8_to_f32(w2[u][r], wf);
#pragma unroll
          for (int i = 0; i < 8; ++i) acc2[r] += xv[i] * wf[i];
        }
      }
    }
  }
#pragma unroll
  for (int r = 0; r < R; ++r) {
    acc[r] = wave_sum(acc[r]);
    if constexpr (EPI == EPI_SWIGLU) acc2[r] = wave_sum(acc2[r]);
  }
  if (norm) ss = wave_sum(ss);
  if (lane == 0) {
#pragma unroll
    for (int r = 0; r < R; ++r) {
      part[0][wid][r] = acc[r];
      part[1][wid][r] = acc2[r];
    }
    ssw[wid] = ss;
  }
  __syncthreads();
  if (threadIdx.x < R && row0 + threadIdx.x < a.N) {
    const int r = threadIdx.x;
    const float sc = norm ? 1.0f / sqrtf((ssw[0] + ssw[1] + ssw[2] + ssw[3]) / static_cast<float>(K) + a.eps) : 1.0f;
    float v = sc * (part[0][0][r] + part[0][1][r] + part[0][2][r] + part[0][3][r]);
    if constexpr (EPI == EPI_SWIGLU) v = silu_ref(v) * (sc * (part[1][0][r] + part[1][1][r] + part[1][2][r] + part[1][3][r]));
    float* dst = a.y + row0 + r;
    if constexpr (EPI == EPI_RESIDUAL) v = *dst + v;
    *dst = v;
  }
}

// Tied / untied LM head for one row with the final RMSNorm as prologue, optional fp32 logits, and a greedy argmax
// with the reference sampler's tie rule (lowest index among equal maxima, Mac/cpu/src/sampler.cpp:42-55).
// The last block to finish reduces the per-block winners, writes the token and advances the decode state.
template <int R, int U>
__global__ __launch_bounds__(256) void k_lm_head_argmax(LmHeadArgs a) {
  extern __shared__ __attribute__((aligned(16))) float xs[];
  __shared__ float red[4];
  __shared__ float bv[4];
  __shared__ int bi[4];
  __shared__ int last;
  stage_x<256>(a.x, nullptr, a.gain, a.eps, a.K, xs, red);
  const int lane = threadIdx.x & (kWave - 1);
  const int wid = threadIdx.x >> 6;
  const int wave = blockIdx.x * 4 + wid;
  const int nwaves = gridDim.x * 4;
  float best = -INFINITY;
  int best_i = 0x7fffffff;
  for (int row0 = wave * R; row0 < a.N; row0 += nwaves * R) {
    float acc[R];
    rows_dot<R, U>(a.w, row0, a.N, a.K, xs, acc);
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int row = row0 + r;
      if (row < a.N) {
        if (acc[r] > best) {  // rows are visited in increasing order within a wave: strict > keeps the lowest index
          best = acc[r];
          best_i = row;
        }
      }
    }
    if (a.logits != nullptr && lane < R && row0 + lane < a.N) {
      float v = acc[0];
#pragma unroll
      for (int r = 1; r < R; ++r)
        if (lane == r) v = acc[r];
      a.logits[row0 + lane] = v;
    }
  }
  // wave winners are uniform across lanes; reduce over the 4 waves, then over blocks
  if (lane == 0) {
    bv[wid] = best;
    bi[wid] = best_i;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    float v = bv[0];
    int i = bi[0];
    for (int w = 1; w < 4; ++w)
      if (bv[w] > v || (bv[w] == v && bi[w] < i)) {
        v = bv[w];
        i = bi[w];
      }
    st_dev(a.part_val + blockIdx.x, v);
    st_dev(a.part_idx + blockIdx.x, i);
    wait_mem();  // the block's candidate is visible device-wide before it is counted
    const int done = atomicAdd(a.counter, 1);
    last = (done == static_cast<int>(gridDim.x) - 1);
  }
  __syncthreads();
  if (!last) return;  // the last block reads every candidate with device-scope loads
  float v = -INFINITY;
  int i = 0x7fffffff;
  for (int b = threadIdx.x; b < static_cast<int>(gridDim.x); b += 256) {
    const float pv = __hip_atomic_load(a.part_val + b, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const int pi = __hip_atomic_load(a.part_idx + b, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
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
  if (lane == 0) {
    bv[wid] = v;
    bi[wid] = i;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int w = 1; w < 4; ++w)
      if (bv[w] > bv[0] || (bv[w] == bv[0] && bi[w] < bi[0])) {
        bv[0] = bv[w];
        bi[0] = bi[w];
      }
    const int tok = bi[0] == 0x7fffffff ? 0 : bi[0];
    if (a.token_out != nullptr) a.token_out[0] = tok;
    if (a.state != nullptr) {
      a.state[0] = tok;      // next input token
      a.state[1] += 1;       // next position
    }
    if (a.ring != nullptr) a.ring[a.ring_pos != nullptr ? a.ring_pos[0] : 0] = tok;
    if (a.ring_pos != nullptr) a.ring_pos[0] += 1;
    st_dev(a.counter, 0);
  }
}

// Group-quantized GEMV/skinny GEMM: y[m][n] = sum_g scale[n][g] * sum_{k in group g} x[m][k] * code[n][k], with
// groups of 64 along K (the product per element is w = float(code) * float(scale), dequant_group's contract).
// BITS = 8: codes int8 [N][K]; BITS = 4: two's complement nibbles, even k in the low nibble, [N][K/2].
//
// Each lane streams 16-byte chunks of a row's codes (16 int8 or 32 int4 codes; a chunk never crosses a scale
// group). The codes become exact fp16 pairs without per-code conversions: the biased code (code + 128, or the
// nibble + 8) is placed in the low mantissa bits of 1024.0 (fp16 0x64xx) by one byte permute (int8) or one
// mask-xor (int4), and one packed fp16 subtract of 1152 (or 1032) leaves the code itself (int4 nibbles in bits
// 4..7: one packed fma by 1/16 minus 72, so that half the nibbles need no shift). v_dot2_f32_f16 then
// accumulates code pairs times fp16 activation pairs in fp32 (products exact), and one fma per chunk applies the
// group scale. The activations are staged once per block in LDS as fp16 pairs in the order the codes unpack
// (int4: k and k + 4 of each group of 8). L lanes share a row (64, or 32 / 16 for short rows) and each lane
// keeps RR rows in flight: 4 rows per wave for tall matrices, one row per lane group when fewer than 4096 rows
// would leave most SIMDs idle.
namespace {
typedef _Float16 qh2 __attribute__((ext_vector_type(2)));
typedef _Float16 sk_qh8 __attribute__((ext_vector_type(8)));

__device__ __forceinline__ qh2 as_qh2(uint32_t v) { return __builtin_bit_cast(qh2, v); }

template <int BITS>
__device__ __forceinline__ void unpack_codes(const u32x4& w, qh2 (&p)[BITS == 8 ? 8 : 16]) {
  if constexpr (BITS == 8) {
    const qh2 bias = {static_cast<_Float16>(-1152.0f), static_cast<_Float16>(-1152.0f)};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const uint32_t u = w[j] ^ 0x80808080u;  // code + 128 per byte
      p[2 * j] = as_qh2(__builtin_amdgcn_perm(0x64646464u, u, 0x04010400u)) + bias;      // k = 4j, 4j + 1
      p[2 * j + 1] = as_qh2(__builtin_amdgcn_perm(0x64646464u, u, 0x04030402u)) + bias;  // k = 4j + 2, 4j + 3
    }
  } else {
    const qh2 bias = {static_cast<_Float16>(-1032.0f), static_cast<_Float16>(-1032.0f)};
    const qh2 bias16 = {static_cast<_Float16>(-72.0f), static_cast<_Float16>(-72.0f)};
    const qh2 sixteenth = {static_cast<_Float16>(0.0625f), static_cast<_Float16>(0.0625f)};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      // k = 8j + i and 8j + i + 4. The mask keeps two nibbles n, the xor adds 8 to them (n ^ 8 = code + 8) and
      // sets the exponent of 1024 in the same step: nibbles i = 0, 2 land in mantissa bits 0..3 (1024 + n - 1032),
      // i = 1, 3 in bits 4..7 (1024 + 16 n, times 1/16 minus 72: exact)
      const uint32_t u = w[j], v = u >> 8;
      p[4 * j + 0] = as_qh2((u & 0x000F000Fu) ^ 0x64086408u) + bias;
      p[4 * j + 1] = as_qh2((u & 0x00F000F0u) ^ 0x64806480u) * sixteenth + bias16;
      p[4 * j + 2] = as_qh2((v & 0x000F000Fu) ^ 0x64086408u) + bias;
      p[4 * j + 3] = as_qh2((v & 0x00F000F0u) ^ 0x64806480u) * sixteenth + bias16;
    }
  }
}
}  // namespace

template <int BITS, int M, int L, int RR>
__global__ __launch_bounds__(256) void k_qmm(QmmArgs a) {
  extern __shared__ __attribute__((aligned(16))) uint32_t xq[];  // [M][K / 2] fp16 pairs
  const int K = a.K, KP = K / 2;
  for (int i = threadIdx.x; i < M * KP; i += 256) {
    const int m = i / KP, p = i - m * KP;
    const int k0 = BITS == 8 ? 2 * p : 8 * (p >> 2) + (p & 3);
    const int k1 = BITS == 8 ? k0 + 1 : k0 + 4;
    const f16* xr = a.x + static_cast<size_t>(m) * K;
    xq[i] = __builtin_bit_cast(uint32_t, qh2{xr[k0], xr[k1]});
  }
  __syncthreads();
  constexpr int CH = BITS == 8 ? 16 : 32;  // codes per 16-byte chunk
  constexpr int NP = CH / 2;               // fp16 pairs per chunk
  constexpr int RP = 64 / L;               // rows side by side in a wave
  constexpr int QR = RR * RP;              // rows per wave per step
  const int lane = threadIdx.x & 63, sub = lane / L, ln = lane % L;
  const int wave = blockIdx.x * 4 + (threadIdx.x >> 6), nwaves = gridDim.x * 4;
  const int nch = K / CH, G = K / 64;
  const size_t rowbytes = BITS == 8 ? static_cast<size_t>(K) : static_cast<size_t>(K) / 2;
  const uint8_t* codes = static_cast<const uint8_t*>(a.codes);
  for (int base = wave * QR; base < a.N; base += nwaves * QR) {
    int rows[RR];
#pragma unroll
    for (int r = 0; r < RR; ++r) rows[r] = min(base + r * RP + sub, a.N - 1);
    float acc[RR][M];
#pragma unroll
    for (int r = 0; r < RR; ++r)
#pragma unroll
      for (int m = 0; m < M; ++m) acc[r][m] = 0.0f;
    for (int c = ln; c < nch; c += L) {
      u32x4 cw[RR];
      float sc[RR];
#pragma unroll
      for (int r = 0; r < RR; ++r) {
        cw[r] = load_stream16(codes + static_cast<size_t>(rows[r]) * rowbytes + static_cast<size_t>(c) * 16);
        sc[r] = static_cast<float>(a.scales[static_cast<size_t>(rows[r]) * G + (c * CH) / 64]);
      }
      qh2 cp[RR][NP];
#pragma unroll
      for (int r = 0; r < RR; ++r) unpack_codes<BITS>(cw[r], cp[r]);
#pragma unroll
      for (int m = 0; m < M; ++m) {
        qh2 xp[NP];
        const u32x4* xs = reinterpret_cast<const u32x4*>(xq + m * KP + c * NP);
#pragma unroll
        for (int q = 0; q < NP / 4; ++q) {
          const u32x4 v = xs[q];
#pragma unroll
          for (int t = 0; t < 4; ++t) xp[4 * q + t] = as_qh2(v[t]);
        }
#pragma unroll
        for (int r = 0; r < RR; ++r) {
          float part = 0.0f;
#pragma unroll
          for (int q = 0; q < NP; ++q) part = __builtin_amdgcn_fdot2(cp[r][q], xp[q], part, false);
          acc[r][m] = fmaf(sc[r], part, acc[r][m]);
        }
      }
    }
#pragma unroll
    for (int r = 0; r < RR; ++r)
#pragma unroll
      for (int m = 0; m < M; ++m) {
        const float v = group_sum<L>(acc[r][m]);
        const int row = base + r * RP + sub;
        if (ln == 0 && row < a.N) a.y[static_cast<size_t>(m) * a.N + row] = v;
      }
  }
}

// The same product for 2 <= M <= 16 rows on matrix cores (v_mfma_f32_16x16x32_f16, D[token][row] = X . W^T): a block
// stages the activations once in LDS and its 8 waves then stream 16-row tiles of codes (tiles blockIdx.x,
// blockIdx.x + gridDim.x, ...), each tile in chunks of eight (int8) or four (int4) 16-byte loads per lane with the
// next chunk (of this or the next tile) in flight. Lane (r, q) = (lane % 16, lane / 16) loads 16 bytes of row r per
// instruction, 64 bytes of the row across the four q: int8: the 16 codes k = 64 g + 16 q + 0..15 of group g; int4:
// the 32 codes k = 128 c + 32 q + 0..31 of groups 2c (q < 2) and 2c + 1 (q >= 2), regrouped by one v_permlane32_swap
// per dword pair so that lane q holds 16 codes of each group at k offset 16 * (0, 2, 1, 3)[q]. The codes unpack
// exactly to fp16 as in k_qmm and are the MFMA's B operand as they come out; its A operand is the token rows, staged
// in LDS as fp16 [16][K + 8] in the same k order (int4: within each 8 k, the order 0 4 1 5 2 6 3 7) and read with
// 16-byte LDS reads (rows M..15 hold zeros, so no lane needs a select). D then holds, per lane,
// tokens 4 q .. 4 q + 3 of row r, so the lane applies its own row's group scales (loaded with the codes). Each
// group's codes go to a fresh accumulator whose sum is scaled and added to the result: the product per element is
// code * scale exactly as in the dequantized weight. Tall matrices only (the LM head): at 151936 x 1024, batch 8,
// int8 runs at 58 % of HBM bandwidth (the dot-product kernel: 24 %), int4 at 52 % (16 %).
template <int BITS>
__global__ __launch_bounds__(512, 4) void k_qmm_mfma(QmmArgs a) {
  extern __shared__ __attribute__((aligned(16))) _Float16 qm_lds[];  // activations [16][K + 8]
  const int K = a.K, G = K / 64, ldx = K + 8;
  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
  const int rl = lane & 15, kq = lane >> 4;
  constexpr int LPC = BITS == 4 ? 4 : 8;           // 16-byte code loads per lane per chunk
  constexpr int GPC = BITS == 8 ? LPC : 2 * LPC;   // scale groups per chunk
  const int nload = BITS == 8 ? G : G / 2;         // code loads per lane over a row (64 bytes of the row each)
  const int nchunk = nload / LPC;                  // G % GPC == 0 (checked at launch)
  const int ntiles = (a.N + 127) / 128;
  const int my_tiles = blockIdx.x < ntiles ? (ntiles - 1 - blockIdx.x) / gridDim.x + 1 : 0;
  const int items = my_tiles * nchunk;
  const size_t rowbytes = BITS == 8 ? static_cast<size_t>(K) : static_cast<size_t>(K) / 2;
  struct Chunk {
    u32x4 w[LPC];
    u32x4 s[GPC / 8];  // the chunk's group scales of the lane's row
  };
  auto tile_row = [&](int item) { return (blockIdx.x + (item / nchunk) * gridDim.x) * 128 + wid * 16; };
  auto load = [&](Chunk& b, int item) {
    const int c = item % nchunk;
    const int row = min(tile_row(item) + rl, a.N - 1);
    const uint8_t* cp = static_cast<const uint8_t*>(a.codes) + row * rowbytes + kq * 16 + static_cast<size_t>(c) * LPC * 64;
#pragma unroll
    for (int s = 0; s < LPC; ++s) b.w[s] = load16(cp + s * 64);
    const f16* sp = a.scales + static_cast<size_t>(row) * G + c * GPC;
#pragma unroll
    for (int s = 0; s < GPC / 8; ++s) b.s[s] = load16(sp + 8 * s);
  };
  Chunk ba, bb;
  // activations: 8-k runs (16-byte load, permuted for int4, 16-byte LDS store), at most XR per thread (K <= 2040).
  // The runs are loaded first and the first code chunk after them: loads complete in issue order, so the staging
  // waits for its own data only and the code stream stays in flight. Rows M..15 are zeros (loaded from row M - 1,
  // not used); 16 K / 8 is a multiple of 512, so every thread has the same number of runs.
  constexpr int XR = 8;
  const int runs = K / 8, nruns = 16 * runs;
  u32x4 xv[XR];
#pragma unroll
  for (int u = 0; u < XR; ++u) {
    const int i = min(tid + 512 * u, nruns - 1);
    const int m = i / runs, k8 = i - m * runs;
    xv[u] = load16(a.x + static_cast<size_t>(min(m, a.M - 1)) * K + 8 * k8);
  }
  __builtin_amdgcn_sched_barrier(0);
  if (items > 0) load(ba, 0);
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int u = 0; u < XR; ++u) {
    const int i = tid + 512 * u;
    if (512 * u >= nruns) break;  // uniform
    const int m = i / runs, k8 = i - m * runs;
    const u32x4 v = m < a.M ? xv[u] : u32x4{0, 0, 0, 0};
    u32x4 o = v;
    if constexpr (BITS == 4) {  // halves 0..7 -> 0 4 1 5 2 6 3 7
      o[0] = __builtin_amdgcn_perm(v[2], v[0], 0x05040100u);
      o[1] = __builtin_amdgcn_perm(v[2], v[0], 0x07060302u);
      o[2] = __builtin_amdgcn_perm(v[3], v[1], 0x05040100u);
      o[3] = __builtin_amdgcn_perm(v[3], v[1], 0x07060302u);
    }
    *reinterpret_cast<u32x4*>(qm_lds + m * ldx + 8 * k8) = o;
  }
  __syncthreads();
  if (items == 0) return;  // no barrier follows

  const int kb = BITS == 8 ? 16 * kq : 16 * ((kq & 1) * 2 + (kq >> 1));
  const _Float16* xr = qm_lds + rl * ldx + kb;
  auto xop = [&](int koff) -> sk_qh8 {  // A operand: 8 activations of the lane's token at k offset koff
    return *reinterpret_cast<const sk_qh8*>(xr + koff);
  };
  auto cop = [](const qh2* p) -> sk_qh8 {
    return sk_qh8{p[0][0], p[0][1], p[1][0], p[1][1], p[2][0], p[2][1], p[3][0], p[3][1]};
  };
  auto scale_of = [](const Chunk& b, int gl) -> float {  // group gl of the chunk
    const uint32_t w = b.s[gl >> 3][(gl >> 1) & 3];
    return static_cast<float>(as_qh2(w)[gl & 1]);
  };
  f32x4 acc = {0.f, 0.f, 0.f, 0.f};
  auto process = [&](Chunk& b, int item) {
    const int c = item % nchunk;
#pragma unroll
    for (int s = 0; s < LPC; ++s) {
      const int idx = c * LPC + s;  // load index within the row
      if constexpr (BITS == 8) {    // group idx: k = 64 idx + 16 kq + 0..15
        qh2 p[8];
        unpack_codes<8>(b.w[s], p);
        f32x4 d = {0.f, 0.f, 0.f, 0.f};
        d = __builtin_amdgcn_mfma_f32_16x16x32_f16(xop(64 * idx), cop(p), d, 0, 0, 0);
        d = __builtin_amdgcn_mfma_f32_16x16x32_f16(xop(64 * idx + 8), cop(p + 4), d, 0, 0, 0);
        const float sc = scale_of(b, s);
#pragma unroll
        for (int i = 0; i < 4; ++i) acc[i] = fmaf(d[i], sc, acc[i]);
      } else {  // dwords 0, 1: group 2 idx at k = 128 idx + kb + 0..15; dwords 2, 3: group 2 idx + 1 (k + 64)
        // in place: the chunk's registers are not read again before the next load into them
        const auto s02 = __builtin_amdgcn_permlane32_swap(b.w[s][0], b.w[s][2], false, false);
        const auto s13 = __builtin_amdgcn_permlane32_swap(b.w[s][1], b.w[s][3], false, false);
        b.w[s] = u32x4{s02[0], s13[0], s02[1], s13[1]};
        const u32x4 w = b.w[s];
        qh2 p[16];
        unpack_codes<4>(w, p);
        f32x4 d0 = {0.f, 0.f, 0.f, 0.f}, d1 = {0.f, 0.f, 0.f, 0.f};
        d0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(xop(128 * idx), cop(p), d0, 0, 0, 0);
        d0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(xop(128 * idx + 8), cop(p + 4), d0, 0, 0, 0);
        d1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(xop(128 * idx + 64), cop(p + 8), d1, 0, 0, 0);
        d1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(xop(128 * idx + 72), cop(p + 12), d1, 0, 0, 0);
        const float s0 = scale_of(b, 2 * s), s1 = scale_of(b, 2 * s + 1);
#pragma unroll
        for (int i = 0; i < 4; ++i) acc[i] = fmaf(d1[i], s1, fmaf(d0[i], s0, acc[i]));
      }
    }
    if (c == nchunk - 1) {  // the tile's row is done: D holds tokens 4 kq + i of row r0 + rl
      const int row = tile_row(item) + rl;
      if (row < a.N) {
#pragma unroll
        for (int i = 0; i < 4; ++i)
          if (4 * kq + i < a.M) a.y[static_cast<size_t>(4 * kq + i) * a.N + row] = acc[i];
      }
      acc = f32x4{0.f, 0.f, 0.f, 0.f};
    }
  };
  for (int it = 0; it < items; it += 2) {
    if (it + 1 < items) load(bb, it + 1);
    process(ba, it);
    if (it + 1 < items) {
      if (it + 2 < items) load(ba, it + 2);
      process(bb, it + 1);
    }
  }
}

// Rows too short for 16 lanes of 16-byte chunks (K < 256 int8 / 512 int4): one lane per 16 k, two rows per wave.
template <int BITS, int M>
__global__ __launch_bounds__(256) void k_qmm_short(QmmArgs a) {
  extern __shared__ __attribute__((aligned(16))) float xs[];  // [M][K]
  for (int m = 0; m < M; ++m)
    for (int i = threadIdx.x; i < a.K; i += 256) xs[m * a.K + i] = static_cast<float>(a.x[static_cast<size_t>(m) * a.K + i]);
  __syncthreads();
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = blockIdx.x * 4 + (threadIdx.x >> 6);
  const int nwaves = gridDim.x * 4;
  constexpr int R = 2;
  const int G = a.K / 64;
  for (int row0 = wave * R; row0 < a.N; row0 += nwaves * R) {
    float acc[R][M];
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
      for (int m = 0; m < M; ++m) acc[r][m] = 0.0f;
    for (int k0 = lane * 16; k0 < a.K; k0 += 1024) {
      float wf[R][16];
#pragma unroll
      for (int r = 0; r < R; ++r) {
        const int row = min(row0 + r, a.N - 1);
        const float sc = static_cast<float>(a.scales[static_cast<size_t>(row) * G + k0 / 64]);
        if constexpr (BITS == 8) {
          const u32x4 c = load_stream16(static_cast<const int8_t*>(a.codes) + static_cast<size_t>(row) * a.K + k0);
#pragma unroll
          for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int b = 0; b < 4; ++b)
              wf[r][j * 4 + b] = static_cast<float>(static_cast<int8_t>((c[j] >> (8 * b)) & 0xff)) * sc;
        } else {
          const uint2 c = *reinterpret_cast<const uint2*>(static_cast<const uint8_t*>(a.codes) +
                                                           static_cast<size_t>(row) * (a.K / 2) + k0 / 2);
          const uint32_t words[2] = {c.x, c.y};
#pragma unroll
          for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int b = 0; b < 8; ++b) {
              const int32_t nib = static_cast<int32_t>((words[j] >> (4 * b)) & 0xf);
              wf[r][j * 8 + b] = static_cast<float>(nib >= 8 ? nib - 16 : nib) * sc;
            }
        }
      }
#pragma unroll
      for (int m = 0; m < M; ++m) {
        float xv[16];
#pragma unroll
        for (int i = 0; i < 16; i += 4)
          *reinterpret_cast<f32x4*>(xv + i) = *reinterpret_cast<const f32x4*>(xs + m * a.K + k0 + i);
#pragma unroll
        for (int r = 0; r < R; ++r) {
          float s = acc[r][m];
#pragma unroll
          for (int i = 0; i < 16; ++i) s += xv[i] * wf[r][i];
          acc[r][m] = s;
        }
      }
    }
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
      for (int m = 0; m < M; ++m) acc[r][m] = wave_sum(acc[r][m]);
    if (lane == 0) {
#pragma unroll
      for (int r = 0; r < R; ++r)
        if (row0 + r < a.N)
#pragma unroll
          for (int m = 0; m < M; ++m) a.y[static_cast<size_t>(m) * a.N + row0 + r] = acc[r][m];
    }
  }
}

// Dequantize codes to fp32 [N][K] (the bit-exact dequant contract, checked element for element).
template <int BITS>
__global__ void k_dequant(const void* codes, const f16* scales, int N, int K, float* w) {
  const size_t total = static_cast<size_t>(N) * K;
  for (size_t idx = blockIdx.x * static_cast<size_t>(blockDim.x) + threadIdx.x; idx < total;
       idx += static_cast<size_t>(gridDim.x) * blockDim.x) {
    const int n = static_cast<int>(idx / K), k = static_cast<int>(idx % K);
    int32_t c;
    if constexpr (BITS == 8) {
      c = static_cast<const int8_t*>(codes)[idx];
    } else {
      const uint8_t byte = static_cast<const uint8_t*>(codes)[static_cast<size_t>(n) * (K / 2) + k / 2];
      const int32_t nib = (k & 1) ? (byte >> 4) : (byte & 0xf);
      c = nib >= 8 ? nib - 16 : nib;
    }
    w[idx] = static_cast<float>(c) * static_cast<float>(scales[static_cast<size_t>(n) * (K / 64) + k / 64]);
  }
}

// Dequantize codes to fp16 [N][K], w = f16(float(code) * float(scale)) rounded to nearest: eight consecutive weights
// of one row (one scale group) per thread and step, a 16-byte store each (K % 64 == 0).
template <int BITS>
__global__ __launch_bounds__(256) void k_dequant_f16(const void* codes, const f16* scales, int N, int K, f16* w) {
  const size_t groups = static_cast<size_t>(N) * (K / 8);
  for (size_t gi = blockIdx.x * static_cast<size_t>(blockDim.x) + threadIdx.x; gi < groups;
       gi += static_cast<size_t>(gridDim.x) * blockDim.x) {
    const size_t idx = gi * 8;
    const int n = static_cast<int>(idx / K), k = static_cast<int>(idx % K);
    const float sc = static_cast<float>(scales[static_cast<size_t>(n) * (K / 64) + k / 64]);
    int32_t c[8];
    if constexpr (BITS == 8) {
      const uint2 b = *reinterpret_cast<const uint2*>(static_cast<const int8_t*>(codes) + idx);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        c[i] = static_cast<int8_t>((b.x >> (8 * i)) & 0xffu);
        c[4 + i] = static_cast<int8_t>((b.y >> (8 * i)) & 0xffu);
      }
    } else {
      const uint32_t b = *reinterpret_cast<const uint32_t*>(static_cast<const uint8_t*>(codes) + idx / 2);
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const int32_t nib = static_cast<int32_t>((b >> (4 * i)) & 0xfu);  // even k in the low nibble
        c[i] = nib >= 8 ? nib - 16 : nib;
      }
    }
    f16x8 v;
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] = static_cast<f16>(static_cast<float>(c[i]) * sc);
    *reinterpret_cast<f16x8*>(w + idx) = v;
  }
}

// ------------------------------------------------------------------------------------------------------------
// Launchers
// ------------------------------------------------------------------------------------------------------------
static int gemv_grid(int N, int R) {
  const int groups = (N + R - 1) / R;
  int blocks = (groups + 3) / 4;
  return blocks < 1024 ? (blocks < 1 ? 1 : blocks) : 1024;
}

hipError_t launch_gemv(const GemvArgs& a, int epi, hipStream_t s) {
  constexpr int R = 4, U = 2;
  const size_t lds = static_cast<size_t>(a.K) * sizeof(float);
  const dim3 grid(gemv_grid(a.N, R)), block(256);
  // K split over the waves of a block, no staging, for all but the tallest matrices; above 16384 row groups the
  // row-per-wave kernel has waves enough to cover its staging
  const int groups = (a.N + (epi == EPI_SWIGLU ? 2 : R) - 1) / (epi == EPI_SWIGLU ? 2 : R);
  const bool ks = groups < 16384;
  const uintptr_t align = reinterpret_cast<uintptr_t>(a.x) | reinterpret_cast<uintptr_t>(a.xh) |
                          reinterpret_cast<uintptr_t>(a.gain) | reinterpret_cast<uintptr_t>(a.w) |
                          reinterpret_cast<uintptr_t>(a.w2);
  if (ks && a.K % 8 == 0 && align % 16 == 0) {  // 16-byte loads of every operand
    switch (epi) {
      case EPI_STORE: hipLaunchKernelGGL((k_gemv_ks<R, U, EPI_STORE>), dim3((a.N + R - 1) / R), block, 0, s, a); break;
      case EPI_RESIDUAL:
        hipLaunchKernelGGL((k_gemv_ks<R, U, EPI_RESIDUAL>), dim3((a.N + R - 1) / R), block, 0, s, a);
        break;
      case EPI_SWIGLU: hipLaunchKernelGGL((k_gemv_ks<2, U, EPI_SWIGLU>), dim3((a.N + 1) / 2), block, 0, s, a); break;
      default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
  }
  switch (epi) {
    case EPI_STORE: hipLaunchKernelGGL((k_gemv<R, U, EPI_STORE>), grid, block, lds, s, a); break;
    case EPI_RESIDUAL: hipLaunchKernelGGL((k_gemv<R, U, EPI_RESIDUAL>), grid, block, lds, s, a); break;
    case EPI_SWIGLU: hipLaunchKernelGGL((k_gemv<2, U, EPI_SWIGLU>), dim3(gemv_grid(a.N, 2)), block, lds, s, a); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

int lm_head_blocks(int N) { return gemv_grid(N, 4) < 512 ? gemv_grid(N, 4) : 512; }

hipError_t launch_lm_head_argmax(const LmHeadArgs& a, hipStream_t s) {
  const size_t lds = static_cast<size_t>(a.K) * sizeof(float);
  hipLaunchKernelGGL((k_lm_head_argmax<4, 2>), dim3(lm_head_blocks(a.N)), dim3(256), lds, s, a);
  return hipGetLastError();
}

// One block per logit row: the greedy token (the first index holding the maximum, like the strict `>` scan of
// Sampler::SampleFromLogits, sampler.cpp:42-48), fed back as the row's next input id at the next position.
// Keeps (v, i) when it beats (bv, bi): larger value, or the same value at a lower index. NaN never wins.
__device__ __forceinline__ void argmax_take(float& bv, int& bi, float v, int i) {
  if (v > bv || (v == bv && i < bi)) {
    bv = v;
    bi = i;
  }
}

__device__ __forceinline__ void argmax_wave(float& bv, int& bi) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) argmax_take(bv, bi, __shfl_xor(bv, o, kWave), __shfl_xor(bi, o, kWave));
}

// Grid (C, n): block (c, row) scans logits [c * chunk, (c + 1) * chunk) of its row. With C > 1 each block publishes
// its candidate, and the last block of the row to arrive (counter per row, reset by that block) picks the winner.
// Within a thread indices rise, so a strict `>` keeps the lowest index of equal maxima; every merge breaks ties
// towards the lower index. A row without a finite maximum (all NaN or -inf) yields token 0.
template <bool VEC>
__global__ __launch_bounds__(256) void k_argmax_rows(const float* logits, int V, int chunk, int32_t* ids,
                                                     int32_t* pos, const int32_t* start, int32_t* ring,
                                                     int ring_stride, float* part_val, int32_t* part_idx,
                                                     int32_t* counters) {
  __shared__ float sv[4];
  __shared__ int si[4];
  __shared__ int last;
  const int c = blockIdx.x, C = gridDim.x, row = blockIdx.y, tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
  const float* x = logits + static_cast<size_t>(row) * V;
  const int lo = c * chunk, hi = min(V, lo + chunk);
  float bv = -INFINITY;
  int bi = 0x7fffffff;
  if (VEC) {  // V and chunk multiples of 4, 16-byte aligned rows: four 16-byte loads in flight per thread
    for (int i = lo + 4 * tid; i < hi; i += 4 * 1024) {
      f32x4 v[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int j = i + 1024 * u;
        v[u] = j < hi ? __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(x + j)) : f32x4(-INFINITY);
      }
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int j = i + 1024 * u;
        if (v[u].x > bv) bv = v[u].x, bi = j;
        if (v[u].y > bv) bv = v[u].y, bi = j + 1;
        if (v[u].z > bv) bv = v[u].z, bi = j + 2;
        if (v[u].w > bv) bv = v[u].w, bi = j + 3;
      }
    }
  } else {
    for (int i = lo + tid; i < hi; i += 256)
      if (x[i] > bv) bv = x[i], bi = i;
  }
  argmax_wave(bv, bi);
  if (lane == 0) {
    sv[wid] = bv;
    si[wid] = bi;
  }
  __syncthreads();
  if (tid == 0) {
    for (int w = 1; w < 4; ++w) argmax_take(bv, bi, sv[w], si[w]);
    if (C > 1) {
      st_dev(part_val + static_cast<size_t>(row) * C + c, bv);
      st_dev(part_idx + static_cast<size_t>(row) * C + c, bi);
      wait_mem();  // the candidate is visible device-wide before it is counted
      last = atomicAdd(counters + row, 1) == C - 1;
    } else {
      last = 1;
      sv[0] = bv;
      si[0] = bi;
    }
  }
  __syncthreads();
  if (!last || tid >= 64) return;
  if (C > 1) {  // C <= 64: one candidate per lane, device-scope loads
    bv = -INFINITY;
    bi = 0x7fffffff;
    if (lane < C) {
      bv = ld_dev(part_val + static_cast<size_t>(row) * C + lane);
      bi = ld_dev(part_idx + static_cast<size_t>(row) * C + lane);
    }
    argmax_wave(bv, bi);
  } else {
    bi = si[0];
  }
  if (lane == 0) {
    if (C > 1) st_dev(counters + row, 0);  // ready for the next step
    if (bi == 0x7fffffff) bi = 0;
    const int p = pos[row];
    const int k = p - start[row];
    if (k >= 0 && k < ring_stride) ring[static_cast<size_t>(row) * ring_stride + k] = bi;
    ids[row] = bi;
    pos[row] = p + 1;
  }
}

int argmax_chunks(int V, int n) {
  // about 512 blocks in all, at most 64 per row and at least 1024 logits per block
  int C = std::min(kArgmaxMaxChunks, std::max(1, (512 + n - 1) / n));
  return std::max(1, std::min(C, V / 1024));
}

hipError_t launch_argmax_rows(const float* logits, int V, int n, int32_t* ids, int32_t* pos, const int32_t* start,
                              int32_t* ring, int ring_stride, float* part_val, int32_t* part_idx, int32_t* counters,
                              hipStream_t s) {
  if (n <= 0 || V <= 0) return hipErrorInvalidValue;
  const int C = argmax_chunks(V, n);
  if (C > 1 && (part_val == nullptr || part_idx == nullptr || counters == nullptr)) return hipErrorInvalidValue;
  const bool vec = V % 4 == 0 && reinterpret_cast<uintptr_t>(logits) % 16 == 0;
  const int chunk = ((V + C - 1) / C + 3) / 4 * 4;
  const dim3 grid(C, n), block(256);
  if (vec)
    hipLaunchKernelGGL(k_argmax_rows<true>, grid, block, 0, s, logits, V, chunk, ids, pos, start, ring, ring_stride,
                       part_val, part_idx, counters);
  else
    hipLaunchKernelGGL(k_argmax_rows<false>, grid, block, 0, s, logits, V, chunk, ids, pos, start, ring,
                       ring_stride, part_val, part_idx, counters);
  return hipGetLastError();
}

// K a multiple of 512 (int8) or 1024 (int4): whole chunks of eight (int8) / four (int4) 16-byte loads per lane and
// 16-byte scale loads; K <= 2040 (the activations fit 64 KB of LDS; at most eight 8-k runs per thread).
bool qmm_mfma_supported(const QmmArgs& a, int bits) {
  const size_t lds = static_cast<size_t>(16) * (a.K + 8) * sizeof(f16);
  return a.M >= 2 && a.M <= 16 && a.K % (bits == 8 ? 512 : 1024) == 0 && lds <= 64 * 1024 &&
         (reinterpret_cast<uintptr_t>(a.x) | reinterpret_cast<uintptr_t>(a.codes) |
          reinterpret_cast<uintptr_t>(a.scales)) % 16 == 0;
}

hipError_t launch_qmm(const QmmArgs& a, int bits, hipStream_t s) {
  const char* mode = std::getenv("SOC_QMM");
  // matrix cores for tall matrices (the LM head); the dot-product kernel keeps the short ones, where a 128-row
  // block per 16 waves would leave most of the chip idle (SOC_QMM=mfma takes the MFMA kernel wherever it applies:
  // the parity tests run it on the short shapes too)
  const bool force_mfma = mode != nullptr && std::strcmp(mode, "mfma") == 0;
  if (qmm_mfma_supported(a, bits) && (force_mfma || a.N >= 16384)) {
    const size_t lds = static_cast<size_t>(16) * (a.K + 8) * sizeof(f16);
    // 8-wave blocks, two resident per CU, tiles looped; int4 (half-size chunks) with 768 blocks, the last third
    // starting as the first blocks finish: 52 % of HBM bandwidth at 151936 x 1024, batch 8, against 48 % with 512
    const dim3 grid(std::min((a.N + 127) / 128, bits == 4 ? 768 : 512)), block(512);
    if (bits == 8) hipLaunchKernelGGL(k_qmm_mfma<8>, grid, block, lds, s, a);
    else hipLaunchKernelGGL(k_qmm_mfma<4>, grid, block, lds, s, a);
    return hipGetLastError();
  }
  const int nch = a.K / (bits == 8 ? 16 : 32);  // 16-byte chunks per row
  if (nch < 16) {
    const size_t lds = static_cast<size_t>(a.M) * a.K * sizeof(float);
    const dim3 grid(gemv_grid(a.N, 2)), block(256);
#define SOC_QMM_SHORT(B, MM)                                                       \
    if (bits == B && a.M == MM) {                                                 \
      hipLaunchKernelGGL((k_qmm_short<B, MM>), grid, block, lds, s, a);            \
      return hipGetLastError();                                                   \
    }
    SOC_QMM_SHORT(8, 1) SOC_QMM_SHORT(8, 2) SOC_QMM_SHORT(8, 4) SOC_QMM_SHORT(8, 8)
    SOC_QMM_SHORT(4, 1) SOC_QMM_SHORT(4, 2) SOC_QMM_SHORT(4, 4) SOC_QMM_SHORT(4, 8)
#undef SOC_QMM_SHORT
    return hipErrorInvalidValue;
  }
  const int L = nch >= 64 ? 64 : nch >= 32 ? 32 : 16;
  const bool tall = a.N >= 4096;
  const int rows_per_wave = tall ? 4 : 64 / L;  // RR = 4 / RP, or 1
  const size_t lds = static_cast<size_t>(a.M) * a.K * sizeof(f16);
  const int waves = (a.N + rows_per_wave - 1) / rows_per_wave;
  const int blocks = std::min((waves + 3) / 4, 2048);
  const dim3 grid(std::max(blocks, 1)), block(256);
#define SOC_QMM_CASE(B, MM, LL)                                                                    \
  if (bits == B && a.M == MM && L == LL) {                                                        \
    if (tall) hipLaunchKernelGGL((k_qmm<B, MM, LL, 4 * LL / 64>), grid, block, lds, s, a);         \
    else hipLaunchKernelGGL((k_qmm<B, MM, LL, 1>), grid, block, lds, s, a);                        \
    return hipGetLastError();                                                                     \
  }
#define SOC_QMM_M(B, LL) SOC_QMM_CASE(B, 1, LL) SOC_QMM_CASE(B, 2, LL) SOC_QMM_CASE(B, 4, LL) SOC_QMM_CASE(B, 8, LL)
  SOC_QMM_M(8, 64) SOC_QMM_M(8, 32) SOC_QMM_M(8, 16)
  SOC_QMM_M(4, 64) SOC_QMM_M(4, 32) SOC_QMM_M(4, 16)
#undef SOC_QMM_M
#undef SOC_QMM_CASE
  return hipErrorInvalidValue;
}

hipError_t launch_dequant_f16(const void* codes, int bits, const f16* scales, int N, int K, f16* w, hipStream_t s) {
  if (N <= 0 || K <= 0 || K % 64 != 0) return hipErrorInvalidValue;
  const size_t groups = static_cast<size_t>(N) * (K / 8);
  const dim3 grid(static_cast<unsigned>(std::min<size_t>((groups + 255) / 256, 4096))), block(256);
  if (bits == 8) hipLaunchKernelGGL((k_dequant_f16<8>), grid, block, 0, s, codes, scales, N, K, w);
  else if (bits == 4) hipLaunchKernelGGL((k_dequant_f16<4>), grid, block, 0, s, codes, scales, N, K, w);
  else return hipErrorInvalidValue;
  return hipGetLastError();
}

hipError_t launch_dequant(const void* codes, int bits, const f16* scales, int N, int K, float* w, hipStream_t s) {
  const dim3 grid(1024), block(256);
  if (bits == 8) hipLaunchKernelGGL((k_dequant<8>), grid, block, 0, s, codes, scales, N, K, w);
  else if (bits == 4) hipLaunchKernelGGL((k_dequant<4>), grid, block, 0, s, codes, scales, N, K, w);
  else return hipErrorInvalidValue;
  return hipGetLastError();
}

}  // namespace soc
