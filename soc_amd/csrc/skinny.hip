// skinny.hip - projections of a ragged decode batch: y[M][N] = x[M][K] . W[N][K]^T with M <= 16 rows of fp32
// activations (one per sequence) and fp16 weights, on MFMA (v_mfma_f32_16x16x32_f16), one launch per projection.
//
// At M <= 16 the work is a weight stream (2 bytes per weight, 2M flops), so the kernel is built around moving W at
// HBM rate: every weight is read once, straight into registers, 16 rows x 256 K per wave per chunk with the next
// chunk in flight, and meets all M activation rows in one MFMA. The activations of the block's K range are split
// once into hi = f16(x) and lo = f16((x - hi) 2^11) in LDS (about 22 bits of each fp32 value; weights are exact), so
// the products track the fp32 reference (Mac/cpu/src/linear.cpp:51-84) up to the order of the sums.
//
// The grid is (row tiles, K splits): the split count is chosen so that the grid covers the chip even for the
// 2560-row projections. Each block writes its partial sums; a second kernel adds the splits in a fixed order (so a
// row's result never depends on the other rows of the batch or on timing) and applies the epilogue: store, residual
// add, SwiGLU of the gate/up halves, or the attention input (per-head q/k RMSNorm, RoPE, KV-cache append). An input
// RMSNorm (rms_norm_module.cpp:56-64) is folded in: the gain multiplies x before the products, the split blocks of
// row tile 0 write the sums of squares of their K range, and the epilogue scales the finished sums by 1 / rms; so no
// separate normalisation or q/k kernel runs.
#include "kernels.h"

#include <cmath>

namespace soc {

namespace {
constexpr int SK_ROWS = 128;    // weight rows per block: 8 waves x 16
constexpr int SK_CHUNK = 256;   // K per register chunk: 8 MFMA steps of 32
constexpr int SK_MAX_KB = 1280; // K per block at most (LDS: 2 x 16 x (1280 + 8) halves = 82 KB)
typedef _Float16 sk_h8 __attribute__((ext_vector_type(8)));
}  // namespace

// Split count for a stacked matrix of `rows` rows and depth K (K % 256 == 0): the divisor d of K / 256 (at most
// SK_MAX_KB of K per block, and at least 512 where K allows: a wave then streams two or more chunks with the next in
// flight; measured 2 % faster per ragged step at Qwen3-4B than one-chunk splits) with the least estimated traffic
// time: weight bytes over the evenness with which the d * tiles blocks fill the chip's block slots (blocks / slots
// over its ceiling; 2 blocks per CU when the block's LDS allows, the kernel's registers allow 2) plus the partial sums
// written and read back (16 rows x 4 bytes x rows x d, twice).
int skinny_splits(int rows, int K) {
  const int n256 = K / SK_CHUNK;
  const int tiles = (rows + SK_ROWS - 1) / SK_ROWS;
  int best = n256;
  double best_cost = 0.0;
  for (int d = 1; d <= n256; ++d) {
    const int kb = K / d;
    if (n256 % d != 0 || kb > SK_MAX_KB || (kb < 2 * SK_CHUNK && K >= 2 * SK_CHUNK)) continue;
    const size_t lds = static_cast<size_t>(2) * 16 * (kb + 8) * sizeof(_Float16);
    const int slots = 256 * (2 * lds <= 160 * 1024 ? 2 : 1);
    const double waves = static_cast<double>(tiles) * d / slots;
    const double eff = waves / std::ceil(waves);
    const double cost = 2.0 * rows * K / eff + 2.0 * 16 * 4 * static_cast<double>(rows) * d;
    if (best_cost == 0.0 || cost < best_cost) {
      best = d;
      best_cost = cost;
    }
  }
  return best;
}

bool skinny_supported(int M, int K) { return M >= 1 && M <= 16 && K % SK_CHUNK == 0 && K >= SK_CHUNK; }

// Rows per tile: 128 (8 waves x 16); SwiGLU tiles hold 64 gate rows (waves 0-3) and the matching 64 up rows
// (waves 4-7).
__host__ __device__ inline int skinny_tiles(int epi, int N0, int Ntot) {
  return epi == EPI_SWIGLU ? (N0 + 63) / 64 : (Ntot + SK_ROWS - 1) / SK_ROWS;
}

// Scratch: the sums of squares [split][16 rows] (64 words reserved per split), then the partials [split][row][Ntot].
__host__ __device__ inline float* sk_part(float* base, int KS) { return base + 64 * KS; }

// grid = (tiles, KS), block = 512, dynamic LDS 2 x 16 x (Kb + 8) halves.
template <int EPI>
__global__ __launch_bounds__(512, 4) void k_skinny_part(SkinnyArgs a) {
  extern __shared__ __attribute__((aligned(16))) _Float16 sk_lds[];
  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
  const int tile = blockIdx.x, ks = blockIdx.y;
  const int k0 = ks * a.Kb;
  const int ld = a.Kb + 8;
  const bool norm = a.gain != nullptr;
  _Float16* xh = sk_lds;
  _Float16* xl = sk_lds + 16 * ld;
  // the wave's 16 weight rows (index in the stacked [w | w2] rows) and the limit of its half
  int r0, lim;
  if constexpr (EPI == EPI_SWIGLU) {
    r0 = (wid < 4 ? 0 : a.N0) + tile * 64 + (wid & 3) * 16;
    lim = wid < 4 ? a.N0 : a.Ntot;
  } else {
    r0 = tile * SK_ROWS + wid * 16;
    lim = a.Ntot;
  }
  const bool active = r0 < lim;
  const int rl = lane & 15, kq = lane >> 4;
  // A operand = W rows r0..r0+15 (lane: row r0 + rl, k = 8 kq + i); rows past the limit repeat its last row, never stored
  const int rr = min(r0 + rl, lim - 1);
  const f16* wrow = (rr < a.N0 ? a.w + static_cast<size_t>(rr) * a.K : a.w2 + static_cast<size_t>(rr - a.N0) * a.K) +
                    k0 + kq * 8;
  const int nch = a.Kb / SK_CHUNK;
  u32x4 wa[8], wb[8];
  // plain (cached) loads: a load instruction covers 64 bytes of each of 16 rows and the next one the adjacent 64,
  // and with the lines allocated in L2 this pattern streams about 15 % faster than with nontemporal loads (measured
  // over a 778 MB matrix on MI355X; the one-launch decode kernels and the GEMV keep nontemporal loads, which are
  // faster there)
  auto load = [&](u32x4* dst, int c) {
#pragma unroll
    for (int s = 0; s < 8; ++s) dst[s] = load16(wrow + c * SK_CHUNK + s * 32);
  };
  // Activations of this K range (times the RMSNorm gain) -> hi/lo fp16 in LDS (rows past M are zero); row m is
  // staged by the 32 threads 32 m .. 32 m + 31, which also sum its squares (written by the blocks of tile 0). The
  // first SU runs of each thread are loaded before the first two weight chunks: loads complete in issue order, so
  // the staging then waits only for its own data while the weight stream stays in flight (a Kb over 128 SU stages
  // the rest afterwards). All loads are unconditional (rows past M and runs past Kb read in-range data that is not
  // used; an inactive wave's weight rows are clamped to valid rows), so no branch splits them. The sum of squares
  // runs in k order.
  constexpr int SU = 5;
  const int m = tid >> 5, j = tid & 31;
  const float* xrow = a.x + static_cast<size_t>(min(m, a.M - 1)) * a.ldx + k0;
  const f16* grow = (norm ? a.gain : reinterpret_cast<const f16*>(a.x)) + k0;  // (not read without a gain)
  f32x4 sv[SU];
  f16x4 sg[SU];
  auto stage_load = [&](int c0) {  // c0: uniform run base
#pragma unroll
    for (int u = 0; u < SU; ++u) {
      const int cc = min(c0 + 128 * u + 4 * j, a.Kb - 4);
      sv[u] = *reinterpret_cast<const f32x4*>(xrow + cc);
      sg[u] = *reinterpret_cast<const f16x4*>(grow + cc);
    }
  };
  float ss = 0.0f;
  auto stage_store = [&](int c0) {
#pragma unroll
    for (int u = 0; u < SU; ++u) {
      if (c0 + 128 * u >= a.Kb) break;  // uniform (Kb % 128 == 0)
      const int cc = c0 + 128 * u + 4 * j;
      f32x4 v = m < a.M ? sv[u] : f32x4{0.f, 0.f, 0.f, 0.f};
      if (norm) {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          ss = fmaf(v[e], v[e], ss);
          v[e] *= static_cast<float>(sg[u][e]);
        }
      }
      f16x4 hi, lo;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const _Float16 h = static_cast<_Float16>(v[e]);
        hi[e] = h;
        lo[e] = static_cast<_Float16>((v[e] - static_cast<float>(h)) * 2048.0f);
      }
      *reinterpret_cast<f16x4*>(&xh[m * ld + cc]) = hi;
      *reinterpret_cast<f16x4*>(&xl[m * ld + cc]) = lo;
    }
  };
  stage_load(0);
  __builtin_amdgcn_sched_barrier(0);  // keep the issue order: staging runs, then weights
  load(wa, 0);
  load(wb, nch > 1 ? 1 : 0);
  __builtin_amdgcn_sched_barrier(0);
  stage_store(0);
  for (int c0 = 128 * SU; c0 < a.Kb; c0 += 128 * SU) {
    stage_load(c0);
    stage_store(c0);
  }
  if (norm) {
    ss = group_sum<32>(ss);
    if (tile == 0 && j == 0) a.part[64 * ks + m] = ss;
  }
  __syncthreads();

  if (!active) return;  // no barrier follows
  const _Float16* bh = xh + rl * ld + kq * 8;  // B operand = x^T (lane: token rl, k = 8 kq + i)
  const _Float16* bl = xl + rl * ld + kq * 8;
  f32x4 acc = {0.f, 0.f, 0.f, 0.f}, accl = {0.f, 0.f, 0.f, 0.f};
  auto mma = [&](const u32x4* src, int c) {
#pragma unroll
    for (int s = 0; s < 8; ++s) {
      const int k = c * SK_CHUNK + s * 32;
      const sk_h8 av = __builtin_bit_cast(sk_h8, src[s]);
      const sk_h8 hv = *reinterpret_cast<const sk_h8*>(bh + k);
      const sk_h8 lv = *reinterpret_cast<const sk_h8*>(bl + k);
      acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(av, hv, acc, 0, 0, 0);
      accl = __builtin_amdgcn_mfma_f32_16x16x32_f16(av, lv, accl, 0, 0, 0);
    }
  };
  for (int c = 0; c < nch; c += 2) {
    if (c > 0 && c + 1 < nch) load(wb, c + 1);  // (chunk 1 went out before the staging)
    mma(wa, c);
    if (c + 1 < nch) {
      if (c + 2 < nch) load(wa, c + 2);
      mma(wb, c + 1);
    }
  }
  // D: lane holds rows row .. row + 3 of token rl (Ntot % 4 == 0 and 16-row alignment: all four or none valid)
  const int row = r0 + 4 * kq;
  if (row < lim) {
    f32x4 v;
#pragma unroll
    for (int i = 0; i < 4; ++i) v[i] = acc[i] + accl[i] * (1.0f / 2048.0f);
    *reinterpret_cast<f32x4*>(sk_part(a.part, a.KS) + (static_cast<size_t>(ks) * 16 + rl) * a.Ntot + row) = v;
  }
}

// Sums, each in split order, of NS streams of n partials (stream i: p[i][0], p[i][st[i]], ...). The loads of all
// streams go out W per stream at a time with no branch between them (indices past n re-read the last partial, which
// is not added), so up to W splits cost one memory round trip however many streams; W is the smallest of 4, 8, 16,
// 32 that covers n (at most 32 per round).
template <int W, int NS>
__device__ __forceinline__ void sum_streams_w(const float* const (&p)[NS], const size_t (&st)[NS], int n,
                                              float (&v)[NS]) {
#pragma unroll
  for (int i = 0; i < NS; ++i) v[i] = 0.0f;
  for (int k = 0; k < n; k += W) {
    float x[NS][W];
#pragma unroll
    for (int i = 0; i < NS; ++i)
#pragma unroll
      for (int u = 0; u < W; ++u) x[i][u] = p[i][static_cast<size_t>(min(k + u, n - 1)) * st[i]];
#pragma unroll
    for (int u = 0; u < W; ++u)
      if (k + u < n)
#pragma unroll
        for (int i = 0; i < NS; ++i) v[i] += x[i][u];
  }
}
template <int NS>
__device__ __forceinline__ void sum_streams(const float* const (&p)[NS], const size_t (&st)[NS], int n,
                                            float (&v)[NS]) {
  if (n <= 4) sum_streams_w<4, NS>(p, st, n, v);
  else if (n <= 8) sum_streams_w<8, NS>(p, st, n, v);
  else if (n <= 16) sum_streams_w<16, NS>(p, st, n, v);
  else sum_streams_w<32, NS>(p, st, n, v);
}

// 1 / rms of an input row from the sum of its splits' sums of squares.
__device__ __forceinline__ float sk_rscale(const SkinnyArgs& a, float ss) {
  return 1.0f / sqrtf(ss / static_cast<float>(a.K) + a.eps);
}

// Store / residual / SwiGLU: one thread per (row m, output n): the KS partials (and, with an input RMSNorm, the
// row's sums of squares) summed in split order, loaded together; then the epilogue.
template <int EPI>
__global__ __launch_bounds__(256) void k_skinny_epi(SkinnyArgs a, int nout) {
  const int n = blockIdx.x * 256 + threadIdx.x, m = blockIdx.y;
  if (n >= nout) return;
  const float* p = sk_part(a.part, a.KS) + static_cast<size_t>(m) * a.Ntot + n;
  const size_t ss_stride = 64, split_stride = static_cast<size_t>(16) * a.Ntot;
  float* dst = a.c + static_cast<size_t>(m) * a.ldc + n;
  // the residual is requested with the partials (read after them it would cost a second memory round trip)
  float prev = 0.0f;
  if constexpr (EPI == EPI_RESIDUAL) prev = *dst;
  float sc = 1.0f, v, u = 0.0f;
  if constexpr (EPI == EPI_SWIGLU) {
    if (a.gain != nullptr) {
      float r[3];
      sum_streams<3>({a.part + m, p, p + a.N0}, {ss_stride, split_stride, split_stride}, a.KS, r);
      sc = sk_rscale(a, r[0]);
      v = r[1];
      u = r[2];
    } else {
      float r[2];
      sum_streams<2>({p, p + a.N0}, {split_stride, split_stride}, a.KS, r);
      v = r[0];
      u = r[1];
    }
  } else {
    if (a.gain != nullptr) {
      float r[2];
      sum_streams<2>({a.part + m, p}, {ss_stride, split_stride}, a.KS, r);
      sc = sk_rscale(a, r[0]);
      v = r[1];
    } else {
      float r[1];
      sum_streams<1>({p}, {split_stride}, a.KS, r);
      v = r[0];
    }
  }
  v *= sc;
  if constexpr (EPI == EPI_SWIGLU) {
    *dst = silu_ref(v) * (sc * u);
  } else if constexpr (EPI == EPI_RESIDUAL) {
    *dst = prev + v;
  } else {
    *dst = v;
  }
}

// The attention input: one wave per (row m, head h): the head's 128 sums (lane: dims lane, lane + 64), scaled by the
// input 1 / rms; q and k heads get their RMSNorm and RoPE at pos[m] (qwen_attention.cpp:168-171; rope.cpp:81-84);
// q -> q_out, k and v -> the fp16 cache of slots[m] at pos[m].
__global__ __launch_bounds__(64) void k_skinny_epi_qkv(SkinnyArgs a) {
  const int m = blockIdx.x, h = blockIdx.y, lane = threadIdx.x;
  const float* p = sk_part(a.part, a.KS) + static_cast<size_t>(m) * a.Ntot + h * 128;
  const size_t ss_stride = 64, split_stride = static_cast<size_t>(16) * a.Ntot;
  // the row's position and slot, the head's gains and the RoPE entries at pos go out before the partials: the
  // table entries wait only for pos, and their round trip overlaps the partials'
  const int pos = a.pos[m], slot = a.slots[m];
  const bool normed = h < a.nq + a.nkv;
  float g0 = 1.0f, g1 = 1.0f, c = 0.0f, sn = 0.0f;
  if (normed) {
    const f16* gn = h < a.nq ? a.q_gain : a.k_gain;
    g0 = static_cast<float>(ld_global(gn, lane));
    g1 = static_cast<float>(ld_global(gn, lane + 64));
    c = a.rope_cos[static_cast<size_t>(pos) * 64 + lane];
    sn = a.rope_sin[static_cast<size_t>(pos) * 64 + lane];
  }
  float x0, x1;
  if (a.gain != nullptr) {
    float r[3];
    sum_streams<3>({a.part + m, p + lane, p + lane + 64}, {ss_stride, split_stride, split_stride}, a.KS, r);
    const float sc = sk_rscale(a, r[0]);
    x0 = sc * r[1];
    x1 = sc * r[2];
  } else {
    float r[2];
    sum_streams<2>({p + lane, p + lane + 64}, {split_stride, split_stride}, a.KS, r);
    x0 = r[0];
    x1 = r[1];
  }
  if (normed) norm_rope_pair(x0, x1, g0, g1, a.eps, c, sn);
  if (h < a.nq) {
    float* dst = a.q_out + static_cast<size_t>(m) * a.nq * 128 + h * 128;
    dst[lane] = x0;
    dst[lane + 64] = x1;
  } else {
    const bool is_k = normed;
    const int g = is_k ? h - a.nq : h - a.nq - a.nkv;
    f16* cache = (is_k ? a.kcache : a.vcache) + static_cast<size_t>(slot) * a.slot_stride +
                 static_cast<size_t>(a.layer) * a.layer_stride + static_cast<size_t>(g) * a.cap * 128 +
                 static_cast<size_t>(pos) * 128;
    cache[lane] = static_cast<f16>(x0);
    cache[lane + 64] = static_cast<f16>(x1);
  }
}

hipError_t launch_skinny(const SkinnyArgs& in, int epi, hipStream_t s) {
  SkinnyArgs a = in;
  if (!skinny_supported(a.M, a.K) || a.Ntot <= 0 || a.N0 <= 0 || a.N0 > a.Ntot) return hipErrorInvalidValue;
  if (epi == EPI_SWIGLU && (a.w2 == nullptr || a.Ntot != 2 * a.N0 || a.N0 % 64 != 0)) return hipErrorInvalidValue;
  if (epi != EPI_SWIGLU && a.Ntot != a.N0) return hipErrorInvalidValue;
  if (epi == EPI_QKV && (a.Ntot != (a.nq + 2 * a.nkv) * 128 || a.pos == nullptr || a.slots == nullptr))
    return hipErrorInvalidValue;
  if (a.ldx % 4 != 0 || a.Ntot % 4 != 0) return hipErrorInvalidValue;
  static const hipError_t configured = skinny_configure();  // allow > 64 KB of dynamic LDS, once per process
  if (configured != hipSuccess) return configured;
  a.KS = skinny_splits(a.Ntot, a.K);
  a.Kb = a.K / a.KS;
  const size_t lds = static_cast<size_t>(2) * 16 * (a.Kb + 8) * sizeof(_Float16);
  const dim3 grid(skinny_tiles(epi, a.N0, a.Ntot), a.KS);
  const int nout = epi == EPI_SWIGLU ? a.N0 : a.Ntot;
  const dim3 g2((nout + 255) / 256, a.M);
  switch (epi) {
    case EPI_STORE:
      hipLaunchKernelGGL(k_skinny_part<EPI_STORE>, grid, dim3(512), lds, s, a);
      hipLaunchKernelGGL(k_skinny_epi<EPI_STORE>, g2, dim3(256), 0, s, a, nout);
      break;
    case EPI_RESIDUAL:
      hipLaunchKernelGGL(k_skinny_part<EPI_RESIDUAL>, grid, dim3(512), lds, s, a);
      hipLaunchKernelGGL(k_skinny_epi<EPI_RESIDUAL>, g2, dim3(256), 0, s, a, nout);
      break;
    case EPI_SWIGLU:
      hipLaunchKernelGGL(k_skinny_part<EPI_SWIGLU>, grid, dim3(512), lds, s, a);
      hipLaunchKernelGGL(k_skinny_epi<EPI_SWIGLU>, g2, dim3(256), 0, s, a, nout);
      break;
    case EPI_QKV:
      hipLaunchKernelGGL(k_skinny_part<EPI_QKV>, grid, dim3(512), lds, s, a);
      hipLaunchKernelGGL(k_skinny_epi_qkv, dim3(a.M, a.nq + 2 * a.nkv), dim3(64), 0, s, a);
      break;
    default:
      return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

size_t skinny_part_floats(int rows, int K) {
  const size_t ks = static_cast<size_t>(skinny_splits(rows, K));
  return 64 * ks + ks * 16 * rows;  // sums of squares, partials
}

hipError_t skinny_configure() {
  const int lds = static_cast<int>(2 * 16 * (SK_MAX_KB + 8) * sizeof(_Float16));
  hipError_t e = hipSuccess;
  for (const void* f : {reinterpret_cast<const void*>(&k_skinny_part<EPI_STORE>),
                        reinterpret_cast<const void*>(&k_skinny_part<EPI_RESIDUAL>),
                        reinterpret_cast<const void*>(&k_skinny_part<EPI_SWIGLU>),
                        reinterpret_cast<const void*>(&k_skinny_part<EPI_QKV>)})
    if (e == hipSuccess) e = hipFuncSetAttribute(f, hipFuncAttributeMaxDynamicSharedMemorySize, lds);
  return e;
}

}  // namespace soc
