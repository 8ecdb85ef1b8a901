// skinny.hip - projections of a ragged decode batch: y[M][N] = x[M][K] . W[N][K]^T with M <= 16 rows of fp32
// activations (one per sequence) and fp16 weights, on MFMA (v_mfma_f32_16x16x32_f16).
//
// At M <= 16 the work is a weight stream (2 bytes per weight, 2M flops), so the kernel is built around moving W at
// HBM rate: every weight is read once, straight into registers, 16 rows x 256 K per wave per chunk with the next
// chunk in flight, and meets all M activation rows in one MFMA. The activations of the block's K range are split
// once into hi = f16(x) and lo = f16((x - hi) 2^11) in LDS (about 22 bits of each fp32 value; weights are exact), so
// the products track the fp32 reference (Mac/cpu/src/linear.cpp:51-84) up to the order of the sums.
//
// The grid is (row tiles of 128, K splits): the split count is chosen so that the grid covers the chip even for the
// 2560-row projections. Each block writes its partial sums; a second kernel adds the splits in a fixed order (so a
// row's result never depends on the other rows of the batch or on timing) and applies the epilogue: store,
// residual add, or SwiGLU of the gate/up halves.
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
// SK_MAX_KB of K per block) with the least estimated traffic time: weight bytes over the evenness with which the
// d * tiles blocks fill the chip's block slots (blocks / slots over its ceiling; 2 blocks per CU when the block's LDS
// allows, the kernel's registers allow 2) plus the partial sums written and read back (16 rows x 4 bytes x rows x d,
// twice).
int skinny_splits(int rows, int K) {
  const int n256 = K / SK_CHUNK;
  const int tiles = (rows + SK_ROWS - 1) / SK_ROWS;
  int best = n256;
  double best_cost = 0.0;
  for (int d = 1; d <= n256; ++d) {
    const int kb = K / d;
    if (n256 % d != 0 || kb > SK_MAX_KB) continue;
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

// grid = (ceil(Ntot / 128), KS), block = 512, dynamic LDS 2 x 16 x (Kb + 8) halves.
__global__ __launch_bounds__(512) void k_skinny_part(SkinnyArgs a) {
  extern __shared__ _Float16 sk_lds[];
  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
  const int ks = blockIdx.y;
  const int k0 = ks * a.Kb;
  const int ld = a.Kb + 8;
  _Float16* xh = sk_lds;
  _Float16* xl = sk_lds + 16 * ld;
  const int r0 = blockIdx.x * SK_ROWS + wid * 16;
  const bool active = r0 < a.Ntot;
  const int rl = lane & 15, kq = lane >> 4;
  // A operand = W rows r0..r0+15 (lane: row r0 + rl, k = 8 kq + i); rows past Ntot repeat the last row, never stored
  const int rr = min(r0 + rl, a.Ntot - 1);
  const f16* wrow = (rr < a.N0 ? a.w + static_cast<size_t>(rr) * a.K : a.w2 + static_cast<size_t>(rr - a.N0) * a.K) +
                    k0 + kq * 8;
  const int nch = a.Kb / SK_CHUNK;
  u32x4 wa[8], wb[8];
  auto load = [&](u32x4* dst, int c) {
#pragma unroll
    for (int s = 0; s < 8; ++s) dst[s] = load_stream16(wrow + c * SK_CHUNK + s * 32);
  };
  // the weight stream does not depend on the activations: start it before staging them
  if (active) load(wa, 0);

  // activations of this K range -> hi/lo fp16 in LDS (rows past M are zero)
  const int q4 = a.Kb / 4;
  for (int i = tid; i < 16 * q4; i += 512) {
    const int m = i / q4, c = (i % q4) * 4;
    const f32x4 v = m < a.M ? *reinterpret_cast<const f32x4*>(a.x + static_cast<size_t>(m) * a.ldx + k0 + c)
                            : f32x4{0.f, 0.f, 0.f, 0.f};
    f16x4 hi, lo;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const _Float16 h = static_cast<_Float16>(v[j]);
      hi[j] = h;
      lo[j] = static_cast<_Float16>((v[j] - static_cast<float>(h)) * 2048.0f);
    }
    *reinterpret_cast<f16x4*>(&xh[m * ld + c]) = hi;
    *reinterpret_cast<f16x4*>(&xl[m * ld + c]) = lo;
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
    if (c + 1 < nch) load(wb, c + 1);
    mma(wa, c);
    if (c + 1 < nch) {
      if (c + 2 < nch) load(wa, c + 2);
      mma(wb, c + 1);
    }
  }
  // D: lane holds rows r0 + 4 kq + i (i = 0..3) of token rl
  const int row = r0 + 4 * kq;
  if (row < a.Ntot) {
    f32x4 v;
#pragma unroll
    for (int i = 0; i < 4; ++i) v[i] = acc[i] + accl[i] * (1.0f / 2048.0f);
    float* dst = a.part + (static_cast<size_t>(ks) * 16 + rl) * a.Ntot + row;
    if (row + 3 < a.Ntot) {
      *reinterpret_cast<f32x4*>(dst) = v;
    } else {
      for (int i = 0; row + i < a.Ntot; ++i) dst[i] = v[i];
    }
  }
}

// Sum of n partials p[0], p[stride], ... in index order, with the loads issued eight at a time.
__device__ __forceinline__ float sum_splits(const float* p, size_t stride, int n) {
  float v = 0.0f;
  int k = 0;
  for (; k + 8 <= n; k += 8) {
    float x[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) x[u] = p[(k + u) * stride];
#pragma unroll
    for (int u = 0; u < 8; ++u) v += x[u];
  }
  for (; k < n; ++k) v += p[k * stride];
  return v;
}

// One thread per (row m, output n): sum of the KS partials in split order, then the epilogue.
template <int EPI>
__global__ __launch_bounds__(256) void k_skinny_epi(SkinnyArgs a, int nout) {
  const int n = blockIdx.x * 256 + threadIdx.x, m = blockIdx.y;
  if (n >= nout) return;
  const float* p = a.part + static_cast<size_t>(m) * a.Ntot + n;
  const size_t split_stride = static_cast<size_t>(16) * a.Ntot;
  const float v = sum_splits(p, split_stride, a.KS);
  float* dst = a.c + static_cast<size_t>(m) * a.ldc + n;
  if constexpr (EPI == EPI_SWIGLU) {
    const float u = sum_splits(p + a.N0, split_stride, a.KS);
    *dst = silu_ref(v) * u;
  } else if constexpr (EPI == EPI_RESIDUAL) {
    *dst += v;
  } else {
    *dst = v;
  }
}

hipError_t launch_skinny(const SkinnyArgs& in, int epi, hipStream_t s) {
  SkinnyArgs a = in;
  if (!skinny_supported(a.M, a.K) || a.Ntot <= 0 || a.N0 <= 0 || a.N0 > a.Ntot) return hipErrorInvalidValue;
  if (epi == EPI_SWIGLU && (a.w2 == nullptr || a.Ntot != 2 * a.N0)) return hipErrorInvalidValue;
  if (epi != EPI_SWIGLU && a.Ntot != a.N0) return hipErrorInvalidValue;
  if (a.ldx % 4 != 0 || a.Ntot % 4 != 0) return hipErrorInvalidValue;
  static const hipError_t configured = skinny_configure();  // allow > 64 KB of dynamic LDS, once per process
  if (configured != hipSuccess) return configured;
  a.KS = skinny_splits(a.Ntot, a.K);
  a.Kb = a.K / a.KS;
  const size_t lds = static_cast<size_t>(2) * 16 * (a.Kb + 8) * sizeof(_Float16);
  const dim3 grid((a.Ntot + SK_ROWS - 1) / SK_ROWS, a.KS);
  hipLaunchKernelGGL(k_skinny_part, grid, dim3(512), lds, s, a);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  const int nout = epi == EPI_SWIGLU ? a.N0 : a.Ntot;
  const dim3 g2((nout + 255) / 256, a.M);
  switch (epi) {
    case EPI_STORE: hipLaunchKernelGGL(k_skinny_epi<EPI_STORE>, g2, dim3(256), 0, s, a, nout); break;
    case EPI_RESIDUAL: hipLaunchKernelGGL(k_skinny_epi<EPI_RESIDUAL>, g2, dim3(256), 0, s, a, nout); break;
    case EPI_SWIGLU: hipLaunchKernelGGL(k_skinny_epi<EPI_SWIGLU>, g2, dim3(256), 0, s, a, nout); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

size_t skinny_part_floats(int rows, int K) {
  return static_cast<size_t>(skinny_splits(rows, K)) * 16 * rows;
}

hipError_t skinny_configure() {
  return hipFuncSetAttribute(reinterpret_cast<const void*>(&k_skinny_part),
                             hipFuncAttributeMaxDynamicSharedMemorySize,
                             static_cast<int>(2 * 16 * (SK_MAX_KB + 8) * sizeof(_Float16)));
}

}  // namespace soc
