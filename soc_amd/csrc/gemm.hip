// gemm.hip - prefill projections C = A . W^T with fp32 activations and fp16 weights.
//
// Reference computation: Linear::Forward over T rows (Mac/cpu/src/linear.cpp:145-157), fp32 accumulation.
// k_gemm_f32a is the LDS-tiled FMA kernel used for every shape (64x64 output tiles, 32-deep K slices staged in
// LDS, 4x4 outputs per thread), with the same epilogues as the decode GEMV.
#include "kernels.h"

namespace soc {

namespace {
constexpr int BM = 64, BN = 64, BK = 32;
}

template <int EPI>
__global__ __launch_bounds__(256) void k_gemm_f32a(GemmArgs g) {
  constexpr int NW = EPI == EPI_SWIGLU ? 2 : 1;
  __shared__ float As[BK][BM + 4];
  __shared__ float Ws[NW][BK][BN + 4];
  const int tid = threadIdx.x;
  const int m0 = blockIdx.y * BM, n0 = blockIdx.x * BN;
  const int tx = tid & 15, ty = tid >> 4;
  float acc[NW][4][4];
#pragma unroll
  for (int w = 0; w < NW; ++w)
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j) acc[w][i][j] = 0.0f;

  for (int k0 = 0; k0 < g.K; k0 += BK) {
    // A tile: 64 rows x 32 k, 8 floats per thread
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const int idx = tid + e * 256;
      const int r = idx / BK, kk = idx % BK;
      const int m = m0 + r, k = k0 + kk;
      As[kk][r] = (m < g.M && k < g.K) ? g.a[static_cast<size_t>(m) * g.lda + k] : 0.0f;
    }
    // W tile(s): 64 rows x 32 k, 8 halves per thread
#pragma unroll
    for (int w = 0; w < NW; ++w) {
      const f16* src = w == 0 ? g.w : g.w2;
      const int r = tid / 4, kk = (tid % 4) * 8;
      const int n = n0 + r;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const int k = k0 + kk + i;
        Ws[w][kk + i][r] = (n < g.N && k < g.K) ? static_cast<float>(src[static_cast<size_t>(n) * g.K + k]) : 0.0f;
      }
    }
    __syncthreads();
#pragma unroll 8
    for (int kk = 0; kk < BK; ++kk) {
      float av[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) av[i] = As[kk][ty * 4 + i];
#pragma unroll
      for (int w = 0; w < NW; ++w) {
        float wv[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) wv[j] = Ws[w][kk][tx * 4 + j];
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
          for (int j = 0; j < 4; ++j) acc[w][i][j] += av[i] * wv[j];
      }
    }
    __syncthreads();
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int m = m0 + ty * 4 + i;
    if (m >= g.M) continue;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int n = n0 + tx * 4 + j;
      if (n >= g.N) continue;
      float* dst = g.c + static_cast<size_t>(m) * g.ldc + n;
      float v = acc[0][i][j];
      if constexpr (EPI == EPI_SWIGLU) v = silu_ref(v) * acc[NW - 1][i][j];
      if constexpr (EPI == EPI_RESIDUAL) v = *dst + v;
      *dst = v;
    }
  }
}

hipError_t launch_gemm_f32a(const GemmArgs& g, int epi, hipStream_t s) {
  const dim3 grid((g.N + BN - 1) / BN, (g.M + BM - 1) / BM), block(256);
  switch (epi) {
    case EPI_STORE: hipLaunchKernelGGL(k_gemm_f32a<EPI_STORE>, grid, block, 0, s, g); break;
    case EPI_RESIDUAL: hipLaunchKernelGGL(k_gemm_f32a<EPI_RESIDUAL>, grid, block, 0, s, g); break;
    case EPI_SWIGLU: hipLaunchKernelGGL(k_gemm_f32a<EPI_SWIGLU>, grid, block, 0, s, g); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

}  // namespace soc
