// qpath.hip - the elementwise steps between the group-quantized projections of a quantized model's forward: the
// projections (k_qmm) take fp16 activation rows and write fp32 rows; these kernels round activations to fp16, add
// a projection into the residual stream, and form SwiGLU (silu(gate) * up, Mac/cpu/src/qwen_mlp.cpp:31) as fp16.
#include <algorithm>

#include "kernels.h"

namespace soc {
namespace {

__global__ void k_f32_to_f16(const float* __restrict__ x, size_t n, f16* __restrict__ y) {
  for (size_t i = blockIdx.x * static_cast<size_t>(blockDim.x) + threadIdx.x; i < n;
       i += static_cast<size_t>(gridDim.x) * blockDim.x)
    y[i] = static_cast<f16>(x[i]);
}

__global__ void k_add_f32(float* __restrict__ x, const float* __restrict__ y, size_t n) {
  for (size_t i = blockIdx.x * static_cast<size_t>(blockDim.x) + threadIdx.x; i < n;
       i += static_cast<size_t>(gridDim.x) * blockDim.x)
    x[i] += y[i];
}

// gu [T][2 I] (gate | up) -> h [T][I] fp16
__global__ void k_swiglu_f16(const float* __restrict__ gu, int T, int I, f16* __restrict__ h) {
  const size_t n = static_cast<size_t>(T) * I;
  for (size_t i = blockIdx.x * static_cast<size_t>(blockDim.x) + threadIdx.x; i < n;
       i += static_cast<size_t>(gridDim.x) * blockDim.x) {
    const size_t t = i / I, c = i % I;
    const float g = gu[t * 2 * I + c], u = gu[t * 2 * I + I + c];
    h[i] = static_cast<f16>(silu_ref(g) * u);
  }
}

int blocks_for(size_t n) { return static_cast<int>(std::min<size_t>((n + 255) / 256, 2048)); }

}  // namespace

hipError_t launch_f32_to_f16(const float* x, size_t n, f16* y, hipStream_t s) {
  hipLaunchKernelGGL(k_f32_to_f16, dim3(blocks_for(n)), dim3(256), 0, s, x, n, y);
  return hipGetLastError();
}

hipError_t launch_add_f32(float* x, const float* y, size_t n, hipStream_t s) {
  hipLaunchKernelGGL(k_add_f32, dim3(blocks_for(n)), dim3(256), 0, s, x, y, n);
  return hipGetLastError();
}

hipError_t launch_swiglu_f16(const float* gu, int T, int I, f16* h, hipStream_t s) {
  hipLaunchKernelGGL(k_swiglu_f16, dim3(blocks_for(static_cast<size_t>(T) * I)), dim3(256), 0, s, gu, T, I, h);
  return hipGetLastError();
}

}  // namespace soc
