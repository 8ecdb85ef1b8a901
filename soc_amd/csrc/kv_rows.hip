// kv_rows.hip - copies K/V rows in the reference's [rows][kv_heads * head_dim] layout (fp32 or fp16) into the fp16
// [kv_head][capacity][head_dim] layout of one (slot, layer) of the cache (KVCache::AppendPrefill /
// AppendDecodeToken, Mac/gpu/src/runtime/kv_cache.mm:78-131, which copies fp32 rows into its fp32 layer buffer).
#include <algorithm>

#include "kernels.h"

namespace soc {
namespace {

template <typename T>
__global__ void k_kv_append_rows(const T* __restrict__ keys, const T* __restrict__ values, int rows, int nkv, int hd,
                                 int cap, int pos, f16* __restrict__ kdst, f16* __restrict__ vdst) {
  const size_t n = static_cast<size_t>(rows) * nkv * hd;
  for (size_t e = blockIdx.x * static_cast<size_t>(blockDim.x) + threadIdx.x; e < n;
       e += static_cast<size_t>(gridDim.x) * blockDim.x) {
    const int d = static_cast<int>(e % hd);
    const int h = static_cast<int>((e / hd) % nkv);
    const int r = static_cast<int>(e / (static_cast<size_t>(hd) * nkv));
    const size_t o = (static_cast<size_t>(h) * cap + pos + r) * hd + d;
    kdst[o] = static_cast<f16>(static_cast<float>(keys[e]));
    vdst[o] = static_cast<f16>(static_cast<float>(values[e]));
  }
}

}  // namespace

hipError_t launch_kv_append_rows(const void* keys, const void* values, bool fp16, int rows, int nkv, int hd, int cap,
                                 int pos, f16* kdst, f16* vdst, hipStream_t s) {
  const size_t n = static_cast<size_t>(rows) * nkv * hd;
  const int blocks = static_cast<int>(std::min<size_t>((n + 255) / 256, 4096));
  if (fp16)
    hipLaunchKernelGGL(k_kv_append_rows<f16>, dim3(blocks), dim3(256), 0, s, static_cast<const f16*>(keys),
                       static_cast<const f16*>(values), rows, nkv, hd, cap, pos, kdst, vdst);
  else
    hipLaunchKernelGGL(k_kv_append_rows<float>, dim3(blocks), dim3(256), 0, s, static_cast<const float*>(keys),
                       static_cast<const float*>(values), rows, nkv, hd, cap, pos, kdst, vdst);
  return hipGetLastError();
}

}  // namespace soc
