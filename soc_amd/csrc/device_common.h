// device_common.h - small device helpers shared by the HIP kernels (gfx950, wave64).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace soc {

typedef _Float16 f16;
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef int32_t i32x4 __attribute__((ext_vector_type(4)));

constexpr int kWave = 64;
constexpr uint64_t kSpinTicks = 20000000ull;  // default bound of a cross-block wait: 200 ms of the 100 MHz counter

// Global-memory view of a pointer. Pointers read from device memory (per-layer weight tables) are generic to the
// compiler, which then emits FLAT loads; FLAT loads also count against lgkmcnt, so every later LDS wait of the wave
// would wait for them too. These helpers are only used on global memory.
typedef const __attribute__((address_space(1))) u32x4 gu32x4;

// 16-byte streaming load from global memory that does not keep the line in the caches (weights are read once per
// step).
__device__ __forceinline__ u32x4 load_stream16(const void* p) { return __builtin_nontemporal_load((gu32x4*)p); }
__device__ __forceinline__ u32x4 load16(const void* p) { return *(gu32x4*)p; }

// Element i of a table in global memory (weight-pointer tables, norm gains) through a global load.
template <typename T>
__device__ __forceinline__ T ld_global(const T* p, size_t i) {
  return ((const __attribute__((address_space(1))) T*)p)[i];
}

__device__ __forceinline__ f16x8 as_f16x8(u32x4 v) { return __builtin_bit_cast(f16x8, v); }

// Exact fp16 -> fp32 of 8 packed halves.
__device__ __forceinline__ void f16x8_to_f32(u32x4 v, float* out) {
  const f16x8 h = as_f16x8(v);
#pragma unroll
  for (int i = 0; i < 8; ++i) out[i] = static_cast<float>(h[i]);
}

// Cross-lane moves inside a row of 16 lanes (DPP, no LDS round trip). CTRL: 0xB1 = quad_perm [1,0,3,2] (lane ^ 1),
// 0x4E = quad_perm [2,3,0,1] (lane ^ 2), 0x141 = row_half_mirror (lane ^ 7 within 8), 0x140 = row_mirror
// (lane ^ 15 within 16).
template <int CTRL>
__device__ __forceinline__ float dpp_mov(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, true));
}

// Sum over aligned groups of `width` lanes (width a power of two <= 64); every lane gets its group's sum.
// Within a 16-lane row: DPP steps (xor 1, xor 2, half mirror, mirror); across rows: lane reads of the row sums.
template <int width>
__device__ __forceinline__ float group_sum(float v) {
  static_assert(width == 1 || width == 2 || width == 4 || width == 8 || width == 16 || width == 32 || width == 64,
                "width must be a power of two <= 64");
  if constexpr (width >= 2) v += dpp_mov<0xB1>(v);
  if constexpr (width >= 4) v += dpp_mov<0x4E>(v);
  if constexpr (width >= 8) v += dpp_mov<0x141>(v);
  if constexpr (width >= 16) v += dpp_mov<0x140>(v);
  if constexpr (width == 32) {
    const float r0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0));
    const float r1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 16));
    const float r2 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32));
    const float r3 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 48));
    v = (threadIdx.x & 32) ? r2 + r3 : r0 + r1;
  } else if constexpr (width == 64) {
    const float r0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0));
    const float r1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 16));
    const float r2 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32));
    const float r3 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 48));
    v = (r0 + r1) + (r2 + r3);
  }
  return v;
}

__device__ __forceinline__ float wave_sum(float v) { return group_sum<64>(v); }

__device__ __forceinline__ float wave_max(float v) {
  v = fmaxf(v, dpp_mov<0xB1>(v));
  v = fmaxf(v, dpp_mov<0x4E>(v));
  v = fmaxf(v, dpp_mov<0x141>(v));
  v = fmaxf(v, dpp_mov<0x140>(v));
  const float r0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0));
  const float r1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 16));
  const float r2 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32));
  const float r3 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 48));
  return fmaxf(fmaxf(r0, r1), fmaxf(r2, r3));
}

// Block-wide sum for blockDim.x == NT threads; `red` must hold NT/64 floats. All threads get the result.
template <int NT>
__device__ __forceinline__ float block_sum(float v, float* red) {
  v = wave_sum(v);
  const int w = threadIdx.x / kWave;
  if ((threadIdx.x & (kWave - 1)) == 0) red[w] = v;
  __syncthreads();
  float s = 0.0f;
#pragma unroll
  for (int i = 0; i < NT / kWave; ++i) s += red[i];
  __syncthreads();
  return s;
}

// Lane l of a wave holds dims (l, l + 64) of one 128-dim head vector: RMSNorm over the 128 values and rotate-half
// RoPE at one table row (cos/sin precomputed on the host in double, then rounded to float, like rope.cpp:77-79).
// The multiply-adds are written as explicit fmaf so that every kernel that inlines this computes the same bits
// (the QKV GEMM epilogue and the stand-alone q/k-norm kernel must agree exactly).
__device__ __forceinline__ void norm_rope_pair(float& x0, float& x1, const f16* gain, float eps, const float* cosr,
                                               const float* sinr, int lane) {
  const float ss = wave_sum(fmaf(x0, x0, x1 * x1));
  const float scale = 1.0f / sqrtf(ss / 128.0f + eps);
  const float y0 = x0 * scale * static_cast<float>(ld_global(gain, lane));
  const float y1 = x1 * scale * static_cast<float>(ld_global(gain, lane + 64));
  const float c = cosr[lane], s = sinr[lane];
  x0 = fmaf(y0, c, -(y1 * s));
  x1 = fmaf(y0, s, y1 * c);
  // Materialise the fp32 results: otherwise a caller's f16 conversion can be folded into the fma
  // (v_fma_mixlo_f16, one rounding straight to f16), which differs from rounding to fp32 first in rare cases and
  // would make the cached keys depend on which kernel wrote them.
  __asm__ volatile("" : "+v"(x0), "+v"(x1));
}

// The same with the gains g0 = gain[lane], g1 = gain[lane + 64] and the table entries c = cosr[lane], s = sinr[lane]
// loaded by the caller (so that it can request them early); the same operations in the same order.
__device__ __forceinline__ void norm_rope_pair(float& x0, float& x1, float g0, float g1, float eps, float c, float s) {
  const float ss = wave_sum(fmaf(x0, x0, x1 * x1));
  const float scale = 1.0f / sqrtf(ss / 128.0f + eps);
  const float y0 = x0 * scale * g0;
  const float y1 = x1 * scale * g1;
  x0 = fmaf(y0, c, -(y1 * s));
  x1 = fmaf(y0, s, y1 * c);
  __asm__ volatile("" : "+v"(x0), "+v"(x1));
}

// SiLU exactly as the reference writes it: v / (1 + exp(-v)) (Mac/cpu/src/qwen_mlp.cpp:31).
__device__ __forceinline__ float silu_ref(float v) { return v / (1.0f + expf(-v)); }

// Relaxed device-scope accesses: on gfx950 these are plain loads/stores with the sc1 bit (coherent across XCDs,
// no cache maintenance instructions). Used for small cross-block hand-offs.
__device__ __forceinline__ void st_dev(float* p, float v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float ld_dev(const float* p) {
  return __hip_atomic_load(const_cast<float*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_dev(int32_t* p, int32_t v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ int32_t ld_dev(const int32_t* p) {
  return __hip_atomic_load(const_cast<int32_t*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Waits until this wave's earlier memory accesses have completed. After device-scope (write-through) stores this
// makes them visible to any agent-scope reader, so a following relaxed counter update publishes them without a
// full release fence (which on gfx950 writes back and invalidates the whole L2 of the XCD).
__device__ __forceinline__ void wait_mem() {
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  __builtin_amdgcn_s_waitcnt(0);
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
}

}  // namespace soc
