// ops.hip - the reference GPU runtime's op kernels (the static Run of Mac/gpu/include/op/*.h: MatMulOp / LinearOp,
// RmsNormOp, RopeOp, SoftmaxOp, EmbeddingOp, ElementwiseMulOp) as gfx950 kernels on caller device pointers, in fp32
// as the reference computes them (gpu_kernels.metal:82-289), and the check every op-level entry point makes of caller
// memory before a kernel reads it.
//
// These serve callers of the reference's op API and the op-level tests; the model's forward passes use the fused
// kernels of the other files.
#include <cmath>
#include <cstring>
#include <string>
#include <vector>

#include "capi_internal.h"
#include "device_common.h"
#include "kernels.h"

namespace soc {

MemRange classify_range(const void* p, size_t bytes) {
  hipPointerAttribute_t attr{};
  if (hipPointerGetAttributes(&attr, p) != hipSuccess) {
    (void)hipGetLastError();  // pageable host memory may fail the query: that is the answer, not an error
    return MemRange::kPageable;
  }
  if (attr.type == hipMemoryTypeHost && attr.devicePointer != p) return MemRange::kPageable;
  if (attr.type != hipMemoryTypeDevice && attr.type != hipMemoryTypeManaged && attr.type != hipMemoryTypeHost)
    return MemRange::kPageable;
  void* base = nullptr;
  size_t size = 0;
  if (hipMemGetAddressRange(&base, &size, const_cast<void*>(p)) != hipSuccess) {
    (void)hipGetLastError();
    return MemRange::kOutside;
  }
  return static_cast<const char*>(p) + bytes <= static_cast<const char*>(base) + size ? MemRange::kDeviceRange
                                                                                       : MemRange::kOutside;
}

int check_device_operand(const char* what, const void* p, size_t bytes) {
  if (bytes == 0) return SOC_OK;
  if (p == nullptr) return fail(SOC_ERR_INVALID, std::string(what) + ": null device pointer");
  const MemRange r = classify_range(p, bytes);
  if (r == MemRange::kDeviceRange) return SOC_OK;
  return fail(SOC_ERR_INVALID, std::string(what) + (r == MemRange::kPageable
                                                        ? " is not in device memory"
                                                        : " extends past the end of its device allocation"));
}

namespace {

// ---- MatMul (matmul_f32_basic, gpu_kernels.metal:253-289): out = lhs . rhs (+ bias) (+ residual), then SiLU ----
// 64 x 64 output tile per 256-thread block, each wave a 32 x 32 quarter as 2 x 2 tiles of v_mfma_f32_16x16x4_f32
// (fp32 operands and accumulation, as the reference's fp32 kernel); K in LDS slices of 16. MFMA operand layout: lane
// l holds A[l % 16][l / 16] and B[l / 16][l % 16]; the 16 x 16 result row 4 (l / 16) + e, column l % 16 sits in
// element e of lane l.
constexpr int kMmBM = 64, kMmBN = 64, kMmBK = 16;

__global__ __launch_bounds__(256) void k_matmul_f32(const float* __restrict__ lhs, const float* __restrict__ rhs,
                                                    const float* bias, const float* residual, float* out, int M, int K,
                                                    int N, int trans, int silu) {
  __shared__ float as[kMmBK][kMmBM + 4];  // [k][m]
  __shared__ float bs[kMmBK][kMmBN + 4];  // [k][n]
  const int tid = threadIdx.x, wid = tid >> 6, lane = tid & 63;
  const int tiles_n = (N + kMmBN - 1) / kMmBN;
  const int m0 = static_cast<int>(blockIdx.x / tiles_n) * kMmBM, n0 = static_cast<int>(blockIdx.x % tiles_n) * kMmBN;
  const int wm = (wid >> 1) * 32, wn = (wid & 1) * 32;
  f32x4 acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
  for (int k0 = 0; k0 < K; k0 += kMmBK) {
    {  // lhs rows m0 .. + 64, columns k0 .. + 16: thread t takes row t / 4, columns 4 (t % 4) .. + 4
      const int m = tid >> 2, kk = (tid & 3) * 4, gm = m0 + m;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int gk = k0 + kk + e;
        as[kk + e][m] = (gm < M && gk < K) ? lhs[static_cast<size_t>(gm) * K + gk] : 0.0f;
      }
    }
    if (!trans) {  // rhs [K][N]: thread t takes row k0 + t / 16, columns 4 (t % 16) .. + 4
      const int kk = tid >> 4, n = (tid & 15) * 4, gk = k0 + kk;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int gn = n0 + n + e;
        bs[kk][n + e] = (gk < K && gn < N) ? rhs[static_cast<size_t>(gk) * N + gn] : 0.0f;
      }
    } else {  // rhs [N][K] read transposed: thread t takes rhs row n0 + t / 4, columns 4 (t % 4) .. + 4
      const int n = tid >> 2, kk = (tid & 3) * 4, gn = n0 + n;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int gk = k0 + kk + e;
        bs[kk + e][n] = (gn < N && gk < K) ? rhs[static_cast<size_t>(gn) * K + gk] : 0.0f;
      }
    }
    __syncthreads();
#pragma unroll
    for (int ks = 0; ks < kMmBK; ks += 4) {
      const int k = ks + (lane >> 4);
      float a[2], b[2];
#pragma unroll
      for (int i = 0; i < 2; ++i) a[i] = as[k][wm + 16 * i + (lane & 15)];
#pragma unroll
      for (int j = 0; j < 2; ++j) b[j] = bs[k][wn + 16 * j + (lane & 15)];
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[i], b[j], acc[i][j], 0, 0, 0);
    }
    __syncthreads();
  }
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int r = m0 + wm + 16 * i + 4 * (lane >> 4) + e, c = n0 + wn + 16 * j + (lane & 15);
        if (r < M && c < N) {
          float v = acc[i][j][e];
          if (bias != nullptr) v += bias[c];
          if (residual != nullptr) v += residual[static_cast<size_t>(r) * N + c];
          if (silu) v = v / (1.0f + expf(-v));
          out[static_cast<size_t>(r) * N + c] = v;
        }
      }
}

// ---- RMSNorm (rms_norm_module.cpp:56-64; rms_norm_f32_rowwise, gpu_kernels.metal:82-102): one block per row ----
__global__ __launch_bounds__(256) void k_rmsnorm_f32(const float* __restrict__ x, const float* __restrict__ w,
                                                     float* y, int n, float eps) {
  __shared__ float red[4];
  const float* xr = x + static_cast<size_t>(blockIdx.x) * n;
  float* yr = y + static_cast<size_t>(blockIdx.x) * n;
  float ss = 0.0f;
  for (int i = threadIdx.x; i < n; i += 256) ss += xr[i] * xr[i];
  ss = block_sum<256>(ss, red);
  const float s = 1.0f / sqrtf(ss / static_cast<float>(n) + eps);
  for (int i = threadIdx.x; i < n; i += 256) yr[i] = __fmul_rn(__fmul_rn(xr[i], s), w[i]);
}

// ---- RoPE (rope.cpp:54-89; rope_f32_qwen, gpu_kernels.metal:138-170) over [rows][heads * head_dim]: rotate-half on
// the first rotary_dim dims of each head with the angle table built on the host in double, the remaining dims copied.
// One thread per (head, pair), so in-place calls are safe. ----
__global__ __launch_bounds__(256) void k_rope_f32(const float* x, float* y, const float* __restrict__ cs,
                                                  const float* __restrict__ sn, int heads, int hd, int rd) {
  const int row = blockIdx.x, half = rd / 2;
  const size_t rbase = static_cast<size_t>(row) * heads * hd;
  for (int t = threadIdx.x; t < heads * half; t += 256) {
    const int h = t / half, i = t % half;
    const size_t b = rbase + static_cast<size_t>(h) * hd;
    const float first = x[b + i], second = x[b + i + half];
    const float c = cs[static_cast<size_t>(row) * half + i], s = sn[static_cast<size_t>(row) * half + i];
    y[b + i] = __fsub_rn(__fmul_rn(first, c), __fmul_rn(second, s));
    y[b + i + half] = __fadd_rn(__fmul_rn(first, s), __fmul_rn(second, c));
  }
  if (x != y && rd < hd)
    for (int t = threadIdx.x; t < heads * (hd - rd); t += 256) {
      const size_t idx = rbase + static_cast<size_t>(t / (hd - rd)) * hd + rd + t % (hd - rd);
      y[idx] = x[idx];
    }
}

// ---- Softmax (softmax_f32_rowwise, gpu_kernels.metal:172-193): max, exp(x - max), sum, divide; one block per row ----
__global__ __launch_bounds__(256) void k_softmax_f32(const float* x, float* y, int n) {
  __shared__ float red[4];
  const float* xr = x + static_cast<size_t>(blockIdx.x) * n;
  float* yr = y + static_cast<size_t>(blockIdx.x) * n;
  float m = -INFINITY;
  for (int i = threadIdx.x; i < n; i += 256) m = fmaxf(m, xr[i]);
  m = wave_max(m);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = m;
  __syncthreads();
  m = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  __syncthreads();
  float sum = 0.0f;
  for (int i = threadIdx.x; i < n; i += 256) {
    const float e = expf(xr[i] - m);
    yr[i] = e;
    sum += e;
  }
  sum = block_sum<256>(sum, red);  // its barriers also order the stores above before the divisions below
  for (int i = threadIdx.x; i < n; i += 256) yr[i] = yr[i] / sum;
}

// ---- Embedding (embedding_f32_lookup / embedding_f16_lookup, gpu_kernels.metal:104-136): an id outside
// [0, vocab) gives a zero row ----
template <typename T>
__global__ __launch_bounds__(256) void k_embedding(const int32_t* __restrict__ ids, const T* __restrict__ table,
                                                   float* out, int hidden, int vocab) {
  const int id = ids[blockIdx.x];
  float* o = out + static_cast<size_t>(blockIdx.x) * hidden;
  const bool ok = id >= 0 && id < vocab;
  for (int i = threadIdx.x; i < hidden; i += 256)
    o[i] = ok ? static_cast<float>(table[static_cast<size_t>(id) * hidden + i]) : 0.0f;
}

// ---- ElementwiseMul (elementwise_mul_f32, gpu_kernels.metal:195-205) ----
__global__ __launch_bounds__(256) void k_mul_f32(const float* a, const float* b, float* y, size_t n) {
  for (size_t i = static_cast<size_t>(blockIdx.x) * 256 + threadIdx.x; i < n; i += static_cast<size_t>(gridDim.x) * 256)
    y[i] = a[i] * b[i];
}

// Token ids from device memory into the forward's id buffer: an id outside [0, vocab) becomes 0 and raises *err
// (the host reads the flag with the call's results and fails the call).
__global__ __launch_bounds__(256) void k_stage_ids(const int32_t* __restrict__ src, int n, int vocab, int32_t* dst,
                                                   int* err) {
  for (int i = blockIdx.x * 256 + threadIdx.x; i < n; i += gridDim.x * 256) {
    const int32_t id = src[i];
    const bool ok = id >= 0 && id < vocab;
    dst[i] = ok ? id : 0;
    if (!ok) *err = 1;
  }
}

// A decode step's inputs: state[0] = the token (the host's, or the validated id at dev_last), state[1] = its
// position, ring position 0.
__global__ void k_decode_prologue(const int32_t* __restrict__ dev_last, int32_t host_last, int32_t pos, int vocab,
                                  int32_t* __restrict__ state, int32_t* __restrict__ ring, int* __restrict__ err) {
  if (threadIdx.x != 0) return;
  int32_t tok = host_last;
  if (dev_last != nullptr) {
    tok = *dev_last;
    if (tok < 0 || tok >= vocab) {
      tok = 0;
      *err = 1;
    }
  }
  state[0] = tok;
  state[1] = pos;
  *ring = 0;
}

// A decode step's results into pinned host words: the next token, the wait error flag, the token id error flag.
__global__ void k_decode_readback(const int32_t* __restrict__ state, const int32_t* __restrict__ wait_err,
                                  const int* __restrict__ id_err, int32_t* __restrict__ host) {
  if (threadIdx.x != 0) return;
  host[0] = state[0];
  host[1] = *wait_err;
  host[2] = id_err != nullptr ? *id_err : 0;
}

struct Words16 {
  int32_t w[16];
};

// dst[0..n) = v.w[0..n), n <= 16, the words travelling in the kernel's arguments.
__global__ void k_write_words(int32_t* __restrict__ dst, int n, Words16 v) {
  const int i = threadIdx.x;
  if (i >= n) return;
  int32_t x = v.w[0];
#pragma unroll
  for (int j = 1; j < 16; ++j) x = i == j ? v.w[j] : x;
  dst[i] = x;
}

int launch_status(const char* what) {
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? SOC_OK : fail(SOC_ERR_HIP, std::string(what) + ": " + hipGetErrorString(e));
}

int sync_status(soc_ctx* ctx, const char* what) {
  const hipError_t e = hipStreamSynchronize(ctx->stream);
  return e == hipSuccess ? SOC_OK : fail(SOC_ERR_HIP, std::string(what) + ": " + hipGetErrorString(e));
}

constexpr int64_t kMaxElems = int64_t{1} << 31;  // element counts the kernels index with 32-bit row offsets

}  // namespace

hipError_t launch_stage_ids(const int32_t* src, int n, int vocab, int32_t* dst, int* err, hipStream_t s) {
  hipLaunchKernelGGL(k_stage_ids, dim3(std::min(64, (n + 255) / 256)), dim3(256), 0, s, src, n, vocab, dst, err);
  return hipGetLastError();
}

hipError_t launch_decode_prologue(const int32_t* dev_last, int32_t host_last, int32_t pos, int vocab, int32_t* state,
                                  int32_t* ring, int* err, hipStream_t s) {
  hipLaunchKernelGGL(k_decode_prologue, dim3(1), dim3(64), 0, s, dev_last, host_last, pos, vocab, state, ring, err);
  return hipGetLastError();
}

hipError_t launch_decode_readback(const int32_t* state, const int32_t* wait_err, const int* id_err, int32_t* host,
                                  hipStream_t s) {
  hipLaunchKernelGGL(k_decode_readback, dim3(1), dim3(64), 0, s, state, wait_err, id_err, host);
  return hipGetLastError();
}

hipError_t launch_write_words(int32_t* dst, const int32_t* src, int n, hipStream_t s) {
  if (n <= 0 || n > 16) return hipErrorInvalidValue;
  Words16 v{};
  std::memcpy(v.w, src, static_cast<size_t>(n) * 4);
  hipLaunchKernelGGL(k_write_words, dim3(1), dim3(64), 0, s, dst, n, v);
  return hipGetLastError();
}

}  // namespace soc

using soc::check_device_operand;
using soc::fail;

int soc_op_matmul(soc_ctx* ctx, const float* lhs, const float* rhs, const float* bias, const float* residual,
                  float* out, int32_t rows, int32_t inner, int32_t cols, int32_t transpose_rhs, int32_t silu) {
  SOC_API_BEGIN
  if (ctx == nullptr) return fail(SOC_ERR_INVALID, "null context");
  if (rows <= 0 || inner <= 0 || cols <= 0) return fail(SOC_ERR_INVALID, "MatMul dimensions must be positive");
  if (int64_t{rows} * inner >= soc::kMaxElems || int64_t{inner} * cols >= soc::kMaxElems ||
      int64_t{rows} * cols >= soc::kMaxElems)
    return fail(SOC_ERR_INVALID, "MatMul operand too large");
  const size_t r = static_cast<size_t>(rows), k = static_cast<size_t>(inner), c = static_cast<size_t>(cols);
  SOC_TRY(check_device_operand("MatMul lhs", lhs, r * k * 4));
  SOC_TRY(check_device_operand("MatMul rhs", rhs, k * c * 4));
  SOC_TRY(check_device_operand("MatMul output", out, r * c * 4));
  if (bias != nullptr) SOC_TRY(check_device_operand("MatMul bias", bias, c * 4));
  if (residual != nullptr) SOC_TRY(check_device_operand("MatMul residual", residual, r * c * 4));
  const int tiles = ((rows + soc::kMmBM - 1) / soc::kMmBM) * ((cols + soc::kMmBN - 1) / soc::kMmBN);
  hipLaunchKernelGGL(soc::k_matmul_f32, dim3(tiles), dim3(256), 0, ctx->stream, lhs, rhs, bias, residual, out, rows,
                     inner, cols, transpose_rhs != 0, silu != 0);
  SOC_TRY(soc::launch_status("MatMul launch"));
  return soc::sync_status(ctx, "MatMul");
  SOC_API_END
}

int soc_op_rmsnorm(soc_ctx* ctx, const float* x, const float* weight, float* y, int32_t rows, int32_t n, float eps) {
  SOC_API_BEGIN
  if (ctx == nullptr) return fail(SOC_ERR_INVALID, "null context");
  if (rows <= 0 || n <= 0) return fail(SOC_ERR_INVALID, "RMSNorm dimensions must be positive");
  const size_t bytes = static_cast<size_t>(rows) * n * 4;
  SOC_TRY(check_device_operand("RMSNorm input", x, bytes));
  SOC_TRY(check_device_operand("RMSNorm weight", weight, static_cast<size_t>(n) * 4));
  SOC_TRY(check_device_operand("RMSNorm output", y, bytes));
  hipLaunchKernelGGL(soc::k_rmsnorm_f32, dim3(rows), dim3(256), 0, ctx->stream, x, weight, y, n, eps);
  SOC_TRY(soc::launch_status("RMSNorm launch"));
  return soc::sync_status(ctx, "RMSNorm");
  SOC_API_END
}

int soc_op_rope(soc_ctx* ctx, const float* x, float* y, int32_t rows, int32_t heads, int32_t head_dim,
                int32_t rotary_dim, int32_t position_offset, double theta) {
  SOC_API_BEGIN
  if (ctx == nullptr) return fail(SOC_ERR_INVALID, "null context");
  if (rows <= 0 || heads <= 0 || head_dim <= 0 || rotary_dim <= 0 || rotary_dim > head_dim || rotary_dim % 2 != 0 ||
      position_offset < 0)
    return fail(SOC_ERR_INVALID, "RoPE params do not match tensor shapes");
  const size_t bytes = static_cast<size_t>(rows) * heads * head_dim * 4;
  SOC_TRY(check_device_operand("RoPE input", x, bytes));
  SOC_TRY(check_device_operand("RoPE output", y, bytes));
  // the angle of rope.cpp:72-79 in double, rounded to float once per factor
  const int half = rotary_dim / 2;
  std::vector<float> cs(static_cast<size_t>(rows) * half), sn(cs.size());
  for (int r = 0; r < rows; ++r)
    for (int i = 0; i < half; ++i) {
      const double exponent = static_cast<double>(i * 2) / static_cast<double>(rotary_dim);
      const double angle = static_cast<double>(position_offset + r) / std::pow(theta, exponent);
      cs[static_cast<size_t>(r) * half + i] = static_cast<float>(std::cos(angle));
      sn[static_cast<size_t>(r) * half + i] = static_cast<float>(std::sin(angle));
    }
  float* d = nullptr;
  hipError_t e = hipMalloc(&d, cs.size() * 8);
  if (e != hipSuccess) return fail(SOC_ERR_NOMEM, "RoPE table allocation failed");
  e = hipMemcpyAsync(d, cs.data(), cs.size() * 4, hipMemcpyHostToDevice, ctx->stream);
  if (e == hipSuccess) e = hipMemcpyAsync(d + cs.size(), sn.data(), sn.size() * 4, hipMemcpyHostToDevice, ctx->stream);
  if (e == hipSuccess) {
    hipLaunchKernelGGL(soc::k_rope_f32, dim3(rows), dim3(256), 0, ctx->stream, x, y, d, d + cs.size(), heads, head_dim,
                       rotary_dim);
    e = hipGetLastError();
  }
  const hipError_t es = hipStreamSynchronize(ctx->stream);
  (void)hipFree(d);
  if (e != hipSuccess) return fail(SOC_ERR_HIP, std::string("RoPE: ") + hipGetErrorString(e));
  if (es != hipSuccess) return fail(SOC_ERR_HIP, std::string("RoPE: ") + hipGetErrorString(es));
  return SOC_OK;
  SOC_API_END
}

int soc_op_softmax(soc_ctx* ctx, const float* x, float* y, int32_t rows, int32_t n) {
  SOC_API_BEGIN
  if (ctx == nullptr) return fail(SOC_ERR_INVALID, "null context");
  if (rows <= 0 || n <= 0) return fail(SOC_ERR_INVALID, "Softmax params do not match tensor shape");
  const size_t bytes = static_cast<size_t>(rows) * n * 4;
  SOC_TRY(check_device_operand("Softmax input", x, bytes));
  SOC_TRY(check_device_operand("Softmax output", y, bytes));
  hipLaunchKernelGGL(soc::k_softmax_f32, dim3(rows), dim3(256), 0, ctx->stream, x, y, n);
  SOC_TRY(soc::launch_status("Softmax launch"));
  return soc::sync_status(ctx, "Softmax");
  SOC_API_END
}

int soc_op_embedding(soc_ctx* ctx, const int32_t* ids, const void* table, int32_t table_dtype, float* out,
                     int32_t tokens, int32_t hidden, int32_t vocab) {
  SOC_API_BEGIN
  if (ctx == nullptr) return fail(SOC_ERR_INVALID, "null context");
  if (table_dtype != SOC_DTYPE_F32 && table_dtype != SOC_DTYPE_F16)
    return fail(SOC_ERR_INVALID, "Embedding table must be float16 or float32");
  if (tokens <= 0 || hidden <= 0 || vocab <= 0) return fail(SOC_ERR_INVALID, "Embedding tensor shapes do not match params");
  SOC_TRY(check_device_operand("Embedding token ids", ids, static_cast<size_t>(tokens) * 4));
  SOC_TRY(check_device_operand("Embedding table", table,
                               static_cast<size_t>(vocab) * hidden * (table_dtype == SOC_DTYPE_F32 ? 4 : 2)));
  SOC_TRY(check_device_operand("Embedding output", out, static_cast<size_t>(tokens) * hidden * 4));
  if (table_dtype == SOC_DTYPE_F32)
    hipLaunchKernelGGL(soc::k_embedding<float>, dim3(tokens), dim3(256), 0, ctx->stream, ids,
                       static_cast<const float*>(table), out, hidden, vocab);
  else
    hipLaunchKernelGGL(soc::k_embedding<soc::f16>, dim3(tokens), dim3(256), 0, ctx->stream, ids,
                       static_cast<const soc::f16*>(table), out, hidden, vocab);
  SOC_TRY(soc::launch_status("Embedding launch"));
  return soc::sync_status(ctx, "Embedding");
  SOC_API_END
}

int soc_op_mul(soc_ctx* ctx, const float* a, const float* b, float* y, int32_t rows, int32_t n) {
  SOC_API_BEGIN
  if (ctx == nullptr) return fail(SOC_ERR_INVALID, "null context");
  if (rows <= 0 || n <= 0) return fail(SOC_ERR_INVALID, "ElementwiseMul params do not match tensor shape");
  const size_t count = static_cast<size_t>(rows) * n;
  SOC_TRY(check_device_operand("ElementwiseMul lhs", a, count * 4));
  SOC_TRY(check_device_operand("ElementwiseMul rhs", b, count * 4));
  SOC_TRY(check_device_operand("ElementwiseMul output", y, count * 4));
  const size_t blocks = std::min<size_t>((count + 255) / 256, 4096);
  hipLaunchKernelGGL(soc::k_mul_f32, dim3(static_cast<unsigned>(blocks)), dim3(256), 0, ctx->stream, a, b, y, count);
  SOC_TRY(soc::launch_status("ElementwiseMul launch"));
  return soc::sync_status(ctx, "ElementwiseMul");
  SOC_API_END
}
