// host_ops.cpp - the reference's op wrappers (include/soc/gpu/ops.h) on the C ABI's op kernels (soc_op_*): the
// tensor checks and messages of Mac/gpu/src/op/*.mm, then one kernel on the tensors' device memory.
#include <algorithm>

#include "soc/gpu/runtime.h"

namespace soc::gpu {

namespace {

bool Fail(std::string* error_message, const char* msg) {
  if (error_message != nullptr) *error_message = msg;
  return false;
}

bool Check(int rc, std::string* error_message) {
  if (rc == SOC_OK) return true;
  if (error_message != nullptr) *error_message = soc_last_error();
  return false;
}

bool IsF32(const DeviceTensor& t) { return t.GetDesc().GetDataType() == DataType::kFloat32; }

// The kernels read row-major tensors: a strided view (the KV cache's layer planes) is not one.
bool Dense(const DeviceTensor& t) { return t.GetDesc().IsContiguous(); }

const float* F(const DeviceTensor& t) { return static_cast<const float*>(t.data()); }
float* Fw(const DeviceTensor& t) { return static_cast<float*>(t.data()); }

}  // namespace

// matmul_op.mm:143-194: the reference's Metal launch shape for these dimensions (the same rules, kept for callers
// that read it; the HIP kernel has one shape).
MatMulExecutionPolicy MatMulOp::SelectPolicy(const MatMulParams& params, std::uint32_t row_count,
                                             std::uint32_t column_count, std::uint32_t inner_dim) {
  auto clamp_to = [](std::uint32_t want, std::uint32_t n) { return std::min(want, std::max<std::uint32_t>(1, n)); };
  MatMulExecutionPolicy p;
  if (params.decode_mode) {
    const std::uint32_t width = column_count <= 4 ? std::max<std::uint32_t>(1, column_count)
                                : (inner_dim >= 128 || column_count >= 16) ? clamp_to(16, column_count)
                                                                            : clamp_to(8, column_count);
    p.threadgroup_width = params.preferred_threadgroup_width != 0
                              ? clamp_to(params.preferred_threadgroup_width, column_count)
                              : width;
    p.threadgroup_height = 1;
    p.tile_columns = params.preferred_tile_columns != 0 ? params.preferred_tile_columns : p.threadgroup_width;
    p.tile_rows = 1;
    p.use_tiled_kernel = inner_dim >= 64 && column_count >= 64 && p.tile_columns <= 32;
    return p;
  }
  std::uint32_t width = 4, height = 2;
  if (column_count >= 16 || inner_dim >= 128) {
    width = row_count <= 8 ? 8 : 16;
    height = 4;
  } else if (column_count >= 8 || inner_dim >= 64) {
    width = 8;
    height = 4;
  }
  p.threadgroup_width = clamp_to(params.preferred_threadgroup_width != 0 ? params.preferred_threadgroup_width : width,
                                 column_count);
  p.threadgroup_height =
      clamp_to(params.preferred_threadgroup_height != 0 ? params.preferred_threadgroup_height : height, row_count);
  p.tile_columns = params.preferred_tile_columns != 0 ? params.preferred_tile_columns : p.threadgroup_width;
  p.tile_rows = params.preferred_tile_rows != 0 ? params.preferred_tile_rows : p.threadgroup_height;
  p.use_tiled_kernel =
      inner_dim >= 64 && column_count >= 64 && row_count >= 2 && p.tile_columns <= 32 && p.tile_rows <= 4;
  return p;
}

// matmul_op.mm:29-100 (ValidateMatMulTensors) and :196-262, then soc_op_matmul
bool MatMulOp::Run(const HipContext& context, PipelineCache* pipeline_cache, const DeviceTensor& lhs,
                   const DeviceTensor& rhs, const DeviceTensor* bias, const DeviceTensor* residual,
                   const DeviceTensor& output, const MatMulParams& params, BufferArena*, std::string* error_message) {
  if (pipeline_cache == nullptr) return Fail(error_message, "Pipeline cache must not be null");
  if (!lhs.IsValid() || !rhs.IsValid() || !output.IsValid())
    return Fail(error_message, "MatMul tensors must be valid device tensors");
  if (!IsF32(lhs) || !IsF32(rhs) || !IsF32(output) || (bias != nullptr && !IsF32(*bias)))
    return Fail(error_message, "MatMul baseline currently supports float32 tensors only");
  if (lhs.GetDesc().Rank() != 2 || rhs.GetDesc().Rank() != 2 || output.GetDesc().Rank() != 2)
    return Fail(error_message, "MatMul baseline expects rank-2 lhs, rhs, and output tensors");
  const auto& ls = lhs.GetDesc().GetShape();
  const auto& rs = rhs.GetDesc().GetShape();
  const auto& os = output.GetDesc().GetShape();
  const std::size_t inner = params.transpose_rhs ? rs[1] : rs[0];
  const std::size_t cols = params.transpose_rhs ? rs[0] : rs[1];
  if (ls[1] != inner) return Fail(error_message, "MatMul inner dimensions must match");
  if (os[0] != ls[0] || os[1] != cols) return Fail(error_message, "MatMul output shape must match lhs_rows x rhs_cols");
  if (bias != nullptr &&
      (!bias->IsValid() || bias->GetDesc().Rank() != 1 || bias->GetDesc().GetShape()[0] != cols))
    return Fail(error_message, "MatMul bias must be a valid rank-1 tensor matching output columns");
  if (residual != nullptr && (!residual->IsValid() || !IsF32(*residual) || residual->GetDesc().Rank() != 2 ||
                              residual->GetDesc().GetShape() != os))
    return Fail(error_message, "MatMul residual must be a valid rank-2 float32 tensor matching the output shape");
  const std::uint32_t rows = params.row_count == 0 ? static_cast<std::uint32_t>(ls[0]) : params.row_count;
  const std::uint32_t k = params.inner_dim == 0 ? static_cast<std::uint32_t>(inner) : params.inner_dim;
  const std::uint32_t n = params.column_count == 0 ? static_cast<std::uint32_t>(cols) : params.column_count;
  if (rows != ls[0] || k != inner || n != cols)
    return Fail(error_message, "Explicit MatMul params must match tensor shapes");
  if (params.use_bias != (bias != nullptr))
    return Fail(error_message, "MatMul params.use_bias must match whether a bias tensor is provided");
  if (params.add_residual != (residual != nullptr))
    return Fail(error_message, "MatMul params.add_residual must match whether a residual tensor is provided");
  if (params.decode_mode && rows != 1)
    return Fail(error_message, "Decode-specialized MatMul currently requires row_count == 1");
  if (!Dense(lhs) || !Dense(rhs) || !Dense(output) || (bias != nullptr && !Dense(*bias)) ||
      (residual != nullptr && !Dense(*residual)))
    return Fail(error_message, "MatMul tensors must be contiguous");
  return Check(soc_op_matmul(context.handle(), F(lhs), F(rhs), bias != nullptr ? F(*bias) : nullptr,
                             residual != nullptr ? F(*residual) : nullptr, Fw(output), static_cast<int32_t>(rows),
                             static_cast<int32_t>(k), static_cast<int32_t>(n), params.transpose_rhs ? 1 : 0,
                             params.enable_silu ? 1 : 0),
               error_message);
}

// linear_op.mm: the activation and residual flags of LinearParams on MatMulOp
bool LinearOp::Run(const HipContext& context, PipelineCache* pipeline_cache, const DeviceTensor& input,
                   const DeviceTensor& weight, const DeviceTensor* bias, const DeviceTensor* residual,
                   const DeviceTensor& output, const LinearParams& params, BufferArena* temporary_arena,
                   std::string* error_message) {
  MatMulParams fused = params.matmul;
  fused.enable_silu = params.activation == LinearActivation::kSiLU;
  fused.add_residual = params.add_residual;
  return MatMulOp::Run(context, pipeline_cache, input, weight, bias, residual, output, fused, temporary_arena,
                       error_message);
}

// rms_norm_op.mm:20-135
bool RmsNormOp::Run(const HipContext& context, PipelineCache* pipeline_cache, const DeviceTensor& input,
                    const DeviceTensor& weight, const DeviceTensor& output, const RmsNormParams& params, BufferArena*,
                    std::string* error_message) {
  if (pipeline_cache == nullptr) return Fail(error_message, "Pipeline cache must not be null");
  if (!input.IsValid() || !weight.IsValid() || !output.IsValid())
    return Fail(error_message, "RMSNorm tensors must be valid device tensors");
  if (!IsF32(input) || !IsF32(weight) || !IsF32(output))
    return Fail(error_message, "RMSNorm baseline currently supports float32 tensors only");
  if (input.GetDesc().Rank() != 2 || output.GetDesc().Rank() != 2 || weight.GetDesc().Rank() != 1)
    return Fail(error_message, "RMSNorm baseline expects input/output rank 2 and weight rank 1");
  const auto& is = input.GetDesc().GetShape();
  if (is != output.GetDesc().GetShape()) return Fail(error_message, "RMSNorm input and output shapes must match");
  if (weight.GetDesc().GetShape()[0] != is[1]) return Fail(error_message, "RMSNorm weight size must match hidden size");
  const std::uint32_t row_size = params.row_size == 0 ? static_cast<std::uint32_t>(is[1]) : params.row_size;
  const std::uint32_t row_count = params.row_count == 0 ? static_cast<std::uint32_t>(is[0]) : params.row_count;
  if (row_size != is[1] || row_count != is[0])
    return Fail(error_message, "Explicit RMSNorm params must match tensor shapes");
  if (!Dense(input) || !Dense(weight) || !Dense(output)) return Fail(error_message, "RMSNorm tensors must be contiguous");
  return Check(soc_op_rmsnorm(context.handle(), F(input), F(weight), Fw(output), static_cast<int32_t>(row_count),
                              static_cast<int32_t>(row_size), params.epsilon),
               error_message);
}

// rope_op.mm:54-100
bool RopeOp::Run(const HipContext& context, PipelineCache* pipeline_cache, const DeviceTensor& input,
                 const DeviceTensor& output, const RopeParams& params, BufferArena*, std::string* error_message) {
  if (pipeline_cache == nullptr) return Fail(error_message, "Pipeline cache must not be null");
  if (!input.IsValid() || !output.IsValid()) return Fail(error_message, "RoPE tensors must be valid");
  if (!IsF32(input) || !IsF32(output)) return Fail(error_message, "RoPE baseline currently supports float32 only");
  if (input.GetDesc().Rank() != 2 || output.GetDesc().Rank() != 2 ||
      input.GetDesc().GetShape() != output.GetDesc().GetShape())
    return Fail(error_message, "RoPE expects matching rank-2 input/output tensors");
  const auto& is = input.GetDesc().GetShape();
  const std::uint32_t rows = params.row_count == 0 ? static_cast<std::uint32_t>(is[0]) : params.row_count;
  const std::uint32_t rotary = params.rotary_dim == 0 ? params.head_dim : params.rotary_dim;
  if (rows != is[0] || params.head_count == 0 || params.head_dim == 0 ||
      static_cast<std::size_t>(params.head_count) * params.head_dim != is[1] || rotary == 0 ||
      rotary > params.head_dim || rotary % 2 != 0)
    return Fail(error_message, "RoPE params do not match tensor shapes");
  if (!Dense(input) || !Dense(output)) return Fail(error_message, "RoPE tensors must be contiguous");
  return Check(soc_op_rope(context.handle(), F(input), Fw(output), static_cast<int32_t>(rows),
                           static_cast<int32_t>(params.head_count), static_cast<int32_t>(params.head_dim),
                           static_cast<int32_t>(rotary), static_cast<int32_t>(params.position_offset),
                           static_cast<double>(params.rope_theta)),
               error_message);
}

// softmax_op.mm:54-85
bool SoftmaxOp::Run(const HipContext& context, PipelineCache* pipeline_cache, const DeviceTensor& input,
                    const DeviceTensor& output, const SoftmaxParams& params, BufferArena*, std::string* error_message) {
  if (pipeline_cache == nullptr) return Fail(error_message, "Pipeline cache must not be null");
  if (!input.IsValid() || !output.IsValid()) return Fail(error_message, "Softmax tensors must be valid");
  if (!IsF32(input) || !IsF32(output) || input.GetDesc().Rank() != 2 || output.GetDesc().Rank() != 2 ||
      input.GetDesc().GetShape() != output.GetDesc().GetShape())
    return Fail(error_message, "Softmax expects matching rank-2 float32 tensors");
  const auto& is = input.GetDesc().GetShape();
  const std::uint32_t rows = params.row_count == 0 ? static_cast<std::uint32_t>(is[0]) : params.row_count;
  const std::uint32_t size = params.row_size == 0 ? static_cast<std::uint32_t>(is[1]) : params.row_size;
  if (rows != is[0] || size != is[1]) return Fail(error_message, "Softmax params do not match tensor shape");
  if (!Dense(input) || !Dense(output)) return Fail(error_message, "Softmax tensors must be contiguous");
  return Check(soc_op_softmax(context.handle(), F(input), Fw(output), static_cast<int32_t>(rows),
                              static_cast<int32_t>(size)),
               error_message);
}

// embedding_op.mm:54-102
bool EmbeddingOp::Run(const HipContext& context, PipelineCache* pipeline_cache, const DeviceTensor& token_ids,
                      const DeviceTensor& embedding_table, const DeviceTensor& output, const EmbeddingParams& params,
                      BufferArena*, std::string* error_message) {
  if (pipeline_cache == nullptr) return Fail(error_message, "Pipeline cache must not be null");
  if (!token_ids.IsValid() || !embedding_table.IsValid() || !output.IsValid())
    return Fail(error_message, "Embedding tensors must be valid");
  if (token_ids.GetDesc().GetDataType() != DataType::kInt32 || !IsF32(output))
    return Fail(error_message, "Embedding expects int32 token ids and float32 output");
  const DataType tdt = embedding_table.GetDesc().GetDataType();
  if (tdt != DataType::kFloat32 && tdt != DataType::kFloat16)
    return Fail(error_message, "Embedding table must be float16 or float32");
  if (token_ids.GetDesc().Rank() != 1 || embedding_table.GetDesc().Rank() != 2 || output.GetDesc().Rank() != 2)
    return Fail(error_message, "Embedding expects rank-1 ids, rank-2 table, and rank-2 output");
  const auto& ts = embedding_table.GetDesc().GetShape();
  const auto& os = output.GetDesc().GetShape();
  const std::uint32_t tokens =
      params.token_count == 0 ? static_cast<std::uint32_t>(token_ids.GetDesc().GetShape()[0]) : params.token_count;
  const std::uint32_t vocab = params.vocab_size == 0 ? static_cast<std::uint32_t>(ts[0]) : params.vocab_size;
  const std::uint32_t hidden = params.hidden_size == 0 ? static_cast<std::uint32_t>(ts[1]) : params.hidden_size;
  if (os[0] != tokens || os[1] != hidden || token_ids.GetDesc().GetShape()[0] != tokens || ts[0] != vocab ||
      ts[1] != hidden)
    return Fail(error_message, "Embedding tensor shapes do not match params");
  if (!Dense(token_ids) || !Dense(embedding_table) || !Dense(output))
    return Fail(error_message, "Embedding tensors must be contiguous");
  return Check(soc_op_embedding(context.handle(), static_cast<const int32_t*>(token_ids.data()), embedding_table.data(),
                                tdt == DataType::kFloat32 ? SOC_DTYPE_F32 : SOC_DTYPE_F16, Fw(output),
                                static_cast<int32_t>(tokens), static_cast<int32_t>(hidden),
                                static_cast<int32_t>(vocab)),
               error_message);
}

// elementwise_mul_op.mm:54-96
bool ElementwiseMulOp::Run(const HipContext& context, PipelineCache* pipeline_cache, const DeviceTensor& lhs,
                           const DeviceTensor& rhs, const DeviceTensor& output, const ElementwiseMulParams& params,
                           BufferArena*, std::string* error_message) {
  if (pipeline_cache == nullptr) return Fail(error_message, "Pipeline cache must not be null");
  if (!lhs.IsValid() || !rhs.IsValid() || !output.IsValid())
    return Fail(error_message, "ElementwiseMul tensors must be valid");
  const auto& ls = lhs.GetDesc().GetShape();
  if (!IsF32(lhs) || !IsF32(rhs) || !IsF32(output) || lhs.GetDesc().Rank() != 2 || rhs.GetDesc().Rank() != 2 ||
      output.GetDesc().Rank() != 2 || ls != rhs.GetDesc().GetShape() || ls != output.GetDesc().GetShape())
    return Fail(error_message, "ElementwiseMul expects matching rank-2 float32 tensors");
  const std::uint32_t rows = params.row_count == 0 ? static_cast<std::uint32_t>(ls[0]) : params.row_count;
  const std::uint32_t size = params.row_size == 0 ? static_cast<std::uint32_t>(ls[1]) : params.row_size;
  if (rows != ls[0] || size != ls[1]) return Fail(error_message, "ElementwiseMul params do not match tensor shape");
  if (!Dense(lhs) || !Dense(rhs) || !Dense(output)) return Fail(error_message, "ElementwiseMul tensors must be contiguous");
  return Check(soc_op_mul(context.handle(), F(lhs), F(rhs), Fw(output), static_cast<int32_t>(rows),
                          static_cast<int32_t>(size)),
               error_message);
}

}  // namespace soc::gpu
