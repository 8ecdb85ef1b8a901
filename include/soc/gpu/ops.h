// ops.h - the reference GPU runtime's op wrappers (Mac/gpu/include/op/*.h: the static Run of MatMulOp, LinearOp,
// RmsNormOp, RopeOp, SoftmaxOp, EmbeddingOp, ElementwiseMulOp) over HIP device tensors. Same parameter structs, the
// same validation and messages (Mac/gpu/src/op/*.mm), fp32 arithmetic as the reference's kernels
// (gpu_kernels.metal:82-289); each runs one gfx950 kernel through the C ABI (soc_op_*) and returns when its output is
// written. Included by soc/gpu/runtime.h.
#pragma once

#include <cstdint>
#include <string>

namespace soc::gpu {

class HipContext;
class PipelineCache;
class DeviceTensor;
class BufferArena;

// matmul_op.h:15-37
struct MatMulParams {
  std::uint32_t row_count = 0;
  std::uint32_t inner_dim = 0;
  std::uint32_t column_count = 0;
  bool use_bias = false;
  bool decode_mode = false;
  bool transpose_rhs = false;
  bool enable_silu = false;
  bool add_residual = false;
  std::uint32_t preferred_threadgroup_width = 0;
  std::uint32_t preferred_threadgroup_height = 0;
  std::uint32_t preferred_tile_columns = 0;
  std::uint32_t preferred_tile_rows = 0;
};

// matmul_op.h:30-36: the reference's Metal launch shape. Kept for callers that inspect it; the HIP kernel tiles its
// output in 64 x 64 blocks whatever the policy says.
struct MatMulExecutionPolicy {
  std::uint32_t threadgroup_width = 1;
  std::uint32_t threadgroup_height = 1;
  std::uint32_t tile_columns = 1;
  std::uint32_t tile_rows = 1;
  bool use_tiled_kernel = false;
};

class MatMulOp {
 public:
  // matmul_op.mm:143-194, the same rules
  static MatMulExecutionPolicy SelectPolicy(const MatMulParams& params, std::uint32_t row_count,
                                            std::uint32_t column_count, std::uint32_t inner_dim);
  // output = lhs [rows][inner] . rhs ([inner][cols], or [cols][inner] with transpose_rhs) (+ bias [cols])
  // (+ residual [rows][cols]), then SiLU with enable_silu; float32 tensors (matmul_op.mm:196-330)
  static bool Run(const HipContext& context, PipelineCache* pipeline_cache, const DeviceTensor& lhs,
                  const DeviceTensor& rhs, const DeviceTensor* bias, const DeviceTensor* residual,
                  const DeviceTensor& output, const MatMulParams& params, BufferArena* temporary_arena,
                  std::string* error_message);
};

enum class LinearActivation { kNone, kSiLU };  // linear_op.h:14-17

struct LinearParams {  // linear_op.h:19-23
  MatMulParams matmul;
  LinearActivation activation = LinearActivation::kNone;
  bool add_residual = false;
};

class LinearOp {
 public:
  // linear_op.mm: MatMulOp with enable_silu from the activation and add_residual from the params
  static bool Run(const HipContext& context, PipelineCache* pipeline_cache, const DeviceTensor& input,
                  const DeviceTensor& weight, const DeviceTensor* bias, const DeviceTensor* residual,
                  const DeviceTensor& output, const LinearParams& params, BufferArena* temporary_arena,
                  std::string* error_message);
};

struct RmsNormParams {  // rms_norm_op.h:12-16
  float epsilon = 1.0e-5f;
  std::uint32_t row_size = 0;
  std::uint32_t row_count = 0;
};

class RmsNormOp {
 public:
  static bool Run(const HipContext& context, PipelineCache* pipeline_cache, const DeviceTensor& input,
                  const DeviceTensor& weight, const DeviceTensor& output, const RmsNormParams& params,
                  BufferArena* temporary_arena, std::string* error_message);
};

struct RopeParams {  // rope_op.h:14-21
  std::uint32_t row_count = 0;
  std::uint32_t head_count = 0;
  std::uint32_t head_dim = 0;
  std::uint32_t rotary_dim = 0;
  std::uint32_t position_offset = 0;
  float rope_theta = 1000000.0f;
};

class RopeOp {
 public:
  static bool Run(const HipContext& context, PipelineCache* pipeline_cache, const DeviceTensor& input,
                  const DeviceTensor& output, const RopeParams& params, BufferArena* temporary_arena,
                  std::string* error_message);
};

struct SoftmaxParams {  // softmax_op.h:14-17
  std::uint32_t row_count = 0;
  std::uint32_t row_size = 0;
};

class SoftmaxOp {
 public:
  static bool Run(const HipContext& context, PipelineCache* pipeline_cache, const DeviceTensor& input,
                  const DeviceTensor& output, const SoftmaxParams& params, BufferArena* temporary_arena,
                  std::string* error_message);
};

struct EmbeddingParams {  // embedding_op.h:14-18
  std::uint32_t token_count = 0;
  std::uint32_t hidden_size = 0;
  std::uint32_t vocab_size = 0;
};

class EmbeddingOp {
 public:
  static bool Run(const HipContext& context, PipelineCache* pipeline_cache, const DeviceTensor& token_ids,
                  const DeviceTensor& embedding_table, const DeviceTensor& output, const EmbeddingParams& params,
                  BufferArena* temporary_arena, std::string* error_message);
};

struct ElementwiseMulParams {  // elementwise_mul_op.h:14-17
  std::uint32_t row_count = 0;
  std::uint32_t row_size = 0;
};

class ElementwiseMulOp {
 public:
  static bool Run(const HipContext& context, PipelineCache* pipeline_cache, const DeviceTensor& lhs,
                  const DeviceTensor& rhs, const DeviceTensor& output, const ElementwiseMulParams& params,
                  BufferArena* temporary_arena, std::string* error_message);
};

}  // namespace soc::gpu
