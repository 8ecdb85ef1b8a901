// capi_internal.h - pieces shared by the translation units that implement the C ABI: the device context, the guard
// that turns C++ exceptions into status codes, and the check of caller pointers before a kernel reads them.
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>
#include <new>
#include <stdexcept>

#include "soc_hip.h"
#include "status.h"

#define SOC_API_BEGIN try {
#define SOC_API_END                                                         \
  }                                                                         \
  catch (const std::bad_alloc&) {                                           \
    return soc::fail(SOC_ERR_NOMEM, "host allocation failed");              \
  }                                                                         \
  catch (const std::exception& e) {                                         \
    return soc::fail(SOC_ERR_INVALID, e.what());                            \
  }

struct soc_ctx {
  int device = 0;
  int num_cus = 0;
  hipStream_t stream = nullptr;
  hipEvent_t ev0 = nullptr, ev1 = nullptr;
  bool timing = false;          // between soc_ctx_timer_start and _stop
  bool stop_recorded = false;   // a forward recorded ev1 before its final synchronisation
  uint32_t* scratch = nullptr;  // device address of this device's copy of `scratch` (soc_decode_steps_noalloc)
  void* sample_ws = nullptr;    // soc_sample_topk: candidate search workspace and its output block
  size_t sample_ws_bytes = 0;
  int* sample_out = nullptr;
  int* sample_host = nullptr;   // pinned host copy of the output block (hipHostMalloc)
  // pinned host words a decode step's readback kernel writes (next token, wait error, token id error), with the
  // address kernels use for them
  int32_t* readback = nullptr;
  int32_t* readback_dev = nullptr;
  // op-level attention (soc_attention_decode): split-key partials and arrival counters, grown on demand
  float* op_part = nullptr;
  size_t op_part_floats = 0;
  int* op_counters = nullptr;
  size_t op_counter_ints = 0;
  // soc_forward with token ids in device memory: set by the staging kernel when an id lies outside [0, vocab)
  int* id_err = nullptr;
};


namespace soc {

// Where `bytes` bytes at p lie. kDeviceRange: in memory a kernel may read (a hipMalloc'd or managed allocation that
// holds the whole range, or pinned host memory mapped for the device). kPageable: host memory the device cannot read
// (a kernel reading it faults on devices without XNACK). kOutside: device memory whose allocation ends before
// p + bytes.
enum class MemRange { kDeviceRange, kPageable, kOutside };
MemRange classify_range(const void* p, size_t bytes);

// SOC_OK when every (pointer, bytes) of a caller's device operands lies inside one device allocation (null pointers
// with 0 bytes pass); otherwise SOC_ERR_INVALID naming the operand. Called before any kernel reads caller memory.
int check_device_operand(const char* what, const void* p, size_t bytes);

}  // namespace soc
