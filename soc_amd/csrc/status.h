// status.h - status codes and the thread-local error message behind soc_last_error().
#pragma once

#include <string>

#include "soc_hip.h"

namespace soc {

// Records `msg` as the calling thread's last error and returns `code`.
int fail(int code, const std::string& msg);
// Clears the calling thread's last error.
void clear_error();

}  // namespace soc

#define SOC_HIP_TRY(expr)                                                                                  \
  do {                                                                                                     \
    hipError_t soc_e_ = (expr);                                                                            \
    if (soc_e_ != hipSuccess)                                                                              \
      return ::soc::fail(SOC_ERR_HIP, std::string(#expr) + ": " + hipGetErrorString(soc_e_));              \
  } while (0)

#define SOC_TRY(expr)            \
  do {                           \
    int soc_rc_ = (expr);        \
    if (soc_rc_ != SOC_OK)       \
      return soc_rc_;            \
  } while (0)
