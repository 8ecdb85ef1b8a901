// status.cpp - the calling thread's last error message (soc::fail, soc::clear_error, soc_last_error). Host only.
#include <string>

#include "soc_hip.h"
#include "status.h"

namespace soc {
namespace {
thread_local std::string g_last_error;
}  // namespace

int fail(int code, const std::string& msg) {
  g_last_error = msg;
  return code;
}

void clear_error() { g_last_error.clear(); }

}  // namespace soc

extern "C" const char* soc_last_error(void) { return soc::g_last_error.c_str(); }
