// Error reporting and version of the C ABI (include/cohere_hip.h).
#include <hip/hip_runtime.h>

#include <string>

#include "cohere_hip.h"

namespace cohere {

namespace {
thread_local std::string g_error;
}

void set_error(const std::string& msg) { g_error = msg; }
void clear_error() { g_error.clear(); }

int check_launch(const char* what) {
  const hipError_t e = hipGetLastError();
  if (e == hipSuccess) return 0;
  g_error = std::string(what) + ": launch failed: " + hipGetErrorString(e);
  return 2;
}

}  // namespace cohere

extern "C" const char* cohere_last_error(void) { return cohere::g_error.c_str(); }

extern "C" const char* cohere_version(void) { return "cohere-inference-amd 0.1 (gfx950)"; }
