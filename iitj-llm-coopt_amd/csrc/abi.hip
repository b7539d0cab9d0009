// Error plumbing and runtime queries of the C ABI (include/coopt_amd.h).
#include "common.h"

namespace coopt {

static thread_local std::string g_last_error;

void set_error(const std::string& msg) { g_last_error = msg; }
void clear_error() { g_last_error.clear(); }

int check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    set_error(std::string(what) + ": " + hipGetErrorString(e));
    return COOPT_EHIP;
  }
  return COOPT_OK;
}

}  // namespace coopt

extern "C" const char* coopt_last_error(void) { return coopt::g_last_error.c_str(); }

extern "C" int coopt_hip_runtime_version(int* version) {
  COOPT_REQUIRE(version != nullptr, "null version pointer");
  hipError_t e = hipRuntimeGetVersion(version);
  if (e != hipSuccess) {
    coopt::set_error(std::string("hipRuntimeGetVersion: ") + hipGetErrorString(e));
    return COOPT_EHIP;
  }
  return COOPT_OK;
}
