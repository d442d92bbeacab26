// capi.hip — error state and version of libhelm_mi355x.so.
#include <string>

#include "helm_common.h"

namespace helm {

static thread_local std::string g_last_error;

void set_error(const std::string& msg) { g_last_error = msg; }

int fail(int code, const std::string& msg) {
  g_last_error = msg;
  return code;
}

int hip_fail(hipError_t e, const char* what) {
  g_last_error = std::string(what) + ": " + hipGetErrorName(e) + " (" + hipGetErrorString(e) + ")";
  return HELM_ERR_HIP;
}

}  // namespace helm

extern "C" const char* helm_last_error(void) { return helm::g_last_error.c_str(); }

extern "C" const char* helm_version(void) { return "helm_mi355x 0.1 gfx950"; }
