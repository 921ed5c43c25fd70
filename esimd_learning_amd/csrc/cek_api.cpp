// cek_api.cpp -- status strings, version and HIP error recording for the C ABI.
#include <hip/hip_runtime.h>

#include <cstdio>

#include "cek.h"

namespace cek {

static thread_local char g_last_hip_error[256] = "";

int record_hip_error(hipError_t e) {
  std::snprintf(g_last_hip_error, sizeof(g_last_hip_error), "%s: %s", hipGetErrorName(e), hipGetErrorString(e));
  return CEK_ERR_HIP;
}

}  // namespace cek

extern "C" const char* cek_error_string(int status) {
  switch (status) {
    case CEK_OK: return "ok";
    case CEK_ERR_INVALID: return "invalid argument (size, pointer, alignment or enum value)";
    case CEK_ERR_UNSUPPORTED: return "unsupported configuration";
    case CEK_ERR_HIP: return "HIP runtime error (see cek_last_hip_error)";
    case CEK_ERR_SCRATCH: return "request needs more than the library's static scratch buffer holds";
    default: return "unknown status";
  }
}

extern "C" const char* cek_last_hip_error(void) { return cek::g_last_hip_error; }

extern "C" int cek_version(void) { return 100; /* 0.1.0 */ }
