// Error reporting and version of the C ABI (include/minillm_hip.h).
#include "common.h"

namespace mllm {

static thread_local std::string g_last_error;

void set_error(const std::string& msg) { g_last_error = msg; }

int fail(int code, const std::string& msg) {
  g_last_error = msg;
  return code;
}

int check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(MLLM_ERR_HIP, std::string(what) + ": " + hipGetErrorString(e));
  return MLLM_OK;
}

}  // namespace mllm

extern "C" int mllm_abi_version(void) { return MLLM_ABI_VERSION; }

extern "C" const char* mllm_last_error(void) { return mllm::g_last_error.c_str(); }
