// Error plumbing and version query of the C ABI.
#include "common.h"

namespace hydra {

static thread_local std::string g_last_error;

void set_error(const std::string& msg) { g_last_error = msg; }

int fail(int code, const std::string& msg) {
  g_last_error = msg;
  return code;
}

int check_launch(const char* what) {
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    return fail(HYDRA_ERR_LAUNCH,
                std::string(what) + ": " + hipGetErrorString(e));
  }
  return HYDRA_OK;
}

bool aligned16(const void* p) {
  return (reinterpret_cast<uintptr_t>(p) & 15u) == 0;
}

int dtype_size(int dtype) {
  switch (dtype) {
    case HYDRA_F32: return 4;
    case HYDRA_BF16: return 2;
    case HYDRA_F16: return 2;
    default: return 0;
  }
}

}  // namespace hydra

extern "C" const char* hydra_last_error(void) {
  return hydra::g_last_error.c_str();
}

extern "C" int hydra_abi_version(void) { return 100; }
