// Library identity and thread-local error state.
#include "mxq_common.h"

namespace mxq {

static thread_local std::string g_last_error;

void set_error(const std::string& msg) { g_last_error = msg; }

int invalid(const std::string& msg) {
  g_last_error = msg;
  return MXQ_EINVAL;
}

int check_launch(const char* what) {
  hipError_t err = hipGetLastError();
  if (err != hipSuccess) {
    g_last_error = std::string(what) + ": " + hipGetErrorString(err);
    return MXQ_EHIP;
  }
  return MXQ_OK;
}

}  // namespace mxq

extern "C" const char* mxq_last_error(void) { return mxq::g_last_error.c_str(); }

extern "C" int mxq_version(void) { return 1; }
