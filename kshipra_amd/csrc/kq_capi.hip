// C-ABI support: version, per-thread error message, launch checking.
#include <string>

#include "kq_common.hpp"

namespace {
thread_local std::string g_last_error;
}

int kq_set_error(int status, const std::string& msg) {
  g_last_error = msg;
  return status;
}

int kq_check_launch(const char* what) {
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess)
    return kq_set_error(KQ_ERR_HIP, std::string(what) + ": " + hipGetErrorString(e));
  return KQ_OK;
}

extern "C" int kq_version(void) { return 103; }

extern "C" const char* kq_last_error(void) { return g_last_error.c_str(); }
