// Boundary bookkeeping: thread-local last error and launch checking.
// Mirrors the reference's int32 status + thread-local message convention
// (native/src/inferfabric_acl.cpp:46-58).
#include "ifattn_internal.h"

#include <string>

namespace ifattn {
namespace {
thread_local std::string g_last_error;
}
int32_t fail(int32_t code, const char *message) {
  g_last_error = message ? message : "";
  return code;
}
int32_t fail(int32_t code, const char *what, const char *message) {
  g_last_error = std::string(what ? what : "") + ": " + (message ? message : "");
  return code;
}
int32_t launch_status(const char *what) {
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    g_last_error = std::string(what) + ": " + hipGetErrorString(e);
    return IFATTN_ELAUNCH;
  }
  return IFATTN_OK;
}
}  // namespace ifattn

extern "C" int32_t ifattn_abi_version(void) { return IFATTN_ABI_VERSION; }
extern "C" const char *ifattn_last_error(void) { return ifattn::g_last_error.c_str(); }
