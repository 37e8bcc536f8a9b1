// Thread-local last-error string and status helpers for the C ABI.
#include "common.hpp"

#include <cstdio>

namespace xmh3 {

static thread_local std::string g_last_error;

void set_last_error(const std::string& msg) { g_last_error = msg; }

int fail(int code, const std::string& msg) {
  g_last_error = msg;
  return code;
}

int check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    return fail(XMH3_EHIP, std::string(what) + ": " + hipGetErrorString(e));
  }
  return XMH3_OK;
}

}  // namespace xmh3

extern "C" const char* xmh3_last_error(void) { return xmh3::g_last_error.c_str(); }

extern "C" int xmh3_abi_version(void) { return 1; }
