// Error plumbing shared by every entry point: a thread-local reason string and the return-code convention
// (0 ok, > 0 hipError_t, < 0 LMOE_E* refusal), as the reference's native C ABI does with mpc_error()
// (native/moe_pipe_cuda.py:95-97).
#include <cstdarg>
#include <cstdio>

#include "lmoe_common.h"

namespace lmoe {

static thread_local std::string g_error;

void set_error(const char *fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  g_error = buf;
}

int fail(int code, const char *fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  g_error = buf;
  return code;
}

int hip_fail(hipError_t e, const char *what) {
  set_error("%s: %s", what, hipGetErrorString(e));
  return int(e) > 0 ? int(e) : 1;
}

}  // namespace lmoe

extern "C" const char *lmoe_error(void) { return lmoe::g_error.c_str(); }

extern "C" int lmoe_abi_version(void) { return 1; }
