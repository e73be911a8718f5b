// Error plumbing shared by every entry point: a thread-local reason string and the return-code convention
// (0 ok, > 0 hipError_t, < 0 LMOE_E* refusal), as the reference's native C ABI does with mpc_error()
// (native/moe_pipe_cuda.py:95-97).
#include <cstdarg>
#include <cstdio>
#include <vector>

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

struct Profile {
  std::vector<hipEvent_t> start, stop;
  int used = 0, armed = 0;
};
static thread_local Profile g_prof;

bool profile_next(hipEvent_t *a, hipEvent_t *b) {
  Profile &p = g_prof;
  if (!p.armed || p.used >= int(p.start.size())) return false;
  *a = p.start[p.used];
  *b = p.stop[p.used];
  ++p.used;
  return true;
}

}  // namespace lmoe

extern "C" const char *lmoe_error(void) { return lmoe::g_error.c_str(); }

extern "C" int lmoe_profile_arm(int max_launches) {
  using namespace lmoe;
  LMOE_REQUIRE(max_launches > 0 && max_launches <= (1 << 16), LMOE_EINVAL, "lmoe_profile_arm: bad count %d",
               max_launches);
  Profile &p = g_prof;
  while (int(p.start.size()) < max_launches) {
    hipEvent_t a, b;
    hipError_t e = hipEventCreate(&a);
    if (e == hipSuccess) e = hipEventCreate(&b);
    if (e != hipSuccess) return hip_fail(e, "lmoe_profile_arm");
    p.start.push_back(a);
    p.stop.push_back(b);
  }
  p.used = 0;
  p.armed = 1;
  return 0;
}

extern "C" int lmoe_profile_read(float *ms, int cap, int *count) {
  using namespace lmoe;
  Profile &p = g_prof;
  LMOE_REQUIRE(cap >= 0 && (ms || cap == 0), LMOE_EINVAL, "lmoe_profile_read: bad buffer");
  for (int i = 0; i < p.used; ++i) {
    hipError_t e = hipEventSynchronize(p.stop[i]);
    float t = 0.0f;
    if (e == hipSuccess) e = hipEventElapsedTime(&t, p.start[i], p.stop[i]);
    if (e != hipSuccess) return hip_fail(e, "lmoe_profile_read");
    if (i < cap) ms[i] = t;
  }
  if (count) *count = p.used;
  p.armed = 0;
  p.used = 0;
  return 0;
}

extern "C" int lmoe_abi_version(void) { return 1; }
