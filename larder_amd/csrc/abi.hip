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

struct TimelineLaunch {
  int kernel, n_wg;
  long long row0;
};
struct Timeline {
  unsigned long long *buf = nullptr;
  long long rows = 0, used = 0;
  std::vector<TimelineLaunch> launches;
};
static thread_local Timeline g_tl;
constexpr int kTimelineMaxLaunches = 1 << 14;

unsigned long long *timeline_next(int kernel, int n_wg) {
  Timeline &t = g_tl;
  if (!t.buf || t.used + n_wg > t.rows || int(t.launches.size()) >= kTimelineMaxLaunches) return nullptr;
  unsigned long long *p = t.buf + size_t(t.used) * 8;
  t.launches.push_back({kernel, n_wg, t.used});
  t.used += n_wg;
  return p;
}

}  // namespace lmoe

extern "C" const char *lmoe_error(void) { return lmoe::g_error.c_str(); }

extern "C" int lmoe_timeline_arm(unsigned long long *buf, long long rows) {
  using namespace lmoe;
  LMOE_REQUIRE(buf && rows > 0, LMOE_EINVAL, "lmoe_timeline_arm: null buffer or no rows");
  LMOE_REQUIRE(aligned16(buf), LMOE_EALIGN, "lmoe_timeline_arm: buffer must be 16-byte aligned");
  g_tl.buf = buf;
  g_tl.rows = rows;
  g_tl.used = 0;
  g_tl.launches.clear();
  return 0;
}

extern "C" int lmoe_timeline_disarm(int *count) {
  using namespace lmoe;
  if (count) *count = int(g_tl.launches.size());
  g_tl.buf = nullptr;
  return 0;
}

extern "C" int lmoe_timeline_launch(int i, int *kernel, long long *row0, int *n_wg) {
  using namespace lmoe;
  LMOE_REQUIRE(i >= 0 && i < int(g_tl.launches.size()), LMOE_EINVAL, "lmoe_timeline_launch: no launch %d", i);
  const TimelineLaunch &l = g_tl.launches[i];
  if (kernel) *kernel = l.kernel;
  if (row0) *row0 = l.row0;
  if (n_wg) *n_wg = l.n_wg;
  return 0;
}

extern "C" int lmoe_timeline_clock_khz(int *khz) {
  using namespace lmoe;
  LMOE_REQUIRE(khz, LMOE_EINVAL, "lmoe_timeline_clock_khz: null pointer");
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e == hipSuccess) e = hipDeviceGetAttribute(khz, hipDeviceAttributeWallClockRate, dev);
  return e == hipSuccess ? 0 : hip_fail(e, "lmoe_timeline_clock_khz");
}

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
