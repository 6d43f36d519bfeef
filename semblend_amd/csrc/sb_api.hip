// Library-wide exports: version string and per-thread error reporting.
#include "sb_common.h"

#include <atomic>
#include <cstring>
#include <mutex>
#include <vector>

namespace sb {

namespace {
thread_local std::string g_last_error;
}

void set_error(const std::string& msg) { g_last_error = msg; }

void clear_error() { g_last_error.clear(); }

int fail(const char* fn, const std::string& msg) {
  g_last_error = std::string(fn) + ": " + msg;
  return SB_ERR_INVALID_ARGUMENT;
}

int check_launch(const char* fn) {
  const hipError_t e = hipGetLastError();
  if (e == hipSuccess) return SB_OK;
  g_last_error = std::string(fn) + ": kernel launch failed: " + hipGetErrorString(e);
  return static_cast<int>(e);
}

// ---------------------------------------------------------------------------------------
// Kernel timing log. Events are recycled through a pool; records hold (name, start, stop).
// ---------------------------------------------------------------------------------------
namespace {

constexpr size_t kMaxTimedLaunches = 65536;

struct TimedLaunch {
  const char* name;
  hipEvent_t start;
  hipEvent_t stop;
};

std::atomic<bool> g_timing{false};
std::mutex g_timing_mu;
std::vector<TimedLaunch> g_log;
std::vector<hipEvent_t> g_event_pool;

hipEvent_t take_event() {
  if (!g_event_pool.empty()) {
    hipEvent_t e = g_event_pool.back();
    g_event_pool.pop_back();
    return e;
  }
  hipEvent_t e = nullptr;
  if (hipEventCreate(&e) != hipSuccess) return nullptr;
  return e;
}

}  // namespace

KernelTimer::KernelTimer(const char* name) {
  if (!g_timing.load(std::memory_order_relaxed)) return;
  std::lock_guard<std::mutex> lock(g_timing_mu);
  if (g_log.size() >= kMaxTimedLaunches) return;
  hipEvent_t start = take_event();
  hipEvent_t stop = take_event();
  if (!start || !stop) {
    if (start) g_event_pool.push_back(start);
    if (stop) g_event_pool.push_back(stop);
    return;
  }
  g_log.push_back({name, start, stop});
  start_ = start;
  stop_ = stop;
}

}  // namespace sb

extern "C" int sb_kernel_timing_enable(int32_t enable) {
  using namespace sb;
  std::lock_guard<std::mutex> lock(g_timing_mu);
  if (enable) {
    for (const TimedLaunch& t : g_log) {
      g_event_pool.push_back(t.start);
      g_event_pool.push_back(t.stop);
    }
    g_log.clear();
  }
  g_timing.store(enable != 0);
  return SB_OK;
}

extern "C" int sb_kernel_timing_read(const char* kernel, double* total_ms, int64_t* launches) {
  using namespace sb;
  if (!kernel || !total_ms || !launches) return fail("sb_kernel_timing_read", "null argument");
  std::lock_guard<std::mutex> lock(g_timing_mu);
  double sum = 0.0;
  int64_t n = 0;
  for (const TimedLaunch& t : g_log) {
    if (std::strcmp(t.name, kernel) != 0) continue;
    float ms = 0.f;
    hipError_t e = hipEventSynchronize(t.stop);
    if (e == hipSuccess) e = hipEventElapsedTime(&ms, t.start, t.stop);
    if (e != hipSuccess) {
      set_error(std::string("sb_kernel_timing_read: ") + hipGetErrorString(e));
      return static_cast<int>(e);
    }
    sum += ms;
    ++n;
  }
  *total_ms = sum;
  *launches = n;
  return SB_OK;
}

extern "C" const char* sb_version(void) { return "semblend_hip 0.1.0 gfx950"; }

extern "C" const char* sb_last_error_string(void) { return sb::g_last_error.c_str(); }
