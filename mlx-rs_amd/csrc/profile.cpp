// Per-kernel launch timing with HIP events.
//
// While a kernel name is armed, every launch of that kernel records one HIP
// event on its stream just before the launch and one just after; reading the
// profile synchronises on the last event and sums the elapsed times.  The
// events are ordinary stream events, so they time the kernel on the stream it
// actually runs on (the caller's), whatever stream the caller's framework
// considers current.  Not for use under stream capture.
#include <hip/hip_runtime.h>

#include <atomic>
#include <mutex>
#include <string>
#include <vector>

#include "kernels.hpp"

namespace mlxr_moe {
namespace {

struct Profile {
  std::atomic<bool> on{false};  // fast path: nothing armed
  std::mutex mu;
  std::string armed;                                   // "" = off
  std::vector<std::pair<hipEvent_t, hipEvent_t>> used; // this session
  std::vector<std::pair<hipEvent_t, hipEvent_t>> pool; // recycled
};

// The events only time: no system-scope fence when they complete (the
// default one writes back and invalidates the caches after the kernel,
// which the elapsed time would include: ~6 us on a 46 us launch).
// Reading the profile still waits for the stop event.
constexpr unsigned kTimingEventFlags = hipEventDisableSystemFence;

Profile& prof() {
  static Profile* p = new Profile();  // never destroyed: events outlive exit
  return *p;
}

}  // namespace

ProfileScope::ProfileScope(const char* kernel, hipStream_t s) {
  Profile& p = prof();
  if (!p.on.load(std::memory_order_relaxed)) return;
  std::lock_guard<std::mutex> lk(p.mu);
  if (p.armed.empty() || p.armed != kernel) return;
  std::pair<hipEvent_t, hipEvent_t> ev{nullptr, nullptr};
  if (!p.pool.empty()) {
    ev = p.pool.back();
    p.pool.pop_back();
  } else if (hipEventCreateWithFlags(&ev.first, kTimingEventFlags) != hipSuccess ||
             hipEventCreateWithFlags(&ev.second, kTimingEventFlags) != hipSuccess) {
    return;
  }
  if (hipEventRecord(ev.first, s) != hipSuccess) {
    p.pool.push_back(ev);
    return;
  }
  stop_ = ev.second;
  stream_ = s;
  p.used.push_back(ev);
}

ProfileScope::~ProfileScope() {
  if (stop_) (void)hipEventRecord(stop_, stream_);
}

int profile_arm(const char* kernel) {
  Profile& p = prof();
  std::lock_guard<std::mutex> lk(p.mu);
  for (auto& ev : p.used) p.pool.push_back(ev);
  p.used.clear();
  p.armed = kernel ? kernel : "";
  p.on.store(!p.armed.empty());
  return 0;
}

int profile_collect(int64_t* launches, double* total_ms, double* min_ms,
                    double* max_ms, std::string* err) {
  Profile& p = prof();
  std::lock_guard<std::mutex> lk(p.mu);
  double tot = 0.0, mn = 0.0, mx = 0.0;
  for (size_t i = 0; i < p.used.size(); ++i) {
    auto& ev = p.used[i];
    hipError_t e = hipEventSynchronize(ev.second);
    float ms = 0.0f;
    if (e == hipSuccess) e = hipEventElapsedTime(&ms, ev.first, ev.second);
    if (e != hipSuccess) {
      *err = std::string("profile: ") + hipGetErrorString(e);
      return -1;
    }
    tot += ms;
    mn = i == 0 ? ms : (ms < mn ? ms : mn);
    mx = i == 0 ? ms : (ms > mx ? ms : mx);
  }
  if (launches) *launches = (int64_t)p.used.size();
  if (total_ms) *total_ms = tot;
  if (min_ms) *min_ms = mn;
  if (max_ms) *max_ms = mx;
  for (auto& ev : p.used) p.pool.push_back(ev);
  p.used.clear();
  p.armed.clear();
  p.on.store(false);
  return 0;
}

}  // namespace mlxr_moe
