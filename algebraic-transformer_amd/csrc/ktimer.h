// Optional per-kernel timing with HIP events (measurement hook for benchmarks).
//
// Disabled by default: a KTimer then costs one relaxed atomic load. When enabled through
// alg_timer_enable(1), each timed launch records a start/stop event pair on its own stream;
// alg_timer_report() synchronises on those events and returns per-kernel launch counts and
// mean durations. Enabling, reporting and timed launches must not race with each other.
#pragma once

#include <hip/hip_runtime.h>

namespace alg {

bool timer_enabled();
void timer_record(const char* name, hipEvent_t start, hipEvent_t stop);

class KTimer {
 public:
  KTimer(const char* name, hipStream_t st) : name_(name), st_(st) {
    if (timer_enabled()) {
      on_ = hipEventCreate(&a_) == hipSuccess && hipEventCreate(&b_) == hipSuccess &&
            hipEventRecord(a_, st_) == hipSuccess;
    }
  }
  ~KTimer() {
    if (on_ && hipEventRecord(b_, st_) == hipSuccess) timer_record(name_, a_, b_);
  }
  KTimer(const KTimer&) = delete;
  KTimer& operator=(const KTimer&) = delete;

 private:
  const char* name_;
  hipStream_t st_;
  hipEvent_t a_{}, b_{};
  bool on_ = false;
};

}  // namespace alg
