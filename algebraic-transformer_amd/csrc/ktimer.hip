// Event-based kernel timer behind alg_timer_enable / alg_timer_report (see ktimer.h).
#include <atomic>
#include <cstdio>
#include <cstring>
#include <map>
#include <mutex>
#include <string>
#include <vector>

#include "algebraic_hip.h"
#include "ktimer.h"

namespace alg {

namespace {
std::atomic<bool> g_on{false};
std::mutex g_mu;
struct Rec { const char* name; hipEvent_t a, b; };
std::vector<Rec> g_recs;
}  // namespace

bool timer_enabled() { return g_on.load(std::memory_order_relaxed); }

void timer_record(const char* name, hipEvent_t start, hipEvent_t stop) {
  std::lock_guard<std::mutex> lk(g_mu);
  g_recs.push_back({name, start, stop});
}

}  // namespace alg

extern "C" {

void alg_timer_enable(int on) {
  alg::g_on.store(on != 0);
}

size_t alg_timer_report(char* out, size_t cap) {
  std::vector<alg::Rec> recs;
  {
    std::lock_guard<std::mutex> lk(alg::g_mu);
    recs.swap(alg::g_recs);
  }
  std::map<std::string, std::pair<long, double>> agg;
  for (const auto& r : recs) {
    float ms = 0.0f;
    if (hipEventSynchronize(r.b) == hipSuccess && hipEventElapsedTime(&ms, r.a, r.b) == hipSuccess) {
      auto& e = agg[r.name];
      e.first += 1;
      e.second += ms;
    }
    (void)hipEventDestroy(r.a);
    (void)hipEventDestroy(r.b);
  }
  std::string s = "{";
  bool first = true;
  for (const auto& kv : agg) {
    char buf[256];
    snprintf(buf, sizeof buf, "%s\"%s\": {\"launches\": %ld, \"mean_ms\": %.6f}", first ? "" : ", ",
             kv.first.c_str(), kv.second.first, kv.second.second / (double)kv.second.first);
    s += buf;
    first = false;
  }
  s += "}";
  if (out && cap) {
    const size_t n = s.size() < cap - 1 ? s.size() : cap - 1;
    std::memcpy(out, s.data(), n);
    out[n] = '\0';
  }
  return s.size() + 1;
}

}  // extern "C"
