// Per-kernel event timing for benchmarking (see timing.h).
#include <stdint.h>
#include <string.h>

#include <atomic>
#include <map>
#include <mutex>
#include <string>
#include <vector>

#include "../../include/naylis_mom.h"
#include "timing.h"

namespace naylis {
namespace {

struct Pending {
  std::string name;
  hipEvent_t start, stop;
};

struct Totals {
  double ms = 0.0;
  int64_t count = 0;
};

std::atomic<int> g_enabled{0};
std::mutex g_mu;
std::vector<Pending> g_pending;
std::vector<hipEvent_t> g_pool;
std::map<std::string, Totals> g_totals;

hipEvent_t take_event() {
  if (!g_pool.empty()) {
    hipEvent_t e = g_pool.back();
    g_pool.pop_back();
    return e;
  }
  hipEvent_t e = nullptr;
  if (hipEventCreate(&e) != hipSuccess) return nullptr;
  return e;
}

// Resolve all pending event pairs into totals (caller holds g_mu).
int drain_locked() {
  int rc = 0;
  for (auto& p : g_pending) {
    float ms = 0.f;
    if (hipEventSynchronize(p.stop) != hipSuccess || hipEventElapsedTime(&ms, p.start, p.stop) != hipSuccess) {
      rc = NAYLIS_ERR_HIP;
    } else {
      Totals& t = g_totals[p.name];
      t.ms += ms;
      t.count += 1;
    }
    g_pool.push_back(p.start);
    g_pool.push_back(p.stop);
  }
  g_pending.clear();
  return rc;
}

}  // namespace

ScopedKernelTimer::ScopedKernelTimer(const char* name, hipStream_t st) : name_(name), st_(st) {
  if (!g_enabled.load(std::memory_order_relaxed)) return;
  std::lock_guard<std::mutex> lk(g_mu);
  start_ = take_event();
  stop_ = take_event();
  if (!start_ || !stop_) {  // timing off for this launch; return what was taken
    if (start_) g_pool.push_back(start_);
    if (stop_) g_pool.push_back(stop_);
    start_ = stop_ = nullptr;
  }
}

// (the launch inside NAYLIS_TIMED recorded both events with the kernel)
ScopedKernelTimer::~ScopedKernelTimer() {
  if (!start_ || !stop_) return;
  std::lock_guard<std::mutex> lk(g_mu);
  g_pending.push_back({name_, start_, stop_});
}

}  // namespace naylis

using namespace naylis;

extern "C" {

void naylis_mom_timing_enable(int on) { g_enabled.store(on ? 1 : 0); }

void naylis_mom_timing_reset(void) {
  std::lock_guard<std::mutex> lk(g_mu);
  drain_locked();
  g_totals.clear();
}

int naylis_mom_timing_get(const char* name, double* total_ms, int64_t* count) {
  std::lock_guard<std::mutex> lk(g_mu);
  const int rc = drain_locked();
  auto it = g_totals.find(name ? name : "");
  *total_ms = it == g_totals.end() ? 0.0 : it->second.ms;
  *count = it == g_totals.end() ? 0 : it->second.count;
  return rc;
}

int naylis_mom_timing_names(char* buf, size_t buf_bytes) {
  std::lock_guard<std::mutex> lk(g_mu);
  const int rc = drain_locked();
  std::string all;
  for (auto& kv : g_totals) {
    if (!all.empty()) all += ",";
    all += kv.first;
  }
  if (buf && buf_bytes) {
    strncpy(buf, all.c_str(), buf_bytes - 1);
    buf[buf_bytes - 1] = 0;
  }
  return rc;
}

}  // extern "C"
