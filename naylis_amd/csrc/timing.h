// Optional per-kernel HIP-event timing (off by default).  When enabled with
// naylis_mom_timing_enable(1), every kernel launch of the library is
// bracketed by two hipEvents recorded on the launch stream; totals per kernel
// name are read back with naylis_mom_timing_get().  Used by bench.py to
// measure each kernel's average duration inside the timed region.
#pragma once
#include <hip/hip_runtime.h>

namespace naylis {

class ScopedKernelTimer {
 public:
  ScopedKernelTimer(const char* name, hipStream_t st);
  ~ScopedKernelTimer();
  ScopedKernelTimer(const ScopedKernelTimer&) = delete;
  ScopedKernelTimer& operator=(const ScopedKernelTimer&) = delete;

 private:
  const char* name_;
  hipStream_t st_;
  hipEvent_t start_ = nullptr, stop_ = nullptr;
};

}  // namespace naylis

// Launch `launch` (a statement) bracketed by the timer of `name` on stream `st`.
#define NAYLIS_TIMED(name, st, ...)                \
  do {                                             \
    ::naylis::ScopedKernelTimer naylis_timer_(name, st); \
    __VA_ARGS__;                                   \
  } while (0)
