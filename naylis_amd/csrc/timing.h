// Optional per-kernel HIP-event timing (off by default).  When enabled with
// naylis_mom_timing_enable(1), every kernel launch of the library goes
// through hipExtLaunchKernel with a start and a stop event bound to the
// kernel's own dispatch, so the pair times the kernel itself (as a profiler
// does), not the wait for the previous work on the stream; totals per kernel
// name are read back with naylis_mom_timing_get().  Used by bench.py to
// measure each kernel's average duration inside the timed region.
#pragma once
#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>

namespace naylis {

class ScopedKernelTimer {
 public:
  ScopedKernelTimer(const char* name, hipStream_t st);
  ~ScopedKernelTimer();
  ScopedKernelTimer(const ScopedKernelTimer&) = delete;
  ScopedKernelTimer& operator=(const ScopedKernelTimer&) = delete;
  bool on() const { return start_ != nullptr && stop_ != nullptr; }
  hipEvent_t start() const { return start_; }
  hipEvent_t stop() const { return stop_; }

 private:
  const char* name_;
  hipStream_t st_;
  hipEvent_t start_ = nullptr, stop_ = nullptr;
};

}  // namespace naylis

// Launch `launch` -- one hipLaunchKernelGGL(kernel, grid, block, lds, stream,
// args...) -- under the timer of `name` on stream `st`: with timing on, the
// same launch through hipExtLaunchKernelGGL with the timer's events (the
// paste takes the launch's tokens before hipLaunchKernelGGL expands).
#define NAYLIS_TIMED(name, st, ...)                      \
  do {                                                   \
    ::naylis::ScopedKernelTimer naylis_timer_(name, st); \
    if (naylis_timer_.on()) {                            \
      NAYLIS_EXT_##__VA_ARGS__;                          \
    } else {                                             \
      __VA_ARGS__;                                       \
    }                                                    \
  } while (0)
#define NAYLIS_EXT_hipLaunchKernelGGL(kernel, grid, block, lds, stream, ...)                                      \
  hipExtLaunchKernelGGL(kernel, grid, block, lds, stream, naylis_timer_.start(), naylis_timer_.stop(), 0, \
                        __VA_ARGS__)
