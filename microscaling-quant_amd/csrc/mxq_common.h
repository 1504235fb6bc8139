// Host-side plumbing shared by the library's translation units: error state and launch checks.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <string>

#include "../../include/mxq_hip.h"

namespace mxq {

void set_error(const std::string& msg);

// Record `msg` and return MXQ_EINVAL.
int invalid(const std::string& msg);

// After a launch: MXQ_OK, or MXQ_EHIP with hipGetLastError's text.
int check_launch(const char* what);

inline hipStream_t as_stream(mxq_stream_t s) { return reinterpret_cast<hipStream_t>(s); }

inline int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }

// One-dimensional grid of `threads` threads in blocks of `block`; grid.x caps at 2^31 - 1 blocks.
inline dim3 grid_for(int64_t threads, int block) { return dim3((unsigned)ceil_div(threads, block)); }

// While mxq_timer_enable(1) is in force, an object of this type brackets one kernel launch with a pair of
// HIP events on the launch's stream, filed under `name` for mxq_timer_read.  Otherwise it does nothing.
class KernelTimer {
 public:
  KernelTimer(const char* name, hipStream_t stream);
  ~KernelTimer();
  KernelTimer(const KernelTimer&) = delete;
  KernelTimer& operator=(const KernelTimer&) = delete;

 private:
  const char* name_;
  hipStream_t stream_;
  hipEvent_t start_ = nullptr;
};

}  // namespace mxq
