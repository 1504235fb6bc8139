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

// Division of n < 2^31 by a divisor d >= 1 fixed at launch, as one multiply-high, an add and a shift
// (Granlund and Montgomery's round-up method): with l = ceil(log2 d) and mul = floor(2^32 (2^l - d) / d) + 1
// (below 2^32, since 2^l - d < d), n / d = (umulhi(n, mul) + n) >> l, and the sum stays below 2^32 because
// umulhi(n, mul) <= n.  A per-wave 64-bit division costs some hundred scalar instructions.
struct DivU31 {
  uint32_t mul, shift, d;
};
inline DivU31 make_divu31(uint32_t d) {
  uint32_t l = 0;
  while ((1ull << l) < d) ++l;
  return DivU31{(uint32_t)(((1ull << 32) * ((1ull << l) - d)) / d + 1), l, d};
}
__device__ __forceinline__ uint32_t divu31(uint32_t n, const DivU31& v) { return (__umulhi(n, v.mul) + n) >> v.shift; }

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
