// Library identity, thread-local error state and the kernel timer.
#include <atomic>
#include <cstring>
#include <mutex>
#include <vector>

#include "mxq_common.h"

namespace mxq {

static thread_local std::string g_last_error;

void set_error(const std::string& msg) { g_last_error = msg; }

int invalid(const std::string& msg) {
  g_last_error = msg;
  return MXQ_EINVAL;
}

int check_launch(const char* what) {
  hipError_t err = hipGetLastError();
  if (err != hipSuccess) {
    g_last_error = std::string(what) + ": " + hipGetErrorString(err);
    return MXQ_EHIP;
  }
  return MXQ_OK;
}

namespace {

struct Timed {
  const char* name;
  hipEvent_t start, stop;
};

std::atomic<int> g_timer_on{0};
std::mutex g_timer_mu;
std::vector<Timed> g_timed;

}  // namespace

KernelTimer::KernelTimer(const char* name, hipStream_t stream) : name_(name), stream_(stream) {
  if (!g_timer_on.load(std::memory_order_relaxed)) return;
  if (hipEventCreate(&start_) != hipSuccess) {
    start_ = nullptr;
    return;
  }
  if (hipEventRecord(start_, stream_) != hipSuccess) {
    (void)hipEventDestroy(start_);
    start_ = nullptr;
  }
}

KernelTimer::~KernelTimer() {
  if (!start_) return;
  hipEvent_t stop = nullptr;
  if (hipEventCreate(&stop) != hipSuccess || hipEventRecord(stop, stream_) != hipSuccess) {
    if (stop) (void)hipEventDestroy(stop);
    (void)hipEventDestroy(start_);
    return;
  }
  std::lock_guard<std::mutex> lock(g_timer_mu);
  g_timed.push_back({name_, start_, stop});
}

}  // namespace mxq

extern "C" int mxq_timer_enable(int32_t on) {
  mxq::g_timer_on.store(on ? 1 : 0);
  return MXQ_OK;
}

extern "C" int mxq_timer_read(const char* kernel, double* total_ms, int64_t* launches) {
  if (!kernel || !total_ms || !launches) return mxq::invalid("mxq_timer_read: NULL argument");
  std::vector<mxq::Timed> mine;
  {
    std::lock_guard<std::mutex> lock(mxq::g_timer_mu);
    std::vector<mxq::Timed> rest;
    for (const auto& t : mxq::g_timed) (std::strcmp(t.name, kernel) == 0 ? mine : rest).push_back(t);
    mxq::g_timed.swap(rest);
  }
  double sum = 0.0;
  int rc = MXQ_OK;
  for (const auto& t : mine) {
    float ms = 0.0f;
    if (rc == MXQ_OK) {
      hipError_t err = hipEventSynchronize(t.stop);
      if (err == hipSuccess) err = hipEventElapsedTime(&ms, t.start, t.stop);
      if (err != hipSuccess) {
        mxq::set_error(std::string("mxq_timer_read: ") + hipGetErrorString(err));
        rc = MXQ_EHIP;
      }
    }
    sum += ms;
    (void)hipEventDestroy(t.start);
    (void)hipEventDestroy(t.stop);
  }
  *total_ms = sum;
  *launches = (int64_t)mine.size();
  return rc;
}

extern "C" const char* mxq_last_error(void) { return mxq::g_last_error.c_str(); }

extern "C" int mxq_version(void) { return MXQ_ABI_VERSION; }
