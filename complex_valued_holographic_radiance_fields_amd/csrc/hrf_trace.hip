// hrf_trace.hip — optional per-stage timing with hipEvents recorded on the
// stream each stage is launched on.  Off by default; when off, a stage scope
// costs one relaxed atomic load.  Each traced stage adds two event records
// to the stream (a few microseconds of queue time each), so a throughput
// measurement traces one stage at most (hrf_trace_only).
#include <hip/hip_runtime.h>

#include <atomic>
#include <cstring>
#include <mutex>
#include <string>
#include <vector>

#include "hrf_internal.h"

namespace hrf {
namespace {

struct Record {
  const char* stage;
  hipEvent_t start, stop;
};

std::atomic<int> g_on{0};
std::mutex g_mu;
// When non-empty, only this stage is traced (guarded by g_mu).
std::string& only() {
  static std::string s;
  return s;
}
std::vector<Record>& records() {
  static std::vector<Record> r;
  return r;
}
std::vector<hipEvent_t>& pool() {
  static std::vector<hipEvent_t> p;
  return p;
}

hipEvent_t take_event() {
  if (!pool().empty()) {
    hipEvent_t e = pool().back();
    pool().pop_back();
    return e;
  }
  hipEvent_t e = nullptr;
  if (hipEventCreate(&e) != hipSuccess) return nullptr;
  return e;
}

}  // namespace

StageTimer::StageTimer(const char* stage, hipStream_t s) : stage_(stage), s_(s) {
  if (!g_on.load(std::memory_order_relaxed)) return;
  std::lock_guard<std::mutex> lock(g_mu);
  if (!only().empty() && only() != stage) return;
  start_ = take_event();
  stop_ = take_event();
  if (start_ && stop_ && hipEventRecord(start_, s_) == hipSuccess) {
    active_ = true;
  }
}

StageTimer::~StageTimer() {
  if (!active_) return;
  std::lock_guard<std::mutex> lock(g_mu);
  if (hipEventRecord(stop_, s_) == hipSuccess) {
    records().push_back(Record{stage_, start_, stop_});
  } else {
    pool().push_back(start_);
    pool().push_back(stop_);
  }
}

}  // namespace hrf

extern "C" {

int hrf_trace_enable(int on) {
  hrf::g_on.store(on ? 1 : 0);
  return HRF_OK;
}

int hrf_trace_only(const char* stage) {
  std::lock_guard<std::mutex> lock(hrf::g_mu);
  hrf::only() = stage ? stage : "";
  return HRF_OK;
}

void hrf_trace_reset(void) {
  std::lock_guard<std::mutex> lock(hrf::g_mu);
  for (auto& r : hrf::records()) {
    hipEventSynchronize(r.stop);
    hrf::pool().push_back(r.start);
    hrf::pool().push_back(r.stop);
  }
  hrf::records().clear();
}

int hrf_trace_read(const char* stage, int64_t* launches, double* total_ms) {
  if (!stage || !launches || !total_ms) {
    hrf::set_error("hrf_trace_read: null argument");
    return HRF_ERR_INVALID;
  }
  std::lock_guard<std::mutex> lock(hrf::g_mu);
  int64_t n = 0;
  double ms = 0.0;
  for (auto& r : hrf::records()) {
    if (std::strcmp(r.stage, stage) != 0) continue;
    HRF_HIP(hipEventSynchronize(r.stop));
    float t = 0.0f;
    HRF_HIP(hipEventElapsedTime(&t, r.start, r.stop));
    ms += t;
    ++n;
  }
  *launches = n;
  *total_ms = ms;
  return HRF_OK;
}

}  // extern "C"
