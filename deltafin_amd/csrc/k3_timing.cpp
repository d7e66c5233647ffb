// Optional per-launch device timing.
//
// While a timing window is open (k3_hip_timing_begin .. k3_hip_timing_end),
// every kernel this library launches goes through hipExtLaunchKernel with a
// pair of hipEvents from a pool created when the window opens; the runtime
// stamps them with that dispatch's own start and end, so the elapsed time is
// the kernel's device duration without the launch overhead around it (the
// figure a kernel trace reports).  Launches beyond the pool are counted as
// dropped rather than timed.  The reference's counterparts are the Metal
// bridge counters (tools/metal_moe.mm:675-681) and the per-layer phase profile
// (native/deltafin/src/engine.rs:4705-4902).
#include <hip/hip_runtime_api.h>
#include <string.h>

#include <algorithm>
#include <atomic>
#include <mutex>
#include <vector>

#include "k3_internal.h"

namespace k3 {
namespace {

const char* const kClassNames[KC_COUNT] = {
    "gemv",        "activate",    "route",       "glu_decode", "down_decode",
    "verify_plan", "glu_verify",  "down_verify", "combine",    "synth",
    "decode_fused", "split_terms", "glu_mfma",   "down_mfma",  "spine_gemv",
    "rms_norm",    "spine_mfma",  "decode_chain",
};

struct TimingState {
  std::mutex mu;
  std::atomic<bool> on{false};
  std::vector<hipEvent_t> events;  // 2 per slot
  std::vector<int> klass;          // per used slot
  int used = 0;
  long long dropped = 0;
};

TimingState& state() {
  static TimingState s;
  return s;
}

void destroy_events_locked(TimingState& s) {
  for (hipEvent_t e : s.events) (void)hipEventDestroy(e);
  s.events.clear();
  s.klass.clear();
  s.used = 0;
  s.dropped = 0;
}

}  // namespace

TimedLaunch::TimedLaunch(int kernel_class, hipStream_t stream) : slot_(-1) {
  (void)stream;
  TimingState& s = state();
  if (!s.on.load(std::memory_order_acquire)) return;
  std::lock_guard<std::mutex> lk(s.mu);
  if (!s.on.load(std::memory_order_relaxed)) return;
  if ((size_t)s.used * 2 >= s.events.size()) {
    ++s.dropped;
    return;
  }
  slot_ = s.used++;
  s.klass.push_back(kernel_class);
}

hipEvent_t TimedLaunch::start() const {
  return slot_ < 0 ? nullptr : state().events[2 * slot_];
}

hipEvent_t TimedLaunch::stop() const {
  return slot_ < 0 ? nullptr : state().events[2 * slot_ + 1];
}

void TimedLaunch::failed() {
  if (slot_ < 0) return;
  TimingState& s = state();
  std::lock_guard<std::mutex> lk(s.mu);
  s.klass[slot_] = -1;
  ++s.dropped;
  slot_ = -1;
}

}  // namespace k3

using namespace k3;

extern "C" {

int k3_hip_timing_begin(int max_launches) {
  if (max_launches <= 0 || max_launches > (1 << 20))
    return fail(K3_HIP_E_INVALID, "timing: max_launches must be in [1, 2^20]");
  TimingState& s = state();
  std::lock_guard<std::mutex> lk(s.mu);
  if (s.on.load()) return fail(K3_HIP_E_INVALID, "timing: a window is already open");
  destroy_events_locked(s);
  s.events.reserve(2 * (size_t)max_launches);
  s.klass.reserve((size_t)max_launches);
  for (int i = 0; i < 2 * max_launches; ++i) {
    hipEvent_t e = nullptr;
    const hipError_t err = hipEventCreate(&e);
    if (err != hipSuccess) {
      destroy_events_locked(s);
      return fail(K3_HIP_E_ALLOC, "timing: event pool: %s", hipGetErrorString(err));
    }
    s.events.push_back(e);
  }
  s.on.store(true, std::memory_order_release);
  return K3_HIP_OK;
}

int k3_hip_timing_end(K3HipKernelTimingV1* out, int capacity, int* n_out,
                      long long* dropped) {
  TimingState& s = state();
  std::lock_guard<std::mutex> lk(s.mu);
  if (!s.on.load()) return fail(K3_HIP_E_INVALID, "timing: no window is open");
  s.on.store(false, std::memory_order_release);
  K3HipKernelTimingV1 acc[KC_COUNT];
  memset(acc, 0, sizeof(acc));
  for (int i = 0; i < s.used; ++i) {
    const int k = s.klass[i];
    if (k < 0 || k >= KC_COUNT) continue;
    hipError_t e = hipEventSynchronize(s.events[2 * i + 1]);
    float ms = 0.0f;
    if (e == hipSuccess) e = hipEventElapsedTime(&ms, s.events[2 * i], s.events[2 * i + 1]);
    if (e != hipSuccess) {  // a pair the runtime never stamped: count it, skip it
      (void)hipGetLastError();
      ++s.dropped;
      continue;
    }
    K3HipKernelTimingV1& a = acc[k];
    if (a.launches == 0) {
      a.min_ms = a.max_ms = ms;
    } else {
      a.min_ms = std::min<double>(a.min_ms, ms);
      a.max_ms = std::max<double>(a.max_ms, ms);
    }
    ++a.launches;
    a.total_ms += ms;
  }
  int n = 0;
  for (int k = 0; k < KC_COUNT; ++k) {
    if (acc[k].launches == 0) continue;
    if (out && n < capacity) {
      out[n] = acc[k];
      strncpy(out[n].kernel, kClassNames[k], sizeof(out[n].kernel) - 1);
    }
    ++n;
  }
  if (n_out) *n_out = std::min(n, std::max(capacity, 0));
  if (dropped) *dropped = s.dropped;
  destroy_events_locked(s);
  return K3_HIP_OK;
}

}  // extern "C"
