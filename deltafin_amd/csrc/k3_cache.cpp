// HBM expert cache: C counterpart of CudaMoeExpertCache
// (native/provider_gate/provider_cuda_moe.{h,cpp}).
//
// * Bookkeeping (policy, budget, slots, strata, plans, fail-closed state,
//   recovery) lives in k3_cache_book.h, free of device calls; this file holds
//   the device side: segments of slots in HBM, the side stream, events,
//   staging and the known-answer qualification.
// * Capacity comes from a budget measured once at first use, free device
//   memory minus a reserve (max(2 GiB, free / 5) by default), capped by the
//   requested expert count (provider_cuda_moe.cpp:668-705); the policy is
//   frozen from then on (:60-74, :571-578).  Slots are allocated in segments
//   as the cache fills, so an allocation can fail while the cache is in use.
// * Such a failure is recoverable (provider_cuda_moe.cpp:545-567, :630-653):
//   the fetch is undone, the copy stream drained, every unpinned entry
//   dropped, unpinned segments given back and the budget re-measured at the
//   next plan; the fetch returns K3_HIP_E_ALLOC and the plan's pinned hits
//   stay readable (k3_hip_cache_materialize_plan) for the caller's exact CPU
//   reconstruction of the tile (provider_moe.cpp:1117-1206).  After two such
//   rebuilds the next failure disables the cache (K3_HIP_E_CAPABILITY).
// * plan() snapshots hits before any miss can be admitted, pinning them for
//   the plan's lifetime (:963-1008); eviction takes the globally least-recent
//   unpinned entry over all layer strata (:707-747).
// * fetch() admits misses with hipMemcpyAsync on the cache's own side stream,
//   so copies overlap compute on the caller's streams; each slot records a
//   ready event that resolve() / ready_subset() make the caller's stream wait
//   on (resolve) or test (ready_subset).  The reference copies on the
//   execution stream through two pinned slabs (:757-805); here pinned sources
//   are copied directly and pageable sources go through a ring of pinned
//   staging slots, filled by a threaded host copy.
// * Because copies run on their own stream, a slot's previous contents may
//   still be read by kernels queued before release(): release() records, for
//   every stream the plan handed its spans to, a per-(slot, stream) event, and
//   a copy into an evicted slot first makes the side stream wait on all of
//   them.
// * Qualification and fail-closed state (provider_cuda_moe.cpp:889-953,
//   :517-533): the first plan runs the reference's device known-answer tests
//   (:291-420) on the cache's stream.  A mismatch disables the cache
//   (K3_HIP_E_CAPABILITY: the caller takes its CPU path); a HIP error, or a
//   caller's k3_hip_cache_poison, makes it terminal (K3_HIP_E_EXEC).  Either
//   way every resident entry is dropped and later calls fail with the reason.
#include <hip/hip_runtime_api.h>
#include <math.h>
#include <string.h>

#include <algorithm>
#include <map>
#include <mutex>
#include <string>
#include <thread>
#include <vector>

#include "k3_cache_book.h"
#include "k3_internal.h"

using namespace k3;

// Slots per device segment (one hipMalloc each).
constexpr int kSegmentSlots = 32;

struct K3HipCache final : CacheBook::Hooks {
  struct SlotDev {
    hipEvent_t ready = nullptr;  // recorded after the slot's last upload
    bool has_ready = false;
    // One event per stream that read the slot, recorded at release.
    std::vector<std::pair<hipStream_t, hipEvent_t>> done;
  };

  K3HipCache(int dev, uint64_t span_bytes, int n_layers, const CachePolicy& policy)
      : device(dev), span(span_bytes), book(((span_bytes + 4095) & ~uint64_t(4095)), n_layers,
                                              kSegmentSlots, policy) {}

  std::mutex mu;
  int device = 0;
  uint64_t span = 0;
  CacheBook book;
  hipStream_t side = nullptr;
  std::vector<uint8_t*> seg_base;
  std::vector<SlotDev> sdev;
  std::vector<hipEvent_t> event_pool;
  std::map<uint64_t, std::vector<hipStream_t>> plan_streams;
  std::vector<uint8_t*> staging;
  std::vector<hipEvent_t> staging_ready;
  std::vector<bool> staging_used;
  int staging_cursor = 0;
  long long uploaded = 0;
  hipError_t hook_error = hipSuccess;  // a device failure inside a hook

  uint8_t* addr(int slot) const {
    int seg = 0, idx = 0;
    book.locate(slot, &seg, &idx);
    return seg_base[seg] + (uint64_t)idx * book.slot_bytes();
  }

  hipEvent_t take_event() {
    if (!event_pool.empty()) {
      hipEvent_t e = event_pool.back();
      event_pool.pop_back();
      return e;
    }
    hipEvent_t e = nullptr;
    if (hipEventCreateWithFlags(&e, hipEventDisableTiming) != hipSuccess) {
      (void)hipGetLastError();
      return nullptr;
    }
    return e;
  }

  // ---- CacheBook::Hooks
  int alloc_segment(int seg, uint64_t bytes) override {
    if (seg != (int)seg_base.size()) {  // segments are made and given back in order
      hook_error = hipErrorInvalidValue;
      return -1;
    }
    uint8_t* p = nullptr;
    const hipError_t e = hipMalloc(reinterpret_cast<void**>(&p), bytes);
    if (e != hipSuccess) {
      (void)hipGetLastError();
      if (e == hipErrorOutOfMemory || e == hipErrorMemoryAllocation) return 1;
      hook_error = e;
      return -1;
    }
    const size_t first = sdev.size(), n = bytes / book.slot_bytes();
    sdev.resize(first + n);
    for (size_t i = first; i < first + n; ++i) {
      const hipError_t ee = hipEventCreateWithFlags(&sdev[i].ready, hipEventDisableTiming);
      if (ee != hipSuccess) {
        (void)hipGetLastError();
        for (size_t j = first; j < i; ++j) (void)hipEventDestroy(sdev[j].ready);
        sdev.resize(first);
        (void)hipFree(p);
        hook_error = ee;
        return -1;
      }
    }
    seg_base.push_back(p);
    return 0;
  }
  void free_segment(int seg) override {
    const int n = book.segment_size(seg);
    const size_t first = sdev.size() - (size_t)n;
    for (size_t i = first; i < sdev.size(); ++i) {
      (void)hipEventDestroy(sdev[i].ready);
      for (auto& d : sdev[i].done) event_pool.push_back(d.second);
    }
    sdev.resize(first);
    (void)hipFree(seg_base[seg]);
    seg_base.resize(seg);
  }
  void wait_slot_idle(int slot) override {
    SlotDev& s = sdev[slot];
    for (auto& d : s.done) (void)hipEventSynchronize(d.second);
    if (s.has_ready) (void)hipEventSynchronize(s.ready);
  }
};

namespace {

int set_device(K3HipCache* c) {
  const hipError_t e = hipSetDevice(c->device);
  return e == hipSuccess ? K3_HIP_OK : hip_fail("cache hipSetDevice", e);
}

// ------------------------------------------------------------ qualification
float e2m1_value(uint8_t code) {
  static const float mag[8] = {0.0f, 0.5f, 1.0f, 1.5f, 2.0f, 3.0f, 4.0f, 6.0f};
  return (code & 8) ? -mag[code & 7] : mag[code & 7];
}

// The reference's two device known-answer tests (provider_cuda_moe.cpp:291-420)
// through this library's own entry points, on `st`: every E2M1 code across two
// generated GEMV rows at two batches (within 2e-4 of a sequential fma sum),
// and a K3 expert with one nonzero per matrix through the single-expert
// launch (out[0] = SiTU(x0, 2 x0), within 2e-5).  Each runs twice and the two
// outputs must match bit for bit.  0 = pass, 1 = mismatch, -1 = HIP error;
// *why names the failure.
int known_answer_tests(hipStream_t st, std::string* why) {
  uint8_t packed[32];
  for (int i = 0; i < 16; ++i) {
    const int ph = (2 * i) % 16;
    packed[i] = (uint8_t)(ph | (((ph + 1) % 16) << 4));
    packed[16 + i] = (uint8_t)((15 - ph) | ((14 - ph) << 4));
  }
  const uint8_t scales[2] = {127, 126};
  float x[64];
  for (int c = 0; c < 32; ++c) {
    x[c] = (float)c / 32.0f;
    x[32 + c] = ((float)c - 15.0f) / 17.0f;
  }
  float want[4];
  for (int b = 0; b < 2; ++b)
    for (int r = 0; r < 2; ++r) {
      float t = 0.0f;
      for (int c = 0; c < 32; ++c) {
        const uint8_t byte = packed[r * 16 + c / 2];
        const uint8_t code = (c & 1) ? (uint8_t)(byte >> 4) : (uint8_t)(byte & 15);
        t = fmaf(ldexpf(e2m1_value(code), (int)scales[r] - 127), x[b * 32 + c], t);
      }
      want[b * 2 + r] = t;
    }
  K3HipGeometryV1 gd;
  k3_hip_geometry_preset(1, &gd);  // K3: hidden 3584, intermediate 3072, SiTU
  const int H = (int)gd.hidden, I = (int)gd.intermediate;
  const uint64_t P = (uint64_t)H * I / 2, S = (uint64_t)I * (H / 32);
  uint8_t *dp = nullptr, *ds = nullptr, *span = nullptr;
  float *dx = nullptr, *o1 = nullptr, *o2 = nullptr, *mx = nullptr, *gate = nullptr,
        *up = nullptr, *m1 = nullptr, *m2 = nullptr;
  std::vector<float> h1(2 * (size_t)H), h2(2 * (size_t)H), mxh(2 * (size_t)H, 0.0f);
  float g1[4], g2[4];
  int result = 0;
  hipError_t e = hipSuccess;
  auto ok = [&](hipError_t v) { return (e = v) == hipSuccess; };
  if (ok(hipMalloc(reinterpret_cast<void**>(&dp), 32)) &&
      ok(hipMalloc(reinterpret_cast<void**>(&ds), 2)) &&
      ok(hipMalloc(reinterpret_cast<void**>(&dx), sizeof(x))) &&
      ok(hipMalloc(reinterpret_cast<void**>(&o1), 16)) &&
      ok(hipMalloc(reinterpret_cast<void**>(&o2), 16)) &&
      ok(hipMalloc(reinterpret_cast<void**>(&span), gd.expert_span)) &&
      ok(hipMalloc(reinterpret_cast<void**>(&mx), 2 * (size_t)H * 4)) &&
      ok(hipMalloc(reinterpret_cast<void**>(&gate), 2 * (size_t)I * 4)) &&
      ok(hipMalloc(reinterpret_cast<void**>(&up), 2 * (size_t)I * 4)) &&
      ok(hipMalloc(reinterpret_cast<void**>(&m1), 2 * (size_t)H * 4)) &&
      ok(hipMalloc(reinterpret_cast<void**>(&m2), 2 * (size_t)H * 4)) &&
      ok(hipMemcpyAsync(dp, packed, 32, hipMemcpyHostToDevice, st)) &&
      ok(hipMemcpyAsync(ds, scales, 2, hipMemcpyHostToDevice, st)) &&
      ok(hipMemcpyAsync(dx, x, sizeof(x), hipMemcpyHostToDevice, st))) {
    // The one-hot expert: code 2 (1.0) at w1 and w2 element 0, code 4 (2.0)
    // at w3 element 0, scale 127 (1.0) for their first groups.
    const uint8_t one = 0x02, two = 0x04, unit = 127;
    mxh[0] = 1.0f;
    mxh[(size_t)H] = -0.5f;
    if (ok(hipMemsetAsync(span, 0, gd.expert_span, st)) &&
        ok(hipMemcpyAsync(span, &one, 1, hipMemcpyHostToDevice, st)) &&
        ok(hipMemcpyAsync(span + P, &unit, 1, hipMemcpyHostToDevice, st)) &&
        ok(hipMemcpyAsync(span + P + S, &one, 1, hipMemcpyHostToDevice, st)) &&
        ok(hipMemcpyAsync(span + 2 * P + S, &unit, 1, hipMemcpyHostToDevice, st)) &&
        ok(hipMemcpyAsync(span + 2 * (P + S), &two, 1, hipMemcpyHostToDevice, st)) &&
        ok(hipMemcpyAsync(span + 3 * P + 2 * S, &unit, 1, hipMemcpyHostToDevice, st)) &&
        ok(hipMemcpyAsync(mx, mxh.data(), 2 * (size_t)H * 4, hipMemcpyHostToDevice, st))) {
      int rc = k3_hip_mxfp4_gemv(dp, ds, dx, o1, 2, 32, 2, st);
      if (rc == K3_HIP_OK) rc = k3_hip_mxfp4_gemv(dp, ds, dx, o2, 2, 32, 2, st);
      if (rc == K3_HIP_OK) rc = k3_hip_moe_launch(&gd, span, mx, 2, gate, up, m1, st);
      if (rc == K3_HIP_OK) rc = k3_hip_moe_launch(&gd, span, mx, 2, gate, up, m2, st);
      if (rc != K3_HIP_OK) {
        *why = std::string("known-answer launch failed: ") + k3_hip_last_error();
        result = -1;
      } else if (ok(hipMemcpyAsync(g1, o1, 16, hipMemcpyDeviceToHost, st)) &&
                 ok(hipMemcpyAsync(g2, o2, 16, hipMemcpyDeviceToHost, st)) &&
                 ok(hipMemcpyAsync(h1.data(), m1, 2 * (size_t)H * 4, hipMemcpyDeviceToHost, st)) &&
                 ok(hipMemcpyAsync(h2.data(), m2, 2 * (size_t)H * 4, hipMemcpyDeviceToHost, st)) &&
                 ok(hipStreamSynchronize(st))) {
        float d1 = 0.0f;
        for (int i = 0; i < 4; ++i) d1 = fmaxf(d1, fabsf(g1[i] - want[i]));
        float d2 = 0.0f;
        for (int b = 0; b < 2; ++b) {
          const float in = b == 0 ? 1.0f : -0.5f, g = in, u = 2.0f * in;
          const float sit = 4.0f * tanhf(g / 4.0f) / (1.0f + expf(-g)) * (25.0f * tanhf(u / 25.0f));
          for (int i = 0; i < H; ++i)
            d2 = fmaxf(d2, fabsf(h1[(size_t)b * H + i] - (i == 0 ? sit : 0.0f)));
        }
        if (memcmp(g1, g2, sizeof(g1)) != 0 || !(d1 <= 2.0e-4f)) {
          *why = "MXFP4 generated-weight known-answer test failed";
          result = 1;
        } else if (memcmp(h1.data(), h2.data(), h1.size() * 4) != 0 || !(d2 <= 2.0e-5f)) {
          *why = "full-expert generated-weight known-answer test failed";
          result = 1;
        }
      }
    }
  }
  if (e != hipSuccess && result == 0) {
    (void)hipGetLastError();
    *why = std::string("known-answer test: ") + hipGetErrorString(e);
    result = -1;
  }
  (void)hipStreamSynchronize(st);
  for (void* q : {(void*)dp, (void*)ds, (void*)dx, (void*)o1, (void*)o2, (void*)span, (void*)mx,
                  (void*)gate, (void*)up, (void*)m1, (void*)m2})
    if (q) (void)hipFree(q);
  return result;
}

// A HIP failure inside a cache call: terminal.
int runtime_fail_locked(K3HipCache* c, const char* what, hipError_t e) {
  (void)hipGetLastError();
  c->book.poison(std::string(what) + ": " + hipGetErrorString(e), true);
  return fail(K3_HIP_E_EXEC, "expert cache disabled after runtime failure: %s",
              c->book.reason().c_str());
}

// The gate every plan / fetch / resolve call passes: qualifies on first use,
// then measures the budget (again after a recovery).
int gate_locked(K3HipCache* c) {
  if (c->book.state() == CacheBook::kUnqualified) {
    c->book.freeze();
    std::string why;
    const int r = known_answer_tests(c->side, &why);
    if (r == 0)
      c->book.enable("known-answer tests passed");
    else
      c->book.poison(why, r < 0);
  }
  if (c->book.state() != CacheBook::kEnabled)
    return fail(c->book.state() == CacheBook::kDisabled ? K3_HIP_E_CAPABILITY : K3_HIP_E_EXEC,
                "expert cache disabled: %s", c->book.reason().c_str());
  if (!c->book.budget_ready()) {
    size_t free_b = 0, total_b = 0;
    const hipError_t e = hipMemGetInfo(&free_b, &total_b);
    if (e != hipSuccess) return runtime_fail_locked(c, "cache budget hipMemGetInfo", e);
    c->book.establish_budget(free_b);
  }
  return K3_HIP_OK;
}

// Host copy of one pageable span into a pinned staging slot, split over a few
// threads: one thread copies ~10 GB/s, well under the host link's ~55 GB/s,
// so a single-threaded copy (as the reference's upload does,
// provider_cuda_moe.cpp:757-805) would bound every pageable miss.
constexpr int kStageCopyThreads = 8;
void staged_copy(uint8_t* dst, const uint8_t* src, uint64_t n) {
  const uint64_t piece = ((n + kStageCopyThreads - 1) / kStageCopyThreads + 4095) & ~uint64_t(4095);
  std::thread workers[kStageCopyThreads - 1];
  int spawned = 0;
  for (int t = 1; t < kStageCopyThreads; ++t) {
    const uint64_t b = (uint64_t)t * piece;
    if (b >= n) break;
    const uint64_t len = std::min(piece, n - b);
    workers[spawned++] = std::thread([=] { memcpy(dst + b, src + b, len); });
  }
  memcpy(dst, src, std::min(piece, n));
  for (int t = 0; t < spawned; ++t) workers[t].join();
}

bool pinned_host(const void* p) {
  hipPointerAttribute_t attr;
  memset(&attr, 0, sizeof(attr));
  if (hipPointerGetAttributes(&attr, p) != hipSuccess) {
    (void)hipGetLastError();
    return false;
  }
  return attr.type == hipMemoryTypeHost;
}

// Remember that the plan handed its spans to `stream` (release orders slot
// reuse after the work queued there).
void note_stream(K3HipCache* c, uint64_t plan_id, hipStream_t stream) {
  auto& v = c->plan_streams[plan_id];
  if (std::find(v.begin(), v.end(), stream) == v.end()) v.push_back(stream);
}

}  // namespace

extern "C" {

K3HipCache* k3_hip_cache_create(int device, uint64_t span_bytes, int capacity_experts,
                                int n_layers, int staging_slots) {
  if (span_bytes == 0 || capacity_experts < 0 || (uint64_t)capacity_experts > kCacheMaxExperts ||
      n_layers <= 0 || n_layers > 4096 || staging_slots < 0 || staging_slots > 16) {
    fail(K3_HIP_E_INVALID, "cache: invalid span/capacity/layers/staging");
    return nullptr;
  }
  if (k3_hip_moe_available(device) != 1) return nullptr;
  CachePolicy policy;
  policy.automatic = capacity_experts == 0;
  policy.capacity = (uint64_t)capacity_experts;
  K3HipCache* c = new K3HipCache(device, span_bytes, n_layers, policy);
  hipError_t e = hipSetDevice(device);
  if (e == hipSuccess) e = hipStreamCreateWithFlags(&c->side, hipStreamNonBlocking);
  for (int i = 0; e == hipSuccess && i < staging_slots; ++i) {
    uint8_t* p = nullptr;
    hipEvent_t ev = nullptr;
    e = hipHostMalloc(reinterpret_cast<void**>(&p), span_bytes, hipHostMallocDefault);
    if (e == hipSuccess) e = hipEventCreateWithFlags(&ev, hipEventDisableTiming);
    if (e == hipSuccess) {
      c->staging.push_back(p);
      c->staging_ready.push_back(ev);
      c->staging_used.push_back(false);
    }
  }
  if (e != hipSuccess) {
    (void)hipGetLastError();
    fail(K3_HIP_E_ALLOC, "cache allocation: %s", hipGetErrorString(e));
    k3_hip_cache_destroy(c);
    return nullptr;
  }
  return c;
}

void k3_hip_cache_destroy(K3HipCache* c) {
  if (!c) return;
  (void)hipSetDevice(c->device);
  if (c->side) (void)hipStreamSynchronize(c->side);
  for (auto& s : c->sdev) {
    for (auto& d : s.done) (void)hipEventSynchronize(d.second);
    if (s.ready) (void)hipEventDestroy(s.ready);
    for (auto& d : s.done) (void)hipEventDestroy(d.second);
  }
  for (hipEvent_t e : c->event_pool) (void)hipEventDestroy(e);
  for (size_t i = 0; i < c->staging.size(); ++i) {
    (void)hipEventDestroy(c->staging_ready[i]);
    (void)hipHostFree(c->staging[i]);
  }
  if (c->side) (void)hipStreamDestroy(c->side);
  for (uint8_t* p : c->seg_base) (void)hipFree(p);
  delete c;
}

int k3_hip_cache_configure(K3HipCache* c, const K3HipCachePolicyV1* p) {
  if (!c || !p || p->abi_version != 1 || p->struct_bytes != sizeof(K3HipCachePolicyV1) ||
      p->automatic_capacity > 1)
    return fail(K3_HIP_E_INVALID, "cache configure: invalid policy header");
  CachePolicy policy;
  policy.automatic = p->automatic_capacity == 1;
  policy.capacity = p->capacity_experts;
  policy.reserve_kind = p->reserve_kind;
  policy.reserve_value = p->reserve_value;
  std::lock_guard<std::mutex> lk(c->mu);
  if (const char* why = c->book.configure(policy))
    return fail(K3_HIP_E_INVALID, "cache configure: %s", why);
  return K3_HIP_OK;
}

int k3_hip_cache_budget(const K3HipCache* c, long long* five) {
  if (!c || !five) return fail(K3_HIP_E_INVALID, "cache budget: null argument");
  K3HipCache* m = const_cast<K3HipCache*>(c);
  std::lock_guard<std::mutex> lk(m->mu);
  five[0] = c->book.budget_ready() ? c->book.capacity() : -1;
  five[1] = c->book.allocated_slots();
  five[2] = (long long)c->book.budget_free();
  five[3] = (long long)c->book.budget_reserve();
  five[4] = c->book.rebuilds_left();
  return c->book.budget_ready() ? 1 : 0;
}

int k3_hip_cache_fail_allocations(K3HipCache* c, int count) {
  if (!c || count < 0) return fail(K3_HIP_E_INVALID, "cache fail allocations: invalid argument");
  std::lock_guard<std::mutex> lk(c->mu);
  c->book.fail_next_allocations(count);
  return K3_HIP_OK;
}

int k3_hip_cache_plan(K3HipCache* c, uint64_t plan_id, int layer, const uint16_t* ids, int n,
                      uint16_t* missing_ids, int* n_missing) {
  if (!c || plan_id == 0 || !ids || n <= 0 || !missing_ids || !n_missing)
    return fail(K3_HIP_E_INVALID, "cache plan: invalid arguments");
  if (layer < 0 || layer >= c->book.n_layers())
    return fail(K3_HIP_E_INVALID, "cache plan: layer %d outside [0, %d)", layer,
                c->book.n_layers());
  for (int i = 1; i < n; ++i)
    if (ids[i - 1] >= ids[i])
      return fail(K3_HIP_E_INVALID, "cache plan: ids must be canonical ascending IDs");
  std::lock_guard<std::mutex> lk(c->mu);
  if (c->book.has_plan(plan_id)) return fail(K3_HIP_E_INVALID, "cache plan: plan id already live");
  int rc = set_device(c);
  if (rc == K3_HIP_OK) rc = gate_locked(c);
  if (rc != K3_HIP_OK) return rc;
  if (n > c->book.capacity())
    return fail(K3_HIP_E_INVALID, "cache plan: %d experts exceed the capacity of %d", n,
                c->book.capacity());
  const CacheBook::Plan& p = c->book.plan(plan_id, layer, ids, n);
  for (size_t i = 0; i < p.missing.size(); ++i) missing_ids[i] = p.missing[i];
  *n_missing = (int)p.missing.size();
  return K3_HIP_OK;
}

int k3_hip_cache_fetch(K3HipCache* c, uint64_t plan_id, const uint8_t* const* sources,
                       int n_sources) {
  if (!c) return fail(K3_HIP_E_INVALID, "cache fetch: null cache");
  std::lock_guard<std::mutex> lk(c->mu);
  CacheBook::Plan* p = c->book.plan_of(plan_id);
  if (!p) return fail(K3_HIP_E_INVALID, "cache fetch: stale or unknown plan");
  if (!p->miss_slots.empty()) return fail(K3_HIP_E_INVALID, "cache fetch: plan already fetched");
  if (n_sources != (int)p->missing.size() || (n_sources > 0 && !sources))
    return fail(K3_HIP_E_INVALID, "cache fetch: %d sources for %zu misses", n_sources,
                p->missing.size());
  for (int i = 0; i < n_sources; ++i)
    if (!sources[i]) return fail(K3_HIP_E_INVALID, "cache fetch: null source %d", i);
  int rc = set_device(c);
  if (rc == K3_HIP_OK) rc = gate_locked(c);
  if (rc != K3_HIP_OK) return rc;
  for (int i = 0; i < n_sources; ++i) {
    bool evicted = false;
    const int slot = c->book.take_slot(*c, &evicted);
    if (slot == -1) {
      c->book.unadmit(*p);
      return fail(K3_HIP_E_ALLOC, "cache fetch: every slot (capacity %d) is pinned by live plans",
                  c->book.capacity());
    }
    if (slot == -2) {
      // Recoverable (provider_cuda_moe.cpp:630-653): undo this fetch, drain
      // the copy stream, rebuild within the bounded retries.
      c->book.unadmit(*p);
      const hipError_t d = hipStreamSynchronize(c->side);
      if (d != hipSuccess) return runtime_fail_locked(c, "cache drain after allocation failure", d);
      const bool alive = c->book.recover(*c, "device allocation of a cache segment failed");
      return fail(K3_HIP_E_ALLOC,
                  "recoverable expert cache allocation failure: the plan's hits stay pinned "
                  "(k3_hip_cache_materialize_plan) for the CPU path; %s",
                  alive ? "the cache re-measures its budget at the next plan"
                        : "the cache is now disabled");
    }
    if (slot < 0) {
      c->book.unadmit(*p);
      return runtime_fail_locked(c, "cache segment allocation", c->hook_error);
    }
    K3HipCache::SlotDev& s = c->sdev[slot];
    uint8_t* dst = c->addr(slot);
    hipError_t e = hipSuccess;
    // Kernels queued on caller streams may still read the slot's previous
    // expert: the copy waits for every release point recorded for it.
    for (auto& d : s.done) {
      if (e == hipSuccess) e = hipStreamWaitEvent(c->side, d.second, 0);
      c->event_pool.push_back(d.second);
    }
    s.done.clear();
    if (e != hipSuccess) return runtime_fail_locked(c, "cache fetch wait for slot reuse", e);
    if (pinned_host(sources[i]) || c->staging.empty()) {
      e = hipMemcpyAsync(dst, sources[i], c->span, hipMemcpyHostToDevice, c->side);
    } else {
      const int k = c->staging_cursor;
      c->staging_cursor = (k + 1) % (int)c->staging.size();
      if (c->staging_used[k]) {
        e = hipEventSynchronize(c->staging_ready[k]);
        if (e != hipSuccess) return runtime_fail_locked(c, "cache staging wait", e);
      }
      staged_copy(c->staging[k], sources[i], c->span);
      e = hipMemcpyAsync(dst, c->staging[k], c->span, hipMemcpyHostToDevice, c->side);
      if (e == hipSuccess) e = hipEventRecord(c->staging_ready[k], c->side);
      c->staging_used[k] = true;
    }
    if (e == hipSuccess) e = hipEventRecord(s.ready, c->side);
    if (e != hipSuccess) {
      (void)hipStreamSynchronize(c->side);
      return runtime_fail_locked(c, "cache fetch copy", e);
    }
    s.has_ready = true;
    c->book.admit(*p, slot);
    c->uploaded += (long long)c->span;
  }
  return K3_HIP_OK;
}

int k3_hip_cache_resolve(K3HipCache* c, uint64_t plan_id, const uint16_t* ids, int n,
                         const uint8_t** device_spans, void* stream) {
  if (!c || !ids || n < 0 || (n > 0 && !device_spans))
    return fail(K3_HIP_E_INVALID, "cache resolve: invalid arguments");
  std::lock_guard<std::mutex> lk(c->mu);
  CacheBook::Plan* p = c->book.plan_of(plan_id);
  if (!p) return fail(K3_HIP_E_INVALID, "cache resolve: stale or unknown plan");
  int rc = set_device(c);
  if (rc == K3_HIP_OK) rc = gate_locked(c);
  if (rc != K3_HIP_OK) return rc;
  hipStream_t st = static_cast<hipStream_t>(stream);
  note_stream(c, plan_id, st);
  for (int i = 0; i < n; ++i) {
    const int slot = CacheBook::plan_slot(*p, ids[i]);
    if (slot == -2) return fail(K3_HIP_E_INVALID, "cache resolve: expert %d outside the plan", ids[i]);
    if (slot < 0) return fail(K3_HIP_E_INVALID, "cache resolve: expert %d not fetched", ids[i]);
    K3HipCache::SlotDev& s = c->sdev[slot];
    if (s.has_ready) {
      const hipError_t e = hipStreamWaitEvent(st, s.ready, 0);
      if (e != hipSuccess) return runtime_fail_locked(c, "cache resolve wait", e);
    }
    device_spans[i] = c->addr(slot);
  }
  return K3_HIP_OK;
}

int k3_hip_cache_ready_subset(K3HipCache* c, uint64_t plan_id, const uint16_t* ids, int n,
                              const uint8_t** device_spans) {
  return k3_hip_cache_ready_subset_v2(c, plan_id, ids, n, device_spans, nullptr);
}

int k3_hip_cache_ready_subset_v2(K3HipCache* c, uint64_t plan_id, const uint16_t* ids, int n,
                                 const uint8_t** device_spans, void* stream) {
  if (!c || !ids || n < 0 || (n > 0 && !device_spans))
    return fail(K3_HIP_E_INVALID, "cache ready: invalid arguments");
  std::lock_guard<std::mutex> lk(c->mu);
  CacheBook::Plan* p = c->book.plan_of(plan_id);
  if (!p) return fail(K3_HIP_E_INVALID, "cache ready: stale or unknown plan");
  int rc = set_device(c);
  if (rc == K3_HIP_OK) rc = gate_locked(c);
  if (rc != K3_HIP_OK) return rc;
  note_stream(c, plan_id, static_cast<hipStream_t>(stream));
  int ready = 0;
  for (int i = 0; i < n; ++i) {
    device_spans[i] = nullptr;
    const int slot = CacheBook::plan_slot(*p, ids[i]);
    if (slot < 0) continue;
    K3HipCache::SlotDev& s = c->sdev[slot];
    if (s.has_ready) {
      const hipError_t q = hipEventQuery(s.ready);
      if (q == hipErrorNotReady) {
        (void)hipGetLastError();
        continue;
      }
      if (q != hipSuccess) return runtime_fail_locked(c, "cache ready query", q);
    }
    device_spans[i] = c->addr(slot);
    ++ready;
  }
  return ready;
}

void k3_hip_cache_release(K3HipCache* c, uint64_t plan_id) {
  if (!c) return;
  std::lock_guard<std::mutex> lk(c->mu);
  CacheBook::Plan* p = c->book.plan_of(plan_id);
  if (!p) return;
  (void)set_device(c);
  auto sit = c->plan_streams.find(plan_id);
  auto mark = [&](int slot) {
    if (slot < 0 || sit == c->plan_streams.end()) return;
    // Everything the caller queued on the plan's streams so far may read the
    // slot; a later copy into it waits for these points.
    K3HipCache::SlotDev& s = c->sdev[slot];
    for (hipStream_t st : sit->second) {
      hipEvent_t ev = nullptr;
      for (auto& d : s.done)
        if (d.first == st) ev = d.second;
      const bool fresh = ev == nullptr;
      if (fresh) ev = c->take_event();
      hipError_t e = ev ? hipEventRecord(ev, st) : hipErrorOutOfMemory;
      if (e == hipSuccess) {
        if (fresh) s.done.emplace_back(st, ev);
        continue;
      }
      // No reuse point for this stream: the host waits for the stream
      // instead, so nothing queued there can still read the slot when it is
      // refilled; if that fails too, the cache fails closed.
      (void)hipGetLastError();
      if (ev && fresh) c->event_pool.push_back(ev);
      if ((e = hipStreamSynchronize(st)) != hipSuccess) {
        (void)runtime_fail_locked(c, "cache release: no reuse point for a stream", e);
        return;
      }
    }
  };
  for (int s : p->hit_slots) mark(s);
  for (int s : p->miss_slots) mark(s);
  if (sit != c->plan_streams.end()) c->plan_streams.erase(sit);
  c->book.release(plan_id);
}

int k3_hip_cache_materialize_plan(K3HipCache* c, uint64_t plan_id, uint16_t* ids_out,
                                  int ids_capacity, uint8_t* host_out, uint64_t host_bytes,
                                  int* n_out) {
  if (!c || !ids_out || !n_out || (host_bytes > 0 && !host_out))
    return fail(K3_HIP_E_INVALID, "cache materialize: invalid arguments");
  std::lock_guard<std::mutex> lk(c->mu);
  CacheBook::Plan* p = c->book.plan_of(plan_id);
  if (!p) return fail(K3_HIP_E_INVALID, "cache materialize: stale or unknown plan");
  const auto hits = c->book.plan_hits(*p);
  if ((int)hits.size() > ids_capacity || host_bytes < (uint64_t)hits.size() * c->span)
    return fail(K3_HIP_E_INVALID, "cache materialize: room for %d ids / %llu bytes, the plan pins %zu",
                ids_capacity, (unsigned long long)host_bytes, hits.size());
  int rc = set_device(c);
  if (rc != K3_HIP_OK) return rc;
  for (size_t i = 0; i < hits.size(); ++i) {
    K3HipCache::SlotDev& s = c->sdev[hits[i].second];
    hipError_t e = s.has_ready ? hipEventSynchronize(s.ready) : hipSuccess;
    if (e == hipSuccess)
      e = hipMemcpy(host_out + i * c->span, c->addr(hits[i].second), c->span,
                    hipMemcpyDeviceToHost);
    if (e != hipSuccess) return runtime_fail_locked(c, "cache materialize copy", e);
    ids_out[i] = hits[i].first;
  }
  *n_out = (int)hits.size();
  return K3_HIP_OK;
}

int k3_hip_cache_state(const K3HipCache* c, char* reason, uint64_t reason_capacity) {
  if (!c) return fail(K3_HIP_E_INVALID, "cache state: null cache");
  K3HipCache* m = const_cast<K3HipCache*>(c);
  std::lock_guard<std::mutex> lk(m->mu);
  if (reason && reason_capacity > 0) {
    const std::string& r = c->book.reason();
    const size_t n = std::min<size_t>(r.size(), (size_t)reason_capacity - 1);
    memcpy(reason, r.data(), n);
    reason[n] = 0;
  }
  switch (c->book.state()) {
    case CacheBook::kEnabled: return 1;
    case CacheBook::kUnqualified: return 0;
    case CacheBook::kDisabled: return K3_HIP_E_CAPABILITY;
    default: return K3_HIP_E_EXEC;
  }
}

void k3_hip_cache_poison(K3HipCache* c, const char* failure) {
  if (!c) return;
  std::lock_guard<std::mutex> lk(c->mu);
  c->book.poison(std::string("poisoned by caller: ") + (failure ? failure : "no detail"), true);
}

void k3_hip_cache_stats(const K3HipCache* c, long long* six) {
  if (!c || !six) return;
  K3HipCache* m = const_cast<K3HipCache*>(c);
  std::lock_guard<std::mutex> lk(m->mu);
  six[0] = c->book.hits();
  six[1] = c->book.misses();
  six[2] = c->book.evictions();
  six[3] = c->book.resident();
  six[4] = c->book.budget_ready() ? c->book.capacity() : (long long)c->book.policy().capacity;
  six[5] = c->uploaded;
}

int k3_hip_cache_read_back(K3HipCache* c, int layer, uint16_t id, uint8_t* host_out,
                           uint64_t bytes) {
  if (!c || !host_out || bytes != c->span || layer < 0 || layer >= c->book.n_layers())
    return fail(K3_HIP_E_INVALID, "cache read back: invalid arguments");
  std::lock_guard<std::mutex> lk(c->mu);
  const int slot = c->book.find(layer, id);
  if (slot < 0)
    return fail(K3_HIP_E_INVALID, "cache read back: expert %d of layer %d is not resident", id, layer);
  int rc = set_device(c);
  if (rc != K3_HIP_OK) return rc;
  K3HipCache::SlotDev& s = c->sdev[slot];
  hipError_t e = s.has_ready ? hipEventSynchronize(s.ready) : hipSuccess;
  if (e == hipSuccess) e = hipMemcpy(host_out, c->addr(slot), bytes, hipMemcpyDeviceToHost);
  return e == hipSuccess ? K3_HIP_OK : hip_fail("cache read back", e);
}

}  // extern "C"
