// HBM expert cache: C counterpart of CudaMoeExpertCache
// (native/provider_gate/provider_cuda_moe.{h,cpp}).
//
// * One slab of capacity x span bytes in HBM; a slot holds one expert span.
// * Entries live in per-layer strata with a global recency clock; eviction picks
//   the globally least-recent entry that no live plan pins
//   (provider_cuda_moe.cpp:707-747).
// * plan() snapshots hits before any miss can be admitted, pinning them for the
//   plan's lifetime (:963-1008).
// * fetch() admits misses with hipMemcpyAsync on the cache's own side stream,
//   so copies overlap compute on the caller's stream; each slot records a ready
//   event that resolve() makes the caller's stream wait on.  The reference
//   copies on the execution stream through two pinned slabs (:757-805); here
//   pinned sources are copied directly and pageable sources go through a ring
//   of pinned staging slots.
// * Because copies run on their own stream, a slot's previous contents may
//   still be read by kernels the caller queued before release(): release()
//   records a per-slot event on the stream the plan was resolved on, and a
//   copy into an evicted slot first makes the side stream wait on it.
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
#include <unordered_map>
#include <vector>

#include "k3_internal.h"

using namespace k3;

struct K3HipCache {
  struct Slot {
    int layer = -1;
    int id = -1;
    uint64_t last_use = 0;
    int pins = 0;
    hipEvent_t ready = nullptr;
    bool has_event = false;
    hipEvent_t done = nullptr;  // recorded at release on the plan's stream
    bool has_done = false;
  };
  struct Plan {
    int layer = 0;
    hipStream_t stream = nullptr;   // set by resolve()
    bool resolved = false;
    std::vector<uint16_t> ids;      // canonical ascending
    std::vector<int> hit_slots;     // pinned at plan time
    std::vector<uint16_t> missing;  // ascending
    std::vector<int> miss_slots;    // filled by fetch
  };

  std::mutex mu;
  int device = 0;
  uint64_t span = 0, slot_bytes = 0;
  int capacity = 0;
  int n_layers = 0;
  uint8_t* slab = nullptr;
  hipStream_t side = nullptr;
  std::vector<Slot> slots;
  std::vector<std::unordered_map<int, int>> strata;  // layer -> id -> slot
  std::map<uint64_t, Plan> plans;
  uint64_t clock = 0;
  std::vector<uint8_t*> staging;
  std::vector<hipEvent_t> staging_ready;
  std::vector<bool> staging_used;
  int staging_cursor = 0;
  long long hits = 0, misses = 0, evictions = 0, uploaded = 0;
  enum State { kUnqualified = 0, kEnabled = 1, kDisabled = 2, kTerminal = 3 };
  int state = kUnqualified;
  std::string reason = "not yet qualified";

  int resident() const {
    int n = 0;
    for (const Slot& s : slots) n += s.id >= 0;
    return n;
  }
};

namespace {

int set_device(K3HipCache* c) {
  const hipError_t e = hipSetDevice(c->device);
  return e == hipSuccess ? K3_HIP_OK : hip_fail("cache hipSetDevice", e);
}

// Free slot, else the globally least-recent unpinned slot (evicted).
int take_slot(K3HipCache* c) {
  int victim = -1;
  for (int i = 0; i < c->capacity; ++i) {
    const K3HipCache::Slot& s = c->slots[i];
    if (s.id < 0 && s.pins == 0) return i;
    if (s.pins == 0 && (victim < 0 || s.last_use < c->slots[victim].last_use)) victim = i;
  }
  if (victim >= 0) {
    K3HipCache::Slot& s = c->slots[victim];
    c->strata[s.layer].erase(s.id);
    s.layer = s.id = -1;
    ++c->evictions;
  }
  return victim;
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

// Fail closed: drop every resident entry and keep the reason.
void poison_locked(K3HipCache* c, const std::string& why, bool terminal) {
  c->state = terminal || c->state == K3HipCache::kTerminal ? K3HipCache::kTerminal
                                                          : K3HipCache::kDisabled;
  c->reason = why;
  for (auto& s : c->slots) s.layer = s.id = -1;
  for (auto& m : c->strata) m.clear();
}

// The gate every plan / fetch / resolve call passes (qualifies on first use).
int gate_locked(K3HipCache* c) {
  if (c->state == K3HipCache::kUnqualified) {
    std::string why;
    const int r = known_answer_tests(c->side, &why);
    if (r == 0) {
      c->state = K3HipCache::kEnabled;
      c->reason = "known-answer tests passed";
    } else {
      poison_locked(c, why, r < 0);
    }
  }
  if (c->state == K3HipCache::kEnabled) return K3_HIP_OK;
  return fail(c->state == K3HipCache::kDisabled ? K3_HIP_E_CAPABILITY : K3_HIP_E_EXEC,
              "expert cache disabled: %s", c->reason.c_str());
}

// A HIP failure inside a cache call: terminal.
int runtime_fail_locked(K3HipCache* c, const char* what, hipError_t e) {
  (void)hipGetLastError();
  poison_locked(c, std::string(what) + ": " + hipGetErrorString(e), true);
  return fail(K3_HIP_E_EXEC, "expert cache disabled after runtime failure: %s",
              c->reason.c_str());
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

}  // namespace

extern "C" {

K3HipCache* k3_hip_cache_create(int device, uint64_t span_bytes, int capacity_experts,
                                int n_layers, int staging_slots) {
  if (span_bytes == 0 || capacity_experts <= 0 || n_layers <= 0 || n_layers > 4096 ||
      staging_slots < 0 || staging_slots > 16) {
    fail(K3_HIP_E_INVALID, "cache: invalid span/capacity/layers/staging");
    return nullptr;
  }
  if (k3_hip_moe_available(device) != 1) return nullptr;
  K3HipCache* c = new K3HipCache();
  c->device = device;
  c->span = span_bytes;
  c->slot_bytes = (span_bytes + 4095) & ~uint64_t(4095);
  c->capacity = capacity_experts;
  c->n_layers = n_layers;
  c->slots.resize(capacity_experts);
  c->strata.resize(n_layers);
  hipError_t e = hipSetDevice(device);
  if (e == hipSuccess) e = hipMalloc(reinterpret_cast<void**>(&c->slab), c->slot_bytes * capacity_experts);
  if (e == hipSuccess) e = hipStreamCreateWithFlags(&c->side, hipStreamNonBlocking);
  for (int i = 0; e == hipSuccess && i < capacity_experts; ++i) {
    e = hipEventCreateWithFlags(&c->slots[i].ready, hipEventDisableTiming);
    if (e == hipSuccess) e = hipEventCreateWithFlags(&c->slots[i].done, hipEventDisableTiming);
  }
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
  for (auto& s : c->slots) {
    if (s.ready) (void)hipEventDestroy(s.ready);
    if (s.done) (void)hipEventDestroy(s.done);
  }
  for (size_t i = 0; i < c->staging.size(); ++i) {
    (void)hipEventDestroy(c->staging_ready[i]);
    (void)hipHostFree(c->staging[i]);
  }
  if (c->side) (void)hipStreamDestroy(c->side);
  if (c->slab) (void)hipFree(c->slab);
  delete c;
}

int k3_hip_cache_plan(K3HipCache* c, uint64_t plan_id, int layer, const uint16_t* ids, int n,
                      uint16_t* missing_ids, int* n_missing) {
  if (!c || plan_id == 0 || !ids || n <= 0 || n > c->capacity || !missing_ids || !n_missing)
    return fail(K3_HIP_E_INVALID, "cache plan: invalid arguments (n must be in [1, capacity])");
  if (layer < 0 || layer >= c->n_layers)
    return fail(K3_HIP_E_INVALID, "cache plan: layer %d outside [0, %d)", layer, c->n_layers);
  for (int i = 1; i < n; ++i)
    if (ids[i - 1] >= ids[i])
      return fail(K3_HIP_E_INVALID, "cache plan: ids must be canonical ascending IDs");
  std::lock_guard<std::mutex> lk(c->mu);
  if (c->plans.count(plan_id)) return fail(K3_HIP_E_INVALID, "cache plan: plan id already live");
  int rc = set_device(c);
  if (rc == K3_HIP_OK) rc = gate_locked(c);
  if (rc != K3_HIP_OK) return rc;
  K3HipCache::Plan p;
  p.layer = layer;
  p.ids.assign(ids, ids + n);
  for (int i = 0; i < n; ++i) {
    auto it = c->strata[layer].find(ids[i]);
    if (it != c->strata[layer].end()) {
      K3HipCache::Slot& s = c->slots[it->second];
      s.last_use = ++c->clock;
      ++s.pins;
      p.hit_slots.push_back(it->second);
      ++c->hits;
    } else {
      p.missing.push_back(ids[i]);
      p.hit_slots.push_back(-1);
      ++c->misses;
    }
  }
  for (size_t i = 0; i < p.missing.size(); ++i) missing_ids[i] = p.missing[i];
  *n_missing = (int)p.missing.size();
  c->plans.emplace(plan_id, std::move(p));
  return K3_HIP_OK;
}

int k3_hip_cache_fetch(K3HipCache* c, uint64_t plan_id, const uint8_t* const* sources,
                       int n_sources) {
  if (!c) return fail(K3_HIP_E_INVALID, "cache fetch: null cache");
  std::lock_guard<std::mutex> lk(c->mu);
  auto pit = c->plans.find(plan_id);
  if (pit == c->plans.end()) return fail(K3_HIP_E_INVALID, "cache fetch: stale or unknown plan");
  K3HipCache::Plan& p = pit->second;
  if (!p.miss_slots.empty()) return fail(K3_HIP_E_INVALID, "cache fetch: plan already fetched");
  if (n_sources != (int)p.missing.size() || (n_sources > 0 && !sources))
    return fail(K3_HIP_E_INVALID, "cache fetch: %d sources for %zu misses", n_sources,
                p.missing.size());
  int rc = set_device(c);
  if (rc == K3_HIP_OK) rc = gate_locked(c);
  if (rc != K3_HIP_OK) return rc;
  for (int i = 0; i < n_sources; ++i) {
    if (!sources[i]) return fail(K3_HIP_E_INVALID, "cache fetch: null source %d", i);
    const int slot = take_slot(c);
    if (slot < 0) return fail(K3_HIP_E_ALLOC, "cache fetch: every slot is pinned by live plans");
    K3HipCache::Slot& s = c->slots[slot];
    uint8_t* dst = c->slab + (uint64_t)slot * c->slot_bytes;
    hipError_t e = hipSuccess;
    // Kernels queued on a caller stream may still read the slot's previous
    // expert: the copy waits for the release point of its last plan.
    if (s.has_done) {
      e = hipStreamWaitEvent(c->side, s.done, 0);
      if (e != hipSuccess) return runtime_fail_locked(c, "cache fetch wait for slot reuse", e);
    }
    if (pinned_host(sources[i]) || c->staging.empty()) {
      e = hipMemcpyAsync(dst, sources[i], c->span, hipMemcpyHostToDevice, c->side);
    } else {
      const int k = c->staging_cursor;
      c->staging_cursor = (k + 1) % (int)c->staging.size();
      if (c->staging_used[k]) {
        e = hipEventSynchronize(c->staging_ready[k]);
        if (e != hipSuccess) return runtime_fail_locked(c, "cache staging wait", e);
      }
      memcpy(c->staging[k], sources[i], c->span);
      e = hipMemcpyAsync(dst, c->staging[k], c->span, hipMemcpyHostToDevice, c->side);
      if (e == hipSuccess) e = hipEventRecord(c->staging_ready[k], c->side);
      c->staging_used[k] = true;
    }
    if (e == hipSuccess) e = hipEventRecord(s.ready, c->side);
    if (e != hipSuccess) {
      (void)hipStreamSynchronize(c->side);
      return runtime_fail_locked(c, "cache fetch copy", e);
    }
    s.has_event = true;
    s.layer = p.layer;
    s.id = p.missing[i];
    s.last_use = ++c->clock;
    ++s.pins;
    c->strata[p.layer][s.id] = slot;
    p.miss_slots.push_back(slot);
    c->uploaded += (long long)c->span;
  }
  return K3_HIP_OK;
}

static int plan_slot(const K3HipCache::Plan& p, uint16_t id) {
  const auto it = std::lower_bound(p.ids.begin(), p.ids.end(), id);
  if (it == p.ids.end() || *it != id) return -2;
  const size_t idx = (size_t)(it - p.ids.begin());
  if (p.hit_slots[idx] >= 0) return p.hit_slots[idx];
  const auto mt = std::lower_bound(p.missing.begin(), p.missing.end(), id);
  const size_t mi = (size_t)(mt - p.missing.begin());
  return mi < p.miss_slots.size() ? p.miss_slots[mi] : -1;
}

int k3_hip_cache_resolve(K3HipCache* c, uint64_t plan_id, const uint16_t* ids, int n,
                         const uint8_t** device_spans, void* stream) {
  if (!c || !ids || n < 0 || (n > 0 && !device_spans))
    return fail(K3_HIP_E_INVALID, "cache resolve: invalid arguments");
  std::lock_guard<std::mutex> lk(c->mu);
  auto pit = c->plans.find(plan_id);
  if (pit == c->plans.end()) return fail(K3_HIP_E_INVALID, "cache resolve: stale or unknown plan");
  int rc = set_device(c);
  if (rc == K3_HIP_OK) rc = gate_locked(c);
  if (rc != K3_HIP_OK) return rc;
  pit->second.stream = static_cast<hipStream_t>(stream);
  pit->second.resolved = true;
  for (int i = 0; i < n; ++i) {
    const int slot = plan_slot(pit->second, ids[i]);
    if (slot == -2) return fail(K3_HIP_E_INVALID, "cache resolve: expert %d outside the plan", ids[i]);
    if (slot < 0) return fail(K3_HIP_E_INVALID, "cache resolve: expert %d not fetched", ids[i]);
    K3HipCache::Slot& s = c->slots[slot];
    if (s.has_event) {
      const hipError_t e = hipStreamWaitEvent(static_cast<hipStream_t>(stream), s.ready, 0);
      if (e != hipSuccess) return runtime_fail_locked(c, "cache resolve wait", e);
    }
    device_spans[i] = c->slab + (uint64_t)slot * c->slot_bytes;
  }
  return K3_HIP_OK;
}

int k3_hip_cache_ready_subset(K3HipCache* c, uint64_t plan_id, const uint16_t* ids, int n,
                              const uint8_t** device_spans) {
  if (!c || !ids || n < 0 || (n > 0 && !device_spans))
    return fail(K3_HIP_E_INVALID, "cache ready: invalid arguments");
  std::lock_guard<std::mutex> lk(c->mu);
  auto pit = c->plans.find(plan_id);
  if (pit == c->plans.end()) return fail(K3_HIP_E_INVALID, "cache ready: stale or unknown plan");
  int rc = set_device(c);
  if (rc == K3_HIP_OK) rc = gate_locked(c);
  if (rc != K3_HIP_OK) return rc;
  int ready = 0;
  for (int i = 0; i < n; ++i) {
    device_spans[i] = nullptr;
    const int slot = plan_slot(pit->second, ids[i]);
    if (slot < 0) continue;
    K3HipCache::Slot& s = c->slots[slot];
    if (s.has_event) {
      const hipError_t q = hipEventQuery(s.ready);
      if (q == hipErrorNotReady) {
        (void)hipGetLastError();
        continue;
      }
      if (q != hipSuccess) return runtime_fail_locked(c, "cache ready query", q);
    }
    device_spans[i] = c->slab + (uint64_t)slot * c->slot_bytes;
    ++ready;
  }
  return ready;
}

void k3_hip_cache_release(K3HipCache* c, uint64_t plan_id) {
  if (!c) return;
  std::lock_guard<std::mutex> lk(c->mu);
  auto pit = c->plans.find(plan_id);
  if (pit == c->plans.end()) return;
  K3HipCache::Plan& p = pit->second;
  (void)set_device(c);
  auto unpin = [&](int s) {
    if (s < 0) return;
    K3HipCache::Slot& slot = c->slots[s];
    // Everything the caller queued on the plan's stream so far may read the
    // slot; a later copy into it waits for this point.
    if (p.resolved) {
      if (hipEventRecord(slot.done, p.stream) == hipSuccess)
        slot.has_done = true;
      else
        (void)hipGetLastError();
    }
    if (slot.pins > 0) --slot.pins;
  };
  for (int s : p.hit_slots) unpin(s);
  for (int s : p.miss_slots) unpin(s);
  c->plans.erase(pit);
}

int k3_hip_cache_state(const K3HipCache* c, char* reason, uint64_t reason_capacity) {
  if (!c) return fail(K3_HIP_E_INVALID, "cache state: null cache");
  K3HipCache* m = const_cast<K3HipCache*>(c);
  std::lock_guard<std::mutex> lk(m->mu);
  if (reason && reason_capacity > 0) {
    const size_t n = std::min<size_t>(c->reason.size(), (size_t)reason_capacity - 1);
    memcpy(reason, c->reason.data(), n);
    reason[n] = 0;
  }
  switch (c->state) {
    case K3HipCache::kEnabled: return 1;
    case K3HipCache::kUnqualified: return 0;
    case K3HipCache::kDisabled: return K3_HIP_E_CAPABILITY;
    default: return K3_HIP_E_EXEC;
  }
}

void k3_hip_cache_poison(K3HipCache* c, const char* failure) {
  if (!c) return;
  std::lock_guard<std::mutex> lk(c->mu);
  poison_locked(c, std::string("poisoned by caller: ") + (failure ? failure : "no detail"), true);
}

void k3_hip_cache_stats(const K3HipCache* c, long long* six) {
  if (!c || !six) return;
  K3HipCache* m = const_cast<K3HipCache*>(c);
  std::lock_guard<std::mutex> lk(m->mu);
  six[0] = c->hits;
  six[1] = c->misses;
  six[2] = c->evictions;
  six[3] = c->resident();
  six[4] = c->capacity;
  six[5] = c->uploaded;
}

int k3_hip_cache_read_back(K3HipCache* c, int layer, uint16_t id, uint8_t* host_out,
                           uint64_t bytes) {
  if (!c || !host_out || bytes != c->span || layer < 0 || layer >= c->n_layers)
    return fail(K3_HIP_E_INVALID, "cache read back: invalid arguments");
  std::lock_guard<std::mutex> lk(c->mu);
  auto it = c->strata[layer].find(id);
  if (it == c->strata[layer].end())
    return fail(K3_HIP_E_INVALID, "cache read back: expert %d of layer %d is not resident", id, layer);
  int rc = set_device(c);
  if (rc != K3_HIP_OK) return rc;
  K3HipCache::Slot& s = c->slots[it->second];
  hipError_t e = s.has_event ? hipEventSynchronize(s.ready) : hipSuccess;
  if (e == hipSuccess)
    e = hipMemcpy(host_out, c->slab + (uint64_t)it->second * c->slot_bytes, bytes,
                  hipMemcpyDeviceToHost);
  return e == hipSuccess ? K3_HIP_OK : hip_fail("cache read back", e);
}

}  // extern "C"
