// Host bookkeeping of the HBM expert cache (k3_cache.cpp), free of device
// calls so the same code runs in the library and in a CPU test
// (tests/c/cache_book_test.cpp): capacity policy and budget, slots in
// device segments, per-layer strata with one global recency clock, plans that
// pin their hits, the fail-closed state and the bounded recovery from an
// allocation failure.  Counterparts: CudaMoeCachePolicy / validate_cache_policy
// / clamp_cache_capacity / establish_budget / evict_global_lru /
// rebuild_after_memory_pressure / poison (provider_cuda_moe.h:16-33,
// provider_cuda_moe.cpp:60-95, :496-567, :668-747).
//
// Device work stays with the caller through Hooks: allocating and freeing a
// segment of slots, and a host-side wait until nothing still reads a slot.
// Every method expects the caller's lock to be held.
#pragma once

#include <stdint.h>

#include <algorithm>
#include <map>
#include <string>
#include <unordered_map>
#include <vector>

namespace k3 {

enum CacheReserveKind : uint32_t { kReserveAuto = 0, kReserveBytes = 1, kReserveRatioPpm = 2 };

struct CachePolicy {
  bool automatic = true;      // capacity = what the budget holds
  uint64_t capacity = 0;      // requested experts (automatic: must be 0)
  uint32_t reserve_kind = kReserveAuto;
  uint64_t reserve_value = 0;  // Auto: 0; Bytes: bytes; RatioPpm: parts per million of free
};

// Most slots a cache may hold: 92 layer strata x 16 routed experts, the
// reference's kCudaMaximumExperts (provider_cuda_moe.cpp:55-57), enforced by
// both the policy check and the budget clamp as there.
constexpr uint64_t kCacheMaxExperts = 92 * 16;
// Recoveries from allocation failure before the cache disables itself
// (rebuilds_remaining, provider_cuda_moe.cpp:879).
constexpr int kCacheRebuilds = 2;

// nullptr when the policy is inside its bounds (validate_cache_policy,
// provider_cuda_moe.cpp:60-74), else the reason.
inline const char* cache_policy_error(const CachePolicy& p) {
  if (p.automatic && p.capacity != 0) return "automatic capacity with a requested expert count";
  if (!p.automatic && p.capacity > kCacheMaxExperts) return "requested capacity above the maximum";
  if (p.reserve_kind == kReserveAuto && p.reserve_value != 0) return "automatic reserve with a value";
  if (p.reserve_kind == kReserveRatioPpm && p.reserve_value > 1000000)
    return "reserve ratio above 1,000,000 ppm";
  if (p.reserve_kind != kReserveAuto && p.reserve_kind != kReserveBytes &&
      p.reserve_kind != kReserveRatioPpm)
    return "unknown reserve kind";
  return nullptr;
}

// Device bytes the budget leaves free (establish_budget,
// provider_cuda_moe.cpp:668-705): Auto max(2 GiB, free / 5), Bytes the value,
// RatioPpm free x value / 1e6 in exact integer arithmetic.
inline uint64_t cache_reserve_bytes(const CachePolicy& p, uint64_t free_bytes) {
  switch (p.reserve_kind) {
    case kReserveBytes:
      return p.reserve_value;
    case kReserveRatioPpm: {
      const uint64_t scale = 1000000, ratio = p.reserve_value;
      return (free_bytes / scale) * ratio + ((free_bytes % scale) * ratio) / scale;
    }
    default:
      return std::max<uint64_t>(uint64_t(2) << 30, free_bytes / 5);
  }
}

// Slots the budget allows (clamp_cache_capacity, provider_cuda_moe.cpp:76-93).
inline uint64_t cache_clamp_capacity(uint64_t free_bytes, uint64_t reserve_bytes, bool automatic,
                                     uint64_t requested, uint64_t slot_bytes) {
  if (slot_bytes == 0) return 0;
  const uint64_t safe_bytes = free_bytes > reserve_bytes ? free_bytes - reserve_bytes : 0;
  const uint64_t safe = std::min<uint64_t>(kCacheMaxExperts, safe_bytes / slot_bytes);
  return automatic ? safe : std::min(safe, requested);
}

class CacheBook {
 public:
  struct Hooks {
    // Make segment `seg` (the next segment; its slots follow the previous
    // segments' in index order) of `bytes` device bytes: 0 ok, 1 out of
    // memory (recoverable), -1 any other failure.
    virtual int alloc_segment(int seg, uint64_t bytes) = 0;
    virtual void free_segment(int seg) = 0;
    // Returns once no queued work still reads `slot` (host-side wait).
    virtual void wait_slot_idle(int slot) = 0;
    virtual ~Hooks() = default;
  };
  struct Slot {
    int layer = -1;
    int id = -1;
    uint64_t last_use = 0;
    int pins = 0;
  };
  struct Plan {
    int layer = 0;
    std::vector<uint16_t> ids;      // canonical ascending
    std::vector<int> hit_slots;     // per id: slot pinned at plan time, or -1
    std::vector<uint16_t> missing;  // ascending
    std::vector<int> miss_slots;    // filled by admissions, in `missing` order
  };
  enum State { kUnqualified = 0, kEnabled = 1, kDisabled = 2, kTerminal = 3 };

  CacheBook(uint64_t slot_bytes, int n_layers, int seg_slots, const CachePolicy& policy)
      : slot_bytes_(slot_bytes), seg_slots_(std::max(1, seg_slots)), policy_(policy),
        strata_(n_layers) {}

  // ------------------------------------------------------------ policy
  // Before first use only (CudaMoeExpertCache::configure, :571-578).
  const char* configure(const CachePolicy& p) {
    if (frozen_) return "the cache policy is frozen after first use";
    if (const char* why = cache_policy_error(p)) return why;
    policy_ = p;
    return nullptr;
  }
  void freeze() { frozen_ = true; }
  bool frozen() const { return frozen_; }
  const CachePolicy& policy() const { return policy_; }

  bool budget_ready() const { return budget_ready_; }
  // Measure the budget from the device's free bytes (establish_budget).  The
  // slots already allocated stay usable; capacity never drops below them
  // while they hold pinned entries.
  void establish_budget(uint64_t free_bytes) {
    freeze();
    budget_free_ = free_bytes;
    budget_reserve_ = cache_reserve_bytes(policy_, free_bytes);
    // Memory this cache already holds counts towards what it may keep.
    const uint64_t held = (uint64_t)allocated_slots() * slot_bytes_;
    capacity_ = (int)cache_clamp_capacity(free_bytes + held, budget_reserve_, policy_.automatic,
                                          policy_.capacity, slot_bytes_);
    budget_ready_ = true;
  }
  int capacity() const { return capacity_; }
  uint64_t budget_free() const { return budget_free_; }
  uint64_t budget_reserve() const { return budget_reserve_; }
  int rebuilds_left() const { return rebuilds_left_; }
  int allocated_slots() const { return (int)slots_.size(); }
  int seg_slots() const { return seg_slots_; }
  uint64_t slot_bytes() const { return slot_bytes_; }

  // ------------------------------------------------------------ state
  int state() const { return state_; }
  const std::string& reason() const { return reason_; }
  void enable(const std::string& why) {
    state_ = kEnabled;
    reason_ = why;
  }
  // Disable (mismatch, exhausted recovery: the caller's CPU path) or make
  // terminal; either way every resident entry is forgotten (poison,
  // provider_cuda_moe.cpp:517-533).
  void poison(const std::string& why, bool terminal) {
    state_ = terminal || state_ == kTerminal ? kTerminal : kDisabled;
    reason_ = why;
    for (Slot& s : slots_) s.layer = s.id = -1;
    for (auto& m : strata_) m.clear();
  }

  // ------------------------------------------------------------ plans
  bool has_plan(uint64_t id) const { return plans_.count(id) != 0; }
  Plan* plan_of(uint64_t id) {
    auto it = plans_.find(id);
    return it == plans_.end() ? nullptr : &it->second;
  }
  // Snapshot hits (pinned, LRU-promoted) before any miss is admitted
  // (provider_cuda_moe.cpp:963-1008).  ids canonical ascending.
  const Plan& plan(uint64_t id, int layer, const uint16_t* ids, int n) {
    Plan p;
    p.layer = layer;
    p.ids.assign(ids, ids + n);
    for (int i = 0; i < n; ++i) {
      auto it = strata_[layer].find(ids[i]);
      if (it != strata_[layer].end()) {
        Slot& s = slots_[it->second];
        s.last_use = ++clock_;
        ++s.pins;
        p.hit_slots.push_back(it->second);
        ++hits_;
      } else {
        p.missing.push_back(ids[i]);
        p.hit_slots.push_back(-1);
        ++misses_;
      }
    }
    return plans_.emplace(id, std::move(p)).first->second;
  }

  // A slot for the plan's next miss: a free allocated slot, else a new
  // segment while under capacity, else the globally least-recent unpinned
  // entry (evict_global_lru, :730-747).  Returns the slot, -1 when every slot
  // is pinned, -2 on a recoverable allocation failure (the caller runs
  // recover()), -3 on any other allocation failure.  *evicted receives
  // whether an entry was dropped to make room.
  int take_slot(Hooks& hk, bool* evicted) {
    *evicted = false;
    for (int i = 0; i < (int)slots_.size(); ++i)
      if (slots_[i].id < 0 && slots_[i].pins == 0) return i;
    if ((int)slots_.size() < capacity_) {
      const int seg = (int)seg_sizes_.size();
      const int n = std::min(seg_slots_, capacity_ - (int)slots_.size());
      int rc;
      if (fail_allocs_ > 0) {
        --fail_allocs_;
        rc = 1;
      } else {
        rc = hk.alloc_segment(seg, (uint64_t)n * slot_bytes_);
      }
      if (rc == 0) {
        const int first = (int)slots_.size();
        slots_.resize(slots_.size() + n);
        seg_sizes_.push_back(n);
        return first;
      }
      return rc == 1 ? -2 : -3;
    }
    int victim = -1;
    for (int i = 0; i < (int)slots_.size(); ++i) {
      const Slot& s = slots_[i];
      if (s.pins == 0 && (victim < 0 || s.last_use < slots_[victim].last_use)) victim = i;
    }
    if (victim < 0) return -1;
    Slot& s = slots_[victim];
    strata_[s.layer].erase(s.id);
    s.layer = s.id = -1;
    ++evictions_;
    *evicted = true;
    return victim;
  }
  // Record the plan's next miss as resident in `slot` (pinned by the plan).
  void admit(Plan& p, int slot) {
    Slot& s = slots_[slot];
    s.layer = p.layer;
    s.id = p.missing[p.miss_slots.size()];
    s.last_use = ++clock_;
    ++s.pins;
    strata_[p.layer][s.id] = slot;
    p.miss_slots.push_back(slot);
  }
  // Undo the plan's admissions (a fetch that failed part way): the entries
  // are forgotten and unpinned.
  void unadmit(Plan& p) {
    for (int slot : p.miss_slots) {
      Slot& s = slots_[slot];
      if (s.id >= 0) strata_[s.layer].erase(s.id);
      s.layer = s.id = -1;
      if (s.pins > 0) --s.pins;
    }
    p.miss_slots.clear();
  }
  // Slot of `id` in the plan: its pinned hit or admitted miss; -1 if not yet
  // admitted, -2 if the id is not in the plan.
  static int plan_slot(const Plan& p, uint16_t id) {
    const auto it = std::lower_bound(p.ids.begin(), p.ids.end(), id);
    if (it == p.ids.end() || *it != id) return -2;
    const size_t idx = (size_t)(it - p.ids.begin());
    if (p.hit_slots[idx] >= 0) return p.hit_slots[idx];
    const auto mt = std::lower_bound(p.missing.begin(), p.missing.end(), id);
    const size_t mi = (size_t)(mt - p.missing.begin());
    return mi < p.miss_slots.size() ? p.miss_slots[mi] : -1;
  }
  // Finish or cancel: unpin every slot the plan holds.
  void release(uint64_t id) {
    auto it = plans_.find(id);
    if (it == plans_.end()) return;
    for (int s : it->second.hit_slots)
      if (s >= 0 && slots_[s].pins > 0) --slots_[s].pins;
    for (int s : it->second.miss_slots)
      if (slots_[s].pins > 0) --slots_[s].pins;
    plans_.erase(it);
  }
  // The plan's pinned hits as (expert id, slot), in canonical order: what
  // materialize_plan_for_cpu copies to the host (:1170-1196).
  std::vector<std::pair<uint16_t, int>> plan_hits(const Plan& p) const {
    std::vector<std::pair<uint16_t, int>> v;
    for (size_t i = 0; i < p.ids.size(); ++i)
      if (p.hit_slots[i] >= 0) v.emplace_back(p.ids[i], p.hit_slots[i]);
    return v;
  }

  // ------------------------------------------------------------ recovery
  // After a recoverable allocation failure (the caller has drained its copy
  // stream): forget every unpinned entry and give back the trailing segments
  // that hold no pinned entry; within the bounded rebuilds the budget is
  // re-measured at the next plan (rebuild_after_memory_pressure, :545-567),
  // past them the cache is disabled (its callers take their CPU path).
  // Pinned entries of live plans stay in place for materialization.  Returns
  // true while the cache stays enabled.
  bool recover(Hooks& hk, const std::string& failure) {
    for (Slot& s : slots_)
      if (s.pins == 0 && s.id >= 0) {
        strata_[s.layer].erase(s.id);
        s.layer = s.id = -1;
      }
    // Give back trailing segments whose slots are all unpinned (segments are
    // indexed by position, so only the tail can shrink).
    while (!seg_sizes_.empty()) {
      const int n = seg_sizes_.back();
      const int first = (int)slots_.size() - n;
      bool pinned = false;
      for (int i = first; i < (int)slots_.size(); ++i) pinned |= slots_[i].pins > 0;
      if (pinned) break;
      for (int i = first; i < (int)slots_.size(); ++i) hk.wait_slot_idle(i);
      hk.free_segment((int)seg_sizes_.size() - 1);
      slots_.resize(first);
      seg_sizes_.pop_back();
    }
    if (rebuilds_left_ == 0) {
      poison("allocation failure after " + std::to_string(kCacheRebuilds) + " rebuilds: " + failure,
             false);
      return false;
    }
    --rebuilds_left_;
    budget_ready_ = false;
    reason_ = "recovered from allocation failure: " + failure;
    return true;
  }
  // Test hook: the next n segment allocations report out of memory without
  // reaching the allocator.
  void fail_next_allocations(int n) { fail_allocs_ = std::max(0, n); }

  // ------------------------------------------------------------ queries
  int find(int layer, uint16_t id) const {
    auto it = strata_[layer].find(id);
    return it == strata_[layer].end() ? -1 : it->second;
  }
  const Slot& slot(int i) const { return slots_[i]; }
  int resident() const {
    int n = 0;
    for (const Slot& s : slots_) n += s.id >= 0;
    return n;
  }
  int n_layers() const { return (int)strata_.size(); }
  long long hits() const { return hits_; }
  long long misses() const { return misses_; }
  long long evictions() const { return evictions_; }
  int segments() const { return (int)seg_sizes_.size(); }
  int segment_size(int seg) const { return seg_sizes_[seg]; }
  // Segment holding `slot` and the slot's index inside it.
  void locate(int slot, int* seg, int* index) const {
    int first = 0, k = 0;
    while (k + 1 < (int)seg_sizes_.size() && slot >= first + seg_sizes_[k]) first += seg_sizes_[k++];
    *seg = k;
    *index = slot - first;
  }

 private:
  uint64_t slot_bytes_;
  int seg_slots_;
  CachePolicy policy_;
  bool frozen_ = false;
  bool budget_ready_ = false;
  uint64_t budget_free_ = 0, budget_reserve_ = 0;
  int capacity_ = 0;
  int rebuilds_left_ = kCacheRebuilds;
  int fail_allocs_ = 0;
  std::vector<Slot> slots_;
  std::vector<int> seg_sizes_;
  std::vector<std::unordered_map<int, int>> strata_;  // layer -> id -> slot
  std::map<uint64_t, Plan> plans_;
  uint64_t clock_ = 0;
  long long hits_ = 0, misses_ = 0, evictions_ = 0;
  int state_ = kUnqualified;
  std::string reason_ = "not yet qualified";
};

}  // namespace k3
