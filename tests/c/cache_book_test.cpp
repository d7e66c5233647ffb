// CPU test of the expert cache's bookkeeping (deltafin_amd/csrc/k3_cache_book.h,
// compiled into the library unchanged): policy bounds, budget arithmetic,
// global LRU over layer strata with plan pinning, and the bounded recovery
// from allocation failure with materialization of a failed plan's hits.
// Device segments are simulated by a host allocator whose failures the test
// forces.  Prints "ok" and exits 0, or names the failed check and exits 1.
#include <stdio.h>
#include <stdlib.h>

#include <set>
#include <string>
#include <vector>

#include "../../deltafin_amd/csrc/k3_cache_book.h"

using namespace k3;

static int failures = 0;
#define CHECK(cond)                                                 \
  do {                                                              \
    if (!(cond)) {                                                  \
      fprintf(stderr, "%s:%d: check failed: %s\n", __FILE__, __LINE__, #cond); \
      ++failures;                                                   \
    }                                                               \
  } while (0)

// Host stand-in for the device side: counts segments, can refuse them.
struct HostHooks : CacheBook::Hooks {
  std::vector<std::vector<unsigned char>> segs;
  int refuse = 0;        // next allocations answered with out-of-memory
  int fatal = 0;         // next allocations answered with a hard failure
  std::set<int> waited;  // slots waited on before a segment went back
  int alloc_segment(int seg, uint64_t bytes) override {
    if (seg != (int)segs.size()) return -1;
    if (fatal > 0) { --fatal; return -1; }
    if (refuse > 0) { --refuse; return 1; }
    segs.emplace_back(bytes);
    return 0;
  }
  void free_segment(int seg) override {
    if (seg == (int)segs.size() - 1) segs.pop_back();
  }
  void wait_slot_idle(int slot) override { waited.insert(slot); }
};

static void test_policy() {
  CachePolicy p;
  CHECK(cache_policy_error(p) == nullptr);
  p.capacity = 3;  // automatic with a requested count
  CHECK(cache_policy_error(p) != nullptr);
  p.automatic = false;
  p.capacity = kCacheMaxExperts;
  CHECK(cache_policy_error(p) == nullptr);
  p.capacity = kCacheMaxExperts + 1;
  CHECK(cache_policy_error(p) != nullptr);
  p.capacity = 4;
  p.reserve_kind = kReserveAuto;
  p.reserve_value = 1;
  CHECK(cache_policy_error(p) != nullptr);
  p.reserve_kind = kReserveRatioPpm;
  p.reserve_value = 1000000;
  CHECK(cache_policy_error(p) == nullptr);
  p.reserve_value = 1000001;
  CHECK(cache_policy_error(p) != nullptr);
  p.reserve_kind = 7;
  p.reserve_value = 0;
  CHECK(cache_policy_error(p) != nullptr);
}

static void test_budget_arithmetic() {
  // The reference's own compile-time checks of clamp_cache_capacity
  // (provider_cuda_moe.cpp:94-97).
  CHECK(cache_clamp_capacity(10, 10, true, 0, 1) == 0);
  CHECK(cache_clamp_capacity(10, 0, false, 0, 1) == 0);
  CHECK(cache_clamp_capacity(10, 0, false, 4, 1) == 4);
  CHECK(cache_clamp_capacity(10, 0, false, 40, 1) == 10);
  CHECK(cache_clamp_capacity(10, 0, true, 0, 0) == 0);
  CachePolicy p;
  const uint64_t gib = uint64_t(1) << 30;
  CHECK(cache_reserve_bytes(p, 5 * gib) == 2 * gib);        // max(2 GiB, free / 5)
  CHECK(cache_reserve_bytes(p, 100 * gib) == 20 * gib);
  p.reserve_kind = kReserveBytes;
  p.reserve_value = 12345;
  CHECK(cache_reserve_bytes(p, 100 * gib) == 12345);
  p.reserve_kind = kReserveRatioPpm;
  p.reserve_value = 250000;
  CHECK(cache_reserve_bytes(p, 4000000) == 1000000);
  p.reserve_value = 333333;  // exact split of the product, no overflow
  const uint64_t big = (uint64_t(1) << 63) + 999999;
  CHECK(cache_reserve_bytes(p, big) == (big / 1000000) * 333333 + ((big % 1000000) * 333333) / 1000000);
  // Automatic capacity from a measured budget: 1000 free, reserve 200
  // (bytes), slot 100 -> 8 slots; a requested 5 is honoured, 50 clamped.
  CachePolicy a;
  a.reserve_kind = kReserveBytes;
  a.reserve_value = 200;
  CacheBook b(100, 1, 4, a);
  b.establish_budget(1000);
  CHECK(b.capacity() == 8 && b.frozen());
  CHECK(b.configure(CachePolicy()) != nullptr);  // frozen after first use
  a.automatic = false;
  a.capacity = 5;
  CacheBook c(100, 1, 4, a);
  CHECK(c.configure(a) == nullptr);
  c.establish_budget(1000);
  CHECK(c.capacity() == 5);
  a.capacity = 50;
  CacheBook d(100, 1, 4, a);
  d.establish_budget(1000);
  CHECK(d.capacity() == 8);
}

static std::vector<uint16_t> admit_all(CacheBook& b, HostHooks& hk, uint64_t id, int layer,
                                       std::vector<uint16_t> ids, int* rc) {
  const CacheBook::Plan& p = b.plan(id, layer, ids.data(), (int)ids.size());
  std::vector<uint16_t> missing = p.missing;
  CacheBook::Plan* pp = b.plan_of(id);
  *rc = 0;
  for (size_t i = 0; i < missing.size(); ++i) {
    bool ev = false;
    const int s = b.take_slot(hk, &ev);
    if (s < 0) {
      b.unadmit(*pp);
      *rc = s;
      break;
    }
    b.admit(*pp, s);
  }
  return missing;
}

static void test_lru_and_pinning() {
  HostHooks hk;
  CachePolicy p;
  p.automatic = false;
  p.capacity = 4;
  p.reserve_kind = kReserveBytes;
  CacheBook b(64, 3, 2, p);
  b.enable("test");
  b.establish_budget(uint64_t(1) << 20);
  CHECK(b.capacity() == 4);
  int rc;
  auto m = admit_all(b, hk, 1, 0, {1, 2}, &rc);  // layer 0: 1, 2
  CHECK(rc == 0 && m.size() == 2 && hk.segs.size() == 1);
  b.release(1);
  m = admit_all(b, hk, 2, 1, {1, 5}, &rc);  // layer 1: 1, 5 (same id, other stratum)
  CHECK(rc == 0 && m.size() == 2 && hk.segs.size() == 2 && b.resident() == 4);
  b.release(2);
  // A hit is pinned at plan time and promoted: (0,1) becomes most recent.
  m = admit_all(b, hk, 3, 0, {1, 9}, &rc);
  CHECK(rc == 0 && m.size() == 1 && m[0] == 9);
  // The globally least-recent unpinned entry, (0, 2), made room for 9.
  CHECK(b.find(0, 2) < 0 && b.find(0, 1) >= 0 && b.find(0, 9) >= 0);
  CHECK(b.evictions() == 1);
  // While plan 3 pins (0,1) and (0,9), two new misses take the two others...
  m = admit_all(b, hk, 4, 2, {7, 8}, &rc);
  CHECK(rc == 0 && b.find(1, 1) < 0 && b.find(1, 5) < 0);
  // ...and a third finds every slot pinned: the fetch is undone.
  m = admit_all(b, hk, 5, 2, {6}, &rc);
  CHECK(rc == -1 && b.find(2, 6) < 0);
  b.release(5);
  b.release(4);
  b.release(3);
  for (int i = 0; i < b.allocated_slots(); ++i) CHECK(b.slot(i).pins == 0);
  CHECK(b.hits() == 1);
}

static void test_recovery() {
  HostHooks hk;
  CachePolicy p;  // automatic capacity
  p.reserve_kind = kReserveBytes;
  CacheBook b(100, 2, 2, p);
  b.enable("test");
  b.establish_budget(600);  // 6 slots, segments of 2
  int rc;
  admit_all(b, hk, 1, 0, {1, 2, 3}, &rc);
  CHECK(rc == 0 && hk.segs.size() == 2);
  b.release(1);
  // Plan 2 hits expert 1, misses 10 and 11; the first needs a new segment,
  // which the device refuses (forced through the book's own hook).
  b.fail_next_allocations(1);
  const CacheBook::Plan& p2 = b.plan(2, 0, std::vector<uint16_t>{1, 10, 11}.data(), 3);
  CHECK(p2.missing.size() == 2);
  CacheBook::Plan* pp = b.plan_of(2);
  bool ev;
  int s = b.take_slot(hk, &ev);  // the free slot left in segment 1
  CHECK(s == 3);
  b.admit(*pp, s);
  s = b.take_slot(hk, &ev);
  CHECK(s == -2);
  b.unadmit(*pp);
  CHECK(b.recover(hk, "forced") && b.state() == CacheBook::kEnabled);
  CHECK(b.rebuilds_left() == kCacheRebuilds - 1 && !b.budget_ready());
  // Unpinned entries are gone, the pinned hit stays for materialization, and
  // the segment without pinned slots went back after its slots were waited on.
  CHECK(b.find(0, 2) < 0 && b.find(0, 3) < 0 && b.find(0, 1) >= 0);
  CHECK(hk.segs.size() == 1 && hk.waited.count(2) && hk.waited.count(3));
  auto hits = b.plan_hits(*pp);
  CHECK(hits.size() == 1 && hits[0].first == 1 && hits[0].second == b.find(0, 1));
  b.release(2);
  // The budget is measured again: the segment still held counts towards it.
  b.establish_budget(300);
  CHECK(b.capacity() == 5);
  // Two more failures: the second rebuild, then the cache disables itself.
  hk.refuse = 1;
  admit_all(b, hk, 3, 1, {4, 5, 6}, &rc);
  CHECK(rc == -2);
  b.release(3);
  CHECK(b.recover(hk, "device") && b.rebuilds_left() == 0);
  b.establish_budget(300);
  hk.refuse = 1;
  admit_all(b, hk, 4, 1, {4, 5, 6}, &rc);
  CHECK(rc == -2);
  CHECK(!b.recover(hk, "device") && b.state() == CacheBook::kDisabled);
  CHECK(b.reason().find("rebuilds") != std::string::npos && b.resident() == 0);
  b.release(4);
  // A hard (non-memory) failure is reported apart from the recoverable kind.
  HostHooks h2;
  CacheBook c(100, 1, 2, p);
  c.establish_budget(1000);
  h2.fatal = 1;
  c.plan(1, 0, std::vector<uint16_t>{1}.data(), 1);
  CHECK(c.take_slot(h2, &ev) == -3);
}

static void test_poison() {
  HostHooks hk;
  CachePolicy p;
  p.reserve_kind = kReserveBytes;
  CacheBook b(10, 1, 4, p);
  b.enable("ok");
  b.establish_budget(100);
  int rc;
  admit_all(b, hk, 1, 0, {3, 4}, &rc);
  b.poison("mismatch", false);
  CHECK(b.state() == CacheBook::kDisabled && b.resident() == 0);
  b.poison("hip error", true);
  CHECK(b.state() == CacheBook::kTerminal);
  b.poison("later", false);  // terminal stays terminal
  CHECK(b.state() == CacheBook::kTerminal);
}

int main() {
  test_policy();
  test_budget_arithmetic();
  test_lru_and_pinning();
  test_recovery();
  test_poison();
  if (failures) {
    fprintf(stderr, "%d check(s) failed\n", failures);
    return 1;
  }
  printf("ok\n");
  return 0;
}
