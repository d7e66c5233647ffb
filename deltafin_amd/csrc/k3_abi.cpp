// Host side of the C ABI declared in include/k3_hip_moe_abi.h.
//
// Surface 2 (device pointers, caller stream) is stateless: it validates, carves
// the caller's workspace and launches.  Surface 1 (host-synchronous
// descriptors) owns one context guarded by a mutex, like the Metal bridge's
// global state (tools/metal_moe.mm:170-200): a stream, pinned staging for
// activations, a device workspace and an HBM cache of uploaded host blobs
// keyed by pointer (the counterpart of the Metal wrap cache, :584-616).
#include <hip/hip_runtime_api.h>
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include <algorithm>
#include <atomic>
#include <mutex>
#include <string>
#include <unordered_map>
#include <vector>

#include "k3_internal.h"

// Per-position decode layers of one call as one position-batched launch pair
// (launch_decode_positions) where supported; 0 keeps one layer per position.
#ifndef K3_BATCH_POSITIONS
#define K3_BATCH_POSITIONS 1
#endif

namespace k3 {

// ---------------------------------------------------------------- errors
namespace {
thread_local char g_last_error[512] = "no error";
}

int fail(int status, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
  return status;
}

int hip_fail(const char* what, hipError_t e) {
  return fail(K3_HIP_E_EXEC, "%s: %s", what, hipGetErrorString(e));
}

#ifndef K3_SIDE_STREAM
#define K3_SIDE_STREAM 1  // 0: everything on the caller's stream
#endif

// The library's second stream on one device (default priority,
// non-blocking), the event that forks work onto it from a caller's stream and
// a pool of join events; created on first use, kept for the process.  Null
// where HIP refused the stream or the fork event: everything then runs on the
// caller's stream.
struct SideStream {
  hipStream_t stream = nullptr;
  hipEvent_t fork = nullptr;
  std::vector<hipEvent_t> free_joins;  // join events not held by a fork
  std::mutex mu;  // one record / wait / launch sequence at a time; the pool
};

SideStream* side_stream() {
  if (!K3_SIDE_STREAM) return nullptr;
  static std::mutex mu;
  static std::unordered_map<int, SideStream*> by_device;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return nullptr;
  std::lock_guard<std::mutex> lock(mu);
  auto it = by_device.find(dev);
  if (it != by_device.end()) return it->second;
  SideStream* bs = new SideStream;
  if (hipStreamCreateWithFlags(&bs->stream, hipStreamNonBlocking) != hipSuccess ||
      hipEventCreateWithFlags(&bs->fork, hipEventDisableTiming) != hipSuccess) {
    if (bs->fork) (void)hipEventDestroy(bs->fork);
    if (bs->stream) (void)hipStreamDestroy(bs->stream);
    delete bs;
    bs = nullptr;
  }
  by_device[dev] = bs;
  return bs;
}

// Work forked from the caller's stream onto the side stream and joined back:
// fork records an event on the caller's stream, the side stream waits on it
// and runs `work`, and a join event of this fork's own (taken from the pool
// while the side stream's mutex is held) records its end; join makes the
// caller's stream wait for exactly that event and returns it to the pool (a
// queued wait keeps the record it saw, so the event may be recorded again).
// Another caller's fork therefore never joins this one, and a caller waits
// only for its own side work.  A SideWork that forked and was not joined
// joins when it goes out of scope, so no return leaves the caller's stream
// ahead of the side work.  The work runs on the caller's stream instead when
// there is no side stream, when no join event could be had, or when the
// caller's stream is being captured into a graph: the shared side stream
// never joins a capture, so another thread's call cannot land in it.
class SideWork {
 public:
  explicit SideWork(hipStream_t st) : st_(st), side_(side_stream()) {}
  ~SideWork() { (void)join(); }
  SideWork(const SideWork&) = delete;
  SideWork& operator=(const SideWork&) = delete;
  bool parallel() const { return side_ != nullptr; }
  template <typename F>
  int fork(F&& work) {
    if (!side_) return work(st_);
    hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(st_, &cap) != hipSuccess || cap != hipStreamCaptureStatusNone)
      return work(st_);
    std::lock_guard<std::mutex> lock(side_->mu);
    hipEvent_t done = nullptr;
    if (!side_->free_joins.empty()) {
      done = side_->free_joins.back();
      side_->free_joins.pop_back();
    } else if (hipEventCreateWithFlags(&done, hipEventDisableTiming) != hipSuccess) {
      return work(st_);
    }
    hipError_t e = hipEventRecord(side_->fork, st_);
    if (e == hipSuccess) e = hipStreamWaitEvent(side_->stream, side_->fork, 0);
    if (e != hipSuccess) {
      side_->free_joins.push_back(done);
      return hip_fail("side stream fork", e);
    }
    // The join event is recorded whether or not `work` launched everything,
    // so an error return still joins what it did launch.
    const int r = work(side_->stream);
    if ((e = hipEventRecord(done, side_->stream)) != hipSuccess) {
      // Nothing to wait on: drain the side stream so no side work outlives
      // the call unjoined.
      (void)hipStreamSynchronize(side_->stream);
      side_->free_joins.push_back(done);
      return hip_fail("side stream join", e);
    }
    done_ = done;
    return r;
  }
  int join() {
    if (!done_) return K3_HIP_OK;
    const hipError_t e = hipStreamWaitEvent(st_, done_, 0);
    if (e != hipSuccess) (void)hipEventSynchronize(done_);  // the host waits instead
    {
      std::lock_guard<std::mutex> lock(side_->mu);
      side_->free_joins.push_back(done_);
    }
    done_ = nullptr;
    return e == hipSuccess ? K3_HIP_OK : hip_fail("side stream join", e);
  }

 private:
  hipStream_t st_;
  SideStream* side_;
  hipEvent_t done_ = nullptr;  // this fork's join event, until joined
};


// ---------------------------------------------------------------- geometry
bool make_geo(const K3HipGeometryV1* d, Geo* out) {
  if (!d || d->abi_version != 1 || d->struct_bytes != sizeof(K3HipGeometryV1) ||
      d->reserved != 0 || d->hidden == 0 || d->intermediate == 0 || d->hidden % 32 != 0 ||
      d->intermediate % 32 != 0 || d->hidden > 8192 || d->intermediate > 8192 ||
      (d->activation != K3_ACT_SITU && d->activation != K3_ACT_SILU))
    return false;
  Geo g;
  g.hidden = (int)d->hidden;
  g.inter = (int)d->intermediate;
  g.act = (int)d->activation;
  const uint64_t w13p = (uint64_t)g.inter * g.hidden / 2, w13s = (uint64_t)g.inter * (g.hidden / 32);
  const uint64_t w2p = (uint64_t)g.hidden * g.inter / 2, w2s = (uint64_t)g.hidden * (g.inter / 32);
  g.w1p = 0;
  g.w1s = w13p;
  g.w2p = g.w1s + w13s;
  g.w2s = g.w2p + w2p;
  g.w3p = g.w2s + w2s;
  g.w3s = g.w3p + w13p;
  g.span = g.w3s + w13s;
  g.layout = K3_LAYOUT_RAW_V1;
  if (d->expert_span != g.span) return false;
  *out = g;
  return true;
}

// ---------------------------------------------------------------- scale4-v2
namespace {
constexpr uint32_t kS4Header = 8192;

uint32_t le32(const uint8_t* p) {
  return (uint32_t)p[0] | (uint32_t)p[1] << 8 | (uint32_t)p[2] << 16 | (uint32_t)p[3] << 24;
}
uint64_t le64(const uint8_t* p) { return (uint64_t)le32(p) | (uint64_t)le32(p + 4) << 32; }
bool all_zero(const uint8_t* p, size_t begin, size_t end) {
  for (size_t i = begin; i < end; ++i)
    if (p[i]) return false;
  return true;
}
}  // namespace

bool make_geo_scale4(const Geo& raw, Geo* out) {
  if (raw.hidden != 3584 || raw.inter != 3072) return false;
  const uint64_t packed = (uint64_t)raw.hidden * raw.inter / 2;
  const uint64_t s4 = (uint64_t)raw.hidden * (raw.inter / 32) / 2;  // same for all three
  Geo g = raw;
  g.w1p = kS4Header;
  g.w1s = g.w1p + packed;
  g.w2p = g.w1s + s4;
  g.w2s = g.w2p + packed;
  g.w3p = g.w2s + s4;
  g.w3s = g.w3p + packed;
  g.span = g.w3s + s4;
  g.layout = K3_LAYOUT_SCALE4_V2;
  if (g.span != K3_SCALE4_V2_EXPERT_SPAN) return false;
  *out = g;
  return true;
}

// The format fixes every field for the K3 geometry: identity and lengths,
// the in-memory payload table (offset, bytes of w1p, w1s, w2p, w2s, w3p,
// w3s), the on-disk sidecar table (offset, bytes of the three index planes),
// zero padding, and per matrix a base <= 240 with the 16-entry table of E8M0
// float bits (base + d) << 23.  Bytes 32-63 (the source digest) are free.
const char* scale4_header_error(const uint8_t* p) {
  static const uint8_t magic[8] = {'K', '3', 'S', 'C', '4', 'V', '2', 0};
  Geo raw, g;
  K3HipGeometryV1 d;
  memset(&d, 0, sizeof(d));
  d.abi_version = 1;
  d.struct_bytes = sizeof(d);
  d.hidden = 3584;
  d.intermediate = 3072;
  d.activation = K3_ACT_SITU;
  d.expert_span = K3_RAW_V1_EXPERT_SPAN;
  if (!make_geo(&d, &raw) || !make_geo_scale4(raw, &g)) return "scale4-v2 geometry";
  if (!p) return "null scale4-v2 header";
  if (memcmp(p, magic, sizeof(magic)) != 0 || le32(p + 8) != 2 || le32(p + 12) != kS4Header ||
      le64(p + 16) != g.span || le64(p + 24) != raw.span)
    return "invalid scale4-v2 header identity or length";
  const uint32_t packed = (uint32_t)(g.w1s - g.w1p), s4 = (uint32_t)(g.w2p - g.w1s);
  const uint32_t payload[12] = {(uint32_t)g.w1p, packed, (uint32_t)g.w1s, s4,
                                (uint32_t)g.w2p, packed, (uint32_t)g.w2s, s4,
                                (uint32_t)g.w3p, packed, (uint32_t)g.w3s, s4};
  for (int i = 0; i < 12; ++i)
    if (le32(p + 72 + 4 * i) != payload[i]) return "invalid scale4-v2 payload table";
  const uint32_t sidecar[6] = {kS4Header, s4, kS4Header + s4, s4, kS4Header + 2 * s4, s4};
  for (int i = 0; i < 6; ++i)
    if (le32(p + 320 + 4 * i) != sidecar[i]) return "invalid scale4-v2 sidecar payload table";
  if (!all_zero(p, 67, 72) || !all_zero(p, 120, 128) || !all_zero(p, 344, kS4Header))
    return "scale4-v2 reserved header bytes are nonzero";
  for (int m = 0; m < 3; ++m) {
    const uint32_t base = p[64 + m];
    if (base > 240) return "scale4-v2 base exceeds the exact uint8 range";
    for (uint32_t delta = 0; delta < 16; ++delta)
      if (le32(p + 128 + 64 * m + 4 * delta) != (base + delta) << 23)
        return "scale4-v2 exponent table does not match its base";
  }
  return nullptr;
}

namespace {
uint64_t align256(uint64_t v) { return (v + 255) & ~uint64_t(255); }
}

uint64_t workspace_bytes(const Geo& g, int max_edges, int max_positions) {
  const uint64_t E = (uint64_t)std::max(max_edges, 1), P = (uint64_t)std::max(max_positions, 1);
  uint64_t b = 0;
  b += align256(E * g.inter * 4);   // h
  b += align256(E * g.hidden * 4);  // y
  b += align256(E * 4);             // ids
  b += align256(E * 4);             // w
  b += align256(E * 8);             // uptr
  b += align256((E + 1) * 4);       // uoff
  b += align256(E * 4);             // uedges
  b += align256(E * 4);             // epos
  b += align256((P + 1) * 4);       // poff
  b += align256(sizeof(VerifyPlanDev));
  b += align256(P * kMaxTerms * g.hidden);         // xq
  b += align256(P * kMaxTerms * (g.hidden / 32));  // xqs
  b += align256(E * kMaxTerms * g.inter);          // hq
  b += align256(E * kMaxTerms * (g.inter / 32));   // hqs
  return b;
}

bool carve_workspace(void* base, uint64_t bytes, const Geo& g, int max_edges, int max_positions,
                     Workspace* ws) {
  if (!base || ((uintptr_t)base & 255u) != 0) return false;
  if (bytes < workspace_bytes(g, max_edges, max_positions)) return false;
  const uint64_t E = (uint64_t)std::max(max_edges, 1), P = (uint64_t)std::max(max_positions, 1);
  uint8_t* p = static_cast<uint8_t*>(base);
  auto take = [&](uint64_t n) {
    uint8_t* r = p;
    p += align256(n);
    return r;
  };
  ws->base = static_cast<uint8_t*>(base);
  ws->bytes = bytes;
  ws->h = reinterpret_cast<float*>(take(E * g.inter * 4));
  ws->y = reinterpret_cast<float*>(take(E * g.hidden * 4));
  ws->ids = reinterpret_cast<int32_t*>(take(E * 4));
  ws->w = reinterpret_cast<float*>(take(E * 4));
  ws->uptr = reinterpret_cast<const uint8_t**>(take(E * 8));
  ws->uoff = reinterpret_cast<int32_t*>(take((E + 1) * 4));
  ws->uedges = reinterpret_cast<int32_t*>(take(E * 4));
  ws->epos = reinterpret_cast<int32_t*>(take(E * 4));
  ws->poff = reinterpret_cast<int32_t*>(take((P + 1) * 4));
  ws->plan = reinterpret_cast<VerifyPlanDev*>(take(sizeof(VerifyPlanDev)));
  ws->xq = take(P * kMaxTerms * g.hidden);
  ws->xqs = take(P * kMaxTerms * (g.hidden / 32));
  ws->hq = take(E * kMaxTerms * g.inter);
  ws->hqs = take(E * kMaxTerms * (g.inter / 32));
  return true;
}

int device_cu_count() {
  static std::mutex mu;
  static std::unordered_map<int, int> cache;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return 256;
  std::lock_guard<std::mutex> lk(mu);
  auto it = cache.find(dev);
  if (it != cache.end()) return it->second;
  int cus = 0;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
      cus <= 0)
    cus = 256;
  cache[dev] = cus;
  return cus;
}

bool lds_fits(const void* kernel, int block, size_t dynamic_lds) {
  static std::mutex mu;
  static std::unordered_map<std::string, bool> cache;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) dev = -1;
  char key[96];
  snprintf(key, sizeof(key), "%p/%d/%zu/%d", kernel, block, dynamic_lds, dev);
  std::lock_guard<std::mutex> lk(mu);
  auto it = cache.find(key);
  if (it != cache.end()) return it->second;
  // Raise the kernel's dynamic-LDS ceiling (a no-op where the runtime needs no
  // opt-in), then ask whether one workgroup of this shape fits on a CU.
  if (hipFuncSetAttribute(kernel, hipFuncAttributeMaxDynamicSharedMemorySize, (int)dynamic_lds) !=
      hipSuccess)
    (void)hipGetLastError();
  int n = 0;
  const bool ok =
      hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, kernel, block, dynamic_lds) == hipSuccess &&
      n >= 1;
  if (!ok) (void)hipGetLastError();
  cache[key] = ok;
  return ok;
}

namespace {

bool geometry_from(const K3HipGeometryV1* g, Geo* out);
int verify_table(const Geo& g, const EdgeTable& tbl, const void* x, int x_dtype, void* out,
                 int out_dtype, const Workspace& ws, hipStream_t st, bool flat);

// ---------------------------------------------------------------- presets
void fill_geometry(uint32_t hidden, uint32_t inter, uint32_t act, K3HipGeometryV1* out) {
  memset(out, 0, sizeof(*out));
  out->abi_version = 1;
  out->struct_bytes = sizeof(K3HipGeometryV1);
  out->hidden = hidden;
  out->intermediate = inter;
  out->activation = act;
  out->expert_span = k3_hip_geometry_span(hidden, inter);
}

// ---------------------------------------------------------------- surface 1 context
struct BlobEntry {
  uint8_t* dev = nullptr;
  uint64_t span = 0;
  uint64_t last_use = 0;
};

struct Context {
  std::mutex mu;
  bool tried = false, ok = false;
  int device = 0;
  hipStream_t stream = nullptr;
  K3HipGeometryV1 gdesc{};
  Geo geo{};
  void* ws = nullptr;
  uint64_t ws_bytes = 0;
  float* dx = nullptr;     // [K3_HIP_MAX_POSITIONS * H] fp32
  float* dout = nullptr;   // [K3_HIP_MAX_POSITIONS * H] fp32
  float* hx = nullptr;     // pinned staging, same size
  float* hout = nullptr;
  uint64_t act_elems = 0;
  int cache_mode = 1;
  uint64_t cache_capacity = 0;  // entries
  std::unordered_map<const uint8_t*, BlobEntry> blobs;
  uint64_t clock = 0;
  long long calls = 0, device_uses = 0, uploads = 0;
};

Context& ctx() {
  static Context c;
  return c;
}

void release_buffers_locked(Context& c) {
  for (auto& kv : c.blobs) (void)hipFree(kv.second.dev);
  c.blobs.clear();
  if (c.ws) (void)hipFree(c.ws);
  if (c.dx) (void)hipFree(c.dx);
  if (c.dout) (void)hipFree(c.dout);
  if (c.hx) (void)hipHostFree(c.hx);
  if (c.hout) (void)hipHostFree(c.hout);
  c.ws = nullptr;
  c.dx = c.dout = c.hx = c.hout = nullptr;
  c.ws_bytes = 0;
  c.act_elems = 0;
}

// (Re)size the geometry-dependent buffers for c.geo.
int allocate_buffers_locked(Context& c) {
  release_buffers_locked(c);
  hipError_t e = hipSetDevice(c.device);
  if (e != hipSuccess) return hip_fail("hipSetDevice", e);
  c.ws_bytes = workspace_bytes(c.geo, K3_HIP_MAX_EDGES, K3_HIP_MAX_POSITIONS);
  c.act_elems = (uint64_t)K3_HIP_MAX_POSITIONS * c.geo.hidden;
  if ((e = hipMalloc(&c.ws, c.ws_bytes)) != hipSuccess ||
      (e = hipMemset(c.ws, 0, c.ws_bytes)) != hipSuccess ||
      (e = hipMalloc(reinterpret_cast<void**>(&c.dx), c.act_elems * 4)) != hipSuccess ||
      (e = hipMalloc(reinterpret_cast<void**>(&c.dout), c.act_elems * 4)) != hipSuccess ||
      (e = hipHostMalloc(reinterpret_cast<void**>(&c.hx), c.act_elems * 4, hipHostMallocDefault)) !=
          hipSuccess ||
      (e = hipHostMalloc(reinterpret_cast<void**>(&c.hout), c.act_elems * 4,
                         hipHostMallocDefault)) != hipSuccess) {
    const int rc = fail(K3_HIP_E_ALLOC, "surface-1 buffer allocation: %s", hipGetErrorString(e));
    release_buffers_locked(c);
    return rc;
  }
  size_t free_b = 0, total_b = 0;
  if (hipMemGetInfo(&free_b, &total_b) != hipSuccess) free_b = 0;
  const uint64_t reserve = std::max<uint64_t>(uint64_t(2) << 30, free_b / 5);
  const uint64_t usable = free_b > reserve ? free_b - reserve : 0;
  // The reference bounds residency at 92 layers x 16 experts
  // (provider_cuda_moe.cpp:54-56); keep the same ceiling.
  c.cache_capacity = std::min<uint64_t>(usable / c.geo.span, 92 * 16);
  return K3_HIP_OK;
}

bool init_locked(Context& c, const char* selector) {
  if (c.tried) return c.ok;
  c.tried = true;
  int count = 0;
  hipError_t e = hipGetDeviceCount(&count);
  if (e != hipSuccess || count <= 0) {
    fail(K3_HIP_E_INIT, "no HIP device: %s", e == hipSuccess ? "count is 0" : hipGetErrorString(e));
    return false;
  }
  int dev = 0;
  if (selector && *selector) {
    char* end = nullptr;
    const long v = strtol(selector, &end, 10);
    if (!end || *end != '\0' || v < 0 || v >= count) {
      fail(K3_HIP_E_INIT, "invalid device selector '%s'", selector);
      return false;
    }
    dev = (int)v;
  }
  if (k3_hip_moe_available(dev) != 1) return false;
  c.device = dev;
  if ((e = hipSetDevice(dev)) != hipSuccess) {
    hip_fail("hipSetDevice", e);
    return false;
  }
  if ((e = hipStreamCreateWithFlags(&c.stream, hipStreamNonBlocking)) != hipSuccess) {
    hip_fail("hipStreamCreate", e);
    return false;
  }
  fill_geometry(3584, 3072, K3_ACT_SITU, &c.gdesc);
  make_geo(&c.gdesc, &c.geo);
  if (allocate_buffers_locked(c) != K3_HIP_OK) return false;
  c.ok = true;
  return true;
}

// Classify a blob pointer: 0 = pageable host, 1 = pinned host, 2 = device.
int classify(const void* p) {
  hipPointerAttribute_t attr;
  memset(&attr, 0, sizeof(attr));
  const hipError_t e = hipPointerGetAttributes(&attr, p);
  if (e != hipSuccess) {
    (void)hipGetLastError();
    return 0;
  }
  if (attr.type == hipMemoryTypeDevice || attr.type == hipMemoryTypeManaged) return 2;
  if (attr.type == hipMemoryTypeHost) return 1;
  return 0;
}

void evict_one_locked(Context& c, const std::vector<const uint8_t*>& keep) {
  auto victim = c.blobs.end();
  for (auto it = c.blobs.begin(); it != c.blobs.end(); ++it) {
    if (std::find(keep.begin(), keep.end(), it->first) != keep.end()) continue;
    if (victim == c.blobs.end() || it->second.last_use < victim->second.last_use) victim = it;
  }
  if (victim != c.blobs.end()) {
    (void)hipFree(victim->second.dev);
    c.blobs.erase(victim);
  }
}

// Device address for one blob; uploads host blobs into the HBM cache.
// `temps` collects uncached uploads to free after the call.
int resolve_blob_locked(Context& c, const Geo& lg, const uint8_t* blob,
                        const std::vector<const uint8_t*>& call, const uint8_t** out,
                        std::vector<uint8_t*>* temps) {
  const int kind = classify(blob);
  if (kind == 2) {
    ++c.device_uses;
    *out = blob;
    return K3_HIP_OK;
  }
  auto it = c.blobs.find(blob);
  if (it != c.blobs.end() && it->second.span == lg.span && c.cache_mode == 1) {
    it->second.last_use = ++c.clock;
    *out = it->second.dev;
    return K3_HIP_OK;
  }
  if (it != c.blobs.end()) {
    (void)hipFree(it->second.dev);
    c.blobs.erase(it);
  }
  const bool keep = c.cache_mode == 1 && c.cache_capacity > 0;
  if (keep) {
    while (c.blobs.size() >= c.cache_capacity && !c.blobs.empty()) {
      const size_t before = c.blobs.size();
      evict_one_locked(c, call);
      if (c.blobs.size() == before) break;
    }
  }
  uint8_t* dev = nullptr;
  hipError_t e = hipMalloc(reinterpret_cast<void**>(&dev), lg.span);
  if (e != hipSuccess) {
    (void)hipGetLastError();
    return fail(K3_HIP_E_ALLOC, "expert upload allocation: %s", hipGetErrorString(e));
  }
  e = kind == 1 ? hipMemcpyAsync(dev, blob, lg.span, hipMemcpyHostToDevice, c.stream)
                : hipMemcpy(dev, blob, lg.span, hipMemcpyHostToDevice);
  if (e != hipSuccess) {
    (void)hipFree(dev);
    return fail(K3_HIP_E_COPY, "expert upload: %s", hipGetErrorString(e));
  }
  ++c.uploads;
  if (keep) {
    BlobEntry be;
    be.dev = dev;
    be.span = lg.span;
    be.last_use = ++c.clock;
    c.blobs[blob] = be;
  } else {
    temps->push_back(dev);
  }
  *out = dev;
  return K3_HIP_OK;
}

int finish_call_locked(Context& c, std::vector<uint8_t*>& temps, int rc) {
  const hipError_t e = hipStreamSynchronize(c.stream);
  for (uint8_t* t : temps) (void)hipFree(t);
  if (rc != K3_HIP_OK) return rc;
  if (e != hipSuccess) return fail(K3_HIP_E_EXEC, "surface-1 execution: %s", hipGetErrorString(e));
  return K3_HIP_OK;
}

// Descriptor validation (tools/metal_moe.mm:407-450): every descriptor of a
// call has the same layout, its byte length is that layout's span, and a
// scale4-v2 blob's header passes scale4_header_error (read from device memory
// when the blob is there).  *lg receives the call's layout geometry.
int check_descriptors(const Context& c, const K3HipExpertDescriptorV1* d, int count,
                      std::vector<const uint8_t*>* blobs, Geo* lg) {
  if (count < 0 || (count > 0 && !d))
    return fail(K3_HIP_E_DESCRIPTOR, "invalid expert descriptor array");
  blobs->clear();
  *lg = c.geo;
  uint32_t selected = 0;
  std::vector<uint8_t> header;
  for (int i = 0; i < count; ++i) {
    if (d[i].abi_version != K3_DESCRIPTOR_ABI_V1 ||
        d[i].struct_bytes != sizeof(K3HipExpertDescriptorV1) || d[i].reserved != 0 ||
        !d[i].blob)
      return fail(K3_HIP_E_DESCRIPTOR, "invalid expert descriptor fields (index %d)", i);
    Geo cand = c.geo;
    if (d[i].layout_id == K3_LAYOUT_SCALE4_V2) {
      if (!make_geo_scale4(c.geo, &cand))
        return fail(K3_HIP_E_CAPABILITY,
                    "scale4-v2 needs the K3 geometry (hidden 3584, intermediate 3072)");
    } else if (d[i].layout_id != K3_LAYOUT_RAW_V1) {
      return fail(K3_HIP_E_DESCRIPTOR, "unknown expert layout (index %d)", i);
    }
    if (d[i].blob_bytes != cand.span)
      return fail(K3_HIP_E_DESCRIPTOR, "expert byte length does not match its layout (index %d)", i);
    if (i == 0) {
      selected = d[i].layout_id;
      *lg = cand;
    } else if (d[i].layout_id != selected) {
      return fail(K3_HIP_E_DESCRIPTOR, "mixed expert layouts are not allowed in one call");
    }
    if (d[i].layout_id == K3_LAYOUT_SCALE4_V2) {
      const uint8_t* hp = d[i].blob;
      if (classify(d[i].blob) == 2) {
        header.resize(8192);
        const hipError_t e = hipMemcpy(header.data(), d[i].blob, 8192, hipMemcpyDeviceToHost);
        if (e != hipSuccess) return hip_fail("scale4-v2 header read", e);
        hp = header.data();
      }
      if (const char* why = scale4_header_error(hp))
        return fail(K3_HIP_E_DESCRIPTOR, "%s (index %d)", why, i);
    }
    blobs->push_back(d[i].blob);
  }
  return K3_HIP_OK;
}

int layer_locked(Context& c, const Geo& lg, const uint8_t* const* blobs, int n,
                 const float* weights, const float* x, float* out) {
  if (!x || !out || n < 0) return fail(K3_HIP_E_INVALID, "layer: null input/output or n < 0");
  const size_t hb = (size_t)c.geo.hidden * 4;
  if (n == 0) {
    memset(out, 0, hb);
    return K3_HIP_OK;
  }
  if (!blobs || !weights) return fail(K3_HIP_E_INVALID, "layer: null blobs or weights");
  if (n > K3_HIP_MAX_TOKEN_EXPERTS)
    return fail(K3_HIP_E_INVALID, "layer: %d experts exceeds %d", n, K3_HIP_MAX_TOKEN_EXPERTS);
  hipError_t e = hipSetDevice(c.device);
  if (e != hipSuccess) return hip_fail("hipSetDevice", e);
  std::vector<const uint8_t*> call(blobs, blobs + n);
  std::vector<uint8_t*> temps;
  TokenRoute route;
  memset(&route, 0, sizeof(route));
  route.n = n;
  for (int i = 0; i < n; ++i) {
    if (!blobs[i]) return fail(K3_HIP_E_INVALID, "layer: null blob %d", i);
    const int rc = resolve_blob_locked(c, lg, blobs[i], call, &route.ptr[i], &temps);
    if (rc != K3_HIP_OK) return finish_call_locked(c, temps, rc);
    route.w[i] = weights[i];
  }
  memcpy(c.hx, x, hb);
  if ((e = hipMemcpyAsync(c.dx, c.hx, hb, hipMemcpyHostToDevice, c.stream)) != hipSuccess)
    return finish_call_locked(c, temps, fail(K3_HIP_E_COPY, "layer input copy: %s", hipGetErrorString(e)));
  Workspace ws;
  carve_workspace(c.ws, c.ws_bytes, c.geo, K3_HIP_MAX_EDGES, K3_HIP_MAX_POSITIONS, &ws);
  int rc = launch_decode_layer(lg, route, c.dx, K3_DTYPE_F32, c.dout, K3_DTYPE_F32, ws, c.stream);
  if (rc == K3_HIP_OK &&
      (e = hipMemcpyAsync(c.hout, c.dout, hb, hipMemcpyDeviceToHost, c.stream)) != hipSuccess)
    rc = fail(K3_HIP_E_COPY, "layer output copy: %s", hipGetErrorString(e));
  rc = finish_call_locked(c, temps, rc);
  if (rc != K3_HIP_OK) return rc;
  memcpy(out, c.hout, hb);
  ++c.calls;
  return K3_HIP_OK;
}

int positions_locked(Context& c, const Geo& lg, const uint8_t* const* blobs, int n_edges,
                     const int* offs, int n_pos, const float* weights, const float* x,
                     float* out, bool flat = false) {
  // Offset validation mirrors tools/metal_moe.mm:852-871.
  if (n_edges < 0 || n_pos < 0) return fail(K3_HIP_E_INVALID, "positions: negative counts");
  // The flat form's bounds (tools/metal_moe.mm:1056-1059): at most 16
  // positions and 16 edges per position on average, else invalid arguments.
  if (flat && (n_pos > 16 || n_edges > n_pos * 16))
    return fail(K3_HIP_E_INVALID, "flat positions: at most 16 positions and 16 x positions edges");
  if (n_pos == 0) return n_edges == 0 ? K3_HIP_OK : fail(K3_HIP_E_INVALID, "positions: edges without positions");
  if (!offs || !x || !out) return fail(K3_HIP_E_INVALID, "positions: null offsets/input/output");
  if (n_pos > K3_HIP_MAX_POSITIONS || n_edges > K3_HIP_MAX_EDGES)
    return fail(K3_HIP_E_INVALID, "positions: at most %d positions and %d edges",
                K3_HIP_MAX_POSITIONS, K3_HIP_MAX_EDGES);
  if (offs[0] != 0) return fail(K3_HIP_E_INVALID, "positions: offsets must start at 0");
  for (int p = 0; p < n_pos; ++p)
    if (offs[p] < 0 || offs[p] > offs[p + 1] || offs[p + 1] > n_edges)
      return fail(K3_HIP_E_INVALID, "positions: offsets are not a partition");
  if (offs[n_pos] != n_edges) return fail(K3_HIP_E_INVALID, "positions: offsets must end at edge count");
  if (n_edges > 0 && (!blobs || !weights)) return fail(K3_HIP_E_INVALID, "positions: null blobs/weights");
  const size_t bytes = (size_t)n_pos * c.geo.hidden * 4;
  if (n_edges == 0) {
    memset(out, 0, bytes);
    return K3_HIP_OK;
  }
  hipError_t e = hipSetDevice(c.device);
  if (e != hipSuccess) return hip_fail("hipSetDevice", e);
  std::vector<const uint8_t*> call(blobs, blobs + n_edges);
  std::vector<uint8_t*> temps;
  EdgeTable tbl;
  memset(&tbl, 0, sizeof(tbl));
  tbl.n_edges = n_edges;
  tbl.n_positions = n_pos;
  for (int p = 0; p <= n_pos; ++p) tbl.pos_off[p] = offs[p];
  for (int i = 0; i < n_edges; ++i) {
    if (!blobs[i]) return fail(K3_HIP_E_INVALID, "positions: null blob %d", i);
    // Repeated blobs resolve to the same device address, so the plan groups them.
    const int rc = resolve_blob_locked(c, lg, blobs[i], call, &tbl.ptr[i], &temps);
    if (rc != K3_HIP_OK) return finish_call_locked(c, temps, rc);
    tbl.w[i] = weights[i];
  }
  memcpy(c.hx, x, bytes);
  if ((e = hipMemcpyAsync(c.dx, c.hx, bytes, hipMemcpyHostToDevice, c.stream)) != hipSuccess)
    return finish_call_locked(c, temps, fail(K3_HIP_E_COPY, "positions input copy: %s", hipGetErrorString(e)));
  Workspace ws;
  carve_workspace(c.ws, c.ws_bytes, c.geo, K3_HIP_MAX_EDGES, K3_HIP_MAX_POSITIONS, &ws);
  // The same path selection as the device surface (k3_hip_set_verify_mode):
  // raw-v1 spans take the matrix-core union path where it applies and pays,
  // scale4-v2 spans run one decode layer per position.
  int rc = verify_table(lg, tbl, c.dx, K3_DTYPE_F32, c.dout, K3_DTYPE_F32, ws, c.stream, flat);
  if (rc == K3_HIP_OK &&
      (e = hipMemcpyAsync(c.hout, c.dout, bytes, hipMemcpyDeviceToHost, c.stream)) != hipSuccess)
    rc = fail(K3_HIP_E_COPY, "positions output copy: %s", hipGetErrorString(e));
  rc = finish_call_locked(c, temps, rc);
  if (rc != K3_HIP_OK) return rc;
  memcpy(out, c.hout, bytes);
  c.calls += n_pos;
  return K3_HIP_OK;
}

bool geometry_from(const K3HipGeometryV1* g, Geo* out) {
  if (g) return make_geo(g, out);
  Context& c = ctx();
  std::lock_guard<std::mutex> lk(c.mu);
  K3HipGeometryV1 d = c.gdesc;
  if (!c.tried) fill_geometry(3584, 3072, K3_ACT_SITU, &d);
  return make_geo(&d, out);
}

int check_dtype(int d) { return d == K3_DTYPE_F32 || d == K3_DTYPE_BF16; }

// Process-wide verify path (k3_hip_set_verify_mode).
std::atomic<int> g_verify_mode{K3_VERIFY_AUTO};

// AUTO picks the matrix-core union path when the batch's unique experts are
// at most this fraction of its edges: per byte the union path (5-6.4 TB/s in
// its two kernels, plus five small launches) costs about 1.08x what one decode
// layer per position does on MI355X (config 3), so it wins once it reads
// under ~92 % of the bytes.
constexpr double kUnionFraction = 0.92;

// Expected unique experts of n_positions independent top_k routes over n_bank
// experts (uniform routing, the least sharing a verify batch can have).
double expected_union(int n_bank, int top_k, int n_positions) {
  const double p = (double)top_k / (double)n_bank;
  double miss = 1.0;
  for (int i = 0; i < n_positions; ++i) miss *= 1.0 - p;
  return (double)n_bank * (1.0 - miss);
}

// Verify over a caller route table, shared by k3_hip_moe_verify_device and
// the descriptor surface's positions call: the matrix-core union path, the
// VALU union kernels or one decode layer per position, as the verify mode and
// the route's sharing say (k3_hip_set_verify_mode).  The union paths read
// raw-v1 spans; other layouts run per position.  Positions without edges get
// zero rows.
int verify_table(const Geo& g, const EdgeTable& tbl, const void* x, int x_dtype, void* out,
                 int out_dtype, const Workspace& ws, hipStream_t st, bool flat) {
  const int n_edges = tbl.n_edges, n_positions = tbl.n_positions;
  const size_t xb = x_dtype == K3_DTYPE_BF16 ? 2 : 4, ob = out_dtype == K3_DTYPE_BF16 ? 2 : 4;
  if (n_edges == 0) return launch_zero(out, (uint64_t)n_positions * g.hidden * ob, st);
  // Distinct experts and the most edges any one of them carries (the
  // matrix-core path takes up to 16 edges, one token column each).
  int n_unique = 0, max_edges_per_expert = 0;
  for (int i = 0; i < n_edges; ++i) {
    bool seen = false;
    for (int j = 0; j < i && !seen; ++j) seen = tbl.ptr[j] == tbl.ptr[i];
    if (seen) continue;
    ++n_unique;
    int c = 0;
    for (int j = i; j < n_edges; ++j) c += tbl.ptr[j] == tbl.ptr[i];
    max_edges_per_expert = std::max(max_edges_per_expert, c);
  }
  const int mode = g_verify_mode.load();
  const bool raw = g.layout == K3_LAYOUT_RAW_V1;
  const bool mfma_ok = raw && verify_mfma_supported(g) && max_edges_per_expert <= 16;
  if (mode == K3_VERIFY_UNION_MFMA && !mfma_ok)
    return fail(K3_HIP_E_CAPABILITY,
                "verify: no matrix-core path (geometry/layout, or an expert with %d > 16 edges)",
                max_edges_per_expert);
  bool mfma = mode == K3_VERIFY_UNION_MFMA ||
              (mode == K3_VERIFY_AUTO && n_positions >= 2 && mfma_ok &&
               n_unique <= kUnionFraction * n_edges);
  // Without the matrix-core path, positions that share most of their experts
  // take the VALU union kernels (each shared expert read once); otherwise one
  // decode layer per position (about twice the streaming rate of the VALU
  // union kernels, so they win unless the union is under half the edges).
  bool valu = raw && (mode == K3_VERIFY_UNION_VALU ||
                      (mode == K3_VERIFY_AUTO && !mfma && !mfma_ok && 2 * n_unique <= n_edges));
  if (flat && !mfma && !valu) {
    // A flat batch runs as one dispatch sequence: per position only when the
    // positions with edges form one run of equal edge counts that the
    // position-batched decode takes (empty positions are zero rows), else
    // the union kernels (raw-v1), else a capability miss.
    int count = -1, runs = 0;
    bool gap = false;
    for (int p = 0; p < n_positions; ++p) {
      const int n = tbl.pos_off[p + 1] - tbl.pos_off[p];
      if (n == 0) {
        gap = runs > 0;
        continue;
      }
      if (n != count || gap) ++runs;
      count = n;
      gap = false;
    }
    const bool one_run = runs == 1 && (n_positions == 1 || (K3_BATCH_POSITIONS &&
                                                            decode_positions_supported(g, count)));
    if (!one_run) {
      if (!raw)
        return fail(K3_HIP_E_CAPABILITY,
                    "flat positions: no single-dispatch form for these edge counts (layout %d)",
                    g.layout);
      mfma = mfma_ok;
      valu = !mfma_ok;
    }
  }
  if (mfma || valu) {
    int rc = launch_verify_plan_table(g, tbl, ws, st, mfma ? x : nullptr, x_dtype);
    if (rc != K3_HIP_OK) return rc;
    return mfma ? launch_verify_mfma(g, n_edges, n_positions, x, x_dtype, out, out_dtype, ws, st,
                                     true)
                : launch_verify_layer(g, n_edges, n_positions, x, x_dtype, out, out_dtype, ws, st);
  }
  // One decode layer per position: a run of two or more consecutive
  // positions with the same edge count runs as one position-batched launch
  // pair (launch_decode_positions over a table-mode route in the workspace);
  // a lone position runs its own layer, and a position with no edges gets a
  // zero row.
  for (int p = 0; p < n_positions;) {
    const int e0 = tbl.pos_off[p], n = tbl.pos_off[p + 1] - e0;
    uint8_t* outp = static_cast<uint8_t*>(out) + (size_t)p * g.hidden * ob;
    const uint8_t* xp = static_cast<const uint8_t*>(x) + (size_t)p * g.hidden * xb;
    if (n == 0) {  // no routed expert: a zero row
      const int rc = launch_zero(outp, (uint64_t)g.hidden * ob, st);
      if (rc != K3_HIP_OK) return rc;
      ++p;
      continue;
    }
    if (n > K3_HIP_MAX_TOKEN_EXPERTS)
      return fail(K3_HIP_E_INVALID, "verify: position %d has %d edges (at most %d)", p, n,
                  K3_HIP_MAX_TOKEN_EXPERTS);
    int run = 1;
    while (p + run < n_positions && tbl.pos_off[p + run + 1] - tbl.pos_off[p + run] == n) ++run;
    if (K3_BATCH_POSITIONS && run > 1 && decode_positions_supported(g, n)) {
      int rc = launch_route_table(tbl, e0, run * n, ws, st);
      if (rc != K3_HIP_OK) return rc;
      TokenRoute route;
      memset(&route, 0, sizeof(route));
      route.pdev = ws.uptr;
      route.wdev = ws.w;
      route.n = n;
      rc = launch_decode_positions(g, route, run, xp, x_dtype, outp, out_dtype, ws, st);
      if (rc != K3_HIP_OK) return rc;
      p += run;
      continue;
    }
    TokenRoute route;
    memset(&route, 0, sizeof(route));
    route.n = n;
    for (int i = 0; i < n; ++i) {
      route.ptr[i] = tbl.ptr[e0 + i];
      route.w[i] = tbl.w[e0 + i];
    }
    const int rc = launch_decode_layer(g, route, xp, x_dtype, outp, out_dtype, ws, st);
    if (rc != K3_HIP_OK) return rc;
    ++p;
  }
  return K3_HIP_OK;
}

// ---------------------------------------------------------------- MoE block
// Positions from which the block's BF16 spine runs on the matrix cores.
#ifndef K3_SPINE_MFMA_MIN_POSITIONS
#define K3_SPINE_MFMA_MIN_POSITIONS 3
#endif
static_assert(sizeof(K3HipMoeSpineV1) == 144, "K3HipMoeSpineV1 layout changed");

// Block workspace: the expert workspace, then logits [P, E], routed_in and
// routed_out [P, R], shared gate and up [P, S] (h overwrites gate), each
// 256-byte aligned.
struct BlockBufs {
  uint8_t* expert_ws;
  uint64_t expert_ws_bytes;
  float* logits;
  float* routed_in;
  float* routed_out;
  float* gate;
  float* up;
  uint8_t* terms;   // BF16 activation terms of the matrix-core spine (P >= 3)
  uint8_t* terms2;  // the hidden rows' terms for the side stream's shared gate/up
};

uint64_t block_layout(const K3HipMoeSpineV1& sp, const Geo& g, int max_positions,
                      uint8_t* base, BlockBufs* b) {
  const uint64_t P = (uint64_t)max_positions;
  uint64_t off = 0;
  const uint64_t ew = align256(workspace_bytes(g, max_positions * (int)sp.top_k, max_positions));
  if (b) {
    b->expert_ws = base;
    b->expert_ws_bytes = ew;
  }
  off += ew;
  auto take = [&](float** dst, uint64_t n) {
    if (b) *dst = reinterpret_cast<float*>(base + off);
    off += align256(n * sizeof(float));
  };
  take(b ? &b->logits : nullptr, P * sp.experts);
  take(b ? &b->routed_in : nullptr, P * sp.routed_hidden);
  take(b ? &b->routed_out : nullptr, P * sp.routed_hidden);
  take(b ? &b->gate : nullptr, P * sp.shared_intermediate);
  take(b ? &b->up : nullptr, P * sp.shared_intermediate);
  const int wmax = (int)std::max(sp.hidden, std::max(sp.routed_hidden, sp.shared_intermediate));
  if (b) b->terms = base + off;
  off += align256(spine_mfma_terms_bytes(max_positions, wmax));
  if (b) b->terms2 = base + off;  // the side stream's: hidden rows, then the shared h
  off += align256(spine_mfma_terms_bytes(
      max_positions, (int)std::max(sp.hidden, sp.shared_intermediate)));
  return off;
}

const char* check_spine(const K3HipMoeSpineV1* sp, const Geo& g) {
  if (!sp) return "null spine";
  if (sp->abi_version != K3_MOE_SPINE_ABI_V1 || sp->struct_bytes != sizeof(K3HipMoeSpineV1))
    return "spine header (abi_version / struct_bytes) mismatch";
  if (sp->matrix_kind != K3_SPINE_MATRIX_BF16 && sp->matrix_kind != K3_SPINE_MATRIX_INT8)
    return "unknown spine matrix kind";
  if (sp->hidden == 0 || sp->routed_hidden == 0 || sp->shared_intermediate == 0 ||
      sp->hidden > (1u << 20) || sp->routed_hidden > (1u << 20) ||
      sp->shared_intermediate > (1u << 20))
    return "spine widths must be in [1, 2^20]";
  if (sp->routed_hidden != (uint32_t)g.hidden)
    return "spine routed_hidden differs from the expert geometry's hidden";
  if (sp->experts == 0 || sp->experts > 4096) return "spine experts must be in [1, 4096]";
  if (sp->top_k == 0 || sp->top_k > K3_HIP_MAX_TOKEN_EXPERTS || sp->top_k > sp->experts)
    return "spine top_k must be in [1, min(32, experts)]";
  if (!sp->router || !sp->router_bias || !sp->routed_down || !sp->routed_norm || !sp->routed_up ||
      !sp->shared_gate || !sp->shared_up || !sp->shared_down)
    return "a spine matrix or vector is null";
  if (sp->matrix_kind == K3_SPINE_MATRIX_INT8 &&
      (!sp->router_scales || !sp->routed_down_scales || !sp->routed_up_scales ||
       !sp->shared_gate_scales || !sp->shared_up_scales || !sp->shared_down_scales))
    return "row-int8 spine matrices need their row scales";
  return nullptr;
}

// A spine-surface status as a K3_HIP_* status, carrying the spine's reason.
int from_spine(int rc, const char* step) {
  if (rc == K3_SPINE_OK) return K3_HIP_OK;
  return fail(rc == K3_SPINE_E_INVALID ? K3_HIP_E_INVALID : K3_HIP_E_EXEC, "MoE block %s: %s",
              step, k3_hip_spine_last_error());
}

// The routed experts of P positions whose routes are already in ws.ids /
// ws.w ([P][top_k]): the union path (plan + matrix-core or VALU kernels) when
// the verify mode asks for it or AUTO expects the union to pay, else one
// decode layer per position on the device route.
int experts_on_device_routes(const Geo& g, const uint8_t* bank, uint64_t stride, int n_bank,
                             int P, int top_k, const float* x, float* out, const Workspace& ws,
                             hipStream_t st) {
  const int n_edges = P * top_k;
  const int mode = g_verify_mode.load();
  if (mode == K3_VERIFY_UNION_MFMA && !verify_mfma_supported(g))
    return fail(K3_HIP_E_CAPABILITY, "MoE block: this geometry/layout has no matrix-core path");
  const bool shared = expected_union(n_bank, top_k, P) <= kUnionFraction * (double)n_edges;
  const bool mfma = P >= 2 && (mode == K3_VERIFY_UNION_MFMA ||
                               (mode == K3_VERIFY_AUTO && shared && verify_mfma_supported(g)));
  if (mfma || (P >= 2 && mode == K3_VERIFY_UNION_VALU)) {
    int rc = launch_verify_plan_bank(g, bank, stride, n_bank, P, top_k, ws, st,
                                     mfma ? x : nullptr, K3_DTYPE_F32);
    if (rc != K3_HIP_OK) return rc;
    return mfma ? launch_verify_mfma(g, n_edges, P, x, K3_DTYPE_F32, out, K3_DTYPE_F32, ws, st,
                                     true)
                : launch_verify_layer(g, n_edges, P, x, K3_DTYPE_F32, out, K3_DTYPE_F32, ws, st);
  }
  TokenRoute route;
  memset(&route, 0, sizeof(route));
  route.bank = bank;
  route.stride = stride;
  route.ids = ws.ids;
  route.wdev = ws.w;
  route.n = top_k;
  if (K3_BATCH_POSITIONS && P > 1 && decode_positions_supported(g, top_k))
    return launch_decode_positions(g, route, P, x, K3_DTYPE_F32, out, K3_DTYPE_F32, ws, st);
  for (int p = 0; p < P; ++p) {
    TokenRoute rp = route;
    rp.ids = ws.ids + (size_t)p * top_k;
    rp.wdev = ws.w + (size_t)p * top_k;
    const int rc = launch_decode_layer(g, rp, x + (size_t)p * g.hidden, K3_DTYPE_F32,
                                       out + (size_t)p * g.hidden, K3_DTYPE_F32, ws, st);
    if (rc != K3_HIP_OK) return rc;
  }
  return K3_HIP_OK;
}

}  // namespace
}  // namespace k3

using namespace k3;

extern "C" {

uint64_t k3_hip_moe_block_workspace_bytes(const K3HipMoeSpineV1* spine,
                                          const K3HipGeometryV1* experts, int max_positions) {
  Geo g;
  if (!geometry_from(experts, &g) || check_spine(spine, g) || max_positions <= 0 ||
      max_positions > K3_HIP_MAX_POSITIONS ||
      max_positions * (int)spine->top_k > K3_HIP_MAX_EDGES)
    return 0;
  return block_layout(*spine, g, max_positions, nullptr, nullptr);
}

int k3_hip_moe_block_device(const K3HipMoeSpineV1* spine, const K3HipGeometryV1* experts,
                            const uint8_t* bank, uint64_t expert_stride, const float* hidden,
                            int n_positions, float* out, int32_t* route_ids,
                            float* route_weights, void* workspace, uint64_t workspace_bytes,
                            void* stream) {
  Geo g;
  if (!geometry_from(experts, &g)) return fail(K3_HIP_E_INVALID, "MoE block: invalid geometry");
  if (const char* why = check_spine(spine, g)) return fail(K3_HIP_E_INVALID, "MoE block: %s", why);
  const K3HipMoeSpineV1& sp = *spine;
  if (!bank || !hidden || !out) return fail(K3_HIP_E_INVALID, "MoE block: null pointer");
  if (expert_stride < g.span || expert_stride % 16 != 0 || ((uintptr_t)bank & 15u) != 0)
    return fail(K3_HIP_E_INVALID, "MoE block: bank must be 16-byte aligned with stride >= span");
  if ((((uintptr_t)hidden | (uintptr_t)out) & 15u) != 0)
    return fail(K3_HIP_E_INVALID, "MoE block: hidden and out must be 16-byte aligned");
  const int top_k = (int)sp.top_k;
  if (n_positions <= 0 || n_positions > K3_HIP_MAX_POSITIONS ||
      n_positions * top_k > K3_HIP_MAX_EDGES)
    return fail(K3_HIP_E_INVALID, "MoE block: positions %d outside [1, %d] (or too many edges)",
                n_positions, K3_HIP_MAX_POSITIONS);
  if (!workspace || ((uintptr_t)workspace & 255u) != 0 ||
      workspace_bytes < block_layout(sp, g, n_positions, nullptr, nullptr))
    return fail(K3_HIP_E_INVALID, "MoE block: workspace missing, misaligned or too small");
  BlockBufs b;
  block_layout(sp, g, n_positions, static_cast<uint8_t*>(workspace), &b);
  Workspace ws;
  if (!carve_workspace(b.expert_ws, b.expert_ws_bytes, g, n_positions * top_k, n_positions, &ws))
    return fail(K3_HIP_E_INVALID, "MoE block: expert workspace carve failed");
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int kind =
      sp.matrix_kind == K3_SPINE_MATRIX_BF16 ? K3_SPINE_KIND_BF16 : K3_SPINE_KIND_INT8;
  const int P = n_positions, H = (int)sp.hidden, R = (int)sp.routed_hidden;
  const int S = (int)sp.shared_intermediate, E = (int)sp.experts;
  int rc;
  // The shared expert's gate/up needs only the hidden rows, so it runs on the
  // side stream where there is one, beside the router, the routed experts and
  // routed_up (the two streams' kernels share the CUs and fill each other's
  // ramps), and the caller's stream waits for it only before shared_down.
  // The next call's fork is recorded after this call's shared_down, so the
  // side stream never overwrites h that is still to be read.  Every return
  // after the fork joins first, so the caller's stream is never ahead of the
  // side work.
  SideWork side(st);
  // 3..16 positions of a BF16 spine: every projection on the matrix cores
  // from BF16 activation terms (the fp32 kernels are bound by LDS and FMAs
  // there); the steps and their order are the same.
  const bool matrices_aligned =
      ((reinterpret_cast<uintptr_t>(sp.router) | reinterpret_cast<uintptr_t>(sp.routed_down) |
        reinterpret_cast<uintptr_t>(sp.routed_up) | reinterpret_cast<uintptr_t>(sp.shared_gate) |
        reinterpret_cast<uintptr_t>(sp.shared_up) | reinterpret_cast<uintptr_t>(sp.shared_down)) &
       15u) == 0;
  if (P >= K3_SPINE_MFMA_MIN_POSITIONS && kind == K3_SPINE_KIND_BF16 && matrices_aligned &&
      spine_mfma_supported(kind, P, R, H) && spine_mfma_supported(kind, P, S, H) &&
      spine_mfma_supported(kind, P, H, R) && spine_mfma_supported(kind, P, H, S)) {
    auto mm = [&](const void* w, const uint8_t* terms, float* y, int rows, int cols, bool acc,
                  hipStream_t s, const char* step) {
      return from_spine(spine_mfma_gemv(w, terms, y, rows, cols, P, acc, s), step);
    };
    auto split = [&](const float* x, int cols, uint8_t* terms, hipStream_t s) {
      return from_spine(spine_mfma_split(x, P, cols, terms, s), "term split");
    };
    // shared gate and up from the hidden rows' terms (already split into
    // `terms` when `split_first` is false), then h = situ(gate, up)
    auto shared_glu = [&](uint8_t* terms, bool split_first, hipStream_t s) -> int {
      int r;
      if ((split_first && (r = split(hidden, H, terms, s))) ||
          (r = mm(sp.shared_gate, terms, b.gate, S, H, false, s, "shared_gate")) ||
          (r = mm(sp.shared_up, terms, b.up, S, H, false, s, "shared_up")))
        return r;
      return launch_activation(b.gate, b.up, b.gate, (int64_t)P * S, K3_ACT_SITU, s);
    };
    // With the side stream the shared expert reads its own copy of the hidden
    // rows' terms (the main stream's buffer is reused for the routed output
    // while the side work may still run), and the side stream also splits
    // its h into that buffer for shared_down, off the main stream's path.
    if (side.parallel() && (rc = side.fork([&](hipStream_t s) {
                              const int r = shared_glu(b.terms2, true, s);
                              return r ? r : split(b.gate, S, b.terms2, s);
                            })))
      return rc;
    // The router logits stay on the fp32 kernels at every P: each position's
    // logit is then summed in the same order whatever the batch (the fp32
    // spine kernels reduce every (row, position) identically), so a hidden row
    // routes to the same experts in a 1-token decode and in a verify batch.
    if ((rc = from_spine(spine_gemv(kind, sp.router, sp.router_scales, hidden, b.logits, E, H, P,
                                    false, st), "router")) ||
        (rc = split(hidden, H, b.terms, st)) ||
        (rc = mm(sp.routed_down, b.terms, b.routed_in, R, H, false, st, "routed_down")) ||
        (!side.parallel() && (rc = shared_glu(b.terms, false, st))))
      return rc;
    if ((rc = launch_route_sigmoid_bias(b.logits, sp.router_bias, E, top_k, P, ws.ids, ws.w,
                                        route_ids, route_weights, st)))
      return rc;
    if ((rc = experts_on_device_routes(g, bank, expert_stride, E, P, top_k, b.routed_in,
                                       b.routed_out, ws, st)))
      return rc;
    // the routed RMS norm writes routed_up's terms in the same launch
    rc = spine_rms_norm_terms(b.routed_out, sp.routed_norm, b.routed_out, P, R, K3_RMS_EPSILON,
                              b.terms, st);
    if (rc == K3_SPINE_E_UNSUPPORTED) {
      if ((rc = from_spine(spine_rms_norm(b.routed_out, sp.routed_norm, b.routed_out, P, R,
                                          K3_RMS_EPSILON, st), "routed RMS norm")) ||
          (rc = split(b.routed_out, R, b.terms, st)))
        return rc;
    } else if ((rc = from_spine(rc, "routed RMS norm"))) {
      return rc;
    }
    if ((rc = mm(sp.routed_up, b.terms, out, H, R, false, st, "routed_up")) ||
        (rc = side.join()))
      return rc;
    if (!side.parallel() && (rc = split(b.gate, S, b.terms, st))) return rc;
    return mm(sp.shared_down, side.parallel() ? b.terms2 : b.terms, out, H, S, true, st,
              "shared_down");
  }
  // the shared expert: h = situ(gate, up), one launch reading each gate row
  // and its up row together (two launches and the activation where the shape
  // has no fused form); h overwrites gate
  auto shared_glu = [&](hipStream_t s) -> int {
    SpineOp glu{};
    glu.w = sp.shared_gate;
    glu.scales = sp.shared_gate_scales;
    glu.w2 = sp.shared_up;
    glu.scales2 = sp.shared_up_scales;
    glu.act = K3_ACT_SITU;
    glu.x = hidden;
    glu.y = b.gate;
    glu.rows = S;
    glu.cols = H;
    glu.positions = P;
    int r = spine_gemv_op(kind, glu, s);
    if (r == K3_SPINE_E_UNSUPPORTED) {
      if ((r = from_spine(spine_gemv(kind, sp.shared_gate, sp.shared_gate_scales, hidden, b.gate,
                                     S, H, P, false, s), "shared_gate")))
        return r;
      if ((r = from_spine(spine_gemv(kind, sp.shared_up, sp.shared_up_scales, hidden, b.up, S,
                                     H, P, false, s), "shared_up")))
        return r;
      return launch_activation(b.gate, b.up, b.gate, (int64_t)P * S, K3_ACT_SITU, s);
    }
    return from_spine(r, "shared gate/up");
  };
  if (side.parallel() && (rc = side.fork(shared_glu))) return rc;
  // prepare: router logits and routed_down (one launch over both matrices,
  // which read the same hidden rows, where the shape allows), then the route
  SpineOp pre{};
  pre.w = sp.router;
  pre.scales = sp.router_scales;
  pre.x = hidden;
  pre.y = b.logits;
  pre.rows = E;
  pre.cols = H;
  pre.positions = P;
  pre.wb = sp.routed_down;
  pre.scales_b = sp.routed_down_scales;
  pre.yb = b.routed_in;
  pre.rows_b = R;
  rc = spine_gemv_op(kind, pre, st);
  if (rc == K3_SPINE_E_UNSUPPORTED) {
    if ((rc = from_spine(spine_gemv(kind, sp.router, sp.router_scales, hidden, b.logits, E, H, P,
                                    false, st), "router")))
      return rc;
    if ((rc = from_spine(spine_gemv(kind, sp.routed_down, sp.routed_down_scales, hidden,
                                    b.routed_in, R, H, P, false, st), "routed_down")))
      return rc;
  } else if ((rc = from_spine(rc, "router + routed_down"))) {
    return rc;
  }
  if ((rc = launch_route_sigmoid_bias(b.logits, sp.router_bias, E, top_k, P, ws.ids, ws.w,
                                      route_ids, route_weights, st)))
    return rc;
  // the routed experts
  if ((rc = experts_on_device_routes(g, bank, expert_stride, E, P, top_k, b.routed_in,
                                     b.routed_out, ws, st)))
    return rc;
  if (!side.parallel() && (rc = shared_glu(st))) return rc;
  // complete: routed_up over the routed RMS norm (staged normalised by the
  // projection itself where the shape allows), + shared_down h (one fp32 add)
  SpineOp up{};
  up.w = sp.routed_up;
  up.scales = sp.routed_up_scales;
  up.x = b.routed_out;
  up.y = out;
  up.rows = H;
  up.cols = R;
  up.positions = P;
  up.norm_w = sp.routed_norm;
  up.eps = K3_RMS_EPSILON;
  rc = spine_gemv_op(kind, up, st);
  if (rc == K3_SPINE_E_UNSUPPORTED) {
    if ((rc = from_spine(spine_rms_norm(b.routed_out, sp.routed_norm, b.routed_out, P, R,
                                        K3_RMS_EPSILON, st), "routed RMS norm")))
      return rc;
    if ((rc = from_spine(spine_gemv(kind, sp.routed_up, sp.routed_up_scales, b.routed_out, out,
                                    H, R, P, false, st), "routed_up")))
      return rc;
  } else if ((rc = from_spine(rc, "routed_up"))) {
    return rc;
  }
  if ((rc = side.join())) return rc;  // h from the side stream
  return from_spine(spine_gemv(kind, sp.shared_down, sp.shared_down_scales, b.gate, out, H, S, P,
                               true, st), "shared_down");
}

uint64_t k3_hip_geometry_span(uint32_t hidden, uint32_t intermediate) {
  if (hidden == 0 || intermediate == 0 || hidden % 32 != 0 || intermediate % 32 != 0) return 0;
  const uint64_t h = hidden, i = intermediate;
  return 2 * (i * h / 2 + i * (h / 32)) + (h * i / 2 + h * (i / 32));
}

int k3_hip_geometry_preset(int preset, K3HipGeometryV1* out) {
  if (!out) return fail(K3_HIP_E_INVALID, "null geometry output");
  if (preset == 1) {
    fill_geometry(3584, 3072, K3_ACT_SITU, out);
    return K3_HIP_OK;
  }
  if (preset == 2) {
    fill_geometry(7168, 2048, K3_ACT_SILU, out);
    return K3_HIP_OK;
  }
  return fail(K3_HIP_E_INVALID, "unknown geometry preset %d", preset);
}

const char* k3_hip_last_error(void) { return g_last_error; }

// ------------------------------------------------------------ surface 1
int k3_hip_init(const char* selector) {
  Context& c = ctx();
  std::lock_guard<std::mutex> lk(c.mu);
  return init_locked(c, selector) ? 0 : -1;
}

int k3_hip_available(void) {
  Context& c = ctx();
  std::lock_guard<std::mutex> lk(c.mu);
  return init_locked(c, nullptr) ? 1 : 0;
}

uint32_t k3_hip_descriptor_abi_version(void) { return K3_DESCRIPTOR_ABI_V1; }

uint64_t k3_hip_layout_capabilities(void) {
  Context& c = ctx();
  std::lock_guard<std::mutex> lk(c.mu);
  if (!init_locked(c, nullptr)) return 0;
  Geo g4;
  return K3_CAP_RAW_V1 | (make_geo_scale4(c.geo, &g4) ? K3_CAP_SCALE4_V2 : 0);
}

int k3_hip_scale4_check_header(const uint8_t* header, uint64_t bytes) {
  if (!header || bytes < 8192) return fail(K3_HIP_E_INVALID, "scale4-v2 header needs 8192 bytes");
  if (const char* why = scale4_header_error(header)) return fail(K3_HIP_E_DESCRIPTOR, "%s", why);
  return K3_HIP_OK;
}

int k3_hip_configure_v1(const K3HipGeometryV1* geometry) {
  Context& c = ctx();
  std::lock_guard<std::mutex> lk(c.mu);
  Geo g;
  if (!make_geo(geometry, &g)) return fail(K3_HIP_E_INVALID, "invalid geometry descriptor");
  if (!init_locked(c, nullptr)) return K3_HIP_E_INIT;
  c.gdesc = *geometry;
  c.geo = g;
  return allocate_buffers_locked(c);
}

void k3_hip_shapes(int* hidden, int* inter, long long* span) {
  Context& c = ctx();
  std::lock_guard<std::mutex> lk(c.mu);
  K3HipGeometryV1 d = c.gdesc;
  if (!c.tried) fill_geometry(3584, 3072, K3_ACT_SITU, &d);
  if (hidden) *hidden = (int)d.hidden;
  if (inter) *inter = (int)d.intermediate;
  if (span) *span = (long long)d.expert_span;
}

void k3_hip_stats(long long* five) {
  Context& c = ctx();
  std::lock_guard<std::mutex> lk(c.mu);
  if (!five) return;
  five[0] = c.calls;
  five[1] = c.device_uses;
  five[2] = c.uploads;
  five[3] = (long long)c.blobs.size();
  five[4] = c.cache_mode;
}

int k3_hip_mode(void) {
  Context& c = ctx();
  std::lock_guard<std::mutex> lk(c.mu);
  return c.cache_mode;
}

int k3_hip_set_mode(int cache_host_blobs) {
  Context& c = ctx();
  std::lock_guard<std::mutex> lk(c.mu);
  if (!init_locked(c, nullptr)) return -1;
  c.cache_mode = cache_host_blobs ? 1 : 0;
  if (!c.cache_mode) {
    for (auto& kv : c.blobs) (void)hipFree(kv.second.dev);
    c.blobs.clear();
  }
  return c.cache_mode;
}

void k3_hip_drop(const uint8_t* blob) {
  Context& c = ctx();
  std::lock_guard<std::mutex> lk(c.mu);
  auto it = c.blobs.find(blob);
  if (it == c.blobs.end()) return;
  (void)hipStreamSynchronize(c.stream);
  (void)hipFree(it->second.dev);
  c.blobs.erase(it);
}

void k3_hip_flush(void) {
  Context& c = ctx();
  std::lock_guard<std::mutex> lk(c.mu);
  if (c.blobs.empty()) return;
  (void)hipStreamSynchronize(c.stream);
  for (auto& kv : c.blobs) (void)hipFree(kv.second.dev);
  c.blobs.clear();
}

int k3_hip_moe_layer_desc_v1(const K3HipExpertDescriptorV1* experts, int expert_count,
                             const float* weights, const float* input, float* output) {
  Context& c = ctx();
  std::lock_guard<std::mutex> lk(c.mu);
  if (!init_locked(c, nullptr)) return K3_HIP_E_INIT;
  std::vector<const uint8_t*> blobs;
  Geo lg;
  const int rc = check_descriptors(c, experts, expert_count, &blobs, &lg);
  if (rc != K3_HIP_OK) return rc;
  return layer_locked(c, lg, blobs.empty() ? nullptr : blobs.data(), expert_count, weights, input,
                      output);
}

int k3_hip_moe_positions_desc_v1(const K3HipExpertDescriptorV1* experts, int edge_count,
                                 const int* position_offsets, int position_count,
                                 const float* weights, const float* input, float* output) {
  Context& c = ctx();
  std::lock_guard<std::mutex> lk(c.mu);
  if (!init_locked(c, nullptr)) return K3_HIP_E_INIT;
  std::vector<const uint8_t*> blobs;
  Geo lg;
  const int rc = check_descriptors(c, experts, edge_count, &blobs, &lg);
  if (rc != K3_HIP_OK) return rc;
  return positions_locked(c, lg, blobs.empty() ? nullptr : blobs.data(), edge_count,
                          position_offsets, position_count, weights, input, output);
}

int k3_hip_moe_positions_flat_desc_v1(const K3HipExpertDescriptorV1* experts, int edge_count,
                                      const int* position_offsets, int position_count,
                                      const float* weights, const float* input, float* output) {
  Context& c = ctx();
  std::lock_guard<std::mutex> lk(c.mu);
  if (!init_locked(c, nullptr)) return K3_HIP_E_INIT;
  std::vector<const uint8_t*> blobs;
  Geo lg;
  const int rc = check_descriptors(c, experts, edge_count, &blobs, &lg);
  if (rc != K3_HIP_OK) return rc;
  return positions_locked(c, lg, blobs.empty() ? nullptr : blobs.data(), edge_count,
                          position_offsets, position_count, weights, input, output, true);
}

int k3_hip_moe_layer(const uint8_t* const* expert_blobs, int n_experts, const float* weights,
                     const float* x, float* out) {
  Context& c = ctx();
  std::lock_guard<std::mutex> lk(c.mu);
  if (!init_locked(c, nullptr)) return K3_HIP_E_INIT;
  return layer_locked(c, c.geo, expert_blobs, n_experts, weights, x, out);
}

int k3_hip_moe_positions(const uint8_t* const* expert_blobs, int n_edges,
                         const int* position_offsets, int n_positions, const float* weights,
                         const float* x, float* out) {
  Context& c = ctx();
  std::lock_guard<std::mutex> lk(c.mu);
  if (!init_locked(c, nullptr)) return K3_HIP_E_INIT;
  return positions_locked(c, c.geo, expert_blobs, n_edges, position_offsets, n_positions, weights,
                          x, out);
}

int k3_hip_moe_positions_flat(const uint8_t* const* expert_blobs, int n_edges,
                              const int* position_offsets, int n_positions, const float* weights,
                              const float* x, float* out) {
  Context& c = ctx();
  std::lock_guard<std::mutex> lk(c.mu);
  if (!init_locked(c, nullptr)) return K3_HIP_E_INIT;
  return positions_locked(c, c.geo, expert_blobs, n_edges, position_offsets, n_positions, weights,
                          x, out, true);
}

// ------------------------------------------------------------ surface 2
uint32_t k3_hip_moe_abi_version(void) { return 1; }

void k3_hip_moe_shapes(int* hidden, int* intermediate, int64_t* expert_span,
                       uint32_t* pointer_layout) {
  int h = 0, i = 0;
  long long s = 0;
  k3_hip_shapes(&h, &i, &s);
  if (hidden) *hidden = h;
  if (intermediate) *intermediate = i;
  if (expert_span) *expert_span = s;
  if (pointer_layout) *pointer_layout = 1;
}

int k3_hip_moe_available(int device) {
  int count = 0;
  hipError_t e = hipGetDeviceCount(&count);
  if (e != hipSuccess) return fail(K3_HIP_E_INIT, "device count query: %s", hipGetErrorString(e));
  if (device < 0 || device >= count)
    return fail(K3_HIP_E_INVALID, "device %d outside the %d visible devices", device, count);
  hipDeviceProp_t prop;
  if ((e = hipGetDeviceProperties(&prop, device)) != hipSuccess)
    return fail(K3_HIP_E_INIT, "device properties: %s", hipGetErrorString(e));
  if (strncmp(prop.gcnArchName, "gfx950", 6) != 0)
    return fail(K3_HIP_E_CAPABILITY, "device %d is %s; this library is built for gfx950 only",
                device, prop.gcnArchName);
  fail(K3_HIP_OK, "available: device %d %s, %d CUs, wave %d", device, prop.gcnArchName,
       prop.multiProcessorCount, prop.warpSize);
  return 1;
}

int k3_hip_mxfp4_gemv(const uint8_t* packed, const uint8_t* scales, const float* x,
                      float* output, int rows, int cols, int batches, void* stream) {
  return launch_gemv(packed, scales, x, K3_DTYPE_F32, output, K3_DTYPE_F32, rows, cols, batches,
                     static_cast<hipStream_t>(stream));
}

int k3_hip_mxfp4_gemv_ex(const uint8_t* packed, const uint8_t* scales, const void* x,
                         int x_dtype, void* output, int out_dtype, int rows, int cols,
                         int batches, void* stream) {
  return launch_gemv(packed, scales, x, x_dtype, output, out_dtype, rows, cols, batches,
                     static_cast<hipStream_t>(stream));
}

int k3_hip_moe_launch(const K3HipGeometryV1* gd, const uint8_t* span, const float* x,
                      int batches, float* gate, float* up, float* out, void* stream) {
  Geo g;
  if (!geometry_from(gd, &g)) return fail(K3_HIP_E_INVALID, "invalid geometry");
  if (!span || !x || !gate || !up || !out)
    return fail(K3_HIP_E_INVALID, "device MoE: null input, scratch, or output pointer");
  if (batches <= 0) return fail(K3_HIP_E_INVALID, "device MoE: batch count must be positive");
  if (((uintptr_t)span & 15u) != 0 || ((uintptr_t)gate & 15u) != 0)
    return fail(K3_HIP_E_INVALID, "device MoE: span and gate must be 16-byte aligned");
  hipStream_t st = static_cast<hipStream_t>(stream);
  int rc = launch_gemv(span + g.w1p, span + g.w1s, x, K3_DTYPE_F32, gate, K3_DTYPE_F32, g.inter,
                       g.hidden, batches, st);
  if (rc == K3_HIP_OK)
    rc = launch_gemv(span + g.w3p, span + g.w3s, x, K3_DTYPE_F32, up, K3_DTYPE_F32, g.inter,
                     g.hidden, batches, st);
  if (rc == K3_HIP_OK)
    rc = launch_activation(gate, up, gate, (int64_t)batches * g.inter, g.act, st);
  if (rc == K3_HIP_OK)
    rc = launch_gemv(span + g.w2p, span + g.w2s, gate, K3_DTYPE_F32, out, K3_DTYPE_F32, g.hidden,
                     g.inter, batches, st);
  return rc;
}

uint64_t k3_hip_moe_workspace_bytes(const K3HipGeometryV1* gd, int max_edges, int max_positions) {
  Geo g;
  if (!geometry_from(gd, &g)) return 0;
  return workspace_bytes(g, max_edges, max_positions);
}

int k3_hip_moe_layer_device(const K3HipGeometryV1* gd, const uint8_t* const* experts,
                            const float* weights, int n_experts, const void* x, int x_dtype,
                            void* out, int out_dtype, void* workspace, uint64_t workspace_bytes,
                            void* stream) {
  Geo g;
  if (!geometry_from(gd, &g)) return fail(K3_HIP_E_INVALID, "invalid geometry");
  if (!experts || !weights || !x || !out)
    return fail(K3_HIP_E_INVALID, "layer: null experts/weights/x/out");
  if (n_experts <= 0 || n_experts > K3_HIP_MAX_TOKEN_EXPERTS)
    return fail(K3_HIP_E_INVALID, "layer: expert count %d outside [1, %d]", n_experts,
                K3_HIP_MAX_TOKEN_EXPERTS);
  if (!check_dtype(x_dtype) || !check_dtype(out_dtype))
    return fail(K3_HIP_E_INVALID, "layer: unknown dtype");
  if (((uintptr_t)x & 15u) != 0) return fail(K3_HIP_E_INVALID, "layer: x must be 16-byte aligned");
  Workspace ws;
  if (!carve_workspace(workspace, workspace_bytes, g, n_experts, 1, &ws))
    return fail(K3_HIP_E_INVALID, "layer: workspace missing, misaligned or smaller than %llu bytes",
                (unsigned long long)k3::workspace_bytes(g, n_experts, 1));
  TokenRoute route;
  memset(&route, 0, sizeof(route));
  route.n = n_experts;
  for (int i = 0; i < n_experts; ++i) {
    if (!experts[i] || ((uintptr_t)experts[i] & 15u) != 0)
      return fail(K3_HIP_E_INVALID, "layer: expert %d span is null or not 16-byte aligned", i);
    route.ptr[i] = experts[i];
    route.w[i] = weights[i];
  }
  return launch_decode_layer(g, route, x, x_dtype, out, out_dtype, ws,
                             static_cast<hipStream_t>(stream));
}

int k3_hip_moe_route_layer_device(const K3HipGeometryV1* gd, const uint8_t* bank,
                                  uint64_t expert_stride, int n_bank, const float* logits,
                                  int top_k, const void* x, int x_dtype, void* out, int out_dtype,
                                  int32_t* route_ids, float* route_weights, void* workspace,
                                  uint64_t workspace_bytes, void* stream) {
  Geo g;
  if (!geometry_from(gd, &g)) return fail(K3_HIP_E_INVALID, "invalid geometry");
  if (!bank || !logits || !x || !out) return fail(K3_HIP_E_INVALID, "route layer: null pointer");
  if (expert_stride < g.span || expert_stride % 16 != 0 || ((uintptr_t)bank & 15u) != 0)
    return fail(K3_HIP_E_INVALID, "route layer: bank must be 16-byte aligned with stride >= span");
  if (!check_dtype(x_dtype) || !check_dtype(out_dtype))
    return fail(K3_HIP_E_INVALID, "route layer: unknown dtype");
  if (((uintptr_t)x & 15u) != 0) return fail(K3_HIP_E_INVALID, "route layer: x must be 16-byte aligned");
  if (top_k <= 0 || top_k > K3_HIP_MAX_TOKEN_EXPERTS || top_k > n_bank)
    return fail(K3_HIP_E_INVALID, "route layer: top_k %d outside [1, min(%d, n_bank)]", top_k,
                K3_HIP_MAX_TOKEN_EXPERTS);
  Workspace ws;
  if (!carve_workspace(workspace, workspace_bytes, g, top_k, 1, &ws))
    return fail(K3_HIP_E_INVALID, "route layer: workspace missing, misaligned or too small");
  if (n_bank > 4096) return fail(K3_HIP_E_INVALID, "route layer: n_bank must be at most 4096");
  hipStream_t st = static_cast<hipStream_t>(stream);
  // Router mode: the gate/up kernel ranks the logits and publishes the route.
  TokenRoute route;
  memset(&route, 0, sizeof(route));
  route.bank = bank;
  route.stride = expert_stride;
  route.logits = logits;
  route.n_bank = n_bank;
  route.ids_pub = ws.ids;
  route.w_pub = ws.w;
  route.ids_user = route_ids;
  route.w_user = route_weights;
  route.n = top_k;
  return launch_decode_layer(g, route, x, x_dtype, out, out_dtype, ws, st);
}

int k3_hip_moe_verify_route_device(const K3HipGeometryV1* gd, const uint8_t* bank,
                                   uint64_t expert_stride, int n_bank, const float* logits,
                                   int n_positions, int top_k, const void* x, int x_dtype,
                                   void* out, int out_dtype, int32_t* route_ids,
                                   float* route_weights, void* workspace,
                                   uint64_t workspace_bytes, void* stream) {
  Geo g;
  if (!geometry_from(gd, &g)) return fail(K3_HIP_E_INVALID, "invalid geometry");
  if (!bank || !logits || !x || !out) return fail(K3_HIP_E_INVALID, "verify: null pointer");
  if (expert_stride < g.span || expert_stride % 16 != 0 || ((uintptr_t)bank & 15u) != 0)
    return fail(K3_HIP_E_INVALID, "verify: bank must be 16-byte aligned with stride >= span");
  if (!check_dtype(x_dtype) || !check_dtype(out_dtype))
    return fail(K3_HIP_E_INVALID, "verify: unknown dtype");
  if (((uintptr_t)x & 15u) != 0) return fail(K3_HIP_E_INVALID, "verify: x must be 16-byte aligned");
  if (n_positions <= 0 || n_positions > K3_HIP_MAX_POSITIONS)
    return fail(K3_HIP_E_INVALID, "verify: positions %d outside [1, %d]", n_positions,
                K3_HIP_MAX_POSITIONS);
  if (top_k <= 0 || top_k > K3_HIP_MAX_TOKEN_EXPERTS || top_k > n_bank ||
      n_positions * top_k > K3_HIP_MAX_EDGES)
    return fail(K3_HIP_E_INVALID, "verify: top_k %d invalid for %d positions", top_k, n_positions);
  const int n_edges = n_positions * top_k;
  Workspace ws;
  if (!carve_workspace(workspace, workspace_bytes, g, n_edges, n_positions, &ws))
    return fail(K3_HIP_E_INVALID, "verify: workspace missing, misaligned or too small");
  if (n_bank > 4096) return fail(K3_HIP_E_INVALID, "verify: n_bank must be at most 4096");
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int mode = g_verify_mode.load();
  if (mode == K3_VERIFY_UNION_MFMA && !verify_mfma_supported(g))
    return fail(K3_HIP_E_CAPABILITY, "verify: this geometry/layout has no matrix-core path");
  // Union paths: route every position (one workgroup each), group the edges
  // by expert, then read each routed expert once for all of its positions.
  // A position's top_k experts are distinct, so no expert has more than
  // n_positions <= 16 edges.
  const bool shared = expected_union(n_bank, top_k, n_positions) <=
                      kUnionFraction * (double)n_edges;
  const bool mfma = mode == K3_VERIFY_UNION_MFMA ||
                    (mode == K3_VERIFY_AUTO && n_positions >= 2 && shared &&
                     verify_mfma_supported(g));
  if (mfma || mode == K3_VERIFY_UNION_VALU) {
    int rc = launch_route(logits, n_bank, top_k, n_positions, ws.ids, ws.w, route_ids,
                          route_weights, st);
    if (rc == K3_HIP_OK)
      rc = launch_verify_plan_bank(g, bank, expert_stride, n_bank, n_positions, top_k, ws, st,
                                   mfma ? x : nullptr, x_dtype);
    if (rc != K3_HIP_OK) return rc;
    return mfma ? launch_verify_mfma(g, n_edges, n_positions, x, x_dtype, out, out_dtype, ws, st,
                                     true)
                : launch_verify_layer(g, n_edges, n_positions, x, x_dtype, out, out_dtype, ws, st);
  }
  // One routed decode layer per position: each position's gate/up workgroups
  // rank its own logits, so the routes equal the per-position router's.  An
  // expert picked by several positions is read once per position.  Where the
  // geometry allows, all positions run as one gate/up launch and one down
  // launch (position on the grid's y axis: one position's workgroups start as
  // the previous one's finish, with no launch boundary between positions);
  // otherwise one layer after another on the stream.
  const size_t xb = x_dtype == K3_DTYPE_BF16 ? 2 : 4, ob = out_dtype == K3_DTYPE_BF16 ? 2 : 4;
  TokenRoute route;
  memset(&route, 0, sizeof(route));
  route.bank = bank;
  route.stride = expert_stride;
  route.logits = logits;
  route.n_bank = n_bank;
  route.ids_pub = ws.ids;
  route.w_pub = ws.w;
  route.ids_user = route_ids;
  route.w_user = route_weights;
  route.n = top_k;
  if (K3_BATCH_POSITIONS && n_positions > 1 && decode_positions_supported(g, top_k))
    return launch_decode_positions(g, route, n_positions, x, x_dtype, out, out_dtype, ws, st);
  for (int p = 0; p < n_positions; ++p) {
    TokenRoute rp = route;
    rp.logits = logits + (size_t)p * n_bank;
    rp.ids_user = route_ids ? route_ids + (size_t)p * top_k : nullptr;
    rp.w_user = route_weights ? route_weights + (size_t)p * top_k : nullptr;
    const int rc = launch_decode_layer(g, rp, static_cast<const uint8_t*>(x) + p * g.hidden * xb,
                                       x_dtype, static_cast<uint8_t*>(out) + p * g.hidden * ob,
                                       out_dtype, ws, st);
    if (rc != K3_HIP_OK) return rc;
  }
  return K3_HIP_OK;
}

int k3_hip_moe_verify_device(const K3HipGeometryV1* gd, const uint8_t* const* edge_experts,
                             const float* edge_weights, const int* position_offsets,
                             int n_positions, const void* x, int x_dtype, void* out,
                             int out_dtype, void* workspace, uint64_t workspace_bytes,
                             void* stream) {
  Geo g;
  if (!geometry_from(gd, &g)) return fail(K3_HIP_E_INVALID, "invalid geometry");
  if (!position_offsets || !x || !out) return fail(K3_HIP_E_INVALID, "verify: null pointer");
  if (!check_dtype(x_dtype) || !check_dtype(out_dtype))
    return fail(K3_HIP_E_INVALID, "verify: unknown dtype");
  if (((uintptr_t)x & 15u) != 0) return fail(K3_HIP_E_INVALID, "verify: x must be 16-byte aligned");
  if (n_positions <= 0 || n_positions > K3_HIP_MAX_POSITIONS)
    return fail(K3_HIP_E_INVALID, "verify: positions %d outside [1, %d]", n_positions,
                K3_HIP_MAX_POSITIONS);
  if (position_offsets[0] != 0) return fail(K3_HIP_E_INVALID, "verify: offsets must start at 0");
  for (int p = 0; p < n_positions; ++p)
    if (position_offsets[p] > position_offsets[p + 1])
      return fail(K3_HIP_E_INVALID, "verify: offsets must be non-decreasing");
  const int n_edges = position_offsets[n_positions];
  if (n_edges < 0 || n_edges > K3_HIP_MAX_EDGES)
    return fail(K3_HIP_E_INVALID, "verify: %d edges outside [0, %d]", n_edges, K3_HIP_MAX_EDGES);
  if (n_edges > 0 && (!edge_experts || !edge_weights))
    return fail(K3_HIP_E_INVALID, "verify: null edge arrays");
  Workspace ws;
  if (!carve_workspace(workspace, workspace_bytes, g, std::max(n_edges, 1), n_positions, &ws))
    return fail(K3_HIP_E_INVALID, "verify: workspace missing, misaligned or too small");
  hipStream_t st = static_cast<hipStream_t>(stream);
  EdgeTable tbl;
  memset(&tbl, 0, sizeof(tbl));
  tbl.n_edges = n_edges;
  tbl.n_positions = n_positions;
  for (int p = 0; p <= n_positions; ++p) tbl.pos_off[p] = position_offsets[p];
  for (int i = 0; i < n_edges; ++i) {
    if (!edge_experts[i] || ((uintptr_t)edge_experts[i] & 15u) != 0)
      return fail(K3_HIP_E_INVALID, "verify: edge %d span is null or misaligned", i);
    tbl.ptr[i] = edge_experts[i];
    tbl.w[i] = edge_weights[i];
  }
  return verify_table(g, tbl, x, x_dtype, out, out_dtype, ws, st, false);
}

int k3_hip_set_fused_decode(int enabled) { return set_fused_decode(enabled); }
int k3_hip_set_decode_chain(int mode) { return set_decode_chain(mode); }

int k3_hip_set_decode_mfma(int mode) { return set_decode_mfma(mode); }

int k3_hip_set_verify_mode(int mode) {
  if (mode < K3_VERIFY_AUTO || mode > K3_VERIFY_UNION_VALU)
    return fail(K3_HIP_E_INVALID, "verify mode %d unknown", mode);
  return g_verify_mode.exchange(mode);
}

int k3_hip_synth_bank(const K3HipGeometryV1* gd, uint8_t* bank, uint64_t expert_stride,
                      int n_experts, uint64_t first_expert, uint64_t seed, int scale_lo,
                      int scale_hi, void* stream) {
  Geo g;
  if (!geometry_from(gd, &g)) return fail(K3_HIP_E_INVALID, "invalid geometry");
  return launch_synth_bank(g, bank, expert_stride, n_experts, first_expert, seed, scale_lo,
                           scale_hi, static_cast<hipStream_t>(stream));
}

int k3_hip_synth_normal(void* out, int dtype, uint64_t n, uint64_t seed, uint64_t stream,
                        void* stream_handle) {
  return launch_synth_normal(out, dtype, n, seed, stream, static_cast<hipStream_t>(stream_handle));
}

}  // extern "C"
