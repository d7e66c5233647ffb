// Allocation-free form of the routed decode layer with the device router
// (k3_hip_moe_route_layer_device).  The caller passes inputs and outputs only;
// the layer's device scratch (the gate/up activations h, the published route
// and the carve-up the layer kernels share) is a file-scope device array of
// K3_HIP_NOALLOC_SCRATCH_BYTES that every call on one GPU shares.  Nothing here
// or in the launch path allocates device or host memory.
//
// Host code never passes `scratch` itself to a kernel: in host code the name
// is a host-side shadow of the device symbol.  Its device address is looked up
// once per device with hipGetSymbolAddress while that device is current, and
// that address is what the layer receives as its workspace.
#include <hip/hip_runtime.h>

#include <mutex>

#include "k3_internal.h"

namespace {

constexpr uint64_t kScratchBytes = K3_HIP_NOALLOC_SCRATCH_BYTES;
static_assert(kScratchBytes % 256 == 0, "scratch size must keep 256-byte carving");

// Held by each device until the process ends.
static __device__ __align__(256) uint8_t scratch[kScratchBytes];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

// Device address of `scratch` on the current device (looked up on the first
// call per device).
int scratch_address(void** out) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return k3::hip_fail("noalloc: hipGetDevice", e);
  if (dev < 0 || dev >= kMaxDevices)
    return k3::fail(K3_HIP_E_INVALID, "noalloc: device %d outside [0, %d)", dev, kMaxDevices);
  std::lock_guard<std::mutex> lk(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p) {
      (void)hipGetLastError();
      return k3::fail(K3_HIP_E_INIT, "noalloc: hipGetSymbolAddress(scratch) on device %d: %s", dev,
                      hipGetErrorString(e));
    }
    if (((uintptr_t)p & 255u) != 0)
      return k3::fail(K3_HIP_E_INIT, "noalloc: scratch on device %d is not 256-byte aligned", dev);
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return K3_HIP_OK;
}

}  // namespace

extern "C" int k3_hip_moe_route_layer_device_noalloc(
    const K3HipGeometryV1* g, const uint8_t* bank, uint64_t expert_stride, int n_bank,
    const float* logits, int top_k, const void* x, int x_dtype, void* out, int out_dtype,
    int32_t* route_ids, float* route_weights, void* stream) {
  if (top_k <= 0 || top_k > K3_HIP_MAX_TOKEN_EXPERTS)
    return k3::fail(K3_HIP_E_INVALID, "noalloc: top_k %d outside [1, %d]", top_k,
                    K3_HIP_MAX_TOKEN_EXPERTS);
  const uint64_t need = k3_hip_moe_workspace_bytes(g, top_k, 1);
  if (need == 0) return k3::fail(K3_HIP_E_INVALID, "noalloc: invalid geometry");
  if (need > kScratchBytes)
    return k3::fail(K3_HIP_E_INVALID,
                    "noalloc: this geometry at top_k %d needs %llu bytes of scratch; the "
                    "allocation-free entry point holds %llu",
                    top_k, (unsigned long long)need, (unsigned long long)kScratchBytes);
  void* ws = nullptr;
  const int rc = scratch_address(&ws);
  if (rc != K3_HIP_OK) return rc;
  return k3_hip_moe_route_layer_device(g, bank, expert_stride, n_bank, logits, top_k, x, x_dtype,
                                       out, out_dtype, route_ids, route_weights, ws,
                                       kScratchBytes, stream);
}
