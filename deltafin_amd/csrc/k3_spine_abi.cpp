// C ABI of the spine surface (include/k3_hip_spine_abi.h): argument checks,
// device qualification and the thread-local error text.  The kernels are in
// k3_spine.hip.
#include <hip/hip_runtime_api.h>
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include "k3_internal.h"

namespace k3 {
namespace {
thread_local char g_spine_error[512] = "no error";
}  // namespace

int spine_fail(int status, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_spine_error, sizeof(g_spine_error), fmt, ap);
  va_end(ap);
  return status;
}

}  // namespace k3

using namespace k3;

extern "C" {

uint32_t k3_hip_spine_bf16_abi_version(void) { return K3_SPINE_ABI_VERSION; }

const char* k3_hip_spine_last_error(void) { return g_spine_error; }

int k3_hip_spine_bf16_available(int device, int* compute_major, int* compute_minor) {
  int count = 0;
  hipError_t e = hipGetDeviceCount(&count);
  if (e != hipSuccess)
    return spine_fail(K3_SPINE_E_RUNTIME, "device count query: %s", hipGetErrorString(e));
  if (device < 0 || device >= count)
    return spine_fail(K3_SPINE_E_UNSUPPORTED,
                      "RAW_BF16 availability: device index is outside the visible range");
  hipDeviceProp_t prop;
  if ((e = hipGetDeviceProperties(&prop, device)) != hipSuccess)
    return spine_fail(K3_SPINE_E_RUNTIME, "device properties: %s", hipGetErrorString(e));
  if (prop.computeMode == hipComputeModeProhibited)
    return spine_fail(K3_SPINE_E_UNSUPPORTED, "RAW_BF16 availability: compute mode is prohibited");
  if (strncmp(prop.gcnArchName, "gfx950", 6) != 0 || prop.warpSize != 64)
    return spine_fail(K3_SPINE_E_UNSUPPORTED,
                      "RAW_BF16 availability: device %d is %s with %d-lane waves; this library "
                      "is built for gfx950 (64-lane) only",
                      device, prop.gcnArchName, prop.warpSize);
  if (compute_major) *compute_major = prop.major;
  if (compute_minor) *compute_minor = prop.minor;
  spine_fail(K3_SPINE_OK, "available: HIP device %d architecture %d.%d (%s)", device, prop.major,
             prop.minor, prop.gcnArchName);
  return 1;
}

int k3_hip_spine_bf16_launch_v1(const uint16_t* weights, const float* activation, float* output,
                                int rows, int columns, int positions, void* stream) {
  return spine_gemv(K3_SPINE_KIND_BF16, weights, nullptr, activation, output, rows, columns,
                    positions, false, static_cast<hipStream_t>(stream));
}

int k3_hip_spine_bf16_decode_bits(const uint16_t* input, uint32_t* output, int count,
                                  void* stream) {
  return spine_decode_bits(input, output, count, static_cast<hipStream_t>(stream));
}

int k3_hip_spine_int8_launch_v1(const int8_t* quantized, const float* row_scales,
                                const float* activation, float* output, int rows, int columns,
                                int positions, void* stream) {
  return spine_gemv(K3_SPINE_KIND_INT8, quantized, row_scales, activation, output, rows, columns,
                    positions, false, static_cast<hipStream_t>(stream));
}

int k3_hip_rms_norm(const float* input, const float* weight, float* output, int rows, int columns,
                    float eps, void* stream) {
  return spine_rms_norm(input, weight, output, rows, columns, eps,
                        static_cast<hipStream_t>(stream));
}

}  // extern "C"
