/* Compiled as plain C11 against include/k3_hip_moe_abi.h and linked to the
 * library, the way a C (or Rust FFI) caller would.  Calls only host-side
 * entry points: no kernel is launched, so it runs without a GPU.
 * Prints "ok" and exits 0 on success. */
#include <stddef.h>
#include <stdio.h>
#include <string.h>

#include "k3_hip_moe_abi.h"

#define CHECK(c)                                                   \
  do {                                                             \
    if (!(c)) {                                                    \
      fprintf(stderr, "check failed: %s (line %d)\n", #c, __LINE__); \
      return 1;                                                    \
    }                                                              \
  } while (0)

_Static_assert(sizeof(K3HipExpertDescriptorV1) == 32, "descriptor size");
_Static_assert(offsetof(K3HipExpertDescriptorV1, blob_bytes) == 16, "descriptor offset");
_Static_assert(offsetof(K3HipExpertDescriptorV1, blob) == 24, "descriptor offset");
_Static_assert(sizeof(K3HipGeometryV1) == 32, "geometry size");
_Static_assert(sizeof(K3HipKernelTimingV1) == 64, "timing row size");

int main(void) {
  K3HipGeometryV1 g;
  CHECK(k3_hip_geometry_span(3584, 3072) == K3_RAW_V1_EXPERT_SPAN);
  CHECK(k3_hip_geometry_span(7168, 2048) == UINT64_C(23396352));
  CHECK(k3_hip_geometry_span(7168, 2047) == 0);
  CHECK(k3_hip_geometry_preset(1, &g) == K3_HIP_OK);
  CHECK(g.hidden == 3584 && g.intermediate == 3072 && g.activation == K3_ACT_SITU);
  CHECK(g.expert_span == K3_RAW_V1_EXPERT_SPAN && g.struct_bytes == 32 && g.abi_version == 1);
  CHECK(k3_hip_geometry_preset(2, &g) == K3_HIP_OK);
  CHECK(g.hidden == 7168 && g.intermediate == 2048 && g.activation == K3_ACT_SILU);
  CHECK(k3_hip_geometry_preset(3, &g) == K3_HIP_E_INVALID);
  CHECK(strstr(k3_hip_last_error(), "preset") != NULL);
  CHECK(k3_hip_descriptor_abi_version() == K3_DESCRIPTOR_ABI_V1);
  CHECK(k3_hip_moe_abi_version() == 1);

  /* Workspace sizing is host arithmetic. */
  k3_hip_geometry_preset(2, &g);
  CHECK(k3_hip_moe_workspace_bytes(&g, 16, 1) > (uint64_t)16 * 2048 * 4);
  CHECK(k3_hip_moe_workspace_bytes(&g, 256, 16) > k3_hip_moe_workspace_bytes(&g, 16, 1));

  /* Argument validation happens before any device work. */
  CHECK(k3_hip_mxfp4_gemv(NULL, NULL, NULL, NULL, 1, 32, 1, NULL) == K3_HIP_E_INVALID);
  {
    static unsigned char buf[64] __attribute__((aligned(16)));
    CHECK(k3_hip_mxfp4_gemv(buf, buf, (const float*)buf, (float*)buf, 1, 33, 1, NULL) ==
          K3_HIP_E_INVALID);
    CHECK(k3_hip_mxfp4_gemv(buf, buf, (const float*)buf, (float*)buf, 0, 32, 1, NULL) ==
          K3_HIP_E_INVALID);
    CHECK(k3_hip_mxfp4_gemv_ex(buf, buf, buf, 7, buf, K3_DTYPE_F32, 1, 32, 1, NULL) ==
          K3_HIP_E_INVALID);
  }
  {
    K3HipGeometryV1 bad = g;
    bad.expert_span += 1;
    CHECK(k3_hip_moe_workspace_bytes(&bad, 16, 1) == 0);
    bad = g;
    bad.reserved = 1;
    CHECK(k3_hip_moe_workspace_bytes(&bad, 16, 1) == 0);
  }
  CHECK(k3_hip_moe_layer_device(&g, NULL, NULL, 0, NULL, K3_DTYPE_BF16, NULL, K3_DTYPE_BF16, NULL,
                                0, NULL) == K3_HIP_E_INVALID);
  CHECK(k3_hip_timing_end(NULL, 0, NULL, NULL) == K3_HIP_E_INVALID);
  CHECK(k3_hip_timing_begin(0) == K3_HIP_E_INVALID);
  printf("ok\n");
  return 0;
}
