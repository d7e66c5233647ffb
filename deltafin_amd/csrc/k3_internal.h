// Internal declarations shared by the kernel and host translation units.
#pragma once

#include <hip/hip_runtime_api.h>
#include <stdint.h>

#include "../../include/k3_hip_moe_abi.h"
#include "../../include/k3_hip_spine_abi.h"

namespace k3 {

// Byte offsets of one expert span: raw-v1 (provider_moe.cpp:217-243), or
// scale4-v2 (tools/metal_moe.mm:127-155), where w1s / w2s / w3s are planes of
// 4-bit scale indices (two per byte, low nibble first, over the flattened
// [rows][groups] scale order) and the E8M0 scale of index d is base + d, the
// three bases being bytes 64, 65, 66 of the span (w1, w2, w3).
struct Geo {
  int hidden;        // H: gate/up columns, down rows, x/out length
  int inter;         // I: gate/up rows, down columns, h length
  int act;           // K3_ACT_*
  uint64_t w1p, w1s, w2p, w2s, w3p, w3s, span;
  int layout;        // K3_LAYOUT_RAW_V1 or K3_LAYOUT_SCALE4_V2
};

bool make_geo(const K3HipGeometryV1* g, Geo* out);
// The scale4-v2 layout of a raw geometry: the reference fixes it for K3 only
// (hidden 3584, intermediate 3072, span 17,039,360); false otherwise.
bool make_geo_scale4(const Geo& raw, Geo* out);
// Header checks of a scale4-v2 span (tools/metal_moe.mm:353-405); p holds the
// span's first 8192 bytes in host memory.  nullptr when valid, else the reason.
const char* scale4_header_error(const uint8_t* p);

// Expert addressing for one token (decode) or one edge set: either a resident
// bank indexed by device-side ids, or explicit span pointers passed by value.
struct TokenRoute {
  const uint8_t* bank;      // bank mode when non-null
  uint64_t stride;          // bank expert stride in bytes
  const int32_t* ids;       // bank mode: device ids [n]
  const float* wdev;        // bank mode: device weights [n]
  // Router mode (bank mode with logits): the kernel that consumes the route
  // computes the top n of logits[n_bank] itself and publishes ids/weights to
  // ids_pub/w_pub (and the optional user copies) for later kernels.
  const float* logits;
  int n_bank;
  int32_t* ids_pub;
  float* w_pub;
  int32_t* ids_user;
  float* w_user;
  // Table mode (no bank, pdev non-null): a caller route already in device
  // memory, span pointers pdev[p * n + e] and weights wdev[p * n + e] for
  // position p (the position-batched decode of caller routes).
  const uint8_t* const* pdev;
  const uint8_t* ptr[K3_HIP_MAX_TOKEN_EXPERTS];
  float w[K3_HIP_MAX_TOKEN_EXPERTS];
  int n;
};

// Verify plan in device workspace, built by k_verify_plan.
struct VerifyPlanDev {
  int n_unique;
  int n_edges;
  int n_positions;
  int pad;
};

// Caller route for verify, passed by value to the plan kernel.
struct EdgeTable {
  const uint8_t* ptr[K3_HIP_MAX_EDGES];
  float w[K3_HIP_MAX_EDGES];
  int pos_off[K3_HIP_MAX_POSITIONS + 1];
  int n_edges;
  int n_positions;
};

// Workspace carve-up (all offsets 256-byte aligned).
struct Workspace {
  uint8_t* base;
  uint64_t bytes;
  float* h;             // [max_edges][I] activations (decode: lane-major per expert)
  float* y;             // [max_edges][H] per-edge expert outputs (verify)
  int32_t* ids;         // [max_edges] route ids
  float* w;             // [max_edges] route weights
  const uint8_t** uptr; // [max_edges] unique expert pointers
  int32_t* uoff;        // [max_edges + 1] unique -> edge-list offsets
  int32_t* uedges;      // [max_edges] edges grouped by unique expert
  int32_t* epos;        // [max_edges] edge -> position
  int32_t* poff;        // [max_positions + 1]
  VerifyPlanDev* plan;  // 1
  // MFMA verify operands: activations split into fp8 (E4M3) terms with one
  // E8M0 scale per 32 elements and term, row-major [row][term][K] bytes and
  // [row][term][K / 32] scale bytes (kMaxTerms terms per row).
  uint8_t* xq;          // [max_positions][kMaxTerms][H]
  uint8_t* xqs;         // [max_positions][kMaxTerms][H / 32]
  uint8_t* hq;          // [max_edges][kMaxTerms][I]
  uint8_t* hqs;         // [max_edges][kMaxTerms][I / 32]
};

// Most fp8 terms an activation row is split into (fp32 rows take three).
constexpr int kMaxTerms = 3;

uint64_t workspace_bytes(const Geo& g, int max_edges, int max_positions);
bool carve_workspace(void* base, uint64_t bytes, const Geo& g, int max_edges,
                     int max_positions, Workspace* ws);

// Thread-local error reporting.
int fail(int status, const char* fmt, ...);
int hip_fail(const char* what, hipError_t e);

// Kernel launchers (k3_kernels.hip).  All validate shapes on the host and
// return a K3_HIP_* status.
int launch_gemv(const uint8_t* packed, const uint8_t* scales, const void* x,
                int x_dtype, void* out, int out_dtype, int rows, int cols,
                int batches, hipStream_t stream);
int launch_activation(const float* gate, const float* up, float* h, int64_t n,
                      int act, hipStream_t stream);
int launch_route(const float* logits, int n_bank, int top_k, int n_positions,
                 int32_t* ids_ws, float* w_ws, int32_t* ids_user,
                 float* w_user, hipStream_t stream);
// K3 router: top_k of sigmoid(logits) + bias per position, weighted by the
// selected sigmoids over their sum + 1e-20 (provider_moe.cpp:1673-1683).
int launch_route_sigmoid_bias(const float* logits, const float* bias, int n_bank, int top_k,
                              int n_positions, int32_t* ids_ws, float* w_ws, int32_t* ids_user,
                              float* w_user, hipStream_t stream);
// Decode layer.  When route.logits is set (router mode) the gate/up kernel
// routes the token itself and publishes the route to ws.ids / ws.w.
int launch_decode_layer(const Geo& g, const TokenRoute& route, const void* x,
                        int x_dtype, void* out, int out_dtype,
                        const Workspace& ws, hipStream_t stream);
// n_positions decode layers of one bank-mode or table-mode route (router
// mode: logits strided by n_bank; caller mode: ids or pdev, and wdev, strided
// by route.n) as one
// gate/up launch and one down launch, position p on blockIdx.y: x and out rows
// strided by hidden, h by route.n * intermediate (ws holds n_positions *
// route.n edges).  Outputs equal n_positions launch_decode_layer calls bit for
// bit.  Only where decode_positions_supported holds (k_down_g64 / k_down_g96
// geometries, at most 16 experts, fused decode off).
bool decode_positions_supported(const Geo& g, int n);
int launch_decode_positions(const Geo& g, const TokenRoute& route, int n_positions,
                            const void* x, int x_dtype, void* out, int out_dtype,
                            const Workspace& ws, hipStream_t stream);
// Process-wide decode path switch (k3_hip_set_fused_decode); returns the
// previous setting.
int set_fused_decode(int enabled);
// One-launch path for one-expert layers (k3_hip_set_decode_chain: 0 off, 1
// on, 2 on with its missing-share fallback taken at once); returns the
// previous setting, or K3_HIP_E_INVALID for another value.
int set_decode_chain(int mode);
// Process-wide choice of the single-token gate/up dots (k3_hip_set_decode_mfma:
// 0 VALU, 1 matrix cores for fp32 activations, 2 also for bf16); returns the
// previous setting, or K3_HIP_E_INVALID for another value.
int set_decode_mfma(int mode);
// LDS bytes the in-kernel router needs for a bank of n_bank logits and top_k.
size_t route_scratch_bytes(int n_bank, int top_k);
// The verify plan (edges grouped by expert) in ws.  x_split (the positions'
// activations, x_dtype bf16 or fp32): the same launch also writes their
// matrix-core terms, and launch_verify_mfma is then called with x_split_done.
int launch_verify_plan_bank(const Geo& g, const uint8_t* bank, uint64_t stride, int n_bank,
                            int n_positions, int top_k, const Workspace& ws,
                            hipStream_t stream, const void* x_split = nullptr,
                            int x_dtype = 0);
int launch_verify_plan_table(const Geo& g, const EdgeTable& table, const Workspace& ws,
                             hipStream_t stream, const void* x_split = nullptr,
                             int x_dtype = 0);
// Edges e0 .. e0 + n - 1 of a caller route table into the workspace as a
// table-mode route (ws.uptr span pointers, ws.w weights).
int launch_route_table(const EdgeTable& table, int e0, int n, const Workspace& ws,
                       hipStream_t stream);
// The VALU union verify kernels over the plan in ws, then the combine.
int launch_verify_layer(const Geo& g, int n_edges, int n_positions,
                        const void* x, int x_dtype, void* out, int out_dtype,
                        const Workspace& ws, hipStream_t stream);
// Per-position route-ordered combine of ws.y (edge outputs) into out.
int launch_verify_combine(const Geo& g, int n_positions, void* out, int out_dtype,
                          const Workspace& ws, hipStream_t stream);
// Matrix-core verify (k3_verify_mfma.hip): split x, gate/up units, split h,
// down units, combine.  Needs a plan in ws whose experts each have at most 16
// edges, and a geometry verify_mfma_supported accepts.
bool verify_mfma_supported(const Geo& g);
int launch_verify_mfma(const Geo& g, int n_edges, int n_positions, const void* x,
                       int x_dtype, void* out, int out_dtype, const Workspace& ws,
                       hipStream_t stream, bool x_split_done = false);
int launch_synth_bank(const Geo& g, uint8_t* bank, uint64_t stride,
                      int n_experts, uint64_t first_expert, uint64_t seed,
                      int lo, int hi, hipStream_t stream);
int launch_synth_normal(void* out, int dtype, uint64_t n, uint64_t seed,
                        uint64_t stream_id, hipStream_t stream);
// Zero `bytes` (a multiple of 4) at a 4-byte aligned device pointer with a
// kernel (graph-capturable, unlike a memset node).
int launch_zero(void* p, uint64_t bytes, hipStream_t stream);

int device_cu_count();
// Whether one workgroup of `kernel` at `block` threads with `dynamic_lds`
// bytes of dynamic LDS fits on a CU of the current device, after raising the
// kernel's dynamic-LDS ceiling (cached per kernel, shape and device).
bool lds_fits(const void* kernel, int block, size_t dynamic_lds);

// Kernel classes for the optional per-launch timing (k3_hip_timing_begin/end).
enum KernelClass : int {
  KC_GEMV = 0,
  KC_ACTIVATE,
  KC_ROUTE,
  KC_GLU_DECODE,
  KC_DOWN_DECODE,
  KC_VERIFY_PLAN,
  KC_GLU_VERIFY,
  KC_DOWN_VERIFY,
  KC_COMBINE,
  KC_SYNTH,
  KC_DECODE_FUSED,
  KC_SPLIT,
  KC_GLU_MFMA,
  KC_DOWN_MFMA,
  KC_SPINE,
  KC_RMS_NORM,
  KC_SPINE_MFMA,
  KC_DECODE_CHAIN,
  KC_COUNT
};

// While timing is enabled, reserves a pair of hipEvents for one kernel launch:
// the launch hands them to hipExtLaunchKernel, which stamps them with the
// kernel's own start and end.  Both are null (an untimed launch) otherwise.
// A launch that fails calls failed() so its unstamped pair is not read.
class TimedLaunch {
 public:
  TimedLaunch(int kernel_class, hipStream_t stream);
  TimedLaunch(const TimedLaunch&) = delete;
  TimedLaunch& operator=(const TimedLaunch&) = delete;
  hipEvent_t start() const;
  hipEvent_t stop() const;
  void failed();

 private:
  int slot_;
};

// Spine projections (k3_spine.hip).  Statuses are the K3_SPINE_* codes of the
// spine surface; failures record their reason through spine_fail.
enum { K3_SPINE_KIND_BF16 = 0, K3_SPINE_KIND_INT8 = 1 };
int spine_fail(int status, const char* fmt, ...);
// accumulate: y += W x instead of y = W x (one fp32 add per output).
int spine_gemv(int kind, const void* weights, const float* row_scales, const float* x,
               float* y, int rows, int cols, int positions, bool accumulate, hipStream_t stream);
// One spine projection with the fused forms: w2 (GLU): y = act(W x, W2 x) per
// row (no accumulate); wb: a second matrix's rows after W's (see below);
// norm_w: x is first RMS-normed per position,
// norm_w * (x * rsqrt(mean(x^2) + eps)).  A fused form the shape cannot take
// returns K3_SPINE_E_UNSUPPORTED before enqueuing anything.
struct SpineOp {
  const void* w;
  const float* scales;
  const void* w2;
  const float* scales2;
  int act;
  const float* x;
  float* y;
  int rows, cols, positions;
  bool accumulate;
  const float* norm_w;
  float eps;
  // A second matrix of the same width over the same x (wb, scales_b: rows_b
  // rows into yb [P][rows_b]), in the same launch; single position group only.
  const void* wb;
  const float* scales_b;
  float* yb;
  int rows_b;
};
int spine_gemv_op(int kind, const SpineOp& op, hipStream_t stream);
// Matrix-core spine (k3_spine_mfma.hip, BF16 matrices, 1..16 positions, cols a
// multiple of 64): split x [P, cols] into BF16 terms (spine_mfma_terms_bytes of
// device memory, 16-byte aligned), then y = W x (+ y) from those terms.
uint64_t spine_mfma_terms_bytes(int positions, int cols);
bool spine_mfma_supported(int kind, int positions, int rows, int cols);
int spine_mfma_split(const float* x, int positions, int cols, void* terms, hipStream_t stream);
int spine_mfma_gemv(const void* w, const void* terms, float* y, int rows, int cols, int positions,
                    bool accumulate, hipStream_t stream);
int spine_decode_bits(const uint16_t* in, uint32_t* out, int count, hipStream_t stream);
int spine_rms_norm(const float* in, const float* weight, float* out, int rows, int cols,
                   float eps, hipStream_t stream);
// The same norm (rows <= 16, cols a multiple of 64, 16-byte aligned), which
// also writes the normalised rows' matrix-core terms (spine_mfma_split's
// layout and values) into terms; K3_SPINE_E_UNSUPPORTED for other shapes.
int spine_rms_norm_terms(const float* in, const float* weight, float* out, int rows, int cols,
                         float eps, void* terms, hipStream_t stream);

}  // namespace k3
