#ifndef K3_HIP_MOE_ABI_H
#define K3_HIP_MOE_ABI_H

/*
 * MI355X (gfx950) routed-expert MXFP4 library: C ABI.
 *
 * Two surfaces, both plain C (pointers, sizes, int status codes):
 *
 *  1. Host-synchronous descriptor surface, the HIP counterpart of the Metal
 *     bridge (tools/metal_moe_abi.h:14-64, tools/metal_moe.mm:17-84).  Calls are
 *     serialised by one library mutex, take host fp32 activations/weights and
 *     return host fp32 outputs.  Expert blobs may live in host memory (they are
 *     staged into an HBM cache keyed by pointer, released by k3_hip_drop) or in
 *     device memory (used in place).
 *
 *  2. Stream-explicit device surface, the HIP counterpart of k3_cuda_*
 *     (tools/cuda_moe_kernels.cu:244-449): device pointers in and out, caller
 *     stream, no allocation, no synchronisation, no retained pointer.
 *
 * Status codes follow tools/metal_moe.mm (0 ok, -1 init, -2 invalid argument,
 * -3 allocation, -4 copy, -5 execution, -6 capability miss, -7 invalid
 * descriptor).  The last failure text is thread-local: k3_hip_last_error().
 *
 * Expert layout (raw-v1 ordering, provider_moe.cpp:217-243): one contiguous
 * span per expert holding w1(gate) packed, w1 scales, w2(down) packed, w2
 * scales, w3(up) packed, w3 scales.  Packed = two E2M1 codes per byte, LOW
 * nibble first; scales = one E8M0 byte per 32 elements (tools/fused_gemv.c:4-6).
 * A scale byte of 255 makes its row NaN (tools/cuda_moe_kernels.cu:128-131).
 */

#include <stddef.h>
#include <stdint.h>

/* ------------------------------------------------------------------ layouts */
/* Same values as tools/metal_moe_abi.h:14-24. */
enum {
  K3_LAYOUT_RAW_V1 = 1,
  K3_LAYOUT_SCALE4_V2 = 2,
  K3_DESCRIPTOR_ABI_V1 = 1,
};

#define K3_RAW_V1_EXPERT_SPAN UINT64_C(17547264)
#define K3_SCALE4_V2_EXPERT_SPAN UINT64_C(17039360)
#define K3_CAP_RAW_V1 (UINT64_C(1) << K3_LAYOUT_RAW_V1)
#define K3_CAP_SCALE4_V2 (UINT64_C(1) << K3_LAYOUT_SCALE4_V2)

/* Status codes (tools/metal_moe.mm ABI comment, :17-84). */
enum {
  K3_HIP_OK = 0,
  K3_HIP_E_INIT = -1,
  K3_HIP_E_INVALID = -2,
  K3_HIP_E_ALLOC = -3,
  K3_HIP_E_COPY = -4,
  K3_HIP_E_EXEC = -5,
  K3_HIP_E_CAPABILITY = -6,
  K3_HIP_E_DESCRIPTOR = -7,
};

/* Activation between gate/up and down.  SiTU is the reference's
 * (provider_moe.cpp:524-533); SiLU-GLU is silu(gate) * up. */
enum { K3_ACT_SITU = 0, K3_ACT_SILU = 1 };
/* Activation / output element types for the device surface. */
enum { K3_DTYPE_F32 = 0, K3_DTYPE_BF16 = 1 };

/* Most experts one token may route to in one device call. */
#define K3_HIP_MAX_TOKEN_EXPERTS 32
/* Verify tiles: positions and edges per call (tools/metal_moe.mm:1056-1059
 * bounds flat position batches at 16 positions x 16 edges). */
#define K3_HIP_MAX_POSITIONS 16
#define K3_HIP_MAX_EDGES 256

/* Expert descriptor: byte-for-byte the layout of K3MetalExpertDescriptorV1
 * (tools/metal_moe_abi.h:35-50), so a caller's descriptor arrays pass through
 * unchanged.  blob_bytes must equal the span of the descriptor's layout at
 * the configured geometry (raw-v1: k3_hip_geometry_span; scale4-v2:
 * K3_SCALE4_V2_EXPERT_SPAN, an 8192-byte header then w1 packed, w1 4-bit
 * scale indices, w2 packed, w2 indices, w3 packed, w3 indices). */
typedef struct K3HipExpertDescriptorV1 {
  uint32_t abi_version;  /* K3_DESCRIPTOR_ABI_V1 */
  uint32_t struct_bytes; /* sizeof(K3HipExpertDescriptorV1) == 32 */
  uint32_t layout_id;    /* K3_LAYOUT_RAW_V1, or K3_LAYOUT_SCALE4_V2 (K3 only;
                            every descriptor of a call has the same layout) */
  uint32_t reserved;     /* 0 */
  uint64_t blob_bytes;
  const uint8_t* blob;   /* host or device pointer */
} K3HipExpertDescriptorV1;

/* Geometry.  The reference hard-codes K3 (hidden 3584, intermediate 3072,
 * tools/cuda_moe_kernels.cu:36-40); this library takes it as data. */
typedef struct K3HipGeometryV1 {
  uint32_t abi_version;  /* 1 */
  uint32_t struct_bytes; /* sizeof(K3HipGeometryV1) == 32 */
  uint32_t hidden;       /* x / output length, positive multiple of 32 */
  uint32_t intermediate; /* h length, positive multiple of 32 */
  uint32_t activation;   /* K3_ACT_* */
  uint32_t reserved;     /* 0 */
  uint64_t expert_span;  /* must equal k3_hip_geometry_span(hidden, intermediate) */
} K3HipGeometryV1;

#ifdef __cplusplus
static_assert(sizeof(K3HipExpertDescriptorV1) == 32, "descriptor ABI drift");
static_assert(offsetof(K3HipExpertDescriptorV1, blob_bytes) == 16, "descriptor ABI drift");
static_assert(offsetof(K3HipExpertDescriptorV1, blob) == 24, "descriptor ABI drift");
static_assert(sizeof(K3HipGeometryV1) == 32, "geometry ABI drift");
extern "C" {
#endif

/* ======================================================= common / geometry */

/* Raw-v1 span for a geometry (provider_moe.cpp:217-243 offsets). 0 if invalid. */
uint64_t k3_hip_geometry_span(uint32_t hidden, uint32_t intermediate);
/* Fill *out with a preset: 1 = K3 (3584/3072/SiTU, 17,547,264 B),
 * 2 = the 16-expert decode benchmark geometry (7168/2048/SiLU, 23,396,352 B).
 * Returns 0 or K3_HIP_E_INVALID. */
int k3_hip_geometry_preset(int preset, K3HipGeometryV1* out);
/* Thread-local text of the last failure on this thread. */
const char* k3_hip_last_error(void);

/* ============================== surface 1: host-synchronous descriptor API */

/* Replaces k3_metal_init (tools/metal_moe.mm:649-652).  selector: NULL/"" =
 * device 0, or a decimal device index.  0 on success, -1 on failure. */
int k3_hip_init(const char* selector);
/* Replaces k3_metal_available (tools/metal_moe.mm:654-657): 1 or 0. */
int k3_hip_available(void);
/* Replaces k3_metal_descriptor_abi_version (tools/metal_moe_abi.h:56). */
uint32_t k3_hip_descriptor_abi_version(void);
/* Replaces k3_metal_layout_capabilities (tools/metal_moe_abi.h:57):
 * K3_CAP_RAW_V1, plus K3_CAP_SCALE4_V2 while the surface-1 geometry is K3
 * (the scale4-v2 format is defined for K3 only, tools/metal_moe.mm:127-155). */
uint64_t k3_hip_layout_capabilities(void);
/* The header checks surface 1 applies to every scale4-v2 descriptor
 * (validate_scale4_header, tools/metal_moe.mm:353-405) on a header in host
 * memory: 0, K3_HIP_E_INVALID (fewer than 8192 bytes) or K3_HIP_E_DESCRIPTOR
 * with the reason in k3_hip_last_error().  No separate reference entry point:
 * the reference runs these checks inside its descriptor calls. */
int k3_hip_scale4_check_header(const uint8_t* header, uint64_t bytes);
/* Sets the geometry used by surface 1 (default preset 1, K3).  Drops every
 * cached blob.  No reference counterpart: the Metal bridge fixes K3. */
int k3_hip_configure_v1(const K3HipGeometryV1* geometry);
/* Replaces k3_metal_shapes (tools/metal_moe.mm:669-673). */
void k3_hip_shapes(int* hidden, int* inter, long long* span);
/* Replaces k3_metal_stats (tools/metal_moe.mm:675-681):
 * [calls, device_resident_uses, host_uploads, cache_entries, cache_mode]. */
void k3_hip_stats(long long* five);
/* Replaces k3_metal_mode / k3_metal_set_mode (:683-693): 1 = keep uploaded
 * host blobs cached in HBM (default), 0 = upload every call. */
int k3_hip_mode(void);
int k3_hip_set_mode(int cache_host_blobs);
/* Replaces k3_metal_drop / k3_metal_flush (:695-707).  A cached host blob must
 * be dropped before its memory is modified, unmapped or freed. */
void k3_hip_drop(const uint8_t* blob);
void k3_hip_flush(void);

/* Replaces k3_metal_moe_layer_desc_v1 (tools/metal_moe_abi.h:59-61):
 * output[hidden] = sum_e weights[e] * expert_e(input[hidden]), summed in
 * descriptor order.  expert_count == 0 writes zeros. */
int k3_hip_moe_layer_desc_v1(const K3HipExpertDescriptorV1* experts,
                             int expert_count, const float* weights,
                             const float* input, float* output);
/* Replaces k3_metal_moe_positions_desc_v1 (tools/metal_moe_abi.h:63-66):
 * position_offsets[position_count+1] partitions the edges; input/output are
 * [position_count, hidden].  Every expert is read once per call however many
 * positions route to it. */
int k3_hip_moe_positions_desc_v1(const K3HipExpertDescriptorV1* experts,
                                 int edge_count, const int* position_offsets,
                                 int position_count, const float* weights,
                                 const float* input, float* output);
/* Raw-pointer forms (tools/metal_moe.mm:829-837, :1023-1032): blobs are spans
 * of the configured geometry. */
int k3_hip_moe_layer(const uint8_t* const* expert_blobs, int n_experts,
                     const float* weights, const float* x, float* out);
int k3_hip_moe_positions(const uint8_t* const* expert_blobs, int n_edges,
                         const int* position_offsets, int n_positions,
                         const float* weights, const float* x, float* out);
/* Flat position batches: replace k3_metal_moe_positions_flat and
 * k3_metal_moe_positions_flat_desc_v1 (tools/metal_moe.mm:1049-1070,
 * :1194-1259), which the provider binds beside the plain positions calls and
 * tries first (native/provider_gate/provider_moe.cpp:141-187, :1406-1478).
 * Same arguments and outputs as the positions calls, run as one batched
 * dispatch sequence over all edges.  Bounds as the Metal bridge's: at most 16
 * positions and 16 x n_positions edges, else K3_HIP_E_INVALID.  Where the
 * batch has no single-dispatch form here (positions with different edge
 * counts over scale4-v2 spans, which have no union kernels) the call returns
 * K3_HIP_E_CAPABILITY (-6) before touching its outputs, and the caller steps
 * down to the positions call, as the provider does. */
int k3_hip_moe_positions_flat(const uint8_t* const* expert_blobs, int n_edges,
                              const int* position_offsets, int n_positions,
                              const float* weights, const float* x, float* out);
int k3_hip_moe_positions_flat_desc_v1(const K3HipExpertDescriptorV1* experts,
                                      int edge_count, const int* position_offsets,
                                      int position_count, const float* weights,
                                      const float* input, float* output);

/* ============================== surface 2: stream-explicit device API */

/* Replaces k3_cuda_moe_abi_version (tools/cuda_moe_kernels.cu:244-246). */
uint32_t k3_hip_moe_abi_version(void);
/* Replaces k3_cuda_moe_shapes (:248-264); reports surface 1's geometry and
 * pointer layout 1. */
void k3_hip_moe_shapes(int* hidden, int* intermediate, int64_t* expert_span,
                       uint32_t* pointer_layout);
/* Replaces k3_cuda_moe_available (:270-329): 1 when `device` is a usable gfx950,
 * else a negative status. */
int k3_hip_moe_available(int device);

/* Replaces k3_cuda_mxfp4_gemv (:331-339): out[b, r] = sum_c W[r, c] x[b, c],
 * x [batches, cols] fp32, out [batches, rows] fp32, cols % 32 == 0.  Each
 * weight row is read once for all batches. */
int k3_hip_mxfp4_gemv(const uint8_t* packed, const uint8_t* scales,
                      const float* x, float* output, int rows, int cols,
                      int batches, void* stream);
/* Same contraction with a bf16 or fp32 activation and output type. */
int k3_hip_mxfp4_gemv_ex(const uint8_t* packed, const uint8_t* scales,
                         const void* x, int x_dtype, void* output,
                         int out_dtype, int rows, int cols, int batches,
                         void* stream);

/* Replaces k3_cuda_moe_launch (:341-417) for geometry g (NULL = surface 1's):
 * gate = W1 x, up = W3 x, gate <- act(gate, up), out = W2 gate, all fp32,
 * x [batches, hidden], gate/up [batches, intermediate], out [batches, hidden]. */
int k3_hip_moe_launch(const K3HipGeometryV1* g, const uint8_t* expert_span,
                      const float* x, int batches, float* gate, float* up,
                      float* expert_output, void* stream);

/* Device workspace bytes needed by the layer / verify calls below for up to
 * max_edges routed edges over max_positions positions.  Its contents need no
 * initialisation.  Calls that share one workspace must not overlap. */
uint64_t k3_hip_moe_workspace_bytes(const K3HipGeometryV1* g, int max_edges,
                                    int max_positions);

/* Whole routed layer for one token (replaces the per-expert launch loop plus
 * ordered_route_reduce, provider_cuda_moe.cpp:1203-1258, :252-289):
 * out[hidden] = sum_{e < n} weights[e] * expert_e(x), summed in route order.
 * experts: host array of n device span pointers; weights: host fp32 [n];
 * x, out: device vectors of x_dtype / out_dtype.  n <= K3_HIP_MAX_TOKEN_EXPERTS. */
int k3_hip_moe_layer_device(const K3HipGeometryV1* g,
                            const uint8_t* const* experts,
                            const float* weights, int n_experts,
                            const void* x, int x_dtype, void* out,
                            int out_dtype, void* workspace,
                            uint64_t workspace_bytes, void* stream);

/* Whole routed layer with the router on the device: the top_k largest of
 * logits[n_bank] (descending, lower index on ties) select experts
 * bank + id * expert_stride, weighted by a softmax over the selected logits.
 * route_ids / route_weights (device, nullable) receive the route. */
int k3_hip_moe_route_layer_device(const K3HipGeometryV1* g,
                                  const uint8_t* bank, uint64_t expert_stride,
                                  int n_bank, const float* logits, int top_k,
                                  const void* x, int x_dtype, void* out,
                                  int out_dtype, int32_t* route_ids,
                                  float* route_weights, void* workspace,
                                  uint64_t workspace_bytes, void* stream);

/* No counterpart in the reference.  For callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc): k3_hip_moe_route_layer_device with the same arguments
 * and results, minus the workspace, which comes from a library-owned static
 * device array of K3_HIP_NOALLOC_SCRATCH_BYTES per GPU (held until the process
 * ends).  Allocates nothing.  A geometry / top_k whose workspace
 * (k3_hip_moe_workspace_bytes(g, top_k, 1)) exceeds that size returns
 * K3_HIP_E_INVALID (1 MiB holds top_k 16 at both presets; the benchmark
 * geometry at top_k 32 needs about 1.4 MB and is refused).  Every call on one GPU shares that GPU's array: calls that
 * overlap on one GPU (two streams, or two threads) race and must be ordered
 * by the caller. */
#define K3_HIP_NOALLOC_SCRATCH_BYTES (UINT64_C(1) << 20)
int k3_hip_moe_route_layer_device_noalloc(const K3HipGeometryV1* g,
                                          const uint8_t* bank,
                                          uint64_t expert_stride, int n_bank,
                                          const float* logits, int top_k,
                                          const void* x, int x_dtype,
                                          void* out, int out_dtype,
                                          int32_t* route_ids,
                                          float* route_weights, void* stream);

/* Batched speculative verify with device routing: positions p < n_positions
 * each route top_k of logits[p, n_bank]; experts are grouped so each routed
 * expert's bytes are read once for all positions that chose it (no reference
 * counterpart amortises this; semantics follow
 * provider_cuda_moe.cpp:1260-1360 and tools/metal_moe.mm:852-1021).
 * x, out: [n_positions, hidden]; route_ids / route_weights (nullable):
 * [n_positions, top_k]. */
int k3_hip_moe_verify_route_device(const K3HipGeometryV1* g,
                                   const uint8_t* bank, uint64_t expert_stride,
                                   int n_bank, const float* logits,
                                   int n_positions, int top_k, const void* x,
                                   int x_dtype, void* out, int out_dtype,
                                   int32_t* route_ids, float* route_weights,
                                   void* workspace, uint64_t workspace_bytes,
                                   void* stream);

/* Batched verify with a caller route: edge e of position p (edges of p are
 * [position_offsets[p], position_offsets[p+1])) uses expert span
 * edge_experts[e] (host array of device pointers) with weight
 * edge_weights[e] (host).  Same grouping and ordered per-position combine. */
int k3_hip_moe_verify_device(const K3HipGeometryV1* g,
                             const uint8_t* const* edge_experts,
                             const float* edge_weights,
                             const int* position_offsets, int n_positions,
                             const void* x, int x_dtype, void* out,
                             int out_dtype, void* workspace,
                             uint64_t workspace_bytes, void* stream);

/* ============================== host-side expert staging (HBM LRU cache) */
/* C counterpart of CudaMoeExpertCache (provider_cuda_moe.h:83-132): a
 * device-resident LRU of expert spans over layer strata, plan-before-I/O
 * snapshots (hits pinned, misses reported), uploads from pinned host memory
 * on a side stream with per-slot ready events. */

typedef struct K3HipCache K3HipCache;

/* A cache over n_layers strata of span_bytes experts.  capacity_experts = 0
 * sizes it from the budget alone (automatic capacity); > 0 requests that many
 * slots, clamped to the budget (CudaMoeCachePolicy, provider_cuda_moe.h:16-28;
 * at most K3_HIP_CACHE_MAX_EXPERTS).  HBM is taken in segments of slots as
 * the cache fills, after the budget is measured at the first plan.
 * staging_slots = pinned host staging buffers used for pageable sources.
 * Returns NULL on failure (see k3_hip_last_error). */
#define K3_HIP_CACHE_MAX_EXPERTS 1472 /* 92 strata x 16: kCudaMaximumExperts, provider_cuda_moe.cpp:55-57 */
K3HipCache* k3_hip_cache_create(int device, uint64_t span_bytes,
                                int capacity_experts, int n_layers,
                                int staging_slots);
void k3_hip_cache_destroy(K3HipCache* cache);

/* Capacity policy (CudaMoeCachePolicy, provider_cuda_moe.h:16-28).  The
 * budget is free device memory at the first plan minus a reserve:
 * K3_CACHE_RESERVE_AUTO max(2 GiB, free / 5), _BYTES reserve_value bytes,
 * _RATIO_PPM free x reserve_value / 1e6 (provider_cuda_moe.cpp:668-705). */
enum { K3_CACHE_RESERVE_AUTO = 0, K3_CACHE_RESERVE_BYTES = 1,
       K3_CACHE_RESERVE_RATIO_PPM = 2 };
typedef struct K3HipCachePolicyV1 {
  uint32_t abi_version;        /* 1 */
  uint32_t struct_bytes;       /* sizeof(K3HipCachePolicyV1) == 32 */
  uint32_t automatic_capacity; /* 1: what the budget holds; 0: capacity_experts */
  uint32_t reserve_kind;       /* K3_CACHE_RESERVE_* */
  uint64_t capacity_experts;   /* 0 when automatic, else <= K3_HIP_CACHE_MAX_EXPERTS */
  uint64_t reserve_value;      /* 0 for AUTO; bytes; or ppm (<= 1,000,000) */
} K3HipCachePolicyV1;
#ifdef __cplusplus
static_assert(sizeof(K3HipCachePolicyV1) == 32, "cache policy ABI drift");
#endif
/* Replaces CudaMoeExpertCache::configure (provider_cuda_moe.h:97-98,
 * validate_cache_policy provider_cuda_moe.cpp:60-74): K3_HIP_E_INVALID for a
 * policy out of bounds, or once the policy is frozen (from the first plan). */
int k3_hip_cache_configure(K3HipCache* cache, const K3HipCachePolicyV1* policy);
/* The budget (CudaMoeResidencyPlanReport::capacity_experts,
 * provider_cuda_moe.h:30-34): five = [capacity in experts (-1 before the
 * first plan), slots allocated, free bytes measured, reserve bytes, rebuilds
 * left].  Returns 1 once measured, 0 before, or K3_HIP_E_INVALID. */
int k3_hip_cache_budget(const K3HipCache* cache, long long* five);
/* Plan (provider_cuda_moe.cpp:963-1008): snapshot hits for `ids` of `layer`
 * (canonical ascending, unique), LRU-promoting them; misses are written to
 * missing_ids (capacity n) and *n_missing.  plan_id must be non-zero and not
 * live.  */
int k3_hip_cache_plan(K3HipCache* cache, uint64_t plan_id, int layer,
                      const uint16_t* ids, int n, uint16_t* missing_ids,
                      int* n_missing);
/* Admit the plan's misses from host memory: sources[i] holds the span of
 * missing_ids[i] (pinned memory is copied directly, pageable memory through
 * a staging slot).  Copies run on the cache's side stream; per-expert ready
 * events are recorded.  Non-blocking for pinned sources.  All or nothing:
 * K3_HIP_E_ALLOC when every slot is pinned by live plans, or on a
 * recoverable device allocation failure (the reference's
 * CudaMoeRecoverableError, provider_cuda_moe.cpp:630-653: the fetch is
 * undone, unpinned entries are dropped and the budget is re-measured at the
 * next plan; after two such rebuilds the cache disables itself).  The plan
 * stays live with its hits pinned: the caller takes its CPU path through
 * k3_hip_cache_materialize_plan, then releases the plan. */
int k3_hip_cache_fetch(K3HipCache* cache, uint64_t plan_id,
                       const uint8_t* const* sources, int n_sources);
/* Device pointers of the plan's experts in `ids` order, and make `stream`
 * wait for every one of them to be resident. */
int k3_hip_cache_resolve(K3HipCache* cache, uint64_t plan_id,
                         const uint16_t* ids, int n,
                         const uint8_t** device_spans, void* stream);
/* Device pointers for the subset of `ids` already resident and ready (no
 * wait); others get NULL.  `stream` is where the caller will read them:
 * release orders the slots' reuse after the work queued there.  Returns the
 * number resident. */
int k3_hip_cache_ready_subset_v2(K3HipCache* cache, uint64_t plan_id,
                                 const uint16_t* ids, int n,
                                 const uint8_t** device_spans, void* stream);
/* The first form, without a stream: the caller reads the spans on the null
 * stream (k3_hip_cache_ready_subset_v2 with stream NULL). */
int k3_hip_cache_ready_subset(K3HipCache* cache, uint64_t plan_id,
                              const uint16_t* ids, int n,
                              const uint8_t** device_spans);
/* Finish or cancel a plan (provider_cuda_moe.cpp:1166-1168).  Slots the plan
 * pinned are reused only after the work queued so far on every stream the
 * plan resolved on (resolve / ready_subset): release records a reuse event on
 * each, and where it cannot, waits on the host for that stream (and fails the
 * cache closed if even that fails). */
void k3_hip_cache_release(K3HipCache* cache, uint64_t plan_id);
/* Bounded device-to-host copy of the plan's pinned hits only, for the
 * caller's exact CPU reconstruction of the tile
 * (CudaMoeExpertCache::materialize_plan_for_cpu, provider_cuda_moe.cpp:1170-1196;
 * used by provider_moe.cpp:1117-1206): ids_out receives their expert ids in
 * canonical order, host_out their spans back to back, *n_out their count.
 * Works on a disabled cache while the plan is live. */
int k3_hip_cache_materialize_plan(K3HipCache* cache, uint64_t plan_id,
                                  uint16_t* ids_out, int ids_capacity,
                                  uint8_t* host_out, uint64_t host_bytes,
                                  int* n_out);
/* Test hook, no reference counterpart: the next `count` device allocations of
 * the cache report out-of-memory without reaching the allocator, so the
 * recoverable path can be exercised on demand. */
int k3_hip_cache_fail_allocations(K3HipCache* cache, int count);
/* [hits, misses, evictions, resident, capacity, bytes_uploaded]. */
void k3_hip_cache_stats(const K3HipCache* cache, long long* six);
/* Qualification and fail-closed state (CudaMoeExpertCache::available / detail,
 * provider_cuda_moe.cpp:889-961).  The first plan runs the reference's device
 * known-answer tests (:291-420) on the cache's stream.  Returns 1 enabled,
 * 0 not yet qualified, K3_HIP_E_CAPABILITY disabled by a known-answer
 * mismatch (the caller takes its CPU path), K3_HIP_E_EXEC terminal (a HIP
 * failure inside a cache call, or k3_hip_cache_poison); once not enabled,
 * plan / fetch / resolve / ready_subset return that status and every resident
 * entry is dropped.  reason (nullable) receives the detail. */
int k3_hip_cache_state(const K3HipCache* cache, char* reason,
                       uint64_t reason_capacity);
/* Mark the cache terminally failed (CudaMoeExpertCache::poison_external,
 * provider_cuda_moe.cpp:1199-1201). */
void k3_hip_cache_poison(K3HipCache* cache, const char* failure);
/* Copy the resident span of (layer, id) to host (bounded D2H, the CPU fallback
 * materialisation of provider_cuda_moe.cpp:1170-1201).  0 or -2 if absent. */
int k3_hip_cache_read_back(K3HipCache* cache, int layer, uint16_t id,
                           uint8_t* host_out, uint64_t bytes);

/* ============================== per-launch device timing */
/* No reference counterpart beyond the Metal bridge counters
 * (tools/metal_moe.mm:675-681) and the per-layer phase profile
 * (native/deltafin/src/engine.rs:4705-4902).  Between begin and end every
 * kernel this library launches, on any stream, is bracketed by two hipEvents
 * recorded on that stream (up to max_launches launches; later ones are
 * counted as dropped).  end synchronises on the recorded events and returns
 * one row per kernel class that ran. */
typedef struct K3HipKernelTimingV1 {
  char kernel[32];   /* kernel class: "glu_decode", "down_decode", ... */
  int64_t launches;
  double total_ms;
  double min_ms;
  double max_ms;
} K3HipKernelTimingV1;

int k3_hip_timing_begin(int max_launches);
int k3_hip_timing_end(K3HipKernelTimingV1* out, int capacity, int* n_out,
                      long long* dropped);

/* ============================== decode kernel selection */
/* No reference counterpart.  A single-token layer call above runs as a
 * gate/up launch and a down launch (the default).  enabled = 1 makes every
 * later call in the process run as one fused launch (router, gate/up, down
 * and ordered combine) where its shape allows it (bf16 x, intermediate 2048,
 * at most 16 experts, one of 64 workspaces per device); 0 restores the
 * default.  Both paths compute bit-identical outputs; the fused one is
 * slower on MI355X.  Returns the previous setting. */
int k3_hip_set_fused_decode(int enabled);

/* No reference counterpart.  A single-token layer call with one routed
 * expert given as a span pointer (bf16 x, raw-v1, intermediate 2048) runs,
 * by default (mode K3_DECODE_CHAIN_ON), as one launch whose workgroups hand h
 * to the down rows through device memory instead of a second launch.
 * K3_DECODE_CHAIN_OFF makes such calls take the two launches;
 * K3_DECODE_CHAIN_FALLBACK runs the one launch with every workgroup computing
 * the gate/up shares it finds missing at once (the path taken when not every
 * workgroup is resident; for tests).  All compute bit-identical outputs.
 * Returns the previous mode, or K3_HIP_E_INVALID for another value. */
#define K3_DECODE_CHAIN_OFF 0
#define K3_DECODE_CHAIN_ON 1
#define K3_DECODE_CHAIN_FALLBACK 2
int k3_hip_set_decode_chain(int mode);

/* No reference counterpart.  Where the single-token gate/up dots of the layer
 * calls above run: K3_DECODE_DOTS_VALU (0) on the vector ALUs for every
 * activation type; K3_DECODE_DOTS_MFMA_F32 (1, the default) on the bf16
 * matrix cores for fp32 activations (x split into three bf16 terms that sum
 * to it exactly, so only the summation order differs) and on the vector ALUs
 * for bf16 ones; K3_DECODE_DOTS_MFMA_ALL (2) on the matrix cores for both.
 * The matrix-core kernel takes raw-v1 spans with hidden a multiple of 256 and
 * 4, 6 or 8 gate/up units of 8 rows per unit pipeline; other shapes keep the
 * vector kernel.  Process-wide; returns the previous setting, or
 * K3_HIP_E_INVALID for another value. */
#define K3_DECODE_DOTS_VALU 0
#define K3_DECODE_DOTS_MFMA_F32 1
#define K3_DECODE_DOTS_MFMA_ALL 2
int k3_hip_set_decode_mfma(int mode);

/* ============================== verify path selection */
/* No reference counterpart.  How the two verify calls above run:
 *   K3_VERIFY_AUTO (default): batches of two or more positions whose unique
 *     experts are at most 92% of their edges (exactly, for a caller route;
 *     the expected union of independent routes, for device routing) go
 *     through the matrix-core union path where it applies (raw-v1 spans,
 *     hidden and intermediate multiples of 256, at most 16 edges per
 *     expert); otherwise one decode layer per position, or the union VALU
 *     kernels when the matrix-core path does not apply and a caller route's
 *     positions share most experts;
 *   K3_VERIFY_POSITIONS: one decode layer per position (an expert chosen by
 *     several positions is read once per position, as in the reference);
 *   K3_VERIFY_UNION_MFMA: every routed expert read once per batch and
 *     multiplied on the block-scaled FP4 matrix cores; a call whose geometry
 *     or route does not allow it returns K3_HIP_E_CAPABILITY;
 *   K3_VERIFY_UNION_VALU: every routed expert read once per batch on the
 *     first-design VALU union kernels.
 * Process-wide; returns the previous mode, or K3_HIP_E_INVALID for an
 * unknown mode (the mode is then unchanged). */
enum { K3_VERIFY_AUTO = 0, K3_VERIFY_POSITIONS = 1, K3_VERIFY_UNION_MFMA = 2,
       K3_VERIFY_UNION_VALU = 3 };
int k3_hip_set_verify_mode(int mode);

/* ============================== synthetic inputs (benchmark support) */
/* No reference counterpart.  Fill device memory with the counter-based
 * synthetic distribution shared with oracle/orc.c: packed bytes uniform,
 * scale bytes uniform in [scale_lo, scale_hi]; expert e of a bank uses
 * matrix streams 3(first_expert+e)+{0,1,2}. */
int k3_hip_synth_bank(const K3HipGeometryV1* g, uint8_t* bank,
                      uint64_t expert_stride, int n_experts,
                      uint64_t first_expert, uint64_t seed, int scale_lo,
                      int scale_hi, void* stream);
/* Normal(0,1) values (fp32 or bf16) from (seed, stream), n elements. */
int k3_hip_synth_normal(void* out, int dtype, uint64_t n, uint64_t seed,
                        uint64_t stream, void* stream_handle);

/* ============================== the whole K3 MoE block on the device */
/* The eight resident spine slots of one MoE layer (MoeSpineT1,
 * native/provider_gate/provider_moe.h:66-100; shapes checked as
 * validate_spine does, provider_moe.cpp:419-450), as device pointers.  Every
 * matrix is row-major [rows, columns] in one storage form: BF16 bits
 * (K3_SPINE_MATRIX_BF16; the *_scales pointers are ignored) or row-int8 with
 * one fp32 scale per row (K3_SPINE_MATRIX_INT8; scales required).  The
 * reference's geometry is hidden 7168, routed_hidden 3584, shared 6144,
 * experts 896, top_k 16 (k3_moe_geometry, provider_moe.h:40-42). */
#define K3_SPINE_MATRIX_BF16 0
#define K3_SPINE_MATRIX_INT8 1
#define K3_MOE_SPINE_ABI_V1 1
typedef struct K3HipMoeSpineV1 {
  uint32_t abi_version;          /* K3_MOE_SPINE_ABI_V1 */
  uint32_t struct_bytes;         /* sizeof(K3HipMoeSpineV1) == 144 */
  uint32_t matrix_kind;          /* K3_SPINE_MATRIX_* */
  uint32_t hidden;               /* H: block input / output width */
  uint32_t routed_hidden;        /* R: expert width (= expert geometry hidden) */
  uint32_t shared_intermediate;  /* S */
  uint32_t experts;              /* E: router rows = bank experts (<= 4096) */
  uint32_t top_k;                /* routed experts per token (<= 32) */
  const void* router;            /* [E, H] */
  const float* router_scales;    /* [E] (int8) */
  const float* router_bias;      /* [E] fp32 correction bias */
  const void* routed_down;       /* [R, H] */
  const float* routed_down_scales;
  const float* routed_norm;      /* [R] fp32 RMS-norm weight */
  const void* routed_up;         /* [H, R] */
  const float* routed_up_scales;
  const void* shared_gate;       /* [S, H] */
  const float* shared_gate_scales;
  const void* shared_up;         /* [S, H] */
  const float* shared_up_scales;
  const void* shared_down;       /* [H, S] */
  const float* shared_down_scales;
} K3HipMoeSpineV1;

/* Workspace bytes of k3_hip_moe_block_device for up to max_positions. */
uint64_t k3_hip_moe_block_workspace_bytes(const K3HipMoeSpineV1* spine,
                                          const K3HipGeometryV1* experts,
                                          int max_positions);

/* The K3 MoE block for n_positions tokens (1..16) in one stream-ordered call,
 * replacing prepare_moe_t1 / complete_moe_t1 and their position forms
 * (provider_moe.cpp:1660-1700, :1970-2014) around the routed expert set:
 *   logits   = router hidden;  scores = sigmoid(logits)
 *   route    = top_k of scores + router_bias (descending, lower index on
 *              ties), weights = scores[route] / (sum + 1e-20)
 *   routed   = sum_{route order} w_e expert_e(routed_down hidden)
 *              (the experts of `experts`, SiTU, from bank + id * stride)
 *   out      = routed_up (routed_norm * rms_norm(routed, eps 1e-5))
 *            + shared_down situ(shared_gate hidden, shared_up hidden)
 * hidden, out: device fp32 [n_positions, H] (16-byte aligned); route_ids /
 * route_weights (device, nullable): [n_positions, top_k].  Every product is
 * fp32 (from 3 positions a 16-byte-aligned BF16 spine runs on the BF16 matrix
 * cores from a three-term BF16 split of each activation, whose products are
 * exact in fp32).  The experts of a batch go through the verify paths
 * (k3_hip_set_verify_mode).  Returns a K3_HIP_* status. */
int k3_hip_moe_block_device(const K3HipMoeSpineV1* spine,
                            const K3HipGeometryV1* experts,
                            const uint8_t* bank, uint64_t expert_stride,
                            const float* hidden, int n_positions, float* out,
                            int32_t* route_ids, float* route_weights,
                            void* workspace, uint64_t workspace_bytes,
                            void* stream);

#ifdef __cplusplus
}
#endif

#endif
