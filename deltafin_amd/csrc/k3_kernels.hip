// gfx950 kernels for the routed-expert MXFP4 path and their host launchers.
//
// Data layout in HBM is the reference's raw-v1 expert span, read in place
// (provider_moe.cpp:217-243): row-major packed E2M1 planes and row-major E8M0
// scale planes.  Every row of every matrix is a run of 16-byte chunks, one
// chunk = one 32-element scale group, so a wave's dwordx4 load covers 64
// consecutive chunks = 1 KiB of contiguous row bytes.
//
// Decode (one token) runs in two launches:
//   A  k_glu_decode   one wave per (expert, 8 gate/up row pairs): the x slice a
//                     lane needs stays in registers across all rows, gate and up
//                     rows of the same index share it, the activation is applied
//                     in registers and h[e][row] is written (fp32).
//   B  k_down_decode  one workgroup per block of output rows, one wave per
//                     routed expert: down rows against h_e (held in registers),
//                     then the route-ordered weighted sum of the experts' rows
//                     out of LDS (tools/metal/moe_mxfp4.metal:410-445 order).
// Verify (M positions) groups edges by expert first, so each routed expert's
// bytes are read once for every position that chose it.
#include <stdarg.h>
#include <stdio.h>

#include <algorithm>
#include <atomic>
#include <mutex>
#include <type_traits>
#include <unordered_map>
#include <vector>

#include <hip/hip_ext.h>

#include "k3_device.h"
#include "k3_internal.h"
#include "k3_launch.h"
#include "k3_terms.h"

namespace k3 {

// ======================================================================
// activation slices
// ======================================================================
template <typename XT>
struct XChunk;

template <>
struct XChunk<uint16_t> {  // bf16 activations
  uint32_t v[16];
  __device__ __forceinline__ void load(const uint16_t* x, int chunk) {
    const uint4* p = reinterpret_cast<const uint4*>(x + (size_t)chunk * 32);
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const uint4 t = p[q];
      v[4 * q + 0] = t.x;
      v[4 * q + 1] = t.y;
      v[4 * q + 2] = t.z;
      v[4 * q + 3] = t.w;
    }
  }
  __device__ __forceinline__ float dot(u32x4 w) const { return chunk_dot_bf16(w, v); }
};

template <>
struct XChunk<float> {
  float v[32];
  __device__ __forceinline__ void load(const float* x, int chunk) {
    const float4* p = reinterpret_cast<const float4*>(x + (size_t)chunk * 32);
#pragma unroll
    for (int q = 0; q < 8; ++q) {
      const float4 t = p[q];
      v[4 * q + 0] = t.x;
      v[4 * q + 1] = t.y;
      v[4 * q + 2] = t.z;
      v[4 * q + 3] = t.w;
    }
  }
  __device__ __forceinline__ float dot(u32x4 w) const { return chunk_dot_f32(w, v); }
};

// A chunk decoded once for several activations.
template <typename XT>
struct WDec;

template <>
struct WDec<uint16_t> {
  v2bf d[16];
  __device__ __forceinline__ void decode(u32x4 w) { chunk_decode_bf16(w, d); }
  __device__ __forceinline__ float dot(const XChunk<uint16_t>& x) const {
    return dot_decoded_bf16(d, x.v);
  }
};

template <>
struct WDec<float> {
  v2f d[16];
  __device__ __forceinline__ void decode(u32x4 w) { chunk_decode_f32(w, d); }
  __device__ __forceinline__ float dot(const XChunk<float>& x) const {
    return dot_decoded_f32(d, x.v);
  }
};

template <typename OT>
__device__ __forceinline__ void store_out(OT* p, float v);
template <>
__device__ __forceinline__ void store_out<float>(float* p, float v) {
  *p = v;
}
template <>
__device__ __forceinline__ void store_out<uint16_t>(uint16_t* p, float v) {
  *p = f32_to_bf16_bits(v);
}

// off: first entry of this route in the device ids / weights (bank mode;
// position-batched kernels route position p at p * n).
__device__ __forceinline__ const uint8_t* route_span(const TokenRoute& r, int e, size_t off = 0) {
  return r.bank ? r.bank + (uint64_t)r.ids[off + e] * r.stride : r.pdev ? r.pdev[off + e] : r.ptr[e];
}
__device__ __forceinline__ float route_weight(const TokenRoute& r, int e, size_t off = 0) {
  return r.bank || r.pdev ? r.wdev[off + e] : r.w[e];
}

// A wave's copy of the route: lane e (< n) holds expert e's span address and
// weight, loaded once so later lookups are register reads (v_readlane) rather
// than memory loads queued behind in-flight weight batches.
struct RouteRegs {
  uint32_t lo, hi;
  float w;
};

__device__ __forceinline__ RouteRegs route_regs(const TokenRoute& r, int lane, size_t off = 0) {
  RouteRegs o;
  o.lo = o.hi = 0u;
  o.w = 0.0f;
  if (lane < r.n) {
    const uint64_t p = reinterpret_cast<uint64_t>(route_span(r, lane, off));
    o.lo = (uint32_t)p;
    o.hi = (uint32_t)(p >> 32);
    o.w = route_weight(r, lane, off);
  }
  return o;
}

// e must be uniform across the wave.
__device__ __forceinline__ const uint8_t* span_of(const RouteRegs& rr, int e) {
  const uint32_t lo = __builtin_amdgcn_readlane(rr.lo, e);
  const uint32_t hi = __builtin_amdgcn_readlane(rr.hi, e);
  return reinterpret_cast<const uint8_t*>(((uint64_t)hi << 32) | lo);
}

__device__ __forceinline__ float weight_of(const RouteRegs& rr, int e) {
  return __uint_as_float(__builtin_amdgcn_readlane(__float_as_uint(rr.w), e));
}

// ======================================================================
// multi-activation GEMV: x rows staged in LDS, each weight chunk decoded once
// and applied to every staged activation
// ======================================================================
constexpr int kMultiMax = 8;

template <typename XT, typename OT, int kRows>
__global__ __launch_bounds__(256) void k_gemv_multi(const uint8_t* __restrict__ packed,
                                                    const uint8_t* __restrict__ scales,
                                                    const XT* __restrict__ x,
                                                    OT* __restrict__ out, int rows, int cols,
                                                    int batches, int group) {
  extern __shared__ uint4 smem_multi[];
  XT* xs = reinterpret_cast<XT*>(smem_multi);
  const int lane = threadIdx.x & 63;
  const int r0 = (blockIdx.x * 4 + (threadIdx.x >> 6)) * kRows;
  const int G = cols >> 5;
  const size_t cp = (size_t)cols >> 1;
  for (int b0 = 0; b0 < batches; b0 += group) {
    const int nb = min(group, batches - b0);
    __syncthreads();
    const int n16 = (int)((size_t)nb * cols * sizeof(XT) / 16);
    const uint4* src = reinterpret_cast<const uint4*>(x + (size_t)b0 * cols);
    // Straight to LDS (global_load_lds_dwordx4: a wave's 64 lanes fill 1 KB),
    // every copy in flight at once; vmcnt(0) before the barrier.
    for (int i0 = (int)threadIdx.x & ~63; i0 < n16; i0 += blockDim.x) {
      const int i = i0 + lane;
      if (i < n16)
        __builtin_amdgcn_global_load_lds(src + i, (__attribute__((address_space(3))) void*)(smem_multi + i0),
                                         16, 0, 0);
    }
    __builtin_amdgcn_s_waitcnt(0x0F70);
    __syncthreads();
    for (int r = 0; r < kRows; ++r) {
      const int row = r0 + r;
      if (row >= rows) break;
      float acc[kMultiMax];
#pragma unroll
      for (int t = 0; t < kMultiMax; ++t) acc[t] = 0.0f;
      const uint8_t* pr = packed + (size_t)row * cp;
      const uint8_t* sr = scales + (size_t)row * G;
      for (int chunk = lane; chunk < G; chunk += 64) {
        WDec<XT> wd;
        wd.decode(load_chunk(pr + (size_t)chunk * 16));
        const float s = e8m0_scale(sr[chunk]);
#pragma unroll
        for (int t = 0; t < kMultiMax; ++t) {
          if (t < nb) {
            XChunk<XT> xv;
            xv.load(xs + (size_t)t * cols, chunk);
            acc[t] = fmaf(wd.dot(xv), s, acc[t]);
          }
        }
      }
#pragma unroll
      for (int t = 0; t < kMultiMax; ++t) {
        if (t < nb) {
          const float v = wave_sum(acc[t]);
          if (lane == 0) store_out(out + (size_t)(b0 + t) * rows + row, v);
        }
      }
    }
  }
}

// ======================================================================
// column split: the S waves of a workgroup share a block of rows, wave w
// owning chunks [w*cw, w*cw + cw) of every row (cw = ceil(G / S) <= 64), so
// each lane holds exactly one activation chunk and every load instruction of a
// wave reads cw * 16 contiguous bytes of one row.  Lanes past the row's end
// load the row's last chunk again (same cache lines, no extra HBM traffic) and
// multiply it by a zero activation, so the load stream has no branches and the
// compiler issues a whole row block's loads back to back.
// ======================================================================
struct ColSplit {
  int cc;      // chunk this lane loads (clamped into the row)
  bool valid;  // lane owns a real chunk
};

__device__ __forceinline__ ColSplit col_split(int G, int S, int wave, int lane) {
  const int cw = (G + S - 1) / S;
  const int c = wave * cw + lane;
  ColSplit r;
  r.valid = lane < cw && c < G;
  r.cc = r.valid ? c : G - 1;
  return r;
}

template <typename XT>
__device__ __forceinline__ void load_x_chunk(XChunk<XT>& xc, const XT* x, const ColSplit& cs);

template <>
__device__ __forceinline__ void load_x_chunk<uint16_t>(XChunk<uint16_t>& xc, const uint16_t* x,
                                                       const ColSplit& cs) {
  xc.load(x, cs.cc);
#pragma unroll
  for (int i = 0; i < 16; ++i) xc.v[i] = cs.valid ? xc.v[i] : 0u;
}

template <>
__device__ __forceinline__ void load_x_chunk<float>(XChunk<float>& xc, const float* x,
                                                    const ColSplit& cs) {
  xc.load(x, cs.cc);
#pragma unroll
  for (int i = 0; i < 32; ++i) xc.v[i] = cs.valid ? xc.v[i] : 0.0f;
}

// ======================================================================
// single-activation GEMV (k3_hip_mxfp4_gemv at one batch): the column split
// above over units of kR rows.  A workgroup holds 4 / S row groups of S waves;
// each lane keeps its one activation chunk in registers, loads the chunk and
// scale byte of all kR rows of its unit at once, and a butterfly reduces the
// kR partials across the wave; the S wave partials meet in LDS.  Every unit
// is one round of loads, so a 2048 x 7168 matrix (512 units of 4 rows, two
// 256-thread workgroups per CU) is one wave of loads over the whole chip.
// Units of 4 rows measured 4.9 us per call at that shape on MI355X, against
// 7.5 us for 8 rows, 7.8 us for 16, 6.7 us for 2 and 9.6 us for 1.
// ======================================================================
template <typename XT, typename OT, int kR>
__global__ __launch_bounds__(256) void k_gemv_cs(const uint8_t* __restrict__ packed,
                                                 const uint8_t* __restrict__ scales,
                                                 const XT* __restrict__ x, OT* __restrict__ out,
                                                 int rows, int cols, int S) {
  constexpr int L = log2c<kR>();
  __shared__ float red[4][kR];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int G = cols >> 5;
  const int groups = 4 / S;
  const int grp = wave / S;
  const int gw = wave - grp * S;
  const bool active = grp < groups;  // S = 3 leaves one wave idle
  const ColSplit cs = col_split(G, S, active ? gw : 0, lane);
  XChunk<XT> xc;
  load_x_chunk<XT>(xc, x, cs);
  const size_t cp = (size_t)cols >> 1;
  const int n_units = (rows + kR - 1) / kR;
  const int per_round = (int)gridDim.x * groups;
  const int iters = (n_units + per_round - 1) / per_round;  // the same in every workgroup
  for (int it = 0; it < iters; ++it) {
    const int u = (it * (int)gridDim.x + (int)blockIdx.x) * groups + grp;
    const int r0 = min(u, n_units - 1) * kR;  // a unit past the end repeats the last one's loads
    u32x4 w[kR];
    uint32_t sc[kR];
#pragma unroll
    for (int r = 0; r < kR; ++r) {
      const int row = min(r0 + r, rows - 1);
      w[r] = load_chunk(packed + (size_t)row * cp + (size_t)cs.cc * 16);
      sc[r] = load_scale(scales + (size_t)row * G + cs.cc);
    }
    float v[kR];
#pragma unroll
    for (int r = 0; r < kR; ++r) v[r] = xc.dot(w[r]) * e8m0_scale(sc[r]);
    wave_reduce_multi<kR>(v, lane);
    if ((lane & ((1 << (6 - L)) - 1)) == 0) red[wave][lane >> (6 - L)] = v[0];
    __syncthreads();
    if (active && gw == 0 && lane < kR && u < n_units && r0 + lane < rows) {
      float t = red[grp * S][lane];
      for (int w2 = 1; w2 < S; ++w2) t += red[grp * S + w2][lane];
      store_out(out + r0 + lane, t);
    }
    __syncthreads();
  }
}


// ======================================================================
// decode phase A: gate/up rows + activation -> h
// A unit is kR (gate row, up row) pairs of one expert; unit u covers pairs
// [u kR, u kR + kR) of the flattened [expert][row] space.  The grid is one
// round of resident workgroups; workgroup b takes units b, b + NB, ... so the
// whole grid sweeps the routed weights as one advancing window.  The S waves
// of a workgroup split every row's chunks (column split above); each wave
// issues its 2 kR row loads at once, forms one partial per row, and a single
// butterfly reduces the 2 kR partials across the wave.  The S wave partials
// meet in LDS (two slots by unit parity, one barrier per unit); kR lanes of
// wave 0 sum them in wave order, apply the activation and store h.
// ======================================================================
// kG (gathered scales): a wave's cw = ceil(G / S) groups of a row are cw
// contiguous scale bytes, so with cw % 4 == 0 and kR * cw <= 256 the kR rows
// of one matrix in a unit are kR * cw / 4 dwords: lane l loads dword l of
// them (one load per matrix instead of kR single-byte loads), and the byte of
// row r for lane l (group c0 + l) is routed to it by a ds_bpermute from lane
// r * cw / 4 + l / 4.
// kS4 (scale4-v2 spans, gathered scales only): sg / su hold gathered index
// dwords and b4 the unit's expert bases (bytes 64-66 of its span).
struct NoBases {};
struct SpanBases {
  uint32_t b4;
};

template <typename XT, int kR, bool kG = false, bool kS4 = false>
struct GluBatch : std::conditional_t<kS4, SpanBases, NoBases> {
  static_assert(!kS4 || kG, "scale4-v2 gate/up loads need gathered scales");
  u32x4 wg[kR], wu[kR];
  uint32_t sg[kG ? 1 : kR], su[kG ? 1 : kR];
};

// Per-lane constants of the gathered-scale loads: byte offset (from the
// unit's first row) of the dword this lane loads, and the ds_bpermute address
// of row 0's source lane (row r adds r * cw).
struct GluGather {
  int off;
  int bp;
};

__device__ __forceinline__ GluGather glu_gather(int G, int S, int wave, int lane, int kR) {
  const int cw = (G + S - 1) / S;
  const int nd = cw >> 2;
  const int u = min(lane / nd, kR - 1);
  const int d = lane < kR * nd ? lane % nd : nd - 1;
  GluGather r;
  r.off = u * G + min(wave * cw + 4 * d, G - 4);
  r.bp = (lane >> 2) << 2;
  return r;
}

// scale4-v2 form of glu_gather: a row's cw groups are cw / 2 index bytes, so
// with G % 8 == 0, cw % 8 == 0 and kR * cw / 8 <= 64 lane l loads dword l of
// the unit's kR * cw / 8 (row u = l / (cw / 8)), and the nibble of group
// c0 + L of row r sits in lane r * cw / 8 + L / 8 at bits 4 (L % 8).
__device__ __forceinline__ GluGather glu_gather4(int G, int S, int wave, int lane, int kR) {
  const int cw = (G + S - 1) / S;
  const int nd = cw >> 3;
  const int u = min(lane / nd, kR - 1);
  const int d = lane < kR * nd ? lane % nd : nd - 1;
  GluGather r;
  r.off = u * (G >> 1) + min(((wave * cw) >> 1) + 4 * d, (G >> 1) - 4);
  r.bp = (lane >> 3) << 2;
  return r;
}

// Rows r0 .. r0 + kR - 1 of the gate and up matrices of the span at `span`.
template <typename XT, int kR, bool kG, bool kS4>
__device__ __forceinline__ void glu_load_rows(GluBatch<XT, kR, kG, kS4>& bt, const uint8_t* span,
                                              const Geo& g, int r0, const ColSplit& cs,
                                              const GluGather& gg) {
  const int G = g.hidden >> 5;
  const size_t cp = (size_t)g.hidden >> 1;
  const uint8_t* gp = span + g.w1p + (size_t)r0 * cp + (size_t)cs.cc * 16;
  const uint8_t* up = span + g.w3p + (size_t)r0 * cp + (size_t)cs.cc * 16;
  if constexpr (kS4) {  // index dwords first, as below
    bt.sg[0] = load_u32(span + g.w1s + (size_t)r0 * (G >> 1) + gg.off);
    bt.su[0] = load_u32(span + g.w3s + (size_t)r0 * (G >> 1) + gg.off);
  } else if constexpr (kG) {  // scale dwords first: waiting for them never waits for the data
    bt.sg[0] = load_u32(span + g.w1s + (size_t)r0 * G + gg.off);
    bt.su[0] = load_u32(span + g.w3s + (size_t)r0 * G + gg.off);
  }
  const uint8_t* gs = span + g.w1s + (size_t)r0 * G + cs.cc;
  const uint8_t* us = span + g.w3s + (size_t)r0 * G + cs.cc;
#pragma unroll
  for (int r = 0; r < kR; ++r) {
    bt.wg[r] = load_chunk(gp + (size_t)r * cp);
    bt.wu[r] = load_chunk(up + (size_t)r * cp);
    if constexpr (!kG) {
      bt.sg[r] = load_scale(gs + (size_t)r * G);
      bt.su[r] = load_scale(us + (size_t)r * G);
    }
  }
}

// Pair index pair0 = e * inter + r0 of routed expert e (route registers;
// kS4: rb4 holds lane e's span bases).
template <typename XT, int kR, bool kG, bool kS4>
__device__ __forceinline__ void glu_load(GluBatch<XT, kR, kG, kS4>& bt, const RouteRegs& rr,
                                         const Geo& g, int pair0, const ColSplit& cs,
                                         const GluGather& gg, uint32_t rb4 = 0u) {
  const int e = pair0 / g.inter;
  glu_load_rows(bt, span_of(rr, e), g, pair0 - e * g.inter, cs, gg);
  if constexpr (kS4) bt.b4 = __builtin_amdgcn_readlane(rb4, e);
}

// Scale byte of row r for this lane from a gathered dword.
__device__ __forceinline__ uint32_t gathered_scale(uint32_t word, int bp, int row_step, int r,
                                                   int lane) {
  const uint32_t w = (uint32_t)__builtin_amdgcn_ds_bpermute(bp + r * row_step, (int)word);
  return (w >> (8 * (lane & 3))) & 0xffu;
}

// scale4-v2: the scale byte base + index of row r for this lane from a
// gathered index dword (row_step4 = cw / 2 bytes of bpermute address per row).
__device__ __forceinline__ uint32_t gathered_scale4(uint32_t word, uint32_t base, int bp,
                                                    int row_step4, int r, int lane) {
  const uint32_t w = (uint32_t)__builtin_amdgcn_ds_bpermute(bp + r * row_step4, (int)word);
  return base + ((w >> (4 * (lane & 7))) & 0xfu);
}

// scale4-v2: lane e (< n) gets the bases dword of its expert's span (bytes
// 64, 65, 66 = w1, w2, w3 bases; byte 67 is zero).
__device__ __forceinline__ uint32_t route_bases(const RouteRegs& rr, int n, int lane) {
  if (lane >= n) return 0u;
  const uint8_t* sp =
      reinterpret_cast<const uint8_t*>(((uint64_t)rr.hi << 32) | (uint64_t)rr.lo);
  return load_u32(sp + 64);
}

__device__ void block_topk(const float* __restrict__ src, int n_bank, int top_k,
                           uint64_t* keys, int* sel, float* wsel, float pre = 0.0f,
                           bool have_pre = false, bool weights = true);
__device__ void block_softmax(const uint64_t* keys, const int* sel, int top_k, float* wsel);
__device__ __forceinline__ float key_value(uint64_t key);

// The route as every wave of the workgroup holds it (lane e: expert e's span
// and weight).  Router mode: the workgroup ranks the logits itself (no
// separate launch; keys is route_scratch_bytes of LDS) and workgroup 0
// publishes the route for later kernels and the caller.  All threads call it.
__device__ __forceinline__ RouteRegs workgroup_route(const TokenRoute& route, uint64_t* keys,
                                                     int* sel, float* wsel, int lane) {
  if (!route.logits) return route_regs(route, lane);
  block_topk(route.logits, route.n_bank, route.n, keys, sel, wsel);
  if (blockIdx.x == 0) {
    for (int j = threadIdx.x; j < route.n; j += blockDim.x) {
      route.ids_pub[j] = sel[j];
      route.w_pub[j] = wsel[j];
      if (route.ids_user) route.ids_user[j] = sel[j];
      if (route.w_user) route.w_user[j] = wsel[j];
    }
  }
  RouteRegs rr;
  rr.lo = rr.hi = 0u;
  rr.w = 0.0f;
  if (lane < route.n) {
    const int id = min(max(sel[lane], 0), route.n_bank - 1);  // bank address in range
    const uint64_t p = reinterpret_cast<uint64_t>(route.bank) + (uint64_t)id * route.stride;
    rr.lo = (uint32_t)p;
    rr.hi = (uint32_t)(p >> 32);
    rr.w = wsel[lane];
  }
  return rr;
}

__device__ __forceinline__ int glu_pair0(int q0, int Q, int n_units, int kR, int it) {
  const int u = q0 + it * Q;
  return (u < n_units ? u : 0) * kR;
}

// The gate/up sweep of one pipeline: pipeline q0 of Q takes units q0, q0 + Q,
// ... (iters of them) with two units in flight, unit it + 1 requested before
// unit it is reduced.  A unit past n_units repeats unit 0's loads and stores
// nothing, so every wave of the workgroup reaches the same iters barriers.
// The S wave partials of a unit meet in red (two slots by unit parity, one
// barrier per unit); kR lanes of the pipeline's wave 0 sum them in wave
// order, apply the activation and store h.  kIters > 0: iters is kIters (the
// loop resolves at compile time, so no wait merges the paths of other counts).
// kTagged (with kDeviceStore): h holds 64-bit entries {value bits, tag}, each
// stored at once, and both units' loads are issued before anything waits.
template <typename XT, int kR, bool kG, bool kDeviceStore = false, int kIters = 0,
          bool kTagged = false>
__device__ __forceinline__ void glu_sweep(const RouteRegs& rr, const Geo& g, const XChunk<XT>& xc,
                                          const ColSplit& cs, const GluGather& gg, int row_step,
                                          int S, int grp, int gw, int wave, int lane, int q0,
                                          int Q, int iters, int n_units, float* __restrict__ h,
                                          float (*red)[16][2 * kR], uint32_t tag = 0u) {
  constexpr int N = 2 * kR;
  constexpr int L = log2c<N>();
  auto unit_pair0 = [&](int it) { return glu_pair0(q0, Q, n_units, kR, it); };
  auto finish = [&](const GluBatch<XT, kR, kG>& bt, int it) {
    const int u = q0 + it * Q;
    const int parity = it & 1;
    float v[N];
#pragma unroll
    for (int r = 0; r < kR; ++r) {
      if constexpr (kG) {
        v[r] = xc.dot(bt.wg[r]) * e8m0_scale(gathered_scale(bt.sg[0], gg.bp, row_step, r, lane));
        v[kR + r] =
            xc.dot(bt.wu[r]) * e8m0_scale(gathered_scale(bt.su[0], gg.bp, row_step, r, lane));
      } else {
        v[r] = xc.dot(bt.wg[r]) * e8m0_scale(bt.sg[r]);
        v[kR + r] = xc.dot(bt.wu[r]) * e8m0_scale(bt.su[r]);
      }
    }
    wave_reduce_multi<N>(v, lane);
    if ((lane & ((1 << (6 - L)) - 1)) == 0) red[parity][wave][lane >> (6 - L)] = v[0];
    lds_barrier();
    if (u < n_units && gw == 0 && lane < kR) {
      const int w0 = grp * S;
      float gv = red[parity][w0][lane], uv = red[parity][w0][kR + lane];
      for (int w = 1; w < S; ++w) {
        gv += red[parity][w0 + w][lane];
        uv += red[parity][w0 + w][kR + lane];
      }
      const float hv = activate(g.act, gv, uv);
      if constexpr (kTagged)
        __hip_atomic_store(reinterpret_cast<uint64_t*>(h) + (size_t)u * kR + lane,
                           ((uint64_t)tag << 32) | __float_as_uint(hv), __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
      else if constexpr (kDeviceStore)  // written through to the device-coherent level
        __hip_atomic_store(h + (size_t)u * kR + lane, hv, __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
      else
        h[(size_t)u * kR + lane] = hv;
    }
  };
  const int n_it = kIters > 0 ? kIters : iters;
  GluBatch<XT, kR, kG> A, B;
  glu_load(A, rr, g, unit_pair0(0), cs, gg);
  glu_load(B, rr, g, unit_pair0(min(1, n_it - 1)), cs, gg);
  // kTagged: both units' loads are issued before anything waits for the first
  if constexpr (kTagged) __builtin_amdgcn_sched_barrier(0);
  for (int it = 0;; it += 2) {
    finish(A, it);
    if (it + 2 >= n_it) {
      if (it + 1 < n_it) finish(B, it + 1);
      break;
    }
    glu_load(A, rr, g, unit_pair0(it + 2), cs, gg);
    finish(B, it + 1);
    if (it + 3 >= n_it) {
      finish(A, it + 2);
      break;
    }
    glu_load(B, rr, g, unit_pair0(it + 3), cs, gg);
  }
}

// Positions along blockIdx.y (kPos kernels, router mode): position p reads
// logits + p n_bank and x + p x, writes h + p h and out + p out, and
// publishes its route at ids/w + p n.  Element strides.
struct PosStride {
  int64_t x, h, out;
};

// Unit pipelines per gate/up workgroup (each S column-split waves) and rows
// per unit; the launch bound follows so the register budget matches the
// resident waves (16 waves/CU -> 128 VGPRs, 8 -> 256).
// k_glu_decode refills a unit's registers with the next unit's loads row by
// row (finish_refill) for fp32 activations: K3 gate/up 37.4 -> 34.9 us on
// MI355X.  With bf16 activations the row-pinned schedule costs more than it
// keeps in flight (the benchmark layer's gate/up 41.1 -> 43.0 us), so those
// keep the unit-at-a-time loop.
#ifndef K3_GLU_REFILL
#define K3_GLU_REFILL 1
#endif
template <typename XT>
constexpr bool kGluRefill = K3_GLU_REFILL && sizeof(XT) == 4;
#ifndef K3_GLU_GROUPS
#define K3_GLU_GROUPS 2
#endif
#ifndef K3_GLU_ROWS
#define K3_GLU_ROWS 4
#endif
constexpr int kGluMaxThreads = 256 * K3_GLU_GROUPS;

// XCD-blocked workgroup order.  MI355X dispatches the workgroups of a launch
// to its 8 XCDs round robin (workgroup k runs on XCD k % 8), and each XCD has
// its own L2 and address-translation cache.  Relabelling workgroup k as
// v = (k % 8) * (G / 8) + k / 8 gives every XCD one contiguous range of v, so
// an XCD reads one contiguous stretch of each matrix instead of every eighth
// slice of all of it.  Only which workgroup computes a row changes; every row
// is computed the same way.  Grids that are not a multiple of 8 keep k.
#ifndef K3_XCD_MAP
#define K3_XCD_MAP 3  // bit 0: gate/up units, bit 1: down row batches
#endif
__device__ __forceinline__ int xcd_block_id(int k, int G) {
  if (!(K3_XCD_MAP & 1) || (G & 7)) return k;
  return (k & 7) * (G >> 3) + (k >> 3);
}

template <typename XT, int kR, bool kG, bool kS4 = false, bool kPos = false>
__global__ __launch_bounds__(kGluMaxThreads) __attribute__((amdgpu_waves_per_eu(1, kGluMaxThreads / 256)))
void k_glu_decode(const TokenRoute route_arg,
                                                     const Geo g,
                                                     const XT* __restrict__ x_arg,
                                                     float* __restrict__ h_arg, int n_units,
                                                     int S, const PosStride pos) {
  // The route is read from the kernel argument itself (a modified copy would
  // live in scratch: its span table is indexed per lane); position pidx's
  // pointers are offsets from it.
  const TokenRoute& route = route_arg;
  const int pidx = kPos ? (int)blockIdx.y : 0;
  const size_t proute = (size_t)pidx * route.n;
  const float* logits = route.logits ? route.logits + (size_t)pidx * route.n_bank : nullptr;
  const XT* __restrict__ x = x_arg + pidx * pos.x;
  float* __restrict__ h = h_arg + pidx * pos.h;
  constexpr int N = 2 * kR;
  constexpr int L = log2c<N>();
  extern __shared__ __attribute__((aligned(16))) uint64_t route_scratch[];
  __shared__ float red[2][16][N];
  __shared__ int sel[K3_HIP_MAX_TOKEN_EXPERTS];
  __shared__ float wsel[K3_HIP_MAX_TOKEN_EXPERTS];
  // The workgroup holds `groups` unit pipelines of S column-split waves; one
  // workgroup per CU, so the router below runs once per CU.
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int groups = blockDim.x / (64 * S);
  const int grp = wave / S;
  const int gw = wave - grp * S;  // wave within its group
  const ColSplit cs = col_split(g.hidden >> 5, S, gw, lane);
  // Only the gathered forms read gg (glu_gather needs cw >= 4).
  const GluGather gg = kS4   ? glu_gather4(g.hidden >> 5, S, gw, lane, kR)
                       : kG ? glu_gather(g.hidden >> 5, S, gw, lane, kR)
                            : GluGather{0, 0};
  // cw (scale4-v2: cw / 2): bpermute bytes per row
  const int row_step = (((g.hidden >> 5) + S - 1) / S) >> (kS4 ? 1 : 0);
  // Router mode: the logits are requested before the activation chunk, so
  // the ranking below waits for them alone.
  const bool pre = logits && route.n_bank <= (int)blockDim.x;
  float logit = 0.0f;
  if (pre && (int)threadIdx.x < route.n_bank) logit = logits[threadIdx.x];
  XChunk<XT> xc;
  load_x_chunk<XT>(xc, x, cs);
  RouteRegs rr;
  if (logits) {
    // Router mode: every workgroup ranks the logits itself (no separate
    // launch) and needs only the experts' ids; workgroup 0 publishes the
    // route for the down kernel.
    block_topk(logits, route.n_bank, route.n, route_scratch, sel, wsel, logit, pre, false);
    rr.lo = rr.hi = 0u;
    rr.w = 0.0f;  // the gate/up units do not weight
    if (lane < route.n) {
      // The ranking writes every sel[j < n]; the clamp keeps a bank address
      // in range whatever LDS holds.
      const int id = min(max(sel[lane], 0), route.n_bank - 1);
      const uint64_t p = reinterpret_cast<uint64_t>(route.bank) + (uint64_t)id * route.stride;
      rr.lo = (uint32_t)p;
      rr.hi = (uint32_t)(p >> 32);
    }
    if (blockIdx.x == 0 && wave == 0) {
      // The route's softmax weights (only the down kernel uses them) and the
      // published route: one wave, the same arithmetic as block_softmax, no
      // barrier; the other workgroups skip them.
      const int j = lane;
      float ex = 0.0f;
      if (j < route.n) {
        const float top = key_value(route_scratch[sel[0]]);
        ex = expf(key_value(route_scratch[sel[j]]) - top);
      }
      const float sum = wave_sum(ex);
      if (j < route.n) {
        const float wj = ex / sum;
        route.ids_pub[proute + j] = sel[j];
        route.w_pub[proute + j] = wj;
        if (route.ids_user) route.ids_user[proute + j] = sel[j];
        if (route.w_user) route.w_user[proute + j] = wj;
      }
    }
  } else {
    rr = route_regs(route, lane, proute);
  }
  const uint32_t rb4 = kS4 ? route_bases(rr, route.n, lane) : 0u;
  // Unit pipelines: global pipeline index q = blockIdx.x * groups + grp takes
  // units q, q + Q, q + 2Q, ... (Q = pipelines in the grid).  Every pipeline
  // of the grid runs the same number of iterations (the host sizes the grid
  // so), which keeps the workgroup-wide barrier below uniform.
  const int Q = gridDim.x * groups;
  const int iters = (n_units + Q - 1) / Q;
  const int q0 = xcd_block_id((int)blockIdx.x, (int)gridDim.x) * groups + grp;
  // Unit of iteration `it` (a unit past the end repeats unit 0's loads and
  // stores nothing, so every wave reaches every barrier).
  auto unit_pair0 = [&](int it) {
    const int u = q0 + it * Q;
    return (u < n_units ? u : 0) * kR;
  };
  auto finish = [&](const GluBatch<XT, kR, kG, kS4>& bt, int it) {
    const int u = q0 + it * Q;
    const int parity = it & 1;
    float v[N];
#pragma unroll
    for (int r = 0; r < kR; ++r) {
      if constexpr (kS4) {  // w1 base in byte 0 of the bases, w3 base in byte 2
        v[r] = xc.dot(bt.wg[r]) *
               e8m0_scale(gathered_scale4(bt.sg[0], bt.b4 & 0xffu, gg.bp, row_step, r, lane));
        v[kR + r] = xc.dot(bt.wu[r]) * e8m0_scale(gathered_scale4(bt.su[0], (bt.b4 >> 16) & 0xffu,
                                                                  gg.bp, row_step, r, lane));
      } else if constexpr (kG) {
        v[r] = xc.dot(bt.wg[r]) * e8m0_scale(gathered_scale(bt.sg[0], gg.bp, row_step, r, lane));
        v[kR + r] =
            xc.dot(bt.wu[r]) * e8m0_scale(gathered_scale(bt.su[0], gg.bp, row_step, r, lane));
      } else {
        v[r] = xc.dot(bt.wg[r]) * e8m0_scale(bt.sg[r]);
        v[kR + r] = xc.dot(bt.wu[r]) * e8m0_scale(bt.su[r]);
      }
    }
    wave_reduce_multi<N>(v, lane);
    if ((lane & ((1 << (6 - L)) - 1)) == 0) red[parity][wave][lane >> (6 - L)] = v[0];
    lds_barrier();
    if (u < n_units && gw == 0 && lane < kR) {
      const int w0 = grp * S;
      float gv = red[parity][w0][lane], uv = red[parity][w0][kR + lane];
      for (int w = 1; w < S; ++w) {
        gv += red[parity][w0 + w][lane];
        uv += red[parity][w0 + w][kR + lane];
      }
      h[(size_t)u * kR + lane] = activate(g.act, gv, uv);
    }
  };
  // Where unit it's loads go: its span and first row, or, past the end, every
  // lane at unit 0's bases (row and lane offsets zero).
  struct UnitAt {
    const uint8_t* span;
    size_t r0, rstep, loff, soff;
    int e;
    bool valid;
  };
  const int G = g.hidden >> 5;
  const size_t cp = (size_t)g.hidden >> 1;
  auto unit_at = [&](int it) {
    UnitAt n;
    const int un = q0 + it * Q;
    n.valid = un < n_units;  // wave-uniform
    const int pair0 = (n.valid ? un : 0) * kR;
    n.e = pair0 / g.inter;
    n.span = span_of(rr, n.e);
    n.r0 = (size_t)(pair0 - n.e * g.inter);
    n.rstep = n.valid ? cp : 0;
    n.loff = n.valid ? (size_t)cs.cc * 16 : 0;
    n.soff = n.valid ? (size_t)gg.off : 0;
    return n;
  };
  // The loads of a unit in one fixed order (scale dwords, then row by row
  // gate and up chunks with their scale bytes), pinned by scheduling barriers,
  // so the wait counts in the loop see the same order from every path.
  auto issue_scales = [&](GluBatch<XT, kR, kG, kS4>& bt, const UnitAt& n) {
    if constexpr (kS4) {
      const size_t so = n.r0 * (size_t)(G >> 1) + n.soff;
      bt.sg[0] = load_u32(n.span + g.w1s + so);
      bt.su[0] = load_u32(n.span + g.w3s + so);
      bt.b4 = __builtin_amdgcn_readlane(rb4, n.e);
    } else if constexpr (kG) {
      const size_t so = n.r0 * (size_t)G + n.soff;
      bt.sg[0] = load_u32(n.span + g.w1s + so);
      bt.su[0] = load_u32(n.span + g.w3s + so);
    }
    __builtin_amdgcn_sched_barrier(0);
  };
  auto issue_row = [&](GluBatch<XT, kR, kG, kS4>& bt, const UnitAt& n, int r) {
    const size_t wo = n.r0 * cp + r * n.rstep + n.loff;
    bt.wg[r] = load_chunk(n.span + g.w1p + wo);
    bt.wu[r] = load_chunk(n.span + g.w3p + wo);
    if constexpr (!kG) {
      const size_t so = n.r0 * (size_t)G + r * (n.valid ? (size_t)G : 0) + (n.valid ? cs.cc : 0);
      bt.sg[r] = load_scale(n.span + g.w1s + so);
      bt.su[r] = load_scale(n.span + g.w3s + so);
    }
    __builtin_amdgcn_sched_barrier(0);
  };
  auto issue_unit = [&](GluBatch<XT, kR, kG, kS4>& bt, int it) {
    const UnitAt n = unit_at(it);
    issue_scales(bt, n);
#pragma unroll
    for (int r = 0; r < kR; ++r) issue_row(bt, n, r);
  };
  if constexpr (kGluRefill<XT>) {
  // Unit it's dots with bt refilled by unit it + 2 as its registers free up:
  // every row's scale first (then the scale registers take the next unit's),
  // then row r's products and right after them row r's next chunks.  The wave
  // so keeps about two units' loads in flight through the products, instead
  // of one between a unit's first product and its buffer's next request.  A
  // unit past the end is requested as one 16-byte line and stores nothing, so
  // every load is unconditional and the wait counts stay exact.  The
  // arithmetic per row is that of finish above.
  auto finish_refill = [&](GluBatch<XT, kR, kG, kS4>& bt, int it) {
    const int u = q0 + it * Q;
    const int parity = it & 1;
    float sgv[kR], suv[kR];
#pragma unroll
    for (int r = 0; r < kR; ++r) {
      if constexpr (kS4) {
        sgv[r] = e8m0_scale(gathered_scale4(bt.sg[0], bt.b4 & 0xffu, gg.bp, row_step, r, lane));
        suv[r] = e8m0_scale(
            gathered_scale4(bt.su[0], (bt.b4 >> 16) & 0xffu, gg.bp, row_step, r, lane));
      } else if constexpr (kG) {
        sgv[r] = e8m0_scale(gathered_scale(bt.sg[0], gg.bp, row_step, r, lane));
        suv[r] = e8m0_scale(gathered_scale(bt.su[0], gg.bp, row_step, r, lane));
      } else {
        sgv[r] = e8m0_scale(bt.sg[r]);
        suv[r] = e8m0_scale(bt.su[r]);
      }
    }
    const UnitAt n = unit_at(it + 2);
    issue_scales(bt, n);
    float v[N];
#pragma unroll
    for (int r = 0; r < kR; ++r) {
      v[r] = xc.dot(bt.wg[r]) * sgv[r];
      v[kR + r] = xc.dot(bt.wu[r]) * suv[r];
      issue_row(bt, n, r);
    }
    wave_reduce_multi<N>(v, lane);
    if ((lane & ((1 << (6 - L)) - 1)) == 0) red[parity][wave][lane >> (6 - L)] = v[0];
    lds_barrier();
    if (u < n_units && gw == 0 && lane < kR) {
      const int w0 = grp * S;
      float gv = red[parity][w0][lane], uv = red[parity][w0][kR + lane];
      for (int w = 1; w < S; ++w) {
        gv += red[parity][w0 + w][lane];
        uv += red[parity][w0 + w][kR + lane];
      }
      h[(size_t)u * kR + lane] = activate(g.act, gv, uv);
    }
  };
  GluBatch<XT, kR, kG, kS4> A, B;
  issue_unit(A, 0);
  issue_unit(B, 1);
  // iters is the same in every pipeline; with iters odd the last B unit is
  // past the end (its loads are the one-line dummy, it stores nothing).
  for (int it = 0; it < iters; it += 2) {
    finish_refill(A, it);
    finish_refill(B, it + 1);
  }
  } else {
  // Two units in flight: unit it + 1 is requested before unit it is reduced.
  // (The compiler merges the loop head's wait counts over the entry and the
  // back edge, so at the head the wave waits for both units; a loop that
  // keeps exactly one unit in flight through every reduction measured slower
  // with bf16 activations: 43.9 against 40.9 us on the benchmark layer.)
  GluBatch<XT, kR, kG, kS4> A, B;
  glu_load(A, rr, g, unit_pair0(0), cs, gg, rb4);
  glu_load(B, rr, g, unit_pair0(min(1, iters - 1)), cs, gg, rb4);
  for (int it = 0;; it += 2) {
    finish(A, it);
    if (it + 2 >= iters) {
      if (it + 1 < iters) finish(B, it + 1);
      break;
    }
    glu_load(A, rr, g, unit_pair0(it + 2), cs, gg, rb4);
    finish(B, it + 1);
    if (it + 3 >= iters) {
      finish(A, it + 2);
      break;
    }
    glu_load(B, rr, g, unit_pair0(it + 3), cs, gg, rb4);
  }
  }
}

// ======================================================================
// decode phase A on the matrix cores: k_glu_mfma
// ======================================================================
// The gate/up rows of k_glu_decode on v_mfma_f32_16x16x32_bf16, for raw-v1
// spans and one token.  Operand layout of that MFMA on gfx950 (measured with a
// one-hot probe): A lane l = row l % 16, K = 8 (l / 16) .. +7; B lane l =
// column l % 16, the same K; D lane l = column l % 16, rows 4 (l / 16) .. +3.
//
// Tiles of 8 weight rows, parity split: lane l (r = l % 16, g = l / 16) loads
// the 16-byte chunk of weight row r / 2 at byte 32 g + 16 (r % 2) of a
// 128-byte line, so one dwordx4 load covers 8 rows x a whole line (256
// columns: a K block) and MFMA row r is weight row r / 2 restricted to the
// block's chunks of parity r % 2.  Dword m of the chunk (columns
// 256 kb + 64 g + 32 (r % 2) + 8 m .. +7) becomes A's 8 bf16 through four
// v_cvt_scalef32_pk_bf16_fp4 with the chunk's scale folded in.  The convert
// applies the exponent field of its fp32 scale operand as an E8M0 scale, so
// the operand is the E8M0 byte shifted into that field (2^(s-127) for s in
// 1..254, NaN for 255, which poisons the row as the reference does); fp4
// times a power of two is exact in bf16.  The reference reads scale byte 0 as
// +0.0 where the convert would apply 2^-127, so a chunk with scale byte 0 has
// its codes zeroed first.
//
// The activation enters as NT bf16 terms whose sum is x exactly (bf16 x: one
// term; fp32 x: t0 = bf16(x), t1 = bf16(x - t0), t2 = bf16(x - t0 - t1), each
// remainder exact in fp32), staged once per workgroup in LDS.  B column t
// (t < NT) holds term t at the K block's even-parity columns and column 8 + t
// the same term at the odd parity; the other columns read a row of zeros.
// Products of a bf16 term with fp4 x 2^k are exact in fp32, so the dot
// differs from the VALU kernel's fp32 chain only in summation order.  Row i's
// dot is D[2 i][t] + D[2 i + 1][8 + t] summed over t: lane (n, g) holds
// D[4 g + j][n] in acc[j], so rows 2 g and 2 g + 1 are the 16-lane sums of
// (n < 8 ? acc[0] : acc[1]) and (n < 8 ? acc[2] : acc[3]); the columns
// without a term are exact zeros.
//
// Work split as in k_glu_decode: a unit is one expert's gate and up tiles (8
// rows each); a pipeline of S waves splits a row's KB K blocks (NB = KB / S
// per wave); pipeline q takes units q, q + Q, ... with two units in flight,
// the S partials meet in LDS and wave 0 of the pipeline applies the
// activation.  A wave's unit is 2 NB dwordx4 weight loads plus NR =
// ceil(NB / 4) scale dwords per tile: in register j, lane l holds dword l % 2
// of the 8 scale bytes of row (l % 16) / 2 in K block 4 j + l / 16, and lane
// (r, g) takes its byte of block b from lane 16 (b % 4) + 2 (r / 2) + g / 2
// of register b / 4 by ds_bpermute.
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

// kS4 (scale4-v2): a row's 8 groups of a K block are 8 index nibbles, one
// dword, so one register per matrix holds 8 blocks x 8 rows (lane l: block
// l / 8, row l % 8) and b4 holds the span's scale bases (byte 0: w1, byte 2:
// w3).
template <int NB, bool kS4>
struct GmUnit : std::conditional_t<kS4, SpanBases, NoBases> {
  static constexpr int NR = kS4 ? (NB + 7) / 8 : (NB + 3) / 4;
  u32x4 wg[NB], wu[NB];
  uint32_t sg[NR], su[NR];
};

// Unit loads at rows r0 .. r0 + 7 of the gate and up matrices of `span`, K
// blocks kb0 .. kb0 + NB - 1 (scale dwords first, so waiting for them never
// waits for the weights).  rstep / loff: the byte step between a lane's rows
// and its lane offset (0 and 0 turn every lane's loads into one line at the
// unit's bases, for a unit past the end); b4: the span's scale bases.
template <int NB, bool kS4>
__device__ __forceinline__ void gm_issue_scales(GmUnit<NB, kS4>& u, const uint8_t* span,
                                                const Geo& g, size_t r0, int kb0, int lane,
                                                bool valid, uint32_t b4) {
  const int G = g.hidden >> 5;
#pragma unroll
  for (int j = 0; j < GmUnit<NB, kS4>::NR; ++j) {
    size_t so;
    if constexpr (kS4) {
      const int bb = min(8 * j + (lane >> 3), NB - 1);
      so = (r0 + (valid ? (size_t)(lane & 7) : 0)) * (size_t)(G >> 1) + 4 * (size_t)(kb0 + bb);
    } else {
      const int bb = min(4 * j + (lane >> 4), NB - 1);
      so = (r0 + (valid ? (size_t)((lane & 15) >> 1) : 0)) * (size_t)G +
           8 * (size_t)(kb0 + bb) + (valid ? 4 * (size_t)(lane & 1) : 0);
    }
    u.sg[j] = load_u32(span + g.w1s + so);
    u.su[j] = load_u32(span + g.w3s + so);
  }
  if constexpr (kS4) u.b4 = b4;
}

// Byte offset of this lane's chunk of K block 0 in the gate (or up) matrix.
__device__ __forceinline__ size_t gm_chunk_off(const Geo& g, size_t r0, int kb0, int lane,
                                               bool valid) {
  return valid ? (r0 + ((lane & 15) >> 1)) * ((size_t)g.hidden >> 1) + 128 * (size_t)kb0 +
                     32 * (lane >> 4) + 16 * (lane & 1)
               : r0 * ((size_t)g.hidden >> 1);
}

template <int NB, bool kS4>
__device__ __forceinline__ void gm_load(GmUnit<NB, kS4>& u, const uint8_t* span, const Geo& g,
                                        size_t r0, int kb0, int lane, bool valid, uint32_t b4) {
  gm_issue_scales<NB, kS4>(u, span, g, r0, kb0, lane, valid, b4);
  const size_t wo = gm_chunk_off(g, r0, kb0, lane, valid);
  const size_t bs = valid ? 128 : 0;
  const uint8_t* gp = span + g.w1p + wo;
  const uint8_t* up = span + g.w3p + wo;
#pragma unroll
  for (int b = 0; b < NB; ++b) {
    u.wg[b] = load_chunk(gp + bs * b);
    u.wu[b] = load_chunk(up + bs * b);
  }
}

// Dword d of a chunk (8 codes) as A's 8 bf16, times the scale whose E8M0 byte
// is in the exponent field of sc.
__device__ __forceinline__ bf16x8 gm_cvt(uint32_t d, float sc) {
  const v2bf a = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(d, sc, 0);
  const v2bf b = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(d, sc, 1);
  const v2bf c = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(d, sc, 2);
  const v2bf e = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(d, sc, 3);
  const u32x4 w = {__builtin_bit_cast(uint32_t, a), __builtin_bit_cast(uint32_t, b),
                   __builtin_bit_cast(uint32_t, c), __builtin_bit_cast(uint32_t, e)};
  return __builtin_bit_cast(bf16x8, w);
}

// A tile's chunk of K block b with its scale byte s (byte 0: all codes zero).
__device__ __forceinline__ u32x4 gm_zero_if(u32x4 w, uint32_t s) {
  const bool z = s == 0u;
  w.x = z ? 0u : w.x;
  w.y = z ? 0u : w.y;
  w.z = z ? 0u : w.z;
  w.w = z ? 0u : w.w;
  return w;
}

// The 16-lane sums of the unit's four per-lane values: (gate row 2 g, gate
// row 2 g + 1, up row 2 g, up row 2 g + 1) of lane group g.  kRefill: the
// registers of u are refilled with the unit at (nspan, nr0) as they free up
// (its scale dwords once every block's scale byte is extracted, block b's
// chunks right after block b's products), so the wave keeps about two units'
// loads in flight through the products instead of one.
template <int NB, bool kS4, bool kRefill>
__device__ __forceinline__ void gm_dots(GmUnit<NB, kS4>& u, const uint8_t* xb, int lane,
                                        float (&v)[4], const uint8_t* nspan, const Geo& g,
                                        size_t nr0, int kb0, bool nvalid, uint32_t nb4) {
  f32x4 ag = {0.f, 0.f, 0.f, 0.f}, au = {0.f, 0.f, 0.f, 0.f};
  uint32_t sgb[NB], sub[NB];
  if constexpr (kS4) {
    // group 2 g + h of row (l % 16) / 2 in block b: nibble 2 g + h of lane
    // 8 b + row's dword
    const int sh = 4 * (2 * (lane >> 4) + (lane & 1));
    const int src = 4 * ((lane & 15) >> 1);
    const uint32_t bg = u.b4 & 0xffu, bu = (u.b4 >> 16) & 0xffu;
#pragma unroll
    for (int b = 0; b < NB; ++b) {
      sgb[b] = bg + (((uint32_t)__builtin_amdgcn_ds_bpermute(src + 32 * (b & 7),
                                                             (int)u.sg[b >> 3]) >> sh) & 0xfu);
      sub[b] = bu + (((uint32_t)__builtin_amdgcn_ds_bpermute(src + 32 * (b & 7),
                                                             (int)u.su[b >> 3]) >> sh) & 0xfu);
    }
  } else {
    const int sh = 8 * (2 * ((lane >> 4) & 1) + (lane & 1));
    const int src = 4 * ((lane & 14) + (lane >> 5));
#pragma unroll
    for (int b = 0; b < NB; ++b) {
      sgb[b] = ((uint32_t)__builtin_amdgcn_ds_bpermute(src + 64 * (b & 3), (int)u.sg[b >> 2]) >>
                sh) & 0xffu;
      sub[b] = ((uint32_t)__builtin_amdgcn_ds_bpermute(src + 64 * (b & 3), (int)u.su[b >> 2]) >>
                sh) & 0xffu;
    }
  }
  const uint8_t* ngp = nullptr;
  const uint8_t* nup = nullptr;
  const size_t bs = nvalid ? 128 : 0;
  if constexpr (kRefill) {
    gm_issue_scales<NB, kS4>(u, nspan, g, nr0, kb0, lane, nvalid, nb4);
    const size_t wo = gm_chunk_off(g, nr0, kb0, lane, nvalid);
    ngp = nspan + g.w1p + wo;
    nup = nspan + g.w3p + wo;
    __builtin_amdgcn_sched_barrier(0);
  }
#pragma unroll
  for (int b = 0; b < NB; ++b) {
    const float cg = e8m0_scale(sgb[b]), cu = e8m0_scale(sub[b]);
    const u32x4 wg = gm_zero_if(u.wg[b], sgb[b]), wu = gm_zero_if(u.wu[b], sub[b]);
#pragma unroll
    for (int m = 0; m < 4; ++m) {
      const bf16x8 bx = *reinterpret_cast<const bf16x8*>(xb + 2 * (256 * b + 8 * m));
      ag = __builtin_amdgcn_mfma_f32_16x16x32_bf16(gm_cvt(wg[m], cg), bx, ag, 0, 0, 0);
      au = __builtin_amdgcn_mfma_f32_16x16x32_bf16(gm_cvt(wu[m], cu), bx, au, 0, 0, 0);
    }
    if constexpr (kRefill) {
      u.wg[b] = load_chunk(ngp + bs * b);
      u.wu[b] = load_chunk(nup + bs * b);
      __builtin_amdgcn_sched_barrier(0);
    }
  }
  const bool lo = (lane & 8) == 0;
  v[0] = lo ? ag[0] : ag[1];
  v[1] = lo ? ag[2] : ag[3];
  v[2] = lo ? au[0] : au[1];
  v[3] = lo ? au[2] : au[3];
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    v[k] += dpp_f32<0xB1>(v[k]);   // quad_perm [1,0,3,2]
    v[k] += dpp_f32<0x4E>(v[k]);   // quad_perm [2,3,0,1]
    v[k] += dpp_f32<0x141>(v[k]);  // row_half_mirror
    v[k] += dpp_f32<0x140>(v[k]);  // row_mirror
  }
}

// Bytes of one activation term row in LDS (16 bytes of padding shift the
// terms' rows to distinct banks).
__host__ __device__ constexpr size_t gm_term_bytes(int hidden) { return 2 * (size_t)hidden + 16; }

constexpr int kGmThreads = 512;

template <typename XT, int NT, int NB, int IT, bool kS4 = false, bool kPos = false>
__global__ __launch_bounds__(kGmThreads) void k_glu_mfma(const TokenRoute route_arg, const Geo g,
                                                         const XT* __restrict__ x_arg,
                                                         float* __restrict__ h_arg, int n_units,
                                                         int S, int xs_off, const PosStride pos) {
  // Positions along blockIdx.y as in k_glu_decode (kPos).
  const TokenRoute& route = route_arg;  // read in place (see k_glu_decode)
  const int pidx = kPos ? (int)blockIdx.y : 0;
  const size_t proute = (size_t)pidx * route.n;
  const float* logits = route.logits ? route.logits + (size_t)pidx * route.n_bank : nullptr;
  const XT* __restrict__ x = x_arg + pidx * pos.x;
  float* __restrict__ h = h_arg + pidx * pos.h;
  extern __shared__ __attribute__((aligned(16))) uint64_t route_scratch[];
  __shared__ float red[2][8][16];
  __shared__ int sel[K3_HIP_MAX_TOKEN_EXPERTS];
  __shared__ float wsel[K3_HIP_MAX_TOKEN_EXPERTS];
  uint8_t* xs = reinterpret_cast<uint8_t*>(route_scratch) + xs_off;
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int groups = kGmThreads / (64 * S);
  const int grp = wave / S;
  const int gw = wave - grp * S;
  const bool pre = logits && route.n_bank <= (int)blockDim.x;
  float logit = 0.0f;
  if (pre && (int)threadIdx.x < route.n_bank) logit = logits[threadIdx.x];
  // The activation, 8 columns per thread and step, requested before the route.
  const int n8 = g.hidden >> 3;
  constexpr int kXSteps = 2;  // hidden <= 8192 (host)
  typedef std::conditional_t<sizeof(XT) == 4, float4, uint4> XV;
  XV xv[kXSteps][sizeof(XT) == 4 ? 2 : 1];
#pragma unroll
  for (int s = 0; s < kXSteps; ++s) {
    const int k = min((int)threadIdx.x + s * kGmThreads, n8 - 1);
    const XV* src = reinterpret_cast<const XV*>(x) + k * (sizeof(XT) == 4 ? 2 : 1);
#pragma unroll
    for (int q = 0; q < (sizeof(XT) == 4 ? 2 : 1); ++q) xv[s][q] = src[q];
  }
  RouteRegs rr;
  if (logits) {
    block_topk(logits, route.n_bank, route.n, route_scratch, sel, wsel, logit, pre, false);
    rr.lo = rr.hi = 0u;
    rr.w = 0.0f;
    if (lane < route.n) {
      const int id = min(max(sel[lane], 0), route.n_bank - 1);
      const uint64_t p = reinterpret_cast<uint64_t>(route.bank) + (uint64_t)id * route.stride;
      rr.lo = (uint32_t)p;
      rr.hi = (uint32_t)(p >> 32);
    }
    if (blockIdx.x == 0 && wave == 0) {
      const int j = lane;
      float ex = 0.0f;
      if (j < route.n) {
        const float top = key_value(route_scratch[sel[0]]);
        ex = expf(key_value(route_scratch[sel[j]]) - top);
      }
      const float sum = wave_sum(ex);
      if (j < route.n) {
        const float wj = ex / sum;
        route.ids_pub[proute + j] = sel[j];
        route.w_pub[proute + j] = wj;
        if (route.ids_user) route.ids_user[proute + j] = sel[j];
        if (route.w_user) route.w_user[proute + j] = wj;
      }
    }
  } else {
    rr = route_regs(route, lane, proute);
  }
  const uint32_t rb4 = kS4 ? route_bases(rr, route.n, lane) : 0u;
  const int tpe = g.inter >> 3;      // tiles per expert
  const int Q = gridDim.x * groups;  // IT = ceil(n_units / Q) (host)
  const int q0 = xcd_block_id((int)blockIdx.x, (int)gridDim.x) * groups + grp;
  const int kb0 = gw * NB;
  // Where unit it's loads go: its span and first row; past the end every lane
  // at unit 0's bases (one line, in bounds), so every load is unconditional.
  struct UnitAt {
    const uint8_t* span;
    size_t r0;
    uint32_t b4;
    bool valid;
  };
  auto unit_at = [&](int it) {
    UnitAt n;
    const int un = q0 + it * Q;
    n.valid = un < n_units;  // wave-uniform
    const int u = n.valid ? un : 0;
    const int e = u / tpe;
    n.span = span_of(rr, e);
    n.r0 = (size_t)(8 * (u - e * tpe));
    n.b4 = kS4 ? (uint32_t)__builtin_amdgcn_readlane(rb4, e) : 0u;
    return n;
  };
  // The scheduling barrier keeps a unit's loads where they are written: sunk
  // into the next unit's dots, they would wait behind that unit's data.
  auto load_unit = [&](GmUnit<NB, kS4>& dst, int it) {
    const UnitAt n = unit_at(it);
    gm_load<NB, kS4>(dst, n.span, g, n.r0, kb0, lane, n.valid, n.b4);
    __builtin_amdgcn_sched_barrier(0);
  };
  // Two units in flight, in a fully unrolled loop of IT iterations with no
  // branches around the loads: a loop-carried pair of buffers would become
  // register copies at the loop head (copying an in-flight register waits for
  // its load), and a load under a runtime condition makes the wait counts
  // after it assume the branch that issued fewer loads.
  GmUnit<NB, kS4> bt[2];
  load_unit(bt[0], 0);
  if constexpr (IT > 1) load_unit(bt[1], 1);
  // Terms into LDS (waits for the activation loads only: they were issued
  // first), then the zero row.
  {
    const size_t tb = gm_term_bytes(g.hidden);
#pragma unroll
    for (int s = 0; s < kXSteps; ++s) {
      const int k = (int)threadIdx.x + s * kGmThreads;
      if (k >= n8) continue;
      uint32_t t[NT][4];
      if constexpr (sizeof(XT) == 4) {
        const float f[8] = {xv[s][0].x, xv[s][0].y, xv[s][0].z, xv[s][0].w,
                            xv[s][1].x, xv[s][1].y, xv[s][1].z, xv[s][1].w};
#pragma unroll
        for (int e = 0; e < 8; e += 2) {
          uint32_t b0[2], b1[2], b2[2];
#pragma unroll
          for (int o = 0; o < 2; ++o) {
            const float v = f[e + o];
            b0[o] = f32_to_bf16_bits(v);
            const float r1 = v - __uint_as_float(b0[o] << 16);
            b1[o] = f32_to_bf16_bits(r1);
            b2[o] = f32_to_bf16_bits(r1 - __uint_as_float(b1[o] << 16));
          }
          t[0][e >> 1] = b0[0] | (b0[1] << 16);
          if constexpr (NT > 1) t[1][e >> 1] = b1[0] | (b1[1] << 16);
          if constexpr (NT > 2) t[2][e >> 1] = b2[0] | (b2[1] << 16);
        }
      } else {
        t[0][0] = xv[s][0].x;
        t[0][1] = xv[s][0].y;
        t[0][2] = xv[s][0].z;
        t[0][3] = xv[s][0].w;
      }
#pragma unroll
      for (int q = 0; q < NT; ++q)
        *reinterpret_cast<uint4*>(xs + q * tb + 16 * (size_t)k) =
            make_uint4(t[q][0], t[q][1], t[q][2], t[q][3]);
      *reinterpret_cast<uint4*>(xs + NT * tb + 16 * (size_t)k) = make_uint4(0u, 0u, 0u, 0u);
    }
  }
  lds_barrier();
  // This lane's B row: term n % 8 (the zero row past NT) at parity n / 8.
  const int n = lane & 15;
  const uint8_t* xb = xs + min(n & 7, NT) * gm_term_bytes(g.hidden) +
                      2 * (256 * kb0 + 64 * (lane >> 4) + 32 * (n >> 3));
  // Unit it's dots (refilling bt with unit it + 2 when kRefill), then its
  // partials through LDS and the activation.
  auto finish = [&](GmUnit<NB, kS4>& bt, int it, auto refill) {
    constexpr bool kRefill = decltype(refill)::value;
    const int u = q0 + it * Q;
    const int parity = it & 1;
    float v[4];
    const UnitAt nx = unit_at(it + 2);
    gm_dots<NB, kS4, kRefill>(bt, xb, lane, v, nx.span, g, nx.r0, kb0, nx.valid, nx.b4);
    if ((lane & 15) == 0) {
      const int gi = lane >> 4;
      red[parity][wave][2 * gi] = v[0];
      red[parity][wave][2 * gi + 1] = v[1];
      red[parity][wave][8 + 2 * gi] = v[2];
      red[parity][wave][8 + 2 * gi + 1] = v[3];
    }
    lds_barrier();
    if (u < n_units && gw == 0 && lane < 8) {
      const int w0 = grp * S;
      float gv = red[parity][w0][lane], uv = red[parity][w0][8 + lane];
      for (int w = 1; w < S; ++w) {
        gv += red[parity][w0 + w][lane];
        uv += red[parity][w0 + w][8 + lane];
      }
      h[(size_t)u * 8 + lane] = activate(g.act, gv, uv);
    }
  };
#pragma unroll
  for (int it = 0; it < IT; ++it) {
    if (it + 2 < IT)
      finish(bt[it & 1], it, std::true_type{});
    else
      finish(bt[it & 1], it, std::false_type{});
  }
}

// ======================================================================
// decode phase B: down rows of every routed expert + ordered combine
// ======================================================================
// kG (gathered scales): with 64 scale groups per row (one chunk per lane) the
// kB = 4 rows of a batch have their scale bytes in one contiguous 256 B run,
// so lane l loads its dword l of the run and each lane's byte of row u
// (byte 64 u + l, held by lane 16 u + l / 4) is routed to it by a
// ds_bpermute: one load instead of kB single-byte loads.
template <int CPL, int kB, bool kG = false>
struct DownBatch {
  static_assert(!kG || (CPL == 1 && kB == 4), "gathered scales need CPL 1, kB 4");
  u32x4 w[kB][CPL];
  uint32_t s[kG ? 1 : kB][CPL];
};

// kS4 (scale4-v2, byte-scale path only): s[u][c] receives the index byte that
// holds the nibble of group cc[c] of row r (flattened index r * GB + cc[c];
// GB is even, so the nibble is the high one exactly when cc[c] is odd), and
// down_dots turns it into base + index.
template <int CPL, int kB, bool kG, bool kS4 = false>
__device__ __forceinline__ void down_load(DownBatch<CPL, kB, kG>& bt, const uint8_t* span,
                                          const Geo& g, const int* cc, int r0, int nrows) {
  static_assert(!kS4 || !kG, "scale4-v2 down loads use the byte-scale path");
  const int GB = g.inter >> 5;
  const size_t cpb = (size_t)g.inter >> 1;
  const uint8_t* dp = span + g.w2p;
  const uint8_t* ds = span + g.w2s;
  if constexpr (kG) {
    // GB == 64 and cc[0] == lane.  Rows past nrows are not in the matrix:
    // their lanes re-read the last dword present (those rows' results are
    // discarded).  Issued first, so waiting for it never waits for the data.
    // Every address is a wave-uniform row base plus a 32-bit lane offset (the
    // scalar-base form of the load: no per-row address registers).
    const int d = min(cc[0], nrows * 16 - 1);
    const uint32_t lo = (uint32_t)cc[0] << 4;
    bt.s[0][0] = load_u32(ds + (size_t)r0 * 64 + 4 * d);
#pragma unroll
    for (int u = 0; u < kB; ++u) {
      const int r = r0 + min(u, nrows - 1);
      bt.w[u][0] = load_chunk(dp + (size_t)r * cpb + lo);
    }
  } else {
#pragma unroll
    for (int u = 0; u < kB; ++u) {
      const int r = r0 + min(u, nrows - 1);
#pragma unroll
      for (int c = 0; c < CPL; ++c) {
        bt.w[u][c] = load_chunk(dp + (size_t)r * cpb + (size_t)cc[c] * 16);
        if constexpr (kS4)
          bt.s[u][c] = load_scale(ds + (((size_t)r * GB + cc[c]) >> 1));
        else
          bt.s[u][c] = load_scale(ds + (size_t)r * GB + cc[c]);
      }
    }
  }
}

// h_e's chunks cc[c] for this lane straight from memory (zero where the lane
// has no chunk).  Each of the 8 float4 loads touches 64 lines 128 B apart.
template <int CPL>
__device__ __forceinline__ void load_h_slice(XChunk<float>* hs, const float* he, const int* cc,
                                             const bool* valid) {
#pragma unroll
  for (int c = 0; c < CPL; ++c) {
    hs[c].load(he, cc[c]);
#pragma unroll
    for (int i = 0; i < 32; ++i) hs[c].v[i] = valid[c] ? hs[c].v[i] : 0.0f;
  }
}

// The same for one chunk per lane (64 chunks per row, chunk = lane), through
// the wave's LDS region: 8 coalesced 1 KB loads of h_e, stored so that lane
// l's chunk (float4s 8 l .. 8 l + 7) sits at float4 9 l .. 9 l + 7 (one float4
// of padding per chunk puts the 16 lanes of a ds_read_b128 pass on distinct
// banks); every access is a base register plus an immediate offset.  A wave's
// LDS operations complete in order, so no barrier is needed.
constexpr int kHSliceF4 = 9 * 64;  // float4s of LDS per wave

// Issue the 8 coalesced loads (float4 64 q + lane of h_e into t[q]) ...
__device__ __forceinline__ void h_slice_issue(float4 (&t)[8], const float* he, int lane) {
  const float4* src = reinterpret_cast<const float4*>(he) + lane;
#pragma unroll
  for (int q = 0; q < 8; ++q) t[q] = src[64 * q];
}

// ... and, once the weight loads behind them are issued too, route them
// through LDS: float4 64 q + lane belongs to chunk 8 q + lane / 8 at position
// lane % 8.
__device__ __forceinline__ void h_slice_transpose(XChunk<float>& hs, const float4 (&t)[8],
                                                  float4* hw, int lane) {
  float4* dst = hw + 9 * (lane >> 3) + (lane & 7);
#pragma unroll
  for (int q = 0; q < 8; ++q) dst[72 * q] = t[q];
  const float4* mine = hw + 9 * lane;
#pragma unroll
  for (int q = 0; q < 8; ++q) {
    const float4 v = mine[q];
    hs.v[4 * q + 0] = v.x;
    hs.v[4 * q + 1] = v.y;
    hs.v[4 * q + 2] = v.z;
    hs.v[4 * q + 3] = v.w;
  }
}

// kS4: base is the expert's w2 base and shift4[c] the nibble position of
// chunk cc[c] (4 when cc[c] is odd).
template <int CPL, int kB, bool kG, bool kS4 = false>
__device__ __forceinline__ float down_dots(const DownBatch<CPL, kB, kG>& bt,
                                           const XChunk<float>* hs, int lane,
                                           uint32_t base = 0u, const int* shift4 = nullptr) {
  float v[kB];
#pragma unroll
  for (int u = 0; u < kB; ++u) {
    if constexpr (kS4) {
      float a = 0.0f;
#pragma unroll
      for (int c = 0; c < CPL; ++c) {
        const uint32_t sc = base + ((bt.s[u][c] >> shift4[c]) & 0xfu);
        a = c == 0 ? hs[0].dot(bt.w[u][0]) * e8m0_scale(sc)
                   : a + hs[c].dot(bt.w[u][c]) * e8m0_scale(sc);
      }
      v[u] = a;
    } else if constexpr (kG) {
      const uint32_t word =
          (uint32_t)__builtin_amdgcn_ds_bpermute((16 * u + (lane >> 2)) << 2, (int)bt.s[0][0]);
      v[u] = hs[0].dot(bt.w[u][0]) * e8m0_scale((word >> (8 * (lane & 3))) & 0xffu);
    } else {
      float a = hs[0].dot(bt.w[u][0]) * e8m0_scale(bt.s[u][0]);
#pragma unroll
      for (int c = 1; c < CPL; ++c) a += hs[c].dot(bt.w[u][c]) * e8m0_scale(bt.s[u][c]);
      v[u] = a;
    }
  }
  wave_reduce_multi<kB>(v, lane);
  return v[0];
}

// k_down_blocks: the output rows are cut into batches of kB rows, and
// workgroup b owns batches b, b + G, b + 2G, ... (G workgroups, one per CU), so
// at any moment the grid reads one contiguous stretch of every routed expert's
// down matrix (DRAM rows are opened once and read whole) while each workgroup
// still owns its output rows outright.  Wave w takes routed experts w, w + nw,
// ... with its h slice in registers and two batches in flight (one butterfly
// per batch); the route-ordered weighted sum out = sum over e in route order of
// w_e * y_e (tools/metal/moe_mxfp4.metal:410-445 order) is formed out of LDS.
constexpr int kDownMaxRows = 64;

#ifndef K3_DOWN_THREADS
#define K3_DOWN_THREADS 1024
#endif
#ifndef K3_DOWN_THREADS_WIDE
#define K3_DOWN_THREADS_WIDE 512
#endif
#ifndef K3_DOWN_BATCH_CPL2
#define K3_DOWN_BATCH_CPL2 2
#endif
template <int CPLB>
constexpr int down_max_threads() {
  return CPLB <= 1 ? K3_DOWN_THREADS : K3_DOWN_THREADS_WIDE;
}

template <typename OT, int CPLB, int kB, bool kS4 = false>
__global__ __launch_bounds__(down_max_threads<CPLB>()) void k_down_blocks(
    const TokenRoute route, const Geo g, const float* __restrict__ h, OT* __restrict__ out) {
  constexpr int L = log2c<kB>();
  __shared__ float ybuf[K3_HIP_MAX_TOKEN_EXPERTS][kDownMaxRows];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform: SGPR
  const int nw = blockDim.x >> 6;
  const int G = gridDim.x;
  const int nbt = (g.hidden + kB - 1) / kB;       // batches in the whole output
  const int nb = (nbt - (int)blockIdx.x + G - 1) / G;  // this workgroup's batches
  const int GB = g.inter >> 5;
  int cc[CPLB];
  bool valid[CPLB];
  int shift4[CPLB];  // scale4-v2: nibble position of chunk cc[c]
#pragma unroll
  for (int c = 0; c < CPLB; ++c) {
    valid[c] = lane + 64 * c < GB;
    cc[c] = min(lane + 64 * c, GB - 1);
    shift4[c] = (cc[c] & 1) * 4;
  }
  // First output row of this workgroup's local batch i, and its row count.
  auto row_of = [&](int i) { return (i * G + (int)blockIdx.x) * kB; };
  auto rows_in = [&](int i) { return min(kB, g.hidden - row_of(i)); };
  const RouteRegs rreg = route_regs(route, lane);
  const uint32_t rb4 = kS4 ? route_bases(rreg, route.n, lane) : 0u;
  const int idx = lane >> (6 - L);
  const bool writer = (lane & ((1 << (6 - L)) - 1)) == 0;
  for (int e = wave; e < route.n; e += nw) {
    const uint8_t* span = span_of(rreg, e);
    const uint32_t base = kS4 ? (__builtin_amdgcn_readlane(rb4, e) >> 8) & 0xffu : 0u;
    // Two batches in flight: batch b + 1 is requested before batch b is
    // reduced.  Loads are unconditional inside the loop (the loop exits
    // instead), so the compiler's wait counts stay partial.
    XChunk<float> hs[CPLB];
    load_h_slice<CPLB>(hs, h + (size_t)e * g.inter, cc, valid);
    DownBatch<CPLB, kB> A, B;
    down_load<CPLB, kB, false, kS4>(A, span, g, cc, row_of(0), rows_in(0));
    const int b1 = min(1, nb - 1);
    down_load<CPLB, kB, false, kS4>(B, span, g, cc, row_of(b1), rows_in(b1));
    for (int b = 0;; b += 2) {
      const float va = down_dots<CPLB, kB, false, kS4>(A, hs, lane, base, shift4);
      if (writer && idx < rows_in(b)) ybuf[e][b * kB + idx] = va;
      if (b + 2 >= nb) {
        if (b + 1 < nb) {
          const float vb = down_dots<CPLB, kB, false, kS4>(B, hs, lane, base, shift4);
          if (writer && idx < rows_in(b + 1)) ybuf[e][(b + 1) * kB + idx] = vb;
        }
        break;
      }
      down_load<CPLB, kB, false, kS4>(A, span, g, cc, row_of(b + 2), rows_in(b + 2));
      const float vb = down_dots<CPLB, kB, false, kS4>(B, hs, lane, base, shift4);
      if (writer && idx < rows_in(b + 1)) ybuf[e][(b + 1) * kB + idx] = vb;
      if (b + 3 >= nb) {
        const float va2 = down_dots<CPLB, kB, false, kS4>(A, hs, lane, base, shift4);
        if (writer && idx < rows_in(b + 2)) ybuf[e][(b + 2) * kB + idx] = va2;
        break;
      }
      down_load<CPLB, kB, false, kS4>(B, span, g, cc, row_of(b + 3), rows_in(b + 3));
    }
  }
  __syncthreads();
  for (int t = threadIdx.x; t < nb * kB; t += blockDim.x) {
    const int row = row_of(t / kB) + (t % kB);
    if (row >= g.hidden) continue;
    float acc = 0.0f;
    for (int e = 0; e < route.n; ++e) acc += weight_of(rreg, e) * ybuf[e][t];
    store_out(out + row, acc);
  }
}

// Down + ordered combine for a few routed experts at intermediate 2048
// (k_down_g64's row batches: 4 rows, one 16-byte chunk per lane, gathered
// scales).  k_down_g64 gives each expert a wave that reloads that expert's
// whole h (8 KB) from L2 for its own batches, which at one expert means 1,792
// one-wave workgroups moving 14.7 MB of h for 7.3 MB of weights.  Here a
// workgroup of kFewWaves waves stages the NE experts' h in LDS once (NE x 8 KB,
// k_down_g64's padded layout) and each wave takes one row batch for every
// expert: it requests the batch's rows of all NE experts up front, then sums
// w_e * y_e over the experts in route order, the order k_down_g64's combine
// uses, with the same per-row dot.
constexpr int kFewWaves = 4;
#ifndef K3_DOWN_FEW_MAX
#define K3_DOWN_FEW_MAX 4  // routed experts up to which k_down_few replaces k_down_g64
#endif

template <typename OT, int NE>
__global__ __launch_bounds__(64 * kFewWaves) void k_down_few(const TokenRoute route_arg,
                                                             const Geo g,
                                                             const float* __restrict__ h,
                                                             OT* __restrict__ out) {
  const TokenRoute& route = route_arg;  // read in place (see k_glu_decode)
  constexpr int kB = 4;
  extern __shared__ float4 hbuf[];  // NE x kHSliceF4
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int nbt = (g.hidden + kB - 1) / kB;
  const int batch = (int)blockIdx.x * kFewWaves + wave;
  const int r0 = min(batch, nbt - 1) * kB;  // a batch past the end re-reads the last one
  const int rows = min(kB, g.hidden - r0);
  // h first (its waits never wait for the weights): 8 floats per thread and
  // expert, float4 f = q 256 + t of expert e
  const float4* h4 = reinterpret_cast<const float4*>(h);
  float4 ht[NE][2];
#pragma unroll
  for (int e = 0; e < NE; ++e)
#pragma unroll
    for (int q = 0; q < 2; ++q) ht[e][q] = h4[(size_t)e * (g.inter >> 2) + q * 256 + threadIdx.x];
  __builtin_amdgcn_sched_barrier(0);
  const RouteRegs rreg = route_regs(route, lane);
  const int cc[1] = {lane};
  DownBatch<1, kB, true> bt[NE];
#pragma unroll
  for (int e = 0; e < NE; ++e) down_load(bt[e], span_of(rreg, e), g, cc, r0, rows);
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int e = 0; e < NE; ++e)
#pragma unroll
    for (int q = 0; q < 2; ++q) {
      const int f = q * 256 + (int)threadIdx.x;
      hbuf[e * kHSliceF4 + 9 * (f >> 3) + (f & 7)] = ht[e][q];
    }
  lds_barrier();
  float acc = 0.0f;
#pragma unroll
  for (int e = 0; e < NE; ++e) {
    XChunk<float> hs;
    const float4* mine = hbuf + e * kHSliceF4 + 9 * lane;
#pragma unroll
    for (int q = 0; q < 8; ++q) {
      const float4 v = mine[q];
      hs.v[4 * q + 0] = v.x;
      hs.v[4 * q + 1] = v.y;
      hs.v[4 * q + 2] = v.z;
      hs.v[4 * q + 3] = v.w;
    }
    const float v = down_dots(bt[e], &hs, lane);
    acc += weight_of(rreg, e) * v;
  }
  const int idx = lane >> 4;
  if ((lane & 15) == 0 && batch < nbt && idx < rows) store_out(out + r0 + idx, acc);
}

// k_down_g64: the same split for intermediate 2048 (64 scale groups per row:
// one chunk per lane, batches of 4 rows with gathered scales, h_e's slice
// transposed through LDS).  Every workgroup runs exactly NB batch slots (a
// slot past its share re-reads its last batch and stores nothing), fully
// unrolled, so the double-buffer schedule is straight-line code: while batch
// b is reduced batch b + 1 is in flight, and batch b + 2 is requested right
// after b's registers are free.
constexpr int kDownG64MaxNB = 8;
// Row batches in flight per wave.  Three measured 22.6 -> 28.0 us for the
// config-2 down kernel (more concurrent DRAM rows per CU), so two.
#ifndef K3_DOWN_INFLIGHT
#define K3_DOWN_INFLIGHT 2
#endif

template <typename OT, int NB, bool kPos = false>
__global__ __launch_bounds__(1024) void k_down_g64(const TokenRoute route_arg, const Geo g,
                                                   const float* __restrict__ h_arg,
                                                   OT* __restrict__ out_arg, const PosStride pos) {
  const TokenRoute& route = route_arg;  // read in place (see k_glu_decode)
  const int pidx = kPos ? (int)blockIdx.y : 0;
  const size_t proute = (size_t)pidx * route.n;
  const float* __restrict__ h = h_arg + pidx * pos.h;
  OT* __restrict__ out = out_arg + pidx * pos.out;
  constexpr int kB = 4;
  __shared__ float ybuf[K3_HIP_MAX_TOKEN_EXPERTS][NB * kB];
  extern __shared__ float4 hbuf[];  // kHSliceF4 float4 per wave
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform: SGPR
  const int G = gridDim.x;
  const int nbt = (g.hidden + kB - 1) / kB;
  const int nb = (nbt - (int)blockIdx.x + G - 1) / G;  // 1 <= nb <= NB (host)
  const int cc[1] = {lane};
  // Batch i of workgroup k is i G + k; XCD-blocked (xcd_block_id) when the
  // grid covers the batches exactly (nbt = G NB): XCD x = k % 8 owns batches
  // x J NB .. (x + 1) J NB - 1 (J = G / 8) and its workgroup j = k / 8 takes
  // x J NB + i J + j, so each XCD reads one contiguous stretch at a time.
  const bool xmap = (K3_XCD_MAP & 2) && (G & 7) == 0 && nbt == G * NB;
  const int xb = xmap ? ((int)blockIdx.x & 7) * (G >> 3) * NB + ((int)blockIdx.x >> 3)
                      : (int)blockIdx.x;
  const int xs = xmap ? (G >> 3) : G;
  auto row_of = [&](int i) { return (min(i, nb - 1) * xs + xb) * kB; };
  auto rows_in = [&](int i) { return min(kB, g.hidden - row_of(i)); };
  const int idx = lane >> 4;
  const bool writer = (lane & 15) == 0;
  // One routed expert per wave (the host launches route.n <= 16 waves).
  // h_e is indexed by route slot, not by the expert's span, so its loads are
  // written ahead of the route; the compiler still issues them after the
  // route's wait, behind the loads of batches 0 and 1 (hipcc 7.2 ISA), and the
  // LDS transpose then waits for them.
  const int e = wave;
  float4 ht[8];
  h_slice_issue(ht, h + (size_t)e * g.inter, lane);
  __builtin_amdgcn_sched_barrier(0);
  const RouteRegs rreg = route_regs(route, lane, proute);
  {
    const uint8_t* span = span_of(rreg, e);
    constexpr int kF = K3_DOWN_INFLIGHT;  // batches in flight per wave
    DownBatch<1, kB, true> bt[kF];
#pragma unroll
    for (int f = 0; f < kF; ++f)
      if (f < NB) down_load(bt[f], span, g, cc, row_of(f), rows_in(f));
    __builtin_amdgcn_sched_barrier(0);
    XChunk<float> hs;
    h_slice_transpose(hs, ht, hbuf + wave * kHSliceF4, lane);
#pragma unroll
    for (int b = 0; b < NB; ++b) {
      const float v = down_dots(bt[b % kF], &hs, lane);
      if (b + kF < NB) down_load(bt[b % kF], span, g, cc, row_of(b + kF), rows_in(b + kF));
      if (writer && b < nb && idx < rows_in(b)) ybuf[e][b * kB + idx] = v;
    }
  }
  __syncthreads();
  for (int t = threadIdx.x; t < nb * kB; t += blockDim.x) {
    const int row = row_of(t / kB) + (t % kB);
    if (row >= g.hidden) continue;
    float acc = 0.0f;
    for (int e = 0; e < route.n; ++e) acc += weight_of(rreg, e) * ybuf[e][t];
    store_out(out + row, acc);
  }
}

// k_down_g96: the same split for intermediate 3072 (96 scale groups per row:
// the K3 geometry).  The batch is a pair of output rows (2 p, 2 p + 1): its
// weights are 3,072 contiguous bytes of the matrix and its scales 192
// contiguous bytes.  Lane l takes group l of both rows (the "head" chunks: two
// coalesced 1 KB loads) and group 64 + l % 32 of row 2 p + l / 32 (the "tail"
// chunk: two 512 B runs), so every lane has three chunks of every pair and
// holds two chunks of h_e (l and 64 + l % 32: 64 floats) instead of three.
// Lane m (< 48) loads dword m of the pair's scales and ds_bpermute hands each
// lane its three bytes: head of row 2 p is byte l, head of row 2 p + 1 byte
// 96 + l, the tail byte 64 + l (l < 32) or 128 + l (l >= 32).  kS4
// (scale4-v2): the pair's 192 index nibbles are 96 bytes (lane m < 24 loads
// dword m) and nibble q sits in dword q / 8 at bit 4 (q % 8), added to the
// expert's base.  One wave per routed expert, NB pair slots unrolled with two
// in flight, h_e's chunks transposed through LDS and the route-ordered
// combine out of LDS, as in k_down_g64.
constexpr int kG96RowBytes = 1536;  // 3072 nibbles
constexpr int kG96ScaleBytes = 96;  // per row (raw-v1)

struct PairBatch {
  u32x4 a, b, c;  // head of row 2 p, head of row 2 p + 1, tail
  uint32_t s;     // the scale dword this lane loaded for the pair
};

template <bool kS4>
__device__ __forceinline__ void pair_load(PairBatch& bt, const uint8_t* span, const Geo& g,
                                          int p, int lane) {
  const uint8_t* dp = span + g.w2p + (size_t)p * (2 * kG96RowBytes);
  const uint8_t* ds = span + g.w2s + (size_t)p * (kS4 ? kG96ScaleBytes : 2 * kG96ScaleBytes);
  bt.s = load_u32(ds + 4 * min(lane, kS4 ? 23 : 47));
  const uint32_t lo = (uint32_t)lane << 4;
  bt.a = load_chunk(dp + lo);
  bt.b = load_chunk(dp + kG96RowBytes + lo);
  bt.c = load_chunk(dp + 1024 + (lane >> 5) * kG96RowBytes + ((uint32_t)(lane & 31) << 4));
}

// E8M0 scale of byte / nibble index q of the pair (see k_down_g96).
template <bool kS4>
__device__ __forceinline__ float pair_scale(uint32_t s, int q, uint32_t base) {
  if constexpr (kS4) {
    const uint32_t word = (uint32_t)__builtin_amdgcn_ds_bpermute((q >> 3) << 2, (int)s);
    return e8m0_scale(base + ((word >> (4 * (q & 7))) & 0xfu));
  } else {
    const uint32_t word = (uint32_t)__builtin_amdgcn_ds_bpermute((q >> 2) << 2, (int)s);
    return e8m0_scale((word >> (8 * (q & 3))) & 0xffu);
  }
}

// Partial sums of rows 2 p and 2 p + 1 over the wave: v[0] in lanes 0-31 holds
// row 2 p, in lanes 32-63 row 2 p + 1.
template <bool kS4>
__device__ __forceinline__ float pair_dots(const PairBatch& bt, const XChunk<float>& hh,
                                           const XChunk<float>& ht, int lane, uint32_t base) {
  const float va = hh.dot(bt.a) * pair_scale<kS4>(bt.s, lane, base);
  const float vb = hh.dot(bt.b) * pair_scale<kS4>(bt.s, 96 + lane, base);
  const float vc = ht.dot(bt.c) * pair_scale<kS4>(bt.s, 64 + lane + ((lane >> 5) << 6), base);
  float v[2] = {va + (lane < 32 ? vc : 0.0f), vb + (lane < 32 ? 0.0f : vc)};
  wave_reduce_multi<2>(v, lane);
  return v[0];
}

template <typename OT, int NB, bool kS4, bool kPos = false>
__global__ __launch_bounds__(1024) void k_down_g96(const TokenRoute route_arg, const Geo g,
                                                   const float* __restrict__ h_arg,
                                                   OT* __restrict__ out_arg, const PosStride pos) {
  const TokenRoute& route = route_arg;  // read in place (see k_glu_decode)
  const int pidx = kPos ? (int)blockIdx.y : 0;
  const size_t proute = (size_t)pidx * route.n;
  const float* __restrict__ h = h_arg + pidx * pos.h;
  OT* __restrict__ out = out_arg + pidx * pos.out;
  __shared__ float ybuf[K3_HIP_MAX_TOKEN_EXPERTS][NB * 2];
  extern __shared__ float4 hbuf[];  // kHSliceF4 float4 per wave
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform: SGPR
  const int G = gridDim.x;
  const int npt = g.hidden >> 1;                       // pairs in the output (hidden even)
  const int nb = (npt - (int)blockIdx.x + G - 1) / G;  // 1 <= nb <= NB (host)
  // XCD-blocked pairs when the grid covers them exactly (as in k_down_g64).
  const bool xmap = (K3_XCD_MAP & 2) && (G & 7) == 0 && npt == G * NB;
  const int xb = xmap ? ((int)blockIdx.x & 7) * (G >> 3) * NB + ((int)blockIdx.x >> 3)
                      : (int)blockIdx.x;
  const int xs = xmap ? (G >> 3) : G;
  auto pair_of = [&](int i) { return min(i, nb - 1) * xs + xb; };
  const int e = wave;  // one routed expert per wave (route.n <= 16 waves)
  const float* he = h + (size_t)e * g.inter;
  // h_e's head (floats 0-2047: float4 64 q + lane) and tail (floats
  // 2048-3071: float4 512 + 64 q + lane), written ahead of the route as in
  // k_down_g64 (and issued, as there, behind the first pairs' loads).
  float4 th[8], tt[4];
  h_slice_issue(th, he, lane);
  {
    const float4* src = reinterpret_cast<const float4*>(he) + 512 + lane;
#pragma unroll
    for (int q = 0; q < 4; ++q) tt[q] = src[64 * q];
  }
  __builtin_amdgcn_sched_barrier(0);
  const RouteRegs rreg = route_regs(route, lane, proute);
  const uint32_t base = kS4 ? (__builtin_amdgcn_readlane(route_bases(rreg, route.n, lane), e) >> 8) & 0xffu
                            : 0u;
  {
    const uint8_t* span = span_of(rreg, e);
    PairBatch bt[2];
    pair_load<kS4>(bt[0], span, g, pair_of(0), lane);
    if constexpr (NB > 1) pair_load<kS4>(bt[1], span, g, pair_of(1), lane);
    __builtin_amdgcn_sched_barrier(0);
    float4* hw = hbuf + wave * kHSliceF4;
    XChunk<float> hh, ht;
    h_slice_transpose(hh, th, hw, lane);
    // The tail reuses the wave's LDS region: a wave's LDS operations run in
    // issue order, so the head's reads above are served before these writes;
    // the empty asm (a compiler memory barrier) keeps the compiler from moving
    // the writes above the reads.
    asm volatile("" ::: "memory");
    {
      float4* dst = hw + 9 * (lane >> 3) + (lane & 7);
#pragma unroll
      for (int q = 0; q < 4; ++q) dst[72 * q] = tt[q];
      const float4* mine = hw + 9 * (lane & 31);
#pragma unroll
      for (int q = 0; q < 8; ++q) {
        const float4 v = mine[q];
        ht.v[4 * q + 0] = v.x;
        ht.v[4 * q + 1] = v.y;
        ht.v[4 * q + 2] = v.z;
        ht.v[4 * q + 3] = v.w;
      }
    }
#pragma unroll
    for (int b = 0; b < NB; ++b) {
      const float v = pair_dots<kS4>(bt[b & 1], hh, ht, lane, base);
      if (b + 2 < NB) pair_load<kS4>(bt[b & 1], span, g, pair_of(b + 2), lane);
      if ((lane & 31) == 0 && b < nb) ybuf[e][2 * b + (lane >> 5)] = v;
    }
  }
  __syncthreads();
  for (int t = threadIdx.x; t < nb * 2; t += blockDim.x) {
    const int row = 2 * pair_of(t >> 1) + (t & 1);
    float acc = 0.0f;
    for (int e2 = 0; e2 < route.n; ++e2) acc += weight_of(rreg, e2) * ybuf[e2][t];
    store_out(out + row, acc);
  }
}

// ======================================================================
// fused decode: router, gate/up and down + combine in one launch
// ======================================================================
// The work of a token is cut into tickets: n_glu gate/up tickets (ticket v is
// the sweep share of one k_glu_decode workgroup: pipelines v * groups .. +
// groups - 1 of Q = n_glu * groups) followed by n_down down tickets (ticket
// d is the output-row share of k_down_g64 workgroup d of n_down).  A
// workgroup claims tickets from a counter one at a time, each claim issued
// while the previous ticket runs, and processes them in claim order.  A down
// ticket waits until every gate/up ticket has released its h stores.  That
// wait always ends: the counter hands out every gate/up ticket before the
// first down ticket, a workgroup holding a gate/up ticket is running and
// finishes it without waiting for anything, so no workgroup waits on work
// that is not already held by a running workgroup, however many workgroups
// are resident.  The wait is still bounded (kFusedSpinLimit polls); a
// workgroup that gives up writes NaN to its output rows.
//
// Cross-workgroup state lives in a slot of g_fused_sync, one slot per caller
// workspace (calls that share a workspace are ordered, so no two launches use
// a slot at once).  Slots are zero when the code object loads, and the last
// workgroup of every launch returns its slot to zero.
//
// Opt-in only: on MI355X at config 2 it takes 76-77 us per token against
// 64-65 us for k_glu_decode + k_down_g64 (the bench's other_decode_path on
// one box).  Per-workgroup phase stamps put the loss in
// three places: 1024-thread workgroups start over ~4 us (512-thread ones over
// 0.8 us) and so finish gate/up later; every down ticket waits for the last
// gate/up ticket plus a poll of the counter; then all workgroups read the
// whole h at device scope at once.
struct FusedSync {
  unsigned ticket;  // tickets claimed
  unsigned done;    // gate/up tickets whose h stores are released
  unsigned exited;  // workgroups finished
  unsigned pad[61];
};
constexpr int kFusedSlots = 64;
constexpr int kFusedSpinLimit = 1 << 20;
static __device__ __align__(256) FusedSync g_fused_sync[kFusedSlots] = {};

struct FusedPlan {
  int n_units;  // gate/up units (route.n * inter / kR)
  int S;        // column-split waves per gate/up pipeline
  int groups;   // gate/up pipelines per workgroup
  int n_glu;    // gate/up tickets
  int n_down;   // down tickets
  int slot;     // g_fused_sync slot
};

// Handing h between workgroups.  K3_FUSED_SYNC 1: h is stored and loaded at
// device scope (written through to, and read from, the level every XCD
// shares), and a store counts once the wave has seen it acknowledged; no
// cache-wide maintenance.  0: plain h accesses ordered by agent-scope
// release / acquire fences (an L2 write-back per storing wave, an L2
// invalidate per waiting workgroup).
#ifndef K3_FUSED_SYNC
#define K3_FUSED_SYNC 1
#endif
constexpr bool kFusedDeviceScope = K3_FUSED_SYNC == 1;

// Wait until every memory operation this wave issued has completed (stores
// and atomics acknowledged); the signal fences keep the compiler from moving
// memory operations across the wait.
__device__ __forceinline__ void wait_vm_complete() {
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0); expcnt and lgkmcnt unconstrained
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
}

// h_e's 8 KB for h_slice_transpose, loaded at device scope (sc1).
__device__ __forceinline__ void h_slice_issue_device(float4 (&t)[8], const float* he, int lane) {
  const Rsrc r = make_rsrc(reinterpret_cast<const uint8_t*>(he), 8192u);
#pragma unroll
  for (int q = 0; q < 8; ++q) {
    const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(r, (uint32_t)lane * 16u,
                                                          (uint32_t)q * 1024u, 16 /* sc1 */);
    t[q] = make_float4(__uint_as_float(v[0]), __uint_as_float(v[1]), __uint_as_float(v[2]),
                       __uint_as_float(v[3]));
  }
}

__device__ __forceinline__ unsigned agent_add(unsigned* p, unsigned v) {
  return __hip_atomic_fetch_add(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Lane 0 of the calling wave polls *c until it reaches target (at most
// kFusedSpinLimit polls); with fences, the wave then acquires at agent scope
// (its caches hold nothing older than the releases it observed).  Returns
// whether the count was reached.
__device__ __forceinline__ bool wait_count(unsigned* c, unsigned target, int lane) {
  int ok = 1;
  if (lane == 0) {
    int i = 0;
    while (__hip_atomic_load(c, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) < target) {
      if (++i == kFusedSpinLimit) {
        ok = 0;
        break;
      }
      __builtin_amdgcn_s_sleep(2);
    }
  }
  if constexpr (kFusedDeviceScope)
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
  else
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
  return __builtin_amdgcn_readfirstlane(ok) != 0;
}

template <typename XT, typename OT, int kR, int NB>
__global__ __launch_bounds__(1024) void k_decode_fused(const TokenRoute route, const Geo g,
                                                       const XT* __restrict__ x, float* h,
                                                       OT* __restrict__ out, const FusedPlan fp) {
  constexpr int kB = 4;
  // Dynamic LDS: the router's keys at the start, then the waves' h slices.
  extern __shared__ __attribute__((aligned(16))) float4 fused_lds[];
  __shared__ float red[2][16][2 * kR];
  __shared__ float ybuf[K3_HIP_MAX_TOKEN_EXPERTS][NB * kB];
  __shared__ int sel[K3_HIP_MAX_TOKEN_EXPERTS];
  __shared__ float wsel[K3_HIP_MAX_TOKEN_EXPERTS];
  __shared__ unsigned s_ticket[2];
  __shared__ int s_ok;
  FusedSync* sy = &g_fused_sync[fp.slot];
  const int S = fp.S;
  const int G = g.hidden >> 5;
  const int row_step = (G + S - 1) / S;
  const unsigned n_glu = (unsigned)fp.n_glu;
  const unsigned n_total = n_glu + (unsigned)fp.n_down;

  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  unsigned claim = 0;
  if (threadIdx.x == 0) claim = agent_add(&sy->ticket, 1u);
  const RouteRegs rr =
      workgroup_route(route, reinterpret_cast<uint64_t*>(fused_lds), sel, wsel, lane);
  if (threadIdx.x == 0) s_ticket[0] = claim;
  __syncthreads();
  unsigned t = s_ticket[0];
  int i = 1;
  // Tickets come in increasing order, so a workgroup's gate/up tickets all
  // precede its down tickets: two loops, each with only its own phase's
  // values live.
  if (t < n_glu) {
    const int grp = wave / S;
    const int gw = wave - grp * S;
    const int Q = fp.n_glu * fp.groups;
    const int iters = (fp.n_units + Q - 1) / Q;
    const ColSplit cs = col_split(G, S, gw, lane);
    const GluGather gg = glu_gather(G, S, gw, lane, kR);
    XChunk<XT> xc;
    load_x_chunk<XT>(xc, x, cs);
    for (; t < n_glu; ++i) {
      if (threadIdx.x == 0) claim = agent_add(&sy->ticket, 1u);
      if (grp < fp.groups) {
        glu_sweep<XT, kR, true, kFusedDeviceScope>(rr, g, xc, cs, gg, row_step, S, grp, gw,
                                                   wave, lane, (int)t * fp.groups + grp, Q,
                                                   iters, fp.n_units, h, red);
        // This wave's h stores are visible device-wide before the ticket
        // counts as done.
        if (gw == 0) {
          if constexpr (kFusedDeviceScope)
            wait_vm_complete();
          else
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
        }
      } else {
        for (int it = 0; it < iters; ++it) lds_barrier();  // the sweep's barriers
      }
      if (threadIdx.x == 0) s_ticket[i & 1] = claim;
      __syncthreads();
      if (threadIdx.x == 0) agent_add(&sy->done, 1u);
      t = s_ticket[i & 1];
    }
  }
  {
    // Down ticket d: output-row batches d, d + n_down, ... (nb <= NB of
    // them), one routed expert per wave.  The expert's first two weight
    // batches are requested before the wait for h.
    const int cc[1] = {lane};
    const int idx = lane >> 4;
    const bool writer = (lane & 15) == 0;
    const int e = wave;
    const bool active = e < route.n;
    const uint8_t* span = span_of(rr, active ? e : 0);
    const int nbt = (g.hidden + kB - 1) / kB;
    for (; t < n_total; ++i) {
      if (threadIdx.x == 0) claim = agent_add(&sy->ticket, 1u);
      const int d = (int)(t - n_glu);
      const int nb = (nbt - d + fp.n_down - 1) / fp.n_down;
      auto row_of = [&](int b) { return (min(b, nb - 1) * fp.n_down + d) * kB; };
      auto rows_in = [&](int b) { return min(kB, g.hidden - row_of(b)); };
      DownBatch<1, kB, true> bt[2];
      if (active) {
        down_load(bt[0], span, g, cc, row_of(0), rows_in(0));
        if constexpr (NB > 1) down_load(bt[1], span, g, cc, row_of(1), rows_in(1));
      }
      if (wave == 0) {
        const bool ok = wait_count(&sy->done, n_glu, lane);
        if (lane == 0) s_ok = ok ? 1 : 0;
      }
      __syncthreads();
      if (active) {
        float4 ht[8];
        if constexpr (kFusedDeviceScope)
          h_slice_issue_device(ht, h + (size_t)e * g.inter, lane);
        else
          h_slice_issue(ht, h + (size_t)e * g.inter, lane);
        XChunk<float> hs;
        h_slice_transpose(hs, ht, fused_lds + wave * kHSliceF4, lane);
#pragma unroll
        for (int b = 0; b < NB; ++b) {
          const float v = down_dots(bt[b & 1], &hs, lane);
          if (b + 2 < NB) down_load(bt[b & 1], span, g, cc, row_of(b + 2), rows_in(b + 2));
          if (writer && b < nb && idx < rows_in(b)) ybuf[e][b * kB + idx] = v;
        }
      }
      __syncthreads();
      const bool ok = s_ok != 0;
      for (int r = threadIdx.x; r < nb * kB; r += blockDim.x) {
        const int row = row_of(r / kB) + (r % kB);
        if (row >= g.hidden) continue;
        float acc = 0.0f;
        for (int k = 0; k < route.n; ++k) acc += weight_of(rr, k) * ybuf[k][r];
        store_out(out + row, ok ? acc : __builtin_nanf(""));
      }
      if (threadIdx.x == 0) s_ticket[i & 1] = claim;
      __syncthreads();
      t = s_ticket[i & 1];
    }
  }
  // Exit: every claim this workgroup made has returned (its value decided the
  // loop), and thread 0's done increments are acknowledged before its exit
  // increment (a workgroup that held no down ticket never waited for them).
  // The last workgroup out returns the slot to zero.
  if (threadIdx.x == 0) {
    unsigned old;
    if constexpr (kFusedDeviceScope) {
      wait_vm_complete();
      old = agent_add(&sy->exited, 1u);
    } else {
      old = __hip_atomic_fetch_add(&sy->exited, 1u, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT);
    }
    if (old == gridDim.x - 1) {
      __hip_atomic_store(&sy->ticket, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      __hip_atomic_store(&sy->done, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      __hip_atomic_store(&sy->exited, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
}

// ======================================================================
// one launch for a one-expert layer: k_expert_chain
// ======================================================================
// A layer with one routed expert (one token, caller route, intermediate 2048)
// is a 23 MB stream that two launches spend mostly on fixed costs: the
// gate/up kernel ends ~5 us after its start, the down kernel starts ~1.1 us
// later and its first row batch arrives ~2.5 us after that (h and weights
// from a cold launch), ~10.8 us per expert on MI355X.  Here one launch of one
// workgroup per CU runs the gate/up sweep of k_glu_decode's few-expert form
// (units of 2 rows, the same per-row arithmetic; the expert's span pointer
// read from the kernel argument at a uniform index, so no load precedes the
// first unit's), then each wave requests its down row batch (k_down_few's
// 4-row batch, one per wave: batch = workgroup + wave x grid; a batch past
// the end re-reads the last one and stores nothing), the workgroup gathers
// the expert's whole h into LDS (k_down_g64's padded layout) as soon as it is
// stored, and each wave forms its rows as k_down_few does.  The outputs are
// the two launches' bit for bit; ~9.3 us per expert.
//
// No counter: h goes through device memory as 64-bit entries {value, tag},
// each a single store written through to the device-coherent level, and a
// reader takes a pair of rows once both entries carry this call's tag (the
// first read through the XCD's L2, re-reads at device scope).  The tag comes
// from a per-workgroup call count (g_chain_calls, one word per workgroup and
// workspace slot, read at the start and advanced at the end): every launch on
// a slot runs one workgroup per CU, so all counts of a slot agree when a
// launch starts, and the tag (a signalling-NaN pattern, which no arithmetic
// result and so no earlier h value carries) differs from the previous
// launch's.  The state stays on the device, so a captured graph replays
// correctly.  (Counters measured slower: 256 increments of one word
// serialize over ~5 us.)
//
// The reads need every gate/up share done, which a workgroup that is not
// resident cannot do; with other work on the GPU (another stream's launch of
// this kernel, say) not every workgroup may be resident.  So after
// poll_limit rounds a waiting workgroup computes the missing shares itself
// (the owner's sweep: bit-identical values and tag, a share done twice is
// harmless), scanning from its own index and re-reading after each.  Every
// loop is bounded; rows still missing after 2 x grid shares become NaN.
struct ChainPlan {
  int S;           // column-split waves per gate/up pipeline
  int groups;      // gate/up pipelines per workgroup
  int n_units;     // 2-row gate/up units (route.n * inter / 2)
  int slot;        // workspace slot (g_chain_calls row)
  int poll_limit;  // read rounds before a workgroup computes missing shares
  int zero;        // 0 (a per-lane offset the compiler cannot fold)
};
#ifndef K3_EXPERT_CHAIN
#define K3_EXPERT_CHAIN 1
#endif
constexpr int kChainMaxGrid = 1024;
constexpr int kChainPollLimit = 256;
constexpr int kChainSlots = 64;
static __device__ __align__(256) unsigned g_chain_calls[kChainSlots][kChainMaxGrid] = {};

// Cache policy of a re-read of tagged h: sc0 and sc1, so that neither the
// CU's vector cache nor the XCD's L2 answers with the copy an earlier read of
// the same lines brought in.
constexpr int kReread = 17;

// Tag of the call whose count is c: a signalling NaN (exponent all ones,
// quiet bit clear, payload 1 .. 2^22 - 1).
__device__ __forceinline__ uint32_t chain_tag(unsigned c) {
  return 0x7F800000u | (1u + c % 0x3FFFFFu);
}

template <typename XT, typename OT, int NE, int kIters>
__global__ __launch_bounds__(kGluMaxThreads) __attribute__((amdgpu_waves_per_eu(1, kGluMaxThreads / 256)))
void k_expert_chain(const TokenRoute route_arg, const Geo g, const XT* __restrict__ x,
                    uint64_t* ht, OT* __restrict__ out, const ChainPlan cp) {
  const TokenRoute& route = route_arg;  // read in place (see k_glu_decode)
  constexpr int kR = 2;
  constexpr int kB = 4;
  constexpr int kMaxPairs = NE * 1024;  // intermediate 2048
  extern __shared__ __attribute__((aligned(16))) float4 hbuf[];  // NE x kHSliceF4
  __shared__ float red[2][16][2 * kR];
  __shared__ uint8_t s_have[kMaxPairs];
  __shared__ int s_miss[2];
  const int lane = threadIdx.x & 63;
  // The call count: loaded per lane (the offset is zero) so that it stays a
  // vector value, waited for only where the first h store needs the tag.
  unsigned* calls = &g_chain_calls[cp.slot][blockIdx.x];
  const unsigned count =
      __hip_atomic_load(calls + lane * cp.zero, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int S = cp.S;
  const int G = g.hidden >> 5;
  const int grp = wave / S;
  const int gw = wave - grp * S;
  const ColSplit cs = col_split(G, S, gw, lane);
  XChunk<XT> xc;
  load_x_chunk<XT>(xc, x, cs);
  // The caller's span pointers and weights, read at uniform indices (scalar
  // loads of the kernel argument), in a wave's route registers.
  RouteRegs rr;
  rr.lo = rr.hi = 0u;
  rr.w = 0.0f;
#pragma unroll
  for (int e = 0; e < NE; ++e) {
    const uint64_t sp = reinterpret_cast<uint64_t>(route.ptr[e]);
    if (lane == e) {
      rr.lo = (uint32_t)sp;
      rr.hi = (uint32_t)(sp >> 32);
      rr.w = route.w[e];
    }
  }
  const uint32_t tag = chain_tag(count);
  const int Q = (int)gridDim.x * cp.groups;
  const int row_step = (G + S - 1) / S;
  auto sweep_as = [&](int b) {  // gate/up share of workgroup b
    const int q0 = xcd_block_id(b, (int)gridDim.x) * cp.groups + grp;
    glu_sweep<XT, kR, false, true, kIters, true>(rr, g, xc, cs, GluGather{0, 0}, row_step, S,
                                                 grp, gw, wave, lane, q0, Q, kIters, cp.n_units,
                                                 reinterpret_cast<float*>(ht), red, tag);
  };
  sweep_as((int)blockIdx.x);
  // down: this wave's row batch of every expert, requested behind the h
  // stores (issued with the gate/up units, the down bytes measured 0.2 us
  // slower per call: they delay the last gate/up units, which everyone waits
  // for)
  const int nbt = (g.hidden + kB - 1) / kB;
  const int batch = (int)blockIdx.x + wave * (int)gridDim.x;
  const int r0 = min(batch, nbt - 1) * kB;
  const int rows = min(kB, g.hidden - r0);
  const int cc[1] = {lane};
  DownBatch<1, kB, true> bt[NE];
#pragma unroll
  for (int e = 0; e < NE; ++e) down_load(bt[e], span_of(rr, e), g, cc, r0, rows);
  __builtin_amdgcn_sched_barrier(0);
  // the tagged h of all NE experts as one buffer; pairs per thread (the host
  // launches at least 384 threads)
  const Rsrc hr = make_rsrc(reinterpret_cast<const uint8_t*>(ht), (uint32_t)(NE * g.inter) * 8u);
  constexpr int kPer = (kMaxPairs + 383) / 384;
  // h into LDS (k_down_g64's padded layout) pair by pair (pair p = rows 2p,
  // 2p + 1 = gate/up unit p, one 16-byte load), once both entries carry the
  // tag: the first round through the L2 (one fetch per XCD), re-reads of the
  // pairs still missing at device scope.  After poll_limit rounds with a pair
  // missing (not every workgroup resident), the workgroup computes the shares
  // it finds missing, scanning from its own index, re-reading after each.
  const int np = NE * (g.inter >> 1);
  const int T = (int)blockDim.x;
  for (int p = threadIdx.x; p < np; p += T) s_have[p] = 0;
  if (threadIdx.x == 0) s_miss[0] = s_miss[1] = 0;
  lds_barrier();
  bool ok = true;
  int polls = 0, shares = 0, next = (int)blockIdx.x + 1;
  for (int round = 0;; ++round) {
    u32x4 v[kPer];
#pragma unroll
    for (int k = 0; k < kPer; ++k) {
      const uint32_t off = (uint32_t)min((int)threadIdx.x + k * T, np - 1) * 16u;
      v[k] = polls == 0 && shares == 0 ? __builtin_amdgcn_raw_buffer_load_b128(hr, off, 0u, 0)
                                       : __builtin_amdgcn_raw_buffer_load_b128(hr, off, 0u, kReread);
    }
    int miss = 0;
#pragma unroll
    for (int k = 0; k < kPer; ++k) {
      const int p = (int)threadIdx.x + k * T;
      if (p >= np || s_have[p]) continue;
      if (v[k][1] == tag && v[k][3] == tag) {
        const int e = p / (g.inter >> 1), j = 2 * (p - e * (g.inter >> 1));  // row of expert e
        const int f = j >> 2;
        float* dst =
            reinterpret_cast<float*>(hbuf + e * kHSliceF4 + 9 * (f >> 3) + (f & 7)) + (j & 3);
        dst[0] = __uint_as_float(v[k][0]);
        dst[1] = __uint_as_float(v[k][2]);
        s_have[p] = 1;
      } else {
        miss = 1;
      }
    }
    // any pair missing in the workgroup? (slot round % 2; the other slot,
    // read by every thread last round, is cleared for the next)
    if (miss) s_miss[round & 1] = 1;
    lds_barrier();
    const bool any_miss = s_miss[round & 1] != 0;
    if (threadIdx.x == 0) s_miss[(round & 1) ^ 1] = 0;
    if (!any_miss) break;
    if (polls < cp.poll_limit) {
      ++polls;
      __builtin_amdgcn_s_sleep(2);
      continue;
    }
    if (shares >= 2 * (int)gridDim.x) {  // rows still missing become NaN
      ok = false;
      break;
    }
    // the next share (from this workgroup's own index on) with a missing unit
    int found = -1;
    for (int k = 0; k < (int)gridDim.x && found < 0; ++k) {
      const int b2 = (next + k) % (int)gridDim.x;
      const int qb = xcd_block_id(b2, (int)gridDim.x) * cp.groups;
      for (int gq = 0; gq < cp.groups; ++gq)
        for (int it = 0; it < kIters; ++it) {
          const int u = qb + gq + it * Q;
          if (u < cp.n_units && !s_have[u]) found = b2;
        }
    }
    if (found < 0) {
      ok = false;
      break;
    }
    next = found + 1;
    ++shares;
    sweep_as(found);
    wait_vm_complete();  // this wave's h stores are done before the re-read
    __syncthreads();
  }
  XChunk<float> hs[NE];
#pragma unroll
  for (int e = 0; e < NE; ++e) {
    const float4* mine = hbuf + e * kHSliceF4 + 9 * lane;
#pragma unroll
    for (int q = 0; q < 8; ++q) {
      const float4 t = mine[q];
      hs[e].v[4 * q + 0] = t.x;
      hs[e].v[4 * q + 1] = t.y;
      hs[e].v[4 * q + 2] = t.z;
      hs[e].v[4 * q + 3] = t.w;
    }
  }
  float acc = 0.0f;
#pragma unroll
  for (int e = 0; e < NE; ++e) {
    const float v = down_dots(bt[e], &hs[e], lane);
    acc += weight_of(rr, e) * v;
  }
  const int idx = lane >> 4;
  if ((lane & 15) == 0 && batch < nbt && idx < rows)
    store_out(out + r0 + idx, ok ? acc : __builtin_nanf(""));
  if (threadIdx.x == 0)
    __hip_atomic_store(calls, count + 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// ======================================================================
// elementwise activation (per-expert launch path)
// ======================================================================
__global__ void k_activate(const float* __restrict__ gate, const float* __restrict__ up,
                           float* __restrict__ hout, int64_t n, int act) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) hout[i] = activate(act, gate[i], up[i]);
}

// ======================================================================
// router: top-k (descending value, lower index on ties, NaN ranked as -inf,
// -0 equal to +0) + softmax over the selected logits; one workgroup per
// position.  Each logit becomes a 64-bit key (order-preserving value bits,
// then the complemented index), so "better" is plain unsigned ">".
//   stage 1: within each 64-logit segment, a logit's rank is the number of
//            larger keys in the segment; ranks < k are candidates (the global
//            top k is always inside the union of the segments' top k);
//   stage 2: each candidate's rank among all candidates is its global rank.
// ======================================================================
constexpr int kRouteMaxBank = 4096;

// Bytes of block_topk's key scratch (the host's route_scratch_bytes).
__device__ __forceinline__ size_t route_scratch_bytes_dev(int n_bank, int top_k) {
  const size_t nseg = (size_t)(n_bank + 63) / 64;
  return (nseg * 64 + ((nseg * (size_t)top_k + 1) & ~(size_t)1)) * sizeof(uint64_t);
}

// Inverse of route_key's value half (NaN comes back as -inf, -0 as +0).
__device__ __forceinline__ float key_value(uint64_t key) {
  uint32_t u = (uint32_t)(key >> 32);
  u = (u & 0x80000000u) ? (u & 0x7fffffffu) : ~u;
  return __uint_as_float(u);
}

__device__ __forceinline__ uint64_t route_key(float v, int i) {
  uint32_t u = __float_as_uint(v);
  if ((u & 0x7fffffffu) > 0x7f800000u) u = 0xff800000u;  // NaN -> -inf
  if (u == 0x80000000u) u = 0u;                           // -0 -> +0
  u = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
  return ((uint64_t)u << 32) | (uint64_t)(~(uint32_t)i);
}

// Block-level top-k + softmax.  keys: nseg*64 + round_up(nseg*top_k, 2) uint64
// of LDS scratch (16-byte aligned); sel/wsel receive the selected ids (rank
// order) and weights.  All threads of the workgroup call it; it ends with a
// barrier.  Comparisons read two keys per 128-bit LDS load.  have_pre: the
// caller already loaded logit threadIdx.x into pre (issued ahead of its other
// loads, so ranking starts as soon as the logits arrive).
__device__ void block_topk(const float* __restrict__ src, int n_bank, int top_k,
                           uint64_t* keys, int* sel, float* wsel, float pre, bool have_pre,
                           bool weights) {
  const int nseg = (n_bank + 63) >> 6;
  const int ncand = nseg * top_k;
  const int ncand2 = (ncand + 1) & ~1;
  uint64_t* cand = keys + (size_t)nseg * 64;
  const int T = blockDim.x;
  int i0 = threadIdx.x;
  if (have_pre) {
    // The preloaded key is stored on its own, so this store waits for that
    // load only (a store shared with the loop below would wait for every
    // load in flight, the caller's later ones included).
    if (i0 < nseg * 64) keys[i0] = i0 < n_bank ? route_key(pre, i0) : 0ull;
    i0 += T;
  }
  for (int i = i0; i < nseg * 64; i += T)
    keys[i] = i < n_bank ? route_key(src[i], i) : 0ull;  // 0 ranks below every real key
  for (int i = threadIdx.x; i < ncand2; i += T) cand[i] = 0ull;
  __syncthreads();
  // stage 1: rank within the 64-key segment
  for (int i = threadIdx.x; i < n_bank; i += T) {
    const uint64_t k = keys[i];
    const ulonglong2* seg = reinterpret_cast<const ulonglong2*>(keys + (i & ~63));
    int rank = 0;
#pragma unroll
    for (int j = 0; j < 32; ++j) {
      const ulonglong2 q = seg[j];
      rank += (q.x > k) + (q.y > k);
    }
    if (rank < top_k) cand[(i >> 6) * top_k + rank] = k;
  }
  __syncthreads();
  // stage 2: rank among the candidates is the global rank.  P adjacent
  // threads share a candidate (P = the largest power of two <= 8 with P
  // threads per candidate available), each counting over its 1/P of the
  // candidate list; the partial counts meet by lane exchange inside the group.
  {
    int lgP = 0;
    while (lgP < 3 && (2 << lgP) * ncand <= T) ++lgP;
    const int P = 1 << lgP;
    const int span2 = ((ncand2 >> 1) + P - 1) >> lgP;  // ulonglong2 per part
    const ulonglong2* c2 = reinterpret_cast<const ulonglong2*>(cand);
    for (int t0 = 0; t0 < ncand * P; t0 += T) {
      const int t = t0 + (int)threadIdx.x;
      const int c = t >> lgP, part = t & (P - 1);
      const bool live = c < ncand;
      const uint64_t k = live ? cand[c] : 0ull;
      const int j0 = part * span2, j1 = min(ncand2 / 2, j0 + span2);
      int rank = 0;
      if (live) {
#pragma unroll 4
        for (int j = j0; j < j1; ++j) {
          const ulonglong2 q = c2[j];
          rank += (q.x > k) + (q.y > k);
        }
      }
      // Every lane of the wave takes part in the exchanges (groups of P
      // lanes are aligned, so a group is wholly live or wholly not).
      for (int m = 1; m < P; m *= 2) rank += __shfl_xor(rank, m);
      if (live && part == 0 && k != 0ull && rank < top_k) sel[rank] = (int)(~(uint32_t)k);
    }
  }
  __syncthreads();
  if (weights) block_softmax(keys, sel, top_k, wsel);
}

// Softmax weights of the selected experts (keys and sel as block_topk leaves
// them): one wave, fixed summation order; the logit is recovered from its key
// (no second global load).  All threads call it.
__device__ void block_softmax(const uint64_t* keys, const int* sel, int top_k, float* wsel) {
  if (threadIdx.x < 64) {
    const int j = threadIdx.x;
    float ex = 0.0f;
    if (j < top_k) {
      const float top = key_value(keys[sel[0]]);
      const float lj = key_value(keys[sel[j]]);
      ex = expf(lj - top);
    }
    const float sum = wave_sum(ex);
    if (j < top_k) wsel[j] = ex / sum;
  }
  __syncthreads();
}

__global__ __launch_bounds__(1024) void k_route(const float* __restrict__ logits, int n_bank,
                                                int top_k, int32_t* __restrict__ ids_ws,
                                                float* __restrict__ w_ws,
                                                int32_t* __restrict__ ids_user,
                                                float* __restrict__ w_user) {
  extern __shared__ __attribute__((aligned(16))) uint64_t rsm[];
  __shared__ int sel[K3_HIP_MAX_TOKEN_EXPERTS];
  __shared__ float wsel[K3_HIP_MAX_TOKEN_EXPERTS];
  const int p = blockIdx.x;
  block_topk(logits + (size_t)p * n_bank, n_bank, top_k, rsm, sel, wsel);
  for (int j = threadIdx.x; j < top_k; j += blockDim.x) {
    const int o = p * top_k + j;
    ids_ws[o] = sel[j];
    w_ws[o] = wsel[j];
    if (ids_user) ids_user[o] = sel[j];
    if (w_user) w_user[o] = wsel[j];
  }
}

// K3 router (prepare_moe_t1, native/provider_gate/provider_moe.cpp:1673-1683):
// scores = sigmoid(logits), choice = scores + correction bias; the top_k
// largest choices (descending, lower index on ties, as block_topk ranks) are
// the route, each weighted by its unbiased score over the selected scores' sum
// + 1e-20 (one wave, fixed order).  choice sits in LDS after the rank keys.
__device__ __forceinline__ float sigmoid_f32(float v) { return 1.0f / (1.0f + expf(-v)); }

__global__ __launch_bounds__(1024) void k_route_sigmoid_bias(
    const float* __restrict__ logits, const float* __restrict__ bias, int n_bank, int top_k,
    int32_t* __restrict__ ids_ws, float* __restrict__ w_ws, int32_t* __restrict__ ids_user,
    float* __restrict__ w_user) {
  extern __shared__ __attribute__((aligned(16))) uint64_t rsm[];
  __shared__ int sel[K3_HIP_MAX_TOKEN_EXPERTS];
  __shared__ float wsel[K3_HIP_MAX_TOKEN_EXPERTS];
  const int p = blockIdx.x;
  const float* lg = logits + (size_t)p * n_bank;
  float* choice = reinterpret_cast<float*>(
      reinterpret_cast<uint8_t*>(rsm) + route_scratch_bytes_dev(n_bank, top_k));
  for (int i = threadIdx.x; i < n_bank; i += blockDim.x) choice[i] = sigmoid_f32(lg[i]) + bias[i];
  __syncthreads();
  block_topk(choice, n_bank, top_k, rsm, sel, wsel);  // its softmax weights are not used
  if (threadIdx.x < 64) {
    const int j = threadIdx.x;
    const float sc = j < top_k ? sigmoid_f32(lg[sel[j]]) : 0.0f;
    const float sum = wave_sum(sc);
    if (j < top_k) {
      const int o = p * top_k + j;
      const float wj = sc / (sum + 1e-20f);
      ids_ws[o] = sel[j];
      w_ws[o] = wj;
      if (ids_user) ids_user[o] = sel[j];
      if (w_user) w_user[o] = wj;
    }
  }
}

// ======================================================================
// verify plan: group edges by expert span (one workgroup, <= 256 edges)
// ======================================================================
// Edge e (thread e) ranks itself by (span pointer, edge index): the sorted
// list groups every expert's edges together, in edge order within a group.
// Group heads are counted with a ballot prefix scan, which numbers the unique
// experts in pointer order.  All loops are over the 256 edges in LDS.
// ranked (workgroup-uniform): rank_in is edge e's rank, computed by the caller.
__device__ void plan_core(const uint8_t* key, int e, int n_edges, int n_positions,
                          const Workspace& ws, bool ranked = false, int rank_in = 0) {
  __shared__ uint64_t kp[K3_HIP_MAX_EDGES];
  __shared__ uint64_t kpe[K3_HIP_MAX_EDGES];  // key * 256 + edge
  __shared__ int srt[K3_HIP_MAX_EDGES];
  __shared__ int wave_heads[K3_HIP_MAX_EDGES / 64];
  __shared__ int wide_keys;
  const uint64_t k = reinterpret_cast<uint64_t>(key);
  if (e == 0) wide_keys = 0;
  __syncthreads();
  if (e < n_edges) {
    kp[e] = k;
    kpe[e] = (k << 8) | (uint64_t)e;
    if ((k >> 56) != 0) wide_keys = 1;
  }
  __syncthreads();
  // Keys below 2^56 (every device address) rank by one 64-bit comparison
  // per pair: key * 256 + edge orders as (key, edge).
  const bool wide = wide_keys != 0;  // uniform
  if (e < n_edges) {
    int rank = rank_in;
    if (!ranked && !wide) {
      rank = 0;
      const uint64_t ke = kpe[e];
#pragma unroll 8
      for (int j = 0; j < n_edges; ++j) rank += kpe[j] < ke;
    } else if (!ranked) {
      rank = 0;
      for (int j = 0; j < n_edges; ++j) {
        const uint64_t kj = kp[j];
        rank += (kj < k) || (kj == k && j < e);
      }
    }
    srt[rank] = e;
  }
  __syncthreads();
  // Sorted position i = thread e: head of a group when its key differs from
  // the previous sorted key.
  const int i = e;
  const bool head = i < n_edges && (i == 0 || kp[srt[i]] != kp[srt[i - 1]]);
  const uint64_t mask = __ballot(head);
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int below = __popcll(mask & ((1ull << lane) - 1ull));
  if (lane == 0) wave_heads[wave] = __popcll(mask);
  __syncthreads();
  int before = 0, total = 0;
  for (int w = 0; w < (int)(blockDim.x >> 6); ++w) {
    before += w < wave ? wave_heads[w] : 0;
    total += wave_heads[w];
  }
  if (i < n_edges) {
    const int edge = srt[i];
    ws.uedges[i] = edge;
    if (head) {
      const int u = before + below;
      ws.uoff[u] = i;
      ws.uptr[u] = reinterpret_cast<const uint8_t*>(kp[edge]);
    }
  }
  if (e == 0) {
    ws.uoff[total] = n_edges;
    ws.plan->n_unique = total;
    ws.plan->n_edges = n_edges;
    ws.plan->n_positions = n_positions;
  }
}

// Exclusive prefix sums of c[0 .. n) in place, n <= 16 * 256, by the 256
// threads of the workgroup (each owns a run of consecutive entries); ends
// with a barrier.
__device__ void scan_bins_256(uint32_t* c, int n) {
  __shared__ uint32_t wtot[4];
  const int t = threadIdx.x, lane = t & 63;
  const int per = (n + 255) >> 8;
  const int b0 = t * per;
  uint32_t s = 0;
  for (int i = 0; i < per; ++i)
    if (b0 + i < n) s += c[b0 + i];
  uint32_t inc = s;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const uint32_t v = __shfl_up(inc, o);
    if (lane >= o) inc += v;
  }
  if (lane == 63) wtot[t >> 6] = inc;
  __syncthreads();
  uint32_t run = inc - s;
  for (int w = 0; w < (t >> 6); ++w) run += wtot[w];
  for (int i = 0; i < per; ++i)
    if (b0 + i < n) {
      const uint32_t v = c[b0 + i];
      c[b0 + i] = run;
      run += v;
    }
  __syncthreads();
}

// The activation's term split (k3_terms.h) that a matrix-core verify call
// needs next, run by workgroups 1 .. of the plan launch beside the plan in
// workgroup 0 (T = 0: none).
template <int T, typename SrcT>
__device__ __forceinline__ bool plan_split_block(const SrcT* xs, int n_rows, int K,
                                                 const Workspace& ws) {
  if constexpr (T > 0) {
    if (blockIdx.x > 0) {
      split_terms_at<T, SrcT>(xs, n_rows, K, ws.xq, ws.xqs,
                              (int)((blockIdx.x - 1) * blockDim.x + threadIdx.x));
      return true;
    }
  }
  return false;
}

constexpr int kPlanMaxBank = 4096;  // experts the counting rank bins

// Bank routes: an edge's key is its expert's span, bank + id * stride, so key
// order is id order and the rank of edge e (position p) is the number of
// edges with a smaller id plus the edges of earlier positions with the same
// id.  A position's ids are distinct (the router ranks distinct experts), so
// a per-expert mask of positions gives the second term; with an id outside
// the bank or a repeated id within a position (the masks' popcounts then
// differ from the edge counts), the comparison rank over every pair of keys
// takes over.  Both give the same order.
template <int T, typename SrcT>
__global__ __launch_bounds__(256) void k_verify_plan_bank(const uint8_t* bank, uint64_t stride,
                                                          int n_bank, int n_positions, int top_k,
                                                          const Workspace ws, const SrcT* xs,
                                                          int K) {
  if (plan_split_block<T, SrcT>(xs, n_positions, K, ws)) return;
  __shared__ uint32_t pmask[kPlanMaxBank];  // bit p: position p routes to the expert
  __shared__ uint32_t pcnt[kPlanMaxBank];   // edges routed to the expert, then their prefix
  __shared__ int fallback;
  const int e = threadIdx.x;
  const int n_edges = n_positions * top_k;
  const uint8_t* key = nullptr;
  int id = -1, p = 0;
  if (e < n_edges) {
    id = ws.ids[e];
    p = e / top_k;
    key = bank + (uint64_t)id * stride;
    ws.epos[e] = p;
  }
  if (e <= n_positions) ws.poff[e] = e * top_k;
  const bool bins = n_bank >= 1 && n_bank <= kPlanMaxBank && stride > 0;  // uniform
  if (bins)
    for (int i = e; i < n_bank; i += blockDim.x) {
      pmask[i] = 0u;
      pcnt[i] = 0u;
    }
  if (e == 0) fallback = bins ? 0 : 1;
  __syncthreads();
  const bool in = bins && e < n_edges && id >= 0 && id < n_bank;
  if (bins && e < n_edges && !in) fallback = 1;
  if (in) {
    atomicOr(&pmask[id], 1u << p);
    atomicAdd(&pcnt[id], 1u);
  }
  __syncthreads();
  if (in && (uint32_t)__popc(pmask[id]) != pcnt[id]) fallback = 1;
  __syncthreads();
  const bool ranked = fallback == 0;  // uniform
  int rank = 0;
  if (ranked) {
    scan_bins_256(pcnt, n_bank);
    if (in) rank = (int)pcnt[id] + __popc(pmask[id] & ((1u << p) - 1u));
  }
  plan_core(key, e, n_edges, n_positions, ws, ranked, rank);
}

template <int T, typename SrcT>
__global__ __launch_bounds__(256) void k_verify_plan_table(const EdgeTable tbl,
                                                           const Workspace ws, const SrcT* xs,
                                                           int K) {
  if (plan_split_block<T, SrcT>(xs, tbl.n_positions, K, ws)) return;
  const int e = threadIdx.x;
  const uint8_t* key = nullptr;
  if (e < tbl.n_edges) {
    key = tbl.ptr[e];
    ws.w[e] = tbl.w[e];
    int p = 0;
    while (p + 1 < tbl.n_positions && tbl.pos_off[p + 1] <= e) ++p;
    ws.epos[e] = p;
  }
  if (e <= tbl.n_positions) ws.poff[e] = tbl.pos_off[e];
  plan_core(key, e, tbl.n_edges, tbl.n_positions, ws);
}

// A caller route table's edges e0 .. e0 + n - 1 as a table-mode route in
// device memory (span pointers and weights, edge order).
__global__ __launch_bounds__(256) void k_route_table(const EdgeTable tbl, int e0, int n,
                                                      const uint8_t** __restrict__ ptr_out,
                                                      float* __restrict__ w_out) {
  for (int i = threadIdx.x; i < n; i += blockDim.x) {
    ptr_out[i] = tbl.ptr[e0 + i];
    w_out[i] = tbl.w[e0 + i];
  }
}

// ======================================================================
// verify phase A on the VALU (the union path where the matrix-core one does
// not apply):
// one workgroup per (unique expert, 32-row block); the expert's positions are
// staged in LDS a group at a time
// ======================================================================
template <typename XT>
struct VerifyA {
  static constexpr int kGroup = sizeof(XT) == 2 ? 4 : 2;
};

template <typename XT, int kRows>
__global__ __launch_bounds__(256) void k_glu_verify_rows(const Geo g, const XT* __restrict__ x,
                                                    const Workspace ws) {
  extern __shared__ uint4 smem_va[];
  XT* xs = reinterpret_cast<XT*>(smem_va);
  constexpr int kG = VerifyA<XT>::kGroup;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform: SGPR
  const int upe = g.inter / (4 * kRows);
  const int u = blockIdx.x / upe;
  if (u >= ws.plan->n_unique) return;
  const int r0 = (blockIdx.x - u * upe) * (4 * kRows) + wave * kRows;
  const int eb = ws.uoff[u], m = ws.uoff[u + 1] - eb;
  const uint8_t* span = ws.uptr[u];
  const int G = g.hidden >> 5;
  const size_t cp = (size_t)g.hidden >> 1;
  for (int t0 = 0; t0 < m; t0 += kG) {
    const int nb = min(kG, m - t0);
    __syncthreads();
    const int per16 = (int)((size_t)g.hidden * sizeof(XT) / 16);
    for (int i = threadIdx.x; i < nb * per16; i += blockDim.x) {
      const int t = i / per16;
      const int pos = ws.epos[ws.uedges[eb + t0 + t]];
      smem_va[i] = reinterpret_cast<const uint4*>(x + (size_t)pos * g.hidden)[i - t * per16];
    }
    __syncthreads();
    for (int r = 0; r < kRows; ++r) {
      const int row = r0 + r;
      float ag[kG], au[kG];
#pragma unroll
      for (int t = 0; t < kG; ++t) ag[t] = au[t] = 0.0f;
      const uint8_t* gp = span + g.w1p + (size_t)row * cp;
      const uint8_t* up = span + g.w3p + (size_t)row * cp;
      const uint8_t* gs = span + g.w1s + (size_t)row * G;
      const uint8_t* us = span + g.w3s + (size_t)row * G;
      for (int chunk = lane; chunk < G; chunk += 64) {
        WDec<XT> dg, du;
        dg.decode(load_chunk(gp + (size_t)chunk * 16));
        du.decode(load_chunk(up + (size_t)chunk * 16));
        const float sg = e8m0_scale(gs[chunk]);
        const float su = e8m0_scale(us[chunk]);
#pragma unroll
        for (int t = 0; t < kG; ++t) {
          if (t < nb) {
            XChunk<XT> xv;
            xv.load(xs + (size_t)t * g.hidden, chunk);
            ag[t] = fmaf(dg.dot(xv), sg, ag[t]);
            au[t] = fmaf(du.dot(xv), su, au[t]);
          }
        }
      }
#pragma unroll
      for (int t = 0; t < kG; ++t) {
        if (t < nb) {
          const float gv = wave_sum(ag[t]);
          const float uv = wave_sum(au[t]);
          if (lane == 0) {
            const int edge = ws.uedges[eb + t0 + t];
            ws.h[(size_t)edge * g.inter + row] = activate(g.act, gv, uv);
          }
        }
      }
    }
  }
}

// ======================================================================
// verify phase B: one workgroup per (unique expert, row block); each wave
// holds the h slices of up to kE edges and streams its rows once per group
// ======================================================================
template <int CPLB, int kRows>
__global__ __launch_bounds__(256) void k_down_verify(const Geo g, const Workspace ws) {
  constexpr int kE = (4 / CPLB) > 0 ? (4 / CPLB) : 1;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform: SGPR
  const int upe = (g.hidden + 4 * kRows - 1) / (4 * kRows);
  const int u = blockIdx.x / upe;
  if (u >= ws.plan->n_unique) return;
  const int r0 = (blockIdx.x - u * upe) * (4 * kRows) + wave * kRows;
  if (r0 >= g.hidden) return;
  const int nrows = min(kRows, g.hidden - r0);
  const int eb = ws.uoff[u], m = ws.uoff[u + 1] - eb;
  const uint8_t* span = ws.uptr[u];
  const int GB = g.inter >> 5;
  const size_t cpb = (size_t)g.inter >> 1;
  for (int t0 = 0; t0 < m; t0 += kE) {
    const int nb = min(kE, m - t0);
    XChunk<float> hs[kE][CPLB];
    int edge[kE];
#pragma unroll
    for (int t = 0; t < kE; ++t) {
      edge[t] = t < nb ? ws.uedges[eb + t0 + t] : 0;
      if (t < nb) {
#pragma unroll
        for (int c = 0; c < CPLB; ++c) {
          const int chunk = lane + 64 * c;
          if (chunk < GB) hs[t][c].load(ws.h + (size_t)edge[t] * g.inter, chunk);
        }
      }
    }
    for (int r = 0; r < nrows; ++r) {
      const int row = r0 + r;
      float acc[kE];
#pragma unroll
      for (int t = 0; t < kE; ++t) acc[t] = 0.0f;
#pragma unroll
      for (int c = 0; c < CPLB; ++c) {
        const int chunk = lane + 64 * c;
        if (chunk < GB) {
          WDec<float> wd;
          wd.decode(load_chunk(span + g.w2p + (size_t)row * cpb + (size_t)chunk * 16));
          const float s = e8m0_scale(span[g.w2s + (size_t)row * GB + chunk]);
#pragma unroll
          for (int t = 0; t < kE; ++t)
            if (t < nb) acc[t] = fmaf(wd.dot(hs[t][c]), s, acc[t]);
        }
      }
#pragma unroll
      for (int t = 0; t < kE; ++t) {
        if (t < nb) {
          const float v = wave_sum(acc[t]);
          if (lane == 0) ws.y[(size_t)edge[t] * g.hidden + row] = v;
        }
      }
    }
  }
}

// Per-position ordered weighted combine of the edge outputs.
template <typename OT>
__global__ void k_combine_positions(const Workspace ws, int hidden, int n_positions,
                                    OT* __restrict__ out) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= (int64_t)hidden * n_positions) return;
  const int p = (int)(i / hidden);
  const int col = (int)(i - (int64_t)p * hidden);
  float acc = 0.0f;
  // Unrolled so that the edges' loads are in flight together; the sum still
  // runs in edge order.
#pragma unroll 8
  for (int e = ws.poff[p]; e < ws.poff[p + 1]; ++e)
    acc += ws.w[e] * ws.y[(size_t)e * hidden + col];
  store_out(out + i, acc);
}

// Zero n 32-bit words (rows of positions with no routed expert).  A kernel
// rather than hipMemsetAsync, so a caller capturing the call into a HIP graph
// records a kernel node.
__global__ void k_zero_words(uint32_t* __restrict__ p, uint64_t n) {
  for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
       i += (uint64_t)gridDim.x * blockDim.x)
    p[i] = 0u;
}

// ======================================================================
// synthetic inputs
// ======================================================================
__device__ __forceinline__ uint64_t mix64(uint64_t z) {
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}
__device__ __forceinline__ uint64_t rand_key(uint64_t seed, uint64_t stream) {
  return mix64(seed ^ mix64(stream ^ 0xD1B54A32D192ED03ull));
}
__device__ __forceinline__ uint64_t rand_at(uint64_t key, uint64_t i) {
  return mix64(key + (i + 1) * 0x9E3779B97F4A7C15ull);
}

__global__ void k_synth_bank(const Geo g, uint8_t* __restrict__ bank, uint64_t stride,
                             uint64_t first_expert, uint64_t seed, int lo, int hi) {
  const uint64_t e = blockIdx.y;
  const uint64_t words = g.span / 8;
  const uint64_t span_lo = (uint64_t)(hi - lo + 1);
  uint64_t* dst = reinterpret_cast<uint64_t*>(bank + e * stride);
  const uint64_t ex = first_expert + e;
  for (uint64_t wi = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; wi < words;
       wi += (uint64_t)gridDim.x * blockDim.x) {
    const uint64_t b = wi * 8;
    uint64_t base, mstream;
    bool is_scale;
    if (b < g.w1s) { base = g.w1p; mstream = 3 * ex + 0; is_scale = false; }
    else if (b < g.w2p) { base = g.w1s; mstream = 3 * ex + 0; is_scale = true; }
    else if (b < g.w2s) { base = g.w2p; mstream = 3 * ex + 1; is_scale = false; }
    else if (b < g.w3p) { base = g.w2s; mstream = 3 * ex + 1; is_scale = true; }
    else if (b < g.w3s) { base = g.w3p; mstream = 3 * ex + 2; is_scale = false; }
    else { base = g.w3s; mstream = 3 * ex + 2; is_scale = true; }
    const uint64_t rel = b - base;
    uint64_t v;
    if (!is_scale) {
      v = rand_at(rand_key(seed, 2 * mstream), rel >> 3);
    } else {
      const uint64_t key = rand_key(seed, 2 * mstream + 1);
      v = 0;
      for (int k = 0; k < 8; ++k) {
        const uint64_t s = (uint64_t)lo + rand_at(key, rel + k) % span_lo;
        v |= (s & 0xffull) << (8 * k);
      }
    }
    dst[wi] = v;
  }
}

__global__ void k_synth_normal(void* out, int dtype, uint64_t n, uint64_t seed, uint64_t stream) {
  const uint64_t key = rand_key(seed, stream);
  for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
       i += (uint64_t)gridDim.x * blockDim.x) {
    const double u1 = ((double)(rand_at(key, 2 * i) >> 11) + 1.0) * 0x1.0p-53;
    const double u2 = (double)(rand_at(key, 2 * i + 1) >> 11) * 0x1.0p-53;
    const float z = (float)(sqrt(-2.0 * log(u1)) * cos(6.283185307179586 * u2));
    if (dtype == K3_DTYPE_BF16)
      reinterpret_cast<uint16_t*>(out)[i] = f32_to_bf16_bits(z);
    else
      reinterpret_cast<float*>(out)[i] = z;
  }
}

// ======================================================================
// host launchers
// ======================================================================
namespace {

constexpr int kRowsGemv = 8;
// Rows per unit of the single-activation GEMV (k_gemv_cs).
#ifndef K3_GEMV_CS_ROWS
#define K3_GEMV_CS_ROWS 4
#endif
constexpr int kRowsGemvCs = K3_GEMV_CS_ROWS;
// Rows per unit of the decode gate/up kernel (gate and up each).
constexpr int kRowsGlu = K3_GLU_ROWS;
// Rows per load batch of the decode down kernel.
#ifndef K3_DOWN_BLOCKS_BATCH
#define K3_DOWN_BLOCKS_BATCH 4
#endif
constexpr int kDownBlocksBatch = K3_DOWN_BLOCKS_BATCH;
constexpr int kRowsVerifyA = 8;
constexpr int kRowsVerifyB = 16;

bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }


template <typename XT, typename OT>
int gemv1_dispatch(const uint8_t* p, const uint8_t* s, const XT* x, OT* y, int rows, int cols,
                   hipStream_t st) {
  const int G = cols / 32;
  const int S = (G + 63) / 64;
  if (S > 4) return -1;  // caller falls back to the LDS kernel
  const int groups = 4 / S;
  const int n_units = (rows + kRowsGemvCs - 1) / kRowsGemvCs;
  const int cus = std::max(1, device_cu_count());
  const int grid = std::max(1, std::min((n_units + groups - 1) / groups, 8 * cus));
  TimedLaunch tl(KC_GEMV, st);
  launch_timed(tl, (k_gemv_cs<XT, OT, kRowsGemvCs>), dim3(grid), dim3(256), 0, st, p, s, x, y,
               rows, cols, S);
  return launched(tl, "mxfp4 GEMV launch");
}

template <typename XT, typename OT>
int gemv_multi_dispatch(const uint8_t* p, const uint8_t* s, const XT* x, OT* y, int rows,
                        int cols, int batches, hipStream_t st) {
  const size_t per = (size_t)cols * sizeof(XT);
  const size_t budget = 64 * 1024;
  int group = (int)std::min<size_t>(budget / per, (size_t)kMultiMax);
  if (group < 1) return fail(K3_HIP_E_INVALID, "mxfp4 GEMV: cols=%d too wide for LDS staging", cols);
  group = std::min(group, batches);
  const int waves = (rows + kRowsGemv - 1) / kRowsGemv;
  TimedLaunch tl(KC_GEMV, st);
  launch_timed(tl, (k_gemv_multi<XT, OT, kRowsGemv>), dim3((waves + 3) / 4), dim3(256),
                     (unsigned)(group * per), st, p, s, x, y, rows, cols, batches, group);
  return launched(tl, "mxfp4 GEMV (multi) launch");
}

template <typename XT, typename OT>
int gemv_typed(const uint8_t* p, const uint8_t* s, const void* x, void* y, int rows, int cols,
               int batches, hipStream_t st) {
  const XT* xt = static_cast<const XT*>(x);
  OT* yt = static_cast<OT*>(y);
  if (batches == 1) {
    const int rc = gemv1_dispatch<XT, OT>(p, s, xt, yt, rows, cols, st);
    if (rc != -1) return rc;
  }
  return gemv_multi_dispatch<XT, OT>(p, s, xt, yt, rows, cols, batches, st);
}

}  // namespace

int launch_gemv(const uint8_t* packed, const uint8_t* scales, const void* x, int x_dtype,
                void* out, int out_dtype, int rows, int cols, int batches, hipStream_t st) {
  if (!packed || !scales || !x || !out)
    return fail(K3_HIP_E_INVALID, "mxfp4 GEMV: null input or output pointer");
  if (rows <= 0 || cols <= 0 || batches <= 0 || cols % 32 != 0)
    return fail(K3_HIP_E_INVALID,
                "mxfp4 GEMV: rows/batches must be positive and cols a positive multiple of 32");
  if (!aligned16(packed) || !aligned16(x))
    return fail(K3_HIP_E_INVALID, "mxfp4 GEMV: packed and x must be 16-byte aligned");
  if ((x_dtype != K3_DTYPE_F32 && x_dtype != K3_DTYPE_BF16) ||
      (out_dtype != K3_DTYPE_F32 && out_dtype != K3_DTYPE_BF16))
    return fail(K3_HIP_E_INVALID, "mxfp4 GEMV: unknown dtype");
  if ((int64_t)rows * batches > INT32_MAX)
    return fail(K3_HIP_E_INVALID, "mxfp4 GEMV: output too large");
  if (x_dtype == K3_DTYPE_F32) {
    return out_dtype == K3_DTYPE_F32
               ? gemv_typed<float, float>(packed, scales, x, out, rows, cols, batches, st)
               : gemv_typed<float, uint16_t>(packed, scales, x, out, rows, cols, batches, st);
  }
  return out_dtype == K3_DTYPE_F32
             ? gemv_typed<uint16_t, float>(packed, scales, x, out, rows, cols, batches, st)
             : gemv_typed<uint16_t, uint16_t>(packed, scales, x, out, rows, cols, batches, st);
}

int launch_activation(const float* gate, const float* up, float* h, int64_t n, int act,
                      hipStream_t st) {
  const int64_t blocks = (n + 255) / 256;
  if (blocks > INT32_MAX) return fail(K3_HIP_E_INVALID, "activation grid too large");
  TimedLaunch tl(KC_ACTIVATE, st);
  launch_timed(tl, k_activate, dim3((unsigned)blocks), dim3(256), 0, st, gate, up, h, n, act);
  return launched(tl, "activation launch");
}

int launch_route(const float* logits, int n_bank, int top_k, int n_positions, int32_t* ids_ws,
                 float* w_ws, int32_t* ids_user, float* w_user, hipStream_t st) {
  if (!logits) return fail(K3_HIP_E_INVALID, "router: null logits");
  if (n_bank <= 0 || n_bank > kRouteMaxBank)
    return fail(K3_HIP_E_INVALID, "router: n_bank must be in [1, %d]", kRouteMaxBank);
  if (top_k <= 0 || top_k > K3_HIP_MAX_TOKEN_EXPERTS || top_k > n_bank)
    return fail(K3_HIP_E_INVALID, "router: top_k must be in [1, min(%d, n_bank)]",
                K3_HIP_MAX_TOKEN_EXPERTS);
  if (n_positions <= 0) return fail(K3_HIP_E_INVALID, "router: no positions");
  const int nseg = (n_bank + 63) / 64;
  const int threads = std::min(1024, nseg * 64);
  const size_t lds = route_scratch_bytes(n_bank, top_k);
  TimedLaunch tl(KC_ROUTE, st);
  launch_timed(tl, k_route, dim3(n_positions), dim3(threads), (unsigned)lds, st, logits, n_bank,
                     top_k, ids_ws, w_ws, ids_user, w_user);
  return launched(tl, "router launch");
}

int launch_route_sigmoid_bias(const float* logits, const float* bias, int n_bank, int top_k,
                              int n_positions, int32_t* ids_ws, float* w_ws, int32_t* ids_user,
                              float* w_user, hipStream_t st) {
  if (!logits || !bias) return fail(K3_HIP_E_INVALID, "K3 router: null logits or bias");
  if (n_bank <= 0 || n_bank > kRouteMaxBank)
    return fail(K3_HIP_E_INVALID, "K3 router: n_bank must be in [1, %d]", kRouteMaxBank);
  if (top_k <= 0 || top_k > K3_HIP_MAX_TOKEN_EXPERTS || top_k > n_bank)
    return fail(K3_HIP_E_INVALID, "K3 router: top_k must be in [1, min(%d, n_bank)]",
                K3_HIP_MAX_TOKEN_EXPERTS);
  if (n_positions <= 0) return fail(K3_HIP_E_INVALID, "K3 router: no positions");
  const int nseg = (n_bank + 63) / 64;
  const int threads = std::min(1024, nseg * 64);
  const size_t lds = route_scratch_bytes(n_bank, top_k) + (size_t)n_bank * sizeof(float);
  TimedLaunch tl(KC_ROUTE, st);
  launch_timed(tl, k_route_sigmoid_bias, dim3(n_positions), dim3(threads), (unsigned)lds, st,
               logits, bias, n_bank, top_k, ids_ws, w_ws, ids_user, w_user);
  return launched(tl, "K3 router launch");
}

namespace {

// Workgroups of k_down_g64 for n routed experts: one per CU, more when a
// workgroup would own more than kDownG64MaxNB batches, and with fewer than 16
// experts 16 / n per CU (a workgroup holds one wave per routed expert, so the
// chip keeps ~16 waves of row batches per CU in flight: one expert at hidden
// 7168 gives 1,792 one-batch workgroups instead of 256 that walk 7 batches
// each); every workgroup owns at least one batch.
int down_g64_blocks(const Geo& g, int n) {
  const int nbt = (g.hidden + 3) / 4;
  const int cus = std::max(1, device_cu_count());
  const int per_cu = std::max(1, 16 / std::max(1, n));
  return std::min(nbt, std::max(cus * per_cu, (nbt + kDownG64MaxNB - 1) / kDownG64MaxNB));
}

// Positions of one launch (kPos kernels along blockIdx.y); n = 1 launches
// the single-position kernels.
struct PosLaunch {
  int n = 1;
  PosStride s{0, 0, 0};
};

template <typename XT, int kR, bool kG, bool kS4 = false>
void glu_go(TimedLaunch& tl, int grid, int threads, size_t lds, hipStream_t st,
            const TokenRoute& route, const Geo& g, const XT* x, float* h, int n_units, int S,
            const PosLaunch& pl) {
  if (pl.n > 1)
    launch_timed(tl, (k_glu_decode<XT, kR, kG, kS4, true>), dim3(grid, pl.n), dim3(threads),
                 (unsigned)lds, st, route, g, x, h, n_units, S, pl.s);
  else
    launch_timed(tl, (k_glu_decode<XT, kR, kG, kS4>), dim3(grid), dim3(threads), (unsigned)lds,
                 st, route, g, x, h, n_units, S, pl.s);
}

// Matrix-core gate/up (k_glu_mfma; k3_hip_set_decode_mfma): 0 never, 1 for
// fp32 activations (the default), 2 for fp32 and bf16 activations.
#ifndef K3_GLU_MFMA
#define K3_GLU_MFMA 1
#endif
std::atomic<int> g_glu_mfma{K3_GLU_MFMA};

// k_glu_mfma when the shape allows it: raw-v1 or scale4-v2 spans, hidden a
// multiple of 256 (at most 8192) split into S waves of 7 or 8 K blocks,
// intermediate a multiple of 8, a 16-byte aligned activation (and position
// stride) and 4, 6 or 8 units per pipeline (the instantiated unrolled loops).
// One position or a position batch (blockIdx.y).  *done says whether it
// launched.
template <typename XT, bool kS4, bool kPos>
void glu_mfma_go(TimedLaunch& tl, int NB, int iters, int grid, size_t lds, hipStream_t st,
                 const TokenRoute& route, const Geo& g, const XT* x, float* h, int n_units, int S,
                 int xo, const PosLaunch& pl) {
  constexpr int NT = sizeof(XT) == 4 ? 3 : 1;
  const dim3 gd(grid, kPos ? pl.n : 1);
#define K3_GM_GO(nb, it)                                                                      \
  if (NB == nb && iters == it)                                                                \
    launch_timed(tl, (k_glu_mfma<XT, NT, nb, it, kS4, kPos>), gd, dim3(kGmThreads),           \
                 (unsigned)lds, st, route, g, x, h, n_units, S, xo, pl.s);
  K3_GM_GO(7, 4) K3_GM_GO(7, 6) K3_GM_GO(7, 8) K3_GM_GO(8, 4) K3_GM_GO(8, 6) K3_GM_GO(8, 8)
#undef K3_GM_GO
}

template <typename XT>
int glu_mfma_try(const Geo& g, const TokenRoute& route, const XT* x, float* h, hipStream_t st,
                 const PosLaunch& pl, bool* done) {
  *done = false;
  constexpr bool f32 = sizeof(XT) == 4;
  constexpr int NT = f32 ? 3 : 1;
  const int mode = g_glu_mfma.load(std::memory_order_relaxed);
  if (mode == 0 || (!f32 && mode < 2)) return K3_HIP_OK;
  const bool s4 = g.layout == K3_LAYOUT_SCALE4_V2;
  if ((g.layout != K3_LAYOUT_RAW_V1 && !s4) || g.hidden % 256 != 0 || g.hidden > 8192 ||
      g.inter % 8 != 0)
    return K3_HIP_OK;
  if (reinterpret_cast<uintptr_t>(x) % 16 != 0 || (pl.s.x * (int64_t)sizeof(XT)) % 16 != 0)
    return K3_HIP_OK;
  const int KB = g.hidden / 256;
  int S = 0;
  for (int s = 1; s <= 8; s *= 2)
    if (KB % s == 0 && KB / s >= 7 && KB / s <= 8) {
      S = s;
      break;
    }
  if (S == 0) return K3_HIP_OK;
  const int NB = KB / S;
  const int groups = kGmThreads / (64 * S);
  const int cus = std::max(1, device_cu_count());
  const int n_units = route.n * (g.inter / 8);
  const int iters = (n_units + cus * groups - 1) / (cus * groups);
  if (iters != 4 && iters != 6 && iters != 8) return K3_HIP_OK;
  const size_t xs_off = route.logits ? (route_scratch_bytes(route.n_bank, route.n) + 15) & ~(size_t)15
                                     : 0;
  const size_t lds = xs_off + (NT + 1) * gm_term_bytes(g.hidden);
  if (lds > 64 * 1024) return K3_HIP_OK;
  TimedLaunch tl(KC_GLU_DECODE, st);
  const int xo = (int)xs_off;
  if (s4) {
    if (pl.n > 1)
      glu_mfma_go<XT, true, true>(tl, NB, iters, cus, lds, st, route, g, x, h, n_units, S, xo, pl);
    else
      glu_mfma_go<XT, true, false>(tl, NB, iters, cus, lds, st, route, g, x, h, n_units, S, xo, pl);
  } else {
    if (pl.n > 1)
      glu_mfma_go<XT, false, true>(tl, NB, iters, cus, lds, st, route, g, x, h, n_units, S, xo, pl);
    else
      glu_mfma_go<XT, false, false>(tl, NB, iters, cus, lds, st, route, g, x, h, n_units, S, xo,
                                    pl);
  }
  *done = true;
  return launched(tl, "decode gate/up launch");
}

template <typename XT>
int glu_decode_dispatch(const Geo& g, const TokenRoute& route, const XT* x, float* h,
                        hipStream_t st, const PosLaunch& pl = PosLaunch{}) {
  {
    bool done = false;
    const int rc = glu_mfma_try(g, route, x, h, st, pl, &done);
    if (done) return rc;
  }
  const int G = g.hidden / 32;
  const int S = (G + 63) / 64;
  if (S > 4) return fail(K3_HIP_E_INVALID, "decode layer: hidden %d exceeds 8192", g.hidden);
  if (g.inter % kRowsGlu != 0) return fail(K3_HIP_E_INVALID, "decode layer: bad intermediate");
  const size_t lds = route.logits ? route_scratch_bytes(route.n_bank, route.n) : 0;
  const int n_units = route.n * (g.inter / kRowsGlu);
  // One workgroup per CU holding up to 16 waves of unit pipelines.
  const int groups = std::max(1, std::min(kGluMaxThreads / (64 * S), 16 / S));
  const int cus = std::max(1, device_cu_count());
  const int grid = std::max(1, std::min(cus, (n_units + groups - 1) / groups));
  const int threads = 64 * S * groups;
  const int cw = (G + S - 1) / S;
  const bool gather = kRowsGlu == 4 && G % 4 == 0 && cw % 4 == 0 && kRowsGlu * cw <= 256;
  TimedLaunch tl(KC_GLU_DECODE, st);
  if (g.layout == K3_LAYOUT_SCALE4_V2) {
    // Index dwords gathered per unit: whole bytes per wave and row, dword
    // aligned, at most one dword per lane.
    if (!(kRowsGlu == 4 && G % 8 == 0 && cw % 8 == 0 && kRowsGlu * (cw / 8) <= 64))
      return fail(K3_HIP_E_CAPABILITY, "scale4-v2: hidden %d is not supported", g.hidden);
    glu_go<XT, kRowsGlu, true, true>(tl, grid, threads, lds, st, route, g, x, h, n_units, S, pl);
    return launched(tl, "decode gate/up launch");
  }
  // Few experts (every pipeline would hold one unit: config 1 is one expert):
  // units of 2 rows, two per pipeline, measured 12.1 -> 10.9 us per expert at
  // hidden 7168 / intermediate 2048 (the second unit's loads are in flight
  // while the first is reduced).  Their scale bytes are loaded per row.
  if (kRowsGlu == 4 && (n_units + groups - 1) / groups <= cus && g.inter % 2 == 0) {
    const int n_units2 = route.n * (g.inter / 2);
    glu_go<XT, 2, false>(tl, grid, threads, lds, st, route, g, x, h, n_units2, S, pl);
    return launched(tl, "decode gate/up launch");
  }
  if (gather)
    glu_go<XT, kRowsGlu, true>(tl, grid, threads, lds, st, route, g, x, h, n_units, S, pl);
  else
    glu_go<XT, kRowsGlu, false>(tl, grid, threads, lds, st, route, g, x, h, n_units, S, pl);
  return launched(tl, "decode gate/up launch");
}

template <typename OT, int CPL, int kB, bool kS4 = false>
int down_blocks_launch(const Geo& g, const TokenRoute& route, const float* h, OT* out,
                       hipStream_t st) {
  // One workgroup per CU, more when a workgroup's batches would overflow its
  // LDS row buffer.
  const int nbt = (g.hidden + kB - 1) / kB;
  const int cus = std::max(1, device_cu_count());
  const int per = std::max(1, std::min((nbt + cus - 1) / cus, kDownMaxRows / kB));
  const int blocks = (nbt + per - 1) / per;
  if ((nbt + blocks - 1) / blocks * kB > kDownMaxRows)
    return fail(K3_HIP_E_INVALID, "decode layer: hidden %d too large for the down kernel", g.hidden);
  const int max_waves = down_max_threads<CPL>() / 64;
  const int nw = std::min(route.n, max_waves);
  TimedLaunch tl(KC_DOWN_DECODE, st);
  launch_timed(tl, (k_down_blocks<OT, CPL, kB, kS4>), dim3(blocks), dim3(64 * nw), 0, st, route, g,
               h, out);
  return launched(tl, "decode down/combine launch");
}

template <typename OT, int NB>
int down_g64_launch(const Geo& g, const TokenRoute& route, const float* h, OT* out, int blocks,
                    hipStream_t st, const PosLaunch& pl) {
  const int nw = route.n;  // one wave per routed expert (route.n <= 16)
  const unsigned lds = (unsigned)(nw * kHSliceF4 * sizeof(float4));
  const void* fn = pl.n > 1 ? (const void*)k_down_g64<OT, NB, true> : (const void*)k_down_g64<OT, NB>;
  if (!lds_fits(fn, 64 * nw, lds))
    return fail(K3_HIP_E_EXEC, "decode layer: %u B of LDS per workgroup not available", lds);
  TimedLaunch tl(KC_DOWN_DECODE, st);
  if (pl.n > 1)
    launch_timed(tl, (k_down_g64<OT, NB, true>), dim3(blocks, pl.n), dim3(64 * nw), lds, st,
                 route, g, h, out, pl.s);
  else
    launch_timed(tl, (k_down_g64<OT, NB>), dim3(blocks), dim3(64 * nw), lds, st, route, g, h, out,
                 pl.s);
  return launched(tl, "decode down/combine launch");
}

template <typename OT>
int down_g64_dispatch(const Geo& g, const TokenRoute& route, const float* h, OT* out,
                      hipStream_t st, const PosLaunch& pl) {
  const int nbt = (g.hidden + 3) / 4;
  if (pl.n == 1 && route.n <= K3_DOWN_FEW_MAX && g.layout == K3_LAYOUT_RAW_V1) {
    // A few experts: h shared per workgroup (k_down_few).
    const unsigned lds = (unsigned)(route.n * kHSliceF4 * sizeof(float4));
    const dim3 grid((nbt + kFewWaves - 1) / kFewWaves), block(64 * kFewWaves);
    TimedLaunch tl(KC_DOWN_DECODE, st);
    switch (route.n) {
      case 1: launch_timed(tl, (k_down_few<OT, 1>), grid, block, lds, st, route, g, h, out); break;
      case 2: launch_timed(tl, (k_down_few<OT, 2>), grid, block, lds, st, route, g, h, out); break;
      case 3: launch_timed(tl, (k_down_few<OT, 3>), grid, block, lds, st, route, g, h, out); break;
      default: launch_timed(tl, (k_down_few<OT, 4>), grid, block, lds, st, route, g, h, out); break;
    }
    return launched(tl, "decode down/combine launch");
  }
  const int blocks = down_g64_blocks(g, route.n);
  const int nb = (nbt + blocks - 1) / blocks;
  switch (nb) {
    case 1: return down_g64_launch<OT, 1>(g, route, h, out, blocks, st, pl);
    case 2: return down_g64_launch<OT, 2>(g, route, h, out, blocks, st, pl);
    case 3: return down_g64_launch<OT, 3>(g, route, h, out, blocks, st, pl);
    case 4: return down_g64_launch<OT, 4>(g, route, h, out, blocks, st, pl);
    case 5: return down_g64_launch<OT, 5>(g, route, h, out, blocks, st, pl);
    case 6: return down_g64_launch<OT, 6>(g, route, h, out, blocks, st, pl);
    case 7: return down_g64_launch<OT, 7>(g, route, h, out, blocks, st, pl);
    case 8: return down_g64_launch<OT, 8>(g, route, h, out, blocks, st, pl);
    default: return fail(K3_HIP_E_INVALID, "decode layer: %d down batches per workgroup", nb);
  }
}

template <typename OT, int NB, bool kS4>
int down_g96_launch(const Geo& g, const TokenRoute& route, const float* h, OT* out, int blocks,
                    hipStream_t st, const PosLaunch& pl) {
  const int nw = route.n;  // one wave per routed expert (route.n <= 16)
  const unsigned lds = (unsigned)(nw * kHSliceF4 * sizeof(float4));
  const void* fn = pl.n > 1 ? (const void*)k_down_g96<OT, NB, kS4, true>
                            : (const void*)k_down_g96<OT, NB, kS4>;
  if (!lds_fits(fn, 64 * nw, lds))
    return fail(K3_HIP_E_EXEC, "decode layer: %u B of LDS per workgroup not available", lds);
  TimedLaunch tl(KC_DOWN_DECODE, st);
  if (pl.n > 1)
    launch_timed(tl, (k_down_g96<OT, NB, kS4, true>), dim3(blocks, pl.n), dim3(64 * nw), lds, st,
                 route, g, h, out, pl.s);
  else
    launch_timed(tl, (k_down_g96<OT, NB, kS4>), dim3(blocks), dim3(64 * nw), lds, st, route, g, h,
                 out, pl.s);
  return launched(tl, "decode down/combine launch");
}

// Workgroups for k_down_g96, sized as for k_down_g64 over row pairs.
template <typename OT, bool kS4>
int down_g96_dispatch(const Geo& g, const TokenRoute& route, const float* h, OT* out,
                      hipStream_t st, const PosLaunch& pl) {
  const int npt = g.hidden / 2;
  const int cus = std::max(1, device_cu_count());
  const int per_cu = std::max(1, 16 / std::max(1, route.n));
  const int blocks =
      std::min(npt, std::max(cus * per_cu, (npt + kDownG64MaxNB - 1) / kDownG64MaxNB));
  const int nb = (npt + blocks - 1) / blocks;
  switch (nb) {
    case 1: return down_g96_launch<OT, 1, kS4>(g, route, h, out, blocks, st, pl);
    case 2: return down_g96_launch<OT, 2, kS4>(g, route, h, out, blocks, st, pl);
    case 3: return down_g96_launch<OT, 3, kS4>(g, route, h, out, blocks, st, pl);
    case 4: return down_g96_launch<OT, 4, kS4>(g, route, h, out, blocks, st, pl);
    case 5: return down_g96_launch<OT, 5, kS4>(g, route, h, out, blocks, st, pl);
    case 6: return down_g96_launch<OT, 6, kS4>(g, route, h, out, blocks, st, pl);
    case 7: return down_g96_launch<OT, 7, kS4>(g, route, h, out, blocks, st, pl);
    case 8: return down_g96_launch<OT, 8, kS4>(g, route, h, out, blocks, st, pl);
    default: return fail(K3_HIP_E_INVALID, "decode layer: %d down pairs per workgroup", nb);
  }
}

// k_down_g96 serves intermediate 3072 with at most 16 routed experts and an
// even hidden width (a build knob keeps k_down_blocks for comparison).
#ifndef K3_DOWN_G96
#define K3_DOWN_G96 1
#endif
bool down_g96_fits(const Geo& g, const TokenRoute& route) {
  return K3_DOWN_G96 && g.inter == 3072 && route.n <= 16 && g.hidden % 2 == 0 && g.w2p % 16 == 0 &&
         g.w2s % 4 == 0;
}

// The down kernels with a position-batched form (k_down_g64, k_down_g96).
bool down_positions_fit(const Geo& g, int n) {
  TokenRoute r{};
  r.n = n;
  return n <= 16 && ((g.inter == 2048 && g.layout != K3_LAYOUT_SCALE4_V2) || down_g96_fits(g, r));
}

template <typename OT>
int down_decode_dispatch(const Geo& g, const TokenRoute& route, const Workspace& ws, OT* out,
                         hipStream_t st, const PosLaunch& pl = PosLaunch{}) {
  const int GB = g.inter / 32;
  if (pl.n > 1 && !down_positions_fit(g, route.n))
    return fail(K3_HIP_E_CAPABILITY, "decode layer: no batched down kernel for this geometry");
  if (g.layout == K3_LAYOUT_SCALE4_V2) {
    // The format is defined for K3 only (96 groups per down row).
    if (GB != 96) return fail(K3_HIP_E_CAPABILITY, "scale4-v2: intermediate %d is not supported", g.inter);
    if (down_g96_fits(g, route)) return down_g96_dispatch<OT, true>(g, route, ws.h, out, st, pl);
    return down_blocks_launch<OT, 2, 2, true>(g, route, ws.h, out, st);
  }
  if (GB == 64 && route.n <= 16) return down_g64_dispatch<OT>(g, route, ws.h, out, st, pl);
  if (down_g96_fits(g, route)) return down_g96_dispatch<OT, false>(g, route, ws.h, out, st, pl);
  switch ((GB + 63) / 64) {
    case 1: return down_blocks_launch<OT, 1, kDownBlocksBatch>(g, route, ws.h, out, st);
    case 2: return down_blocks_launch<OT, 2, K3_DOWN_BATCH_CPL2>(g, route, ws.h, out, st);
    case 3: return down_blocks_launch<OT, 3, 2>(g, route, ws.h, out, st);
    case 4: return down_blocks_launch<OT, 4, 1>(g, route, ws.h, out, st);
    default: return fail(K3_HIP_E_INVALID, "decode layer: intermediate %d exceeds 8192", g.inter);
  }
}

// Fused decode (k_decode_fused) when selected (k3_hip_set_fused_decode; off
// by default: it measures slower than the two launches, see the kernel's
// comment) and its shape holds: intermediate 2048 (64 scale groups per down
// row), at most 16 routed experts, gathered gate/up scales, and a free
// g_fused_sync slot for the workspace.  *ran tells the caller whether it
// launched; otherwise the two-launch path runs.
#ifndef K3_FUSED_DECODE
#define K3_FUSED_DECODE 0
#endif
#ifndef K3_FUSED_GLU_GROUPS
#define K3_FUSED_GLU_GROUPS 2
#endif

std::atomic<int> g_fused_enabled{K3_FUSED_DECODE};

// Slot of g_fused_sync for a workspace on the current device, -1 once every
// slot is taken.  A workspace keeps its slot for the life of the process.
int fused_slot(const void* ws_base) {
  static std::mutex mu;
  static std::unordered_map<int, std::vector<const void*>> table;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return -1;
  std::lock_guard<std::mutex> lock(mu);
  std::vector<const void*>& v = table[dev];
  for (size_t i = 0; i < v.size(); ++i)
    if (v[i] == ws_base) return (int)i;
  if ((int)v.size() >= kFusedSlots) return -1;
  v.push_back(ws_base);
  return (int)v.size() - 1;
}

// Launched for bf16 activations only (fused_decode): an fp32 x slice (32
// registers) does not fit the 1024-thread register budget next to the
// gate/up batches.
template <typename OT, int NB>
int fused_launch(const Geo& g, const TokenRoute& route, const uint16_t* x, float* h, OT* out,
                 const FusedPlan& fp, int grid, hipStream_t st, bool* ran) {
  const size_t keys = route.logits ? route_scratch_bytes(route.n_bank, route.n) : 0;
  const size_t lds = std::max(keys, (size_t)16 * kHSliceF4 * sizeof(float4));
  const void* kernel = (const void*)k_decode_fused<uint16_t, OT, kRowsGlu, NB>;
  if (!lds_fits(kernel, 1024, lds)) return K3_HIP_OK;  // two-launch path
  *ran = true;
  TimedLaunch tl(KC_DECODE_FUSED, st);
  launch_timed(tl, (k_decode_fused<uint16_t, OT, kRowsGlu, NB>), dim3(grid), dim3(1024),
               (unsigned)lds, st, route, g, x, h, out, fp);
  return launched(tl, "fused decode launch");
}

template <typename OT>
int fused_decode(const Geo& g, const TokenRoute& route, const float* x, OT* out,
                 const Workspace& ws, hipStream_t st, bool* ran) {
  *ran = false;  // fp32 activations: two-launch path
  return K3_HIP_OK;
}

template <typename OT>
int fused_decode(const Geo& g, const TokenRoute& route, const uint16_t* x, OT* out,
                 const Workspace& ws, hipStream_t st, bool* ran) {
  *ran = false;
  if (!g_fused_enabled.load(std::memory_order_relaxed)) return K3_HIP_OK;
  const int G = g.hidden / 32;
  const int S = (G + 63) / 64;
  const int cw = (G + S - 1) / S;
  const bool gather = kRowsGlu == 4 && G % 4 == 0 && cw % 4 == 0 && kRowsGlu * cw <= 256;
  if (S > 4 || !gather || g.inter != 64 * 32 || route.n > 16) return K3_HIP_OK;
  const int slot = fused_slot(ws.base);
  if (slot < 0) return K3_HIP_OK;
  const int cus = std::max(1, device_cu_count());
  FusedPlan fp;
  fp.S = S;
  fp.groups = std::max(1, std::min(K3_FUSED_GLU_GROUPS, 16 / S));
  fp.n_units = route.n * (g.inter / kRowsGlu);
  fp.n_glu = std::max(1, std::min(cus, (fp.n_units + fp.groups - 1) / fp.groups));
  const int nbt = (g.hidden + 3) / 4;
  fp.n_down = std::min(nbt, std::max(cus, (nbt + kDownG64MaxNB - 1) / kDownG64MaxNB));
  fp.slot = slot;
  const int nb = (nbt + fp.n_down - 1) / fp.n_down;
  const int grid = std::min(cus, std::max(fp.n_glu, fp.n_down));
  switch (nb) {
    case 1: return fused_launch<OT, 1>(g, route, x, ws.h, out, fp, grid, st, ran);
    case 2: return fused_launch<OT, 2>(g, route, x, ws.h, out, fp, grid, st, ran);
    case 3: return fused_launch<OT, 3>(g, route, x, ws.h, out, fp, grid, st, ran);
    case 4: return fused_launch<OT, 4>(g, route, x, ws.h, out, fp, grid, st, ran);
    case 5: return fused_launch<OT, 5>(g, route, x, ws.h, out, fp, grid, st, ran);
    case 6: return fused_launch<OT, 6>(g, route, x, ws.h, out, fp, grid, st, ran);
    case 7: return fused_launch<OT, 7>(g, route, x, ws.h, out, fp, grid, st, ran);
    case 8: return fused_launch<OT, 8>(g, route, x, ws.h, out, fp, grid, st, ran);
    default: return K3_HIP_OK;
  }
}

// One launch for a one-expert layer (k_expert_chain) where the two-launch
// path would run k_glu_decode's 2-row units and k_down_few<OT, 1>: one
// token, caller span pointers, bf16 activations (fp32 ones may take the
// matrix-core gate/up, whose sums are ordered differently), raw-v1,
// intermediate 2048, one workgroup per CU whose waves cover the down row
// batches, and the workspace's h and y areas (the decode layer does not use
// y) holding the tagged h.  g_chain_mode: 0 off, 1 on, 2 on with the
// missing-share fallback taken at once (a test of that path).  *ran tells the
// caller whether it launched.
std::atomic<int> g_chain_mode{K3_EXPERT_CHAIN};

template <typename OT>
int chain_decode(const Geo& g, const TokenRoute& route, const float* x, OT* out,
                 const Workspace& ws, hipStream_t st, bool* ran) {
  *ran = false;
  return K3_HIP_OK;
}

template <typename OT>
int chain_decode(const Geo& g, const TokenRoute& route, const uint16_t* x, OT* out,
                 const Workspace& ws, hipStream_t st, bool* ran) {
  *ran = false;
  const int mode = g_chain_mode.load(std::memory_order_relaxed);
  if (mode == 0) return K3_HIP_OK;
  if (route.logits || route.bank || route.pdev || route.n != 1 ||
      g.layout != K3_LAYOUT_RAW_V1 || g.inter != 2048 || g.hidden % 32 != 0)
    return K3_HIP_OK;
  constexpr int NE = 1;
  if (reinterpret_cast<const uint8_t*>(ws.ids) - reinterpret_cast<const uint8_t*>(ws.h) <
      (ptrdiff_t)NE * g.inter * 8)
    return K3_HIP_OK;
  const int G = g.hidden / 32;
  const int S = (G + 63) / 64;
  if (S > 4) return K3_HIP_OK;
  // glu_decode_dispatch's few-expert condition (2-row units)
  const int groups = std::max(1, std::min(kGluMaxThreads / (64 * S), 16 / S));
  const int cus = std::max(1, device_cu_count());
  const int n_units4 = route.n * (g.inter / kRowsGlu);
  if (!(kRowsGlu == 4 && (n_units4 + groups - 1) / groups <= cus)) return K3_HIP_OK;
  ChainPlan cp;
  cp.S = S;
  cp.groups = groups;
  cp.n_units = route.n * (g.inter / 2);
  cp.poll_limit = mode == 2 ? 0 : kChainPollLimit;
  cp.zero = 0;
  const int grid = std::max(1, std::min(cus, (cp.n_units + groups - 1) / groups));
  const int threads = 64 * S * groups;
  const int nbt = (g.hidden + 3) / 4;
  if (grid < cus || grid > kChainMaxGrid || threads < 384 || (int64_t)grid * (threads / 64) < nbt)
    return K3_HIP_OK;
  const int iters = (cp.n_units + grid * groups - 1) / (grid * groups);
  if (iters != 1 && iters != 2) return K3_HIP_OK;
  const void* kernel = iters == 1 ? (const void*)k_expert_chain<uint16_t, OT, NE, 1>
                                  : (const void*)k_expert_chain<uint16_t, OT, NE, 2>;
  const unsigned lds = (unsigned)(NE * kHSliceF4 * sizeof(float4));
  if (!lds_fits(kernel, threads, lds)) return K3_HIP_OK;
  cp.slot = fused_slot(ws.base);
  if (cp.slot < 0 || cp.slot >= kChainSlots) return K3_HIP_OK;
  *ran = true;
  uint64_t* ht = reinterpret_cast<uint64_t*>(ws.h);
  TimedLaunch tl(KC_DECODE_CHAIN, st);
  if (iters == 1)
    launch_timed(tl, (k_expert_chain<uint16_t, OT, NE, 1>), dim3(grid), dim3(threads), lds, st,
                 route, g, x, ht, out, cp);
  else
    launch_timed(tl, (k_expert_chain<uint16_t, OT, NE, 2>), dim3(grid), dim3(threads), lds, st,
                 route, g, x, ht, out, cp);
  return launched(tl, "one-expert decode launch");
}

}  // namespace

int set_fused_decode(int enabled) {
  return g_fused_enabled.exchange(enabled ? 1 : 0);
}

int set_decode_chain(int mode) {
  if (mode < 0 || mode > 2) return fail(K3_HIP_E_INVALID, "decode chain mode %d unknown", mode);
  return g_chain_mode.exchange(mode);
}

int set_decode_mfma(int mode) {
  if (mode < 0 || mode > 2) return fail(K3_HIP_E_INVALID, "decode dot mode %d unknown", mode);
  return g_glu_mfma.exchange(mode);
}

size_t route_scratch_bytes(int n_bank, int top_k) {
  const size_t nseg = (size_t)(n_bank + 63) / 64;
  return (nseg * 64 + ((nseg * (size_t)top_k + 1) & ~(size_t)1)) * sizeof(uint64_t);
}

int launch_decode_layer(const Geo& g, const TokenRoute& route, const void* x, int x_dtype,
                        void* out, int out_dtype, const Workspace& ws, hipStream_t st) {
  if (route.n <= 0 || route.n > K3_HIP_MAX_TOKEN_EXPERTS)
    return fail(K3_HIP_E_INVALID, "decode layer: expert count %d outside [1, %d]", route.n,
                K3_HIP_MAX_TOKEN_EXPERTS);
  bool ran = false;
  const int frc =
      x_dtype == K3_DTYPE_BF16
          ? (out_dtype == K3_DTYPE_BF16
                 ? fused_decode(g, route, static_cast<const uint16_t*>(x),
                                static_cast<uint16_t*>(out), ws, st, &ran)
                 : fused_decode(g, route, static_cast<const uint16_t*>(x),
                                static_cast<float*>(out), ws, st, &ran))
          : (out_dtype == K3_DTYPE_BF16
                 ? fused_decode(g, route, static_cast<const float*>(x),
                                static_cast<uint16_t*>(out), ws, st, &ran)
                 : fused_decode(g, route, static_cast<const float*>(x), static_cast<float*>(out),
                                ws, st, &ran));
  if (frc != K3_HIP_OK || ran) return frc;
  const int crc =
      x_dtype == K3_DTYPE_BF16
          ? (out_dtype == K3_DTYPE_BF16
                 ? chain_decode(g, route, static_cast<const uint16_t*>(x),
                                static_cast<uint16_t*>(out), ws, st, &ran)
                 : chain_decode(g, route, static_cast<const uint16_t*>(x),
                                static_cast<float*>(out), ws, st, &ran))
          : (out_dtype == K3_DTYPE_BF16
                 ? chain_decode(g, route, static_cast<const float*>(x),
                                static_cast<uint16_t*>(out), ws, st, &ran)
                 : chain_decode(g, route, static_cast<const float*>(x), static_cast<float*>(out),
                                ws, st, &ran));
  if (crc != K3_HIP_OK || ran) return crc;
  int rc = x_dtype == K3_DTYPE_BF16
               ? glu_decode_dispatch<uint16_t>(g, route, static_cast<const uint16_t*>(x), ws.h, st)
               : glu_decode_dispatch<float>(g, route, static_cast<const float*>(x), ws.h, st);
  if (rc != K3_HIP_OK) return rc;
  // The down kernel reads the route the gate/up kernel published.
  TokenRoute down_route = route;
  if (route.logits) {
    down_route.logits = nullptr;
    down_route.ids = ws.ids;
    down_route.wdev = ws.w;
  }
  return out_dtype == K3_DTYPE_BF16
             ? down_decode_dispatch<uint16_t>(g, down_route, ws, static_cast<uint16_t*>(out), st)
             : down_decode_dispatch<float>(g, down_route, ws, static_cast<float*>(out), st);
}

bool decode_positions_supported(const Geo& g, int n) {
  return n >= 1 && n <= 16 && down_positions_fit(g, n) && g_fused_enabled.load() == 0;
}

int launch_decode_positions(const Geo& g, const TokenRoute& route, int n_positions,
                            const void* x, int x_dtype, void* out, int out_dtype,
                            const Workspace& ws, hipStream_t st) {
  if (!(route.bank || route.pdev) || n_positions < 1 || !decode_positions_supported(g, route.n))
    return fail(K3_HIP_E_CAPABILITY, "decode positions: no batched form for this call");
  PosLaunch pl;
  pl.n = n_positions;
  pl.s.x = g.hidden;
  pl.s.h = (int64_t)route.n * g.inter;
  pl.s.out = g.hidden;
  int rc = x_dtype == K3_DTYPE_BF16
               ? glu_decode_dispatch<uint16_t>(g, route, static_cast<const uint16_t*>(x), ws.h, st, pl)
               : glu_decode_dispatch<float>(g, route, static_cast<const float*>(x), ws.h, st, pl);
  if (rc != K3_HIP_OK) return rc;
  TokenRoute down_route = route;
  if (route.logits) {
    down_route.logits = nullptr;
    down_route.ids = ws.ids;
    down_route.wdev = ws.w;
  }
  return out_dtype == K3_DTYPE_BF16
             ? down_decode_dispatch<uint16_t>(g, down_route, ws, static_cast<uint16_t*>(out), st, pl)
             : down_decode_dispatch<float>(g, down_route, ws, static_cast<float*>(out), st, pl);
}

// Workgroups of the plan launch: the plan, plus the activation split's when
// x_split is set (one thread per 8 elements of the n_rows x hidden rows).
static dim3 plan_grid(const Geo& g, int n_rows, const void* x_split) {
  const int64_t threads = x_split ? (int64_t)n_rows * (g.hidden / 32) * 4 : 0;
  return dim3((unsigned)(1 + (threads + 255) / 256));
}

int launch_verify_plan_bank(const Geo& g, const uint8_t* bank, uint64_t stride, int n_bank,
                            int n_positions, int top_k, const Workspace& ws, hipStream_t st,
                            const void* x_split, int x_dtype) {
  // Rank-sorted plan: unique experts in span-pointer order, each expert's
  // edges in edge order (every union kernel takes any expert order).
  TimedLaunch tl(KC_VERIFY_PLAN, st);
  const dim3 grid = plan_grid(g, n_positions, x_split);
  if (!x_split)
    launch_timed(tl, (k_verify_plan_bank<0, float>), grid, dim3(256), 0, st, bank, stride,
                 n_bank, n_positions, top_k, ws, nullptr, g.hidden);
  else if (x_dtype == K3_DTYPE_BF16)
    launch_timed(tl, (k_verify_plan_bank<2, uint16_t>), grid, dim3(256), 0, st, bank, stride,
                 n_bank, n_positions, top_k, ws, static_cast<const uint16_t*>(x_split),
                 g.hidden);
  else
    launch_timed(tl, (k_verify_plan_bank<3, float>), grid, dim3(256), 0, st, bank, stride,
                 n_bank, n_positions, top_k, ws, static_cast<const float*>(x_split), g.hidden);
  return launched(tl, "verify plan launch");
}

int launch_verify_plan_table(const Geo& g, const EdgeTable& table, const Workspace& ws,
                             hipStream_t st, const void* x_split, int x_dtype) {
  TimedLaunch tl(KC_VERIFY_PLAN, st);
  const dim3 grid = plan_grid(g, table.n_positions, x_split);
  if (!x_split)
    launch_timed(tl, (k_verify_plan_table<0, float>), grid, dim3(256), 0, st, table, ws, nullptr,
                 g.hidden);
  else if (x_dtype == K3_DTYPE_BF16)
    launch_timed(tl, (k_verify_plan_table<2, uint16_t>), grid, dim3(256), 0, st, table, ws,
                 static_cast<const uint16_t*>(x_split), g.hidden);
  else
    launch_timed(tl, (k_verify_plan_table<3, float>), grid, dim3(256), 0, st, table, ws,
                 static_cast<const float*>(x_split), g.hidden);
  return launched(tl, "verify plan launch");
}

int launch_route_table(const EdgeTable& table, int e0, int n, const Workspace& ws, hipStream_t st) {
  if (e0 < 0 || n < 1 || e0 + n > table.n_edges)
    return fail(K3_HIP_E_INVALID, "route table: edges %d .. %d outside the table", e0, e0 + n);
  TimedLaunch tl(KC_VERIFY_PLAN, st);
  launch_timed(tl, k_route_table, dim3(1), dim3(256), 0, st, table, e0, n, ws.uptr, ws.w);
  return launched(tl, "route table launch");
}

namespace {

template <typename XT>
int glu_verify_dispatch(const Geo& g, int n_edges, const XT* x, const Workspace& ws,
                        hipStream_t st) {
  constexpr int kG = VerifyA<XT>::kGroup;
  const size_t lds = (size_t)kG * g.hidden * sizeof(XT);
  if (lds > 96 * 1024) return fail(K3_HIP_E_INVALID, "verify: hidden %d too wide", g.hidden);
  const int upe = g.inter / (4 * kRowsVerifyA);
  TimedLaunch tl(KC_GLU_VERIFY, st);
  launch_timed(tl, (k_glu_verify_rows<XT, kRowsVerifyA>), dim3(upe * n_edges), dim3(256),
               (unsigned)lds, st, g, x, ws);
  return launched(tl, "verify gate/up launch");
}

int down_verify_dispatch(const Geo& g, int n_edges, const Workspace& ws, hipStream_t st) {
  const int GB = g.inter / 32;
  const int cplb = (GB + 63) / 64;
  const int upe = (g.hidden + 4 * kRowsVerifyB - 1) / (4 * kRowsVerifyB);
  const dim3 grid(upe * n_edges), block(256);
  if (cplb > 4) return fail(K3_HIP_E_INVALID, "verify: intermediate %d exceeds 8192", g.inter);
  TimedLaunch tl(KC_DOWN_VERIFY, st);
  switch (cplb) {
    case 1: launch_timed(tl, (k_down_verify<1, kRowsVerifyB>), grid, block, 0, st, g, ws); break;
    case 2: launch_timed(tl, (k_down_verify<2, kRowsVerifyB>), grid, block, 0, st, g, ws); break;
    case 3: launch_timed(tl, (k_down_verify<3, kRowsVerifyB>), grid, block, 0, st, g, ws); break;
    case 4: launch_timed(tl, (k_down_verify<4, kRowsVerifyB>), grid, block, 0, st, g, ws); break;
    default: return fail(K3_HIP_E_INVALID, "verify: intermediate %d exceeds 8192", g.inter);
  }
  return launched(tl, "verify down launch");
}

}  // namespace

int launch_verify_layer(const Geo& g, int n_edges, int n_positions, const void* x, int x_dtype,
                        void* out, int out_dtype, const Workspace& ws, hipStream_t st) {
  if (g.inter % (4 * kRowsVerifyA) != 0)
    return fail(K3_HIP_E_INVALID, "verify: intermediate must be a multiple of 32");
  int rc = x_dtype == K3_DTYPE_BF16
               ? glu_verify_dispatch<uint16_t>(g, n_edges, static_cast<const uint16_t*>(x), ws, st)
               : glu_verify_dispatch<float>(g, n_edges, static_cast<const float*>(x), ws, st);
  if (rc != K3_HIP_OK) return rc;
  rc = down_verify_dispatch(g, n_edges, ws, st);
  if (rc != K3_HIP_OK) return rc;
  return launch_verify_combine(g, n_positions, out, out_dtype, ws, st);
}

int launch_verify_combine(const Geo& g, int n_positions, void* out, int out_dtype,
                          const Workspace& ws, hipStream_t st) {
  const int64_t n = (int64_t)g.hidden * n_positions;
  const dim3 grid((unsigned)((n + 255) / 256)), block(256);
  TimedLaunch tl(KC_COMBINE, st);
  if (out_dtype == K3_DTYPE_BF16)
    launch_timed(tl, k_combine_positions<uint16_t>, grid, block, 0, st, ws, g.hidden,
                       n_positions, static_cast<uint16_t*>(out));
  else
    launch_timed(tl, k_combine_positions<float>, grid, block, 0, st, ws, g.hidden, n_positions,
                       static_cast<float*>(out));
  return launched(tl, "verify combine launch");
}

int launch_synth_bank(const Geo& g, uint8_t* bank, uint64_t stride, int n_experts,
                      uint64_t first_expert, uint64_t seed, int lo, int hi, hipStream_t st) {
  if (!bank || n_experts <= 0 || n_experts > 65535 || stride < g.span || stride % 8 != 0 ||
      ((uintptr_t)bank & 7u) != 0 || lo < 0 || hi > 255 || lo > hi)
    return fail(K3_HIP_E_INVALID, "synth bank: invalid arguments");
  TimedLaunch tl(KC_SYNTH, st);
  launch_timed(tl, k_synth_bank, dim3(1024, n_experts), dim3(256), 0, st, g, bank, stride,
                     first_expert, seed, lo, hi);
  return launched(tl, "synth bank launch");
}

int launch_synth_normal(void* out, int dtype, uint64_t n, uint64_t seed, uint64_t stream_id,
                        hipStream_t st) {
  if (!out || (dtype != K3_DTYPE_F32 && dtype != K3_DTYPE_BF16))
    return fail(K3_HIP_E_INVALID, "synth normal: invalid arguments");
  if (n == 0) return K3_HIP_OK;
  const uint64_t blocks = std::min<uint64_t>((n + 255) / 256, 4096);
  TimedLaunch tl(KC_SYNTH, st);
  launch_timed(tl, k_synth_normal, dim3((unsigned)blocks), dim3(256), 0, st, out, dtype, n, seed,
                     stream_id);
  return launched(tl, "synth normal launch");
}

int launch_zero(void* p, uint64_t bytes, hipStream_t st) {
  if (!p || bytes % 4 != 0 || ((uintptr_t)p & 3u) != 0)
    return fail(K3_HIP_E_INVALID, "zero fill: needs a 4-byte aligned pointer and size");
  if (bytes == 0) return K3_HIP_OK;
  const uint64_t n = bytes / 4;
  const uint64_t blocks = std::min<uint64_t>((n + 255) / 256, 1024);
  TimedLaunch tl(KC_COMBINE, st);
  launch_timed(tl, k_zero_words, dim3((unsigned)blocks), dim3(256), 0, st,
               static_cast<uint32_t*>(p), n);
  return launched(tl, "zero fill launch");
}

}  // namespace k3
