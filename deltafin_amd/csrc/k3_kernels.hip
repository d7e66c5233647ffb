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

#include "k3_device.h"
#include "k3_internal.h"

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

__device__ __forceinline__ const uint8_t* route_span(const TokenRoute& r, int e) {
  return r.bank ? r.bank + (uint64_t)r.ids[e] * r.stride : r.ptr[e];
}
__device__ __forceinline__ float route_weight(const TokenRoute& r, int e) {
  return r.bank ? r.wdev[e] : r.w[e];
}

// ======================================================================
// single-activation GEMV: one wave per kRows rows, x slice in registers
// ======================================================================
template <typename XT, typename OT, int CPL, int kRows>
__global__ __launch_bounds__(256) void k_gemv1(const uint8_t* __restrict__ packed,
                                               const uint8_t* __restrict__ scales,
                                               const XT* __restrict__ x,
                                               OT* __restrict__ out, int rows, int cols) {
  const int lane = threadIdx.x & 63;
  const int r0 = (blockIdx.x * 4 + (threadIdx.x >> 6)) * kRows;
  if (r0 >= rows) return;
  const int G = cols >> 5;
  const size_t cp = (size_t)cols >> 1;

  XChunk<XT> xs[CPL];
#pragma unroll
  for (int c = 0; c < CPL; ++c) {
    const int chunk = lane + 64 * c;
    if (chunk < G) xs[c].load(x, chunk);
  }
  float acc[kRows];
#pragma unroll
  for (int r = 0; r < kRows; ++r) {
    float a = 0.0f;
    if (r0 + r < rows) {
      const uint8_t* pr = packed + (size_t)(r0 + r) * cp;
      const uint8_t* sr = scales + (size_t)(r0 + r) * G;
#pragma unroll
      for (int c = 0; c < CPL; ++c) {
        const int chunk = lane + 64 * c;
        if (chunk < G) {
          const u32x4 w = load_chunk(pr + (size_t)chunk * 16);
          a = fmaf(xs[c].dot(w), e8m0_scale(sr[chunk]), a);
        }
      }
    }
    acc[r] = a;
  }
#pragma unroll
  for (int r = 0; r < kRows; ++r) {
    const float v = wave_sum(acc[r]);
    if (lane == 0 && r0 + r < rows) store_out(out + r0 + r, v);
  }
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
    for (int i = threadIdx.x; i < n16; i += blockDim.x) smem_multi[i] = src[i];
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
// decode phase A: gate/up rows of one expert + activation -> h
// ======================================================================
template <typename XT, int CPL, int kRows>
__global__ __launch_bounds__(256) void k_glu_decode(const TokenRoute route, const Geo g,
                                                    const XT* __restrict__ x,
                                                    float* __restrict__ h) {
  const int lane = threadIdx.x & 63;
  const int unit = blockIdx.x * 4 + (threadIdx.x >> 6);
  const int upe = g.inter / kRows;
  if (unit >= route.n * upe) return;
  const int e = unit / upe;
  const int r0 = (unit - e * upe) * kRows;
  const int G = g.hidden >> 5;
  const size_t cp = (size_t)g.hidden >> 1;
  const uint8_t* span = route_span(route, e);
  const uint8_t* gp = span + g.w1p + (size_t)r0 * cp;
  const uint8_t* gs = span + g.w1s + (size_t)r0 * G;
  const uint8_t* up = span + g.w3p + (size_t)r0 * cp;
  const uint8_t* us = span + g.w3s + (size_t)r0 * G;

  XChunk<XT> xs[CPL];
#pragma unroll
  for (int c = 0; c < CPL; ++c) {
    const int chunk = lane + 64 * c;
    if (chunk < G) xs[c].load(x, chunk);
  }
  float ag[kRows], au[kRows];
#pragma unroll
  for (int r = 0; r < kRows; ++r) {
    float a = 0.0f, b = 0.0f;
#pragma unroll
    for (int c = 0; c < CPL; ++c) {
      const int chunk = lane + 64 * c;
      if (chunk < G) {
        const u32x4 wg = load_chunk(gp + (size_t)r * cp + (size_t)chunk * 16);
        const u32x4 wu = load_chunk(up + (size_t)r * cp + (size_t)chunk * 16);
        const float sg = e8m0_scale(gs[(size_t)r * G + chunk]);
        const float su = e8m0_scale(us[(size_t)r * G + chunk]);
        a = fmaf(xs[c].dot(wg), sg, a);
        b = fmaf(xs[c].dot(wu), su, b);
      }
    }
    ag[r] = a;
    au[r] = b;
  }
  float* hrow = h + (size_t)e * g.inter + r0;
#pragma unroll
  for (int r = 0; r < kRows; ++r) {
    const float gv = wave_sum(ag[r]);
    const float uv = wave_sum(au[r]);
    if (lane == 0) hrow[r] = activate(g.act, gv, uv);
  }
}

// ======================================================================
// decode phase B: down rows of every routed expert + ordered combine
// ======================================================================
constexpr int kDownMaxRows = 64;

template <typename OT, int CPLB>
__global__ __launch_bounds__(1024) void k_down_decode(const TokenRoute route, const Geo g,
                                                      const float* __restrict__ h,
                                                      OT* __restrict__ out,
                                                      int rows_per_block) {
  __shared__ float ybuf[K3_HIP_MAX_TOKEN_EXPERTS][kDownMaxRows];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int nw = blockDim.x >> 6;
  const int row0 = blockIdx.x * rows_per_block;
  const int nrows = min(rows_per_block, g.hidden - row0);
  const int GB = g.inter >> 5;
  const size_t cpb = (size_t)g.inter >> 1;

  for (int e = wave; e < route.n; e += nw) {
    const uint8_t* span = route_span(route, e);
    const uint8_t* dp = span + g.w2p + (size_t)row0 * cpb;
    const uint8_t* ds = span + g.w2s + (size_t)row0 * GB;
    XChunk<float> hs[CPLB];
#pragma unroll
    for (int c = 0; c < CPLB; ++c) {
      const int chunk = lane + 64 * c;
      if (chunk < GB) hs[c].load(h + (size_t)e * g.inter, chunk);
    }
    for (int r = 0; r < nrows; ++r) {
      float a = 0.0f;
#pragma unroll
      for (int c = 0; c < CPLB; ++c) {
        const int chunk = lane + 64 * c;
        if (chunk < GB) {
          const u32x4 w = load_chunk(dp + (size_t)r * cpb + (size_t)chunk * 16);
          a = fmaf(hs[c].dot(w), e8m0_scale(ds[(size_t)r * GB + chunk]), a);
        }
      }
      a = wave_sum(a);
      if (lane == 0) ybuf[e][r] = a;
    }
  }
  __syncthreads();
  for (int t = threadIdx.x; t < nrows; t += blockDim.x) {
    float acc = 0.0f;
    for (int e = 0; e < route.n; ++e) acc += route_weight(route, e) * ybuf[e][t];
    store_out(out + row0 + t, acc);
  }
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
// router: top-k (descending, lower index on ties, NaN never selected ahead of
// a number) + softmax over the selected logits; one workgroup per position
// ======================================================================
__global__ __launch_bounds__(256) void k_route(const float* __restrict__ logits, int n_bank,
                                               int top_k, int32_t* __restrict__ ids_ws,
                                               float* __restrict__ w_ws,
                                               int32_t* __restrict__ ids_user,
                                               float* __restrict__ w_user) {
  extern __shared__ float lg[];
  __shared__ int sel[K3_HIP_MAX_TOKEN_EXPERTS];
  const int p = blockIdx.x;
  const float* src = logits + (size_t)p * n_bank;
  for (int i = threadIdx.x; i < n_bank; i += blockDim.x) {
    const float v = src[i];
    lg[i] = (v != v) ? -INFINITY : v;
  }
  __syncthreads();
  for (int i = threadIdx.x; i < n_bank; i += blockDim.x) {
    const float li = lg[i];
    int rank = 0;
    for (int j = 0; j < n_bank; ++j) {
      const float lj = lg[j];
      rank += (lj > li) || (lj == li && j < i);
    }
    if (rank < top_k) sel[rank] = i;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    const float top = lg[sel[0]];
    float ex[K3_HIP_MAX_TOKEN_EXPERTS];
    float sum = 0.0f;
    for (int j = 0; j < top_k; ++j) {
      ex[j] = expf(lg[sel[j]] - top);
      sum += ex[j];
    }
    for (int j = 0; j < top_k; ++j) {
      const float w = ex[j] / sum;
      const int o = p * top_k + j;
      ids_ws[o] = sel[j];
      w_ws[o] = w;
      if (ids_user) ids_user[o] = sel[j];
      if (w_user) w_user[o] = w;
    }
  }
}

// ======================================================================
// verify plan: group edges by expert span (one workgroup, <= 256 edges)
// ======================================================================
__device__ void plan_core(const uint8_t* key, int e, int n_edges, int n_positions,
                          const Workspace& ws) {
  __shared__ const uint8_t* kp[K3_HIP_MAX_EDGES];
  __shared__ int first[K3_HIP_MAX_EDGES];
  __shared__ int uid_of_first[K3_HIP_MAX_EDGES];
  __shared__ int ucount[K3_HIP_MAX_EDGES];
  __shared__ int uoff[K3_HIP_MAX_EDGES + 1];
  if (e < n_edges) kp[e] = key;
  __syncthreads();
  int f = e;
  if (e < n_edges) {
    for (int j = 0; j < e; ++j) {
      if (kp[j] == key) {
        f = j;
        break;
      }
    }
    first[e] = f;
  }
  __syncthreads();
  if (e < n_edges && f == e) {
    int u = 0, cnt = 0;
    for (int j = 0; j < n_edges; ++j) {
      u += (j < e) && (first[j] == j);
      cnt += (kp[j] == key);
    }
    uid_of_first[e] = u;
    ucount[u] = cnt;
    ws.uptr[u] = key;
  }
  __syncthreads();
  if (e == 0) {
    int u = 0, off = 0;
    for (int j = 0; j < n_edges; ++j) {
      if (first[j] == j) {
        uoff[u] = off;
        ws.uoff[u] = off;
        off += ucount[u];
        ++u;
      }
    }
    uoff[u] = off;
    ws.uoff[u] = off;
    ws.plan->n_unique = u;
    ws.plan->n_edges = n_edges;
    ws.plan->n_positions = n_positions;
  }
  __syncthreads();
  if (e < n_edges) {
    int rank = 0;
    for (int j = 0; j < e; ++j) rank += (kp[j] == key);
    ws.uedges[uoff[uid_of_first[first[e]]] + rank] = e;
  }
}

__global__ __launch_bounds__(256) void k_verify_plan_bank(const uint8_t* bank, uint64_t stride,
                                                          int n_positions, int top_k,
                                                          const Workspace ws) {
  const int e = threadIdx.x;
  const int n_edges = n_positions * top_k;
  const uint8_t* key = nullptr;
  if (e < n_edges) {
    key = bank + (uint64_t)ws.ids[e] * stride;
    ws.epos[e] = e / top_k;
  }
  if (e <= n_positions) ws.poff[e] = e * top_k;
  plan_core(key, e, n_edges, n_positions, ws);
}

__global__ __launch_bounds__(256) void k_verify_plan_table(const EdgeTable tbl,
                                                           const Workspace ws) {
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

// ======================================================================
// verify phase A: one workgroup per (unique expert, 32-row block); the
// expert's positions are staged in LDS a group at a time
// ======================================================================
template <typename XT>
struct VerifyA {
  static constexpr int kGroup = sizeof(XT) == 2 ? 4 : 2;
};

template <typename XT, int kRows>
__global__ __launch_bounds__(256) void k_glu_verify(const Geo g, const XT* __restrict__ x,
                                                    const Workspace ws) {
  extern __shared__ uint4 smem_va[];
  XT* xs = reinterpret_cast<XT*>(smem_va);
  constexpr int kG = VerifyA<XT>::kGroup;
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
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
  const int wave = threadIdx.x >> 6;
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
  for (int e = ws.poff[p]; e < ws.poff[p + 1]; ++e)
    acc += ws.w[e] * ws.y[(size_t)e * hidden + col];
  store_out(out + i, acc);
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
constexpr int kRowsGlu = 8;
constexpr int kRowsVerifyA = 8;
constexpr int kRowsVerifyB = 16;

bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

int launched(const char* what) {
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? K3_HIP_OK : hip_fail(what, e);
}

template <typename XT, typename OT>
int gemv1_dispatch(const uint8_t* p, const uint8_t* s, const XT* x, OT* y, int rows, int cols,
                   hipStream_t st) {
  const int G = cols / 32;
  const int cpl = (G + 63) / 64;
  const int waves = (rows + kRowsGemv - 1) / kRowsGemv;
  const dim3 grid((waves + 3) / 4), block(256);
  switch (cpl) {
    case 1: hipLaunchKernelGGL((k_gemv1<XT, OT, 1, kRowsGemv>), grid, block, 0, st, p, s, x, y, rows, cols); break;
    case 2: hipLaunchKernelGGL((k_gemv1<XT, OT, 2, kRowsGemv>), grid, block, 0, st, p, s, x, y, rows, cols); break;
    case 3: hipLaunchKernelGGL((k_gemv1<XT, OT, 3, kRowsGemv>), grid, block, 0, st, p, s, x, y, rows, cols); break;
    case 4: hipLaunchKernelGGL((k_gemv1<XT, OT, 4, kRowsGemv>), grid, block, 0, st, p, s, x, y, rows, cols); break;
    default: return -1;  // caller falls back to the LDS kernel
  }
  return launched("mxfp4 GEMV launch");
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
  hipLaunchKernelGGL((k_gemv_multi<XT, OT, kRowsGemv>), dim3((waves + 3) / 4), dim3(256),
                     (unsigned)(group * per), st, p, s, x, y, rows, cols, batches, group);
  return launched("mxfp4 GEMV (multi) launch");
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
  hipLaunchKernelGGL(k_activate, dim3((unsigned)blocks), dim3(256), 0, st, gate, up, h, n, act);
  return launched("activation launch");
}

int launch_route(const float* logits, int n_bank, int top_k, int n_positions, int32_t* ids_ws,
                 float* w_ws, int32_t* ids_user, float* w_user, hipStream_t st) {
  if (!logits) return fail(K3_HIP_E_INVALID, "router: null logits");
  if (n_bank <= 0 || n_bank > 16384)
    return fail(K3_HIP_E_INVALID, "router: n_bank must be in [1, 16384]");
  if (top_k <= 0 || top_k > K3_HIP_MAX_TOKEN_EXPERTS || top_k > n_bank)
    return fail(K3_HIP_E_INVALID, "router: top_k must be in [1, min(%d, n_bank)]",
                K3_HIP_MAX_TOKEN_EXPERTS);
  hipLaunchKernelGGL(k_route, dim3(n_positions), dim3(256), (unsigned)(n_bank * sizeof(float)),
                     st, logits, n_bank, top_k, ids_ws, w_ws, ids_user, w_user);
  return launched("router launch");
}

namespace {

template <typename XT>
int glu_decode_dispatch(const Geo& g, const TokenRoute& route, const XT* x, float* h,
                        hipStream_t st) {
  const int G = g.hidden / 32;
  const int cpl = (G + 63) / 64;
  const int units = route.n * (g.inter / kRowsGlu);
  const dim3 grid((units + 3) / 4), block(256);
  switch (cpl) {
    case 1: hipLaunchKernelGGL((k_glu_decode<XT, 1, kRowsGlu>), grid, block, 0, st, route, g, x, h); break;
    case 2: hipLaunchKernelGGL((k_glu_decode<XT, 2, kRowsGlu>), grid, block, 0, st, route, g, x, h); break;
    case 3: hipLaunchKernelGGL((k_glu_decode<XT, 3, kRowsGlu>), grid, block, 0, st, route, g, x, h); break;
    case 4: hipLaunchKernelGGL((k_glu_decode<XT, 4, kRowsGlu>), grid, block, 0, st, route, g, x, h); break;
    default: return fail(K3_HIP_E_INVALID, "decode layer: hidden %d exceeds 8192", g.hidden);
  }
  return launched("decode gate/up launch");
}

template <typename OT>
int down_decode_dispatch(const Geo& g, const TokenRoute& route, const float* h, OT* out,
                         hipStream_t st) {
  const int GB = g.inter / 32;
  const int cplb = (GB + 63) / 64;
  const int cus = std::max(1, device_cu_count());
  int rpb = (g.hidden + cus - 1) / cus;
  rpb = std::min(std::max(rpb, 1), kDownMaxRows);
  const int blocks = (g.hidden + rpb - 1) / rpb;
  const int nw = std::min(route.n, 16);
  const dim3 grid(blocks), block(64 * nw);
  switch (cplb) {
    case 1: hipLaunchKernelGGL((k_down_decode<OT, 1>), grid, block, 0, st, route, g, h, out, rpb); break;
    case 2: hipLaunchKernelGGL((k_down_decode<OT, 2>), grid, block, 0, st, route, g, h, out, rpb); break;
    case 3: hipLaunchKernelGGL((k_down_decode<OT, 3>), grid, block, 0, st, route, g, h, out, rpb); break;
    case 4: hipLaunchKernelGGL((k_down_decode<OT, 4>), grid, block, 0, st, route, g, h, out, rpb); break;
    default: return fail(K3_HIP_E_INVALID, "decode layer: intermediate %d exceeds 8192", g.inter);
  }
  return launched("decode down/combine launch");
}

}  // namespace

int launch_decode_layer(const Geo& g, const TokenRoute& route, const void* x, int x_dtype,
                        void* out, int out_dtype, const Workspace& ws, hipStream_t st) {
  if (route.n <= 0 || route.n > K3_HIP_MAX_TOKEN_EXPERTS)
    return fail(K3_HIP_E_INVALID, "decode layer: expert count %d outside [1, %d]", route.n,
                K3_HIP_MAX_TOKEN_EXPERTS);
  if (g.inter % kRowsGlu != 0) return fail(K3_HIP_E_INVALID, "decode layer: bad intermediate");
  int rc = x_dtype == K3_DTYPE_BF16
               ? glu_decode_dispatch<uint16_t>(g, route, static_cast<const uint16_t*>(x), ws.h, st)
               : glu_decode_dispatch<float>(g, route, static_cast<const float*>(x), ws.h, st);
  if (rc != K3_HIP_OK) return rc;
  return out_dtype == K3_DTYPE_BF16
             ? down_decode_dispatch<uint16_t>(g, route, ws.h, static_cast<uint16_t*>(out), st)
             : down_decode_dispatch<float>(g, route, ws.h, static_cast<float*>(out), st);
}

int launch_verify_plan_bank(const Geo& g, const uint8_t* bank, uint64_t stride, int n_positions,
                            int top_k, const Workspace& ws, hipStream_t st) {
  (void)g;
  hipLaunchKernelGGL(k_verify_plan_bank, dim3(1), dim3(256), 0, st, bank, stride, n_positions,
                     top_k, ws);
  return launched("verify plan launch");
}

int launch_verify_plan_table(const EdgeTable& table, const Workspace& ws, hipStream_t st) {
  hipLaunchKernelGGL(k_verify_plan_table, dim3(1), dim3(256), 0, st, table, ws);
  return launched("verify plan launch");
}

namespace {

template <typename XT>
int glu_verify_dispatch(const Geo& g, int n_edges, const XT* x, const Workspace& ws,
                        hipStream_t st) {
  constexpr int kG = VerifyA<XT>::kGroup;
  const size_t lds = (size_t)kG * g.hidden * sizeof(XT);
  if (lds > 96 * 1024) return fail(K3_HIP_E_INVALID, "verify: hidden %d too wide", g.hidden);
  const int upe = g.inter / (4 * kRowsVerifyA);
  hipLaunchKernelGGL((k_glu_verify<XT, kRowsVerifyA>), dim3(upe * n_edges), dim3(256),
                     (unsigned)lds, st, g, x, ws);
  return launched("verify gate/up launch");
}

int down_verify_dispatch(const Geo& g, int n_edges, const Workspace& ws, hipStream_t st) {
  const int GB = g.inter / 32;
  const int cplb = (GB + 63) / 64;
  const int upe = (g.hidden + 4 * kRowsVerifyB - 1) / (4 * kRowsVerifyB);
  const dim3 grid(upe * n_edges), block(256);
  switch (cplb) {
    case 1: hipLaunchKernelGGL((k_down_verify<1, kRowsVerifyB>), grid, block, 0, st, g, ws); break;
    case 2: hipLaunchKernelGGL((k_down_verify<2, kRowsVerifyB>), grid, block, 0, st, g, ws); break;
    case 3: hipLaunchKernelGGL((k_down_verify<3, kRowsVerifyB>), grid, block, 0, st, g, ws); break;
    case 4: hipLaunchKernelGGL((k_down_verify<4, kRowsVerifyB>), grid, block, 0, st, g, ws); break;
    default: return fail(K3_HIP_E_INVALID, "verify: intermediate %d exceeds 8192", g.inter);
  }
  return launched("verify down launch");
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
  const int64_t n = (int64_t)g.hidden * n_positions;
  const dim3 grid((unsigned)((n + 255) / 256)), block(256);
  if (out_dtype == K3_DTYPE_BF16)
    hipLaunchKernelGGL(k_combine_positions<uint16_t>, grid, block, 0, st, ws, g.hidden,
                       n_positions, static_cast<uint16_t*>(out));
  else
    hipLaunchKernelGGL(k_combine_positions<float>, grid, block, 0, st, ws, g.hidden, n_positions,
                       static_cast<float*>(out));
  return launched("verify combine launch");
}

int launch_synth_bank(const Geo& g, uint8_t* bank, uint64_t stride, int n_experts,
                      uint64_t first_expert, uint64_t seed, int lo, int hi, hipStream_t st) {
  if (!bank || n_experts <= 0 || n_experts > 65535 || stride < g.span || stride % 8 != 0 ||
      ((uintptr_t)bank & 7u) != 0 || lo < 0 || hi > 255 || lo > hi)
    return fail(K3_HIP_E_INVALID, "synth bank: invalid arguments");
  hipLaunchKernelGGL(k_synth_bank, dim3(1024, n_experts), dim3(256), 0, st, g, bank, stride,
                     first_expert, seed, lo, hi);
  return launched("synth bank launch");
}

int launch_synth_normal(void* out, int dtype, uint64_t n, uint64_t seed, uint64_t stream_id,
                        hipStream_t st) {
  if (!out || (dtype != K3_DTYPE_F32 && dtype != K3_DTYPE_BF16))
    return fail(K3_HIP_E_INVALID, "synth normal: invalid arguments");
  if (n == 0) return K3_HIP_OK;
  const uint64_t blocks = std::min<uint64_t>((n + 255) / 256, 4096);
  hipLaunchKernelGGL(k_synth_normal, dim3((unsigned)blocks), dim3(256), 0, st, out, dtype, n, seed,
                     stream_id);
  return launched("synth normal launch");
}

}  // namespace k3
