// Batched speculative verify on CDNA4's block-scaled matrix cores.
//
// The reference runs verify one routed expert at a time and re-reads that
// expert's rows for every token that chose it (tools/cuda_moe_kernels.cu:110-124,
// provider_cuda_moe.cpp:1010-1164).  Here the verify plan (k_verify_plan_*)
// groups the batch's edges by expert span, and each unique expert's bytes are
// streamed from HBM once for all of its tokens, as a small-M contraction on
// v_mfma_scale_f32_16x16x128_f8f6f4:
//
//   A (16 x 128) = 16 weight rows, MXFP4 exactly as stored: lane l holds row
//                  l % 16, 32-element block l / 16 of the K step = one 16-byte
//                  chunk of the row, with that chunk's E8M0 byte as its scale.
//                  No dequantisation instruction touches the weights.
//   B (128 x 16) = up to 16 tokens' activations as fp8 E4M3 terms with one
//                  E8M0 scale per 32 elements.  Lane l (token l % 16, g = l / 16)
//                  holds two 16-element runs of the K step, K = 16 g .. 16 g + 15
//                  in bytes 0-15 and K = 64 + 16 g .. + 15 in bytes 16-31, and
//                  the scale of block g (K = 32 g .. 32 g + 31).  With an fp4 A
//                  operand this is how gfx950 pairs the operands (measured on
//                  the device: lane group g of A meets bytes 16 (g / 2) + j % 16
//                  of B lane group 2 (g % 2) + j / 16 for its nibble j).
//                  An activation row is split into T terms (k_split_terms):
//                  bf16 x is exact in two, fp32 rows (fp32 x, h) keep about 12
//                  bits in three.
//   D (16 x 16)  = fp32, lane l: token l % 16, rows 4 (l / 16) .. + 3.
// The unit sums a K step's products at about 2^-14 of its largest product
// (measured), far inside the 1e-3 output bar.
//
// Phase A (gate/up) produces h[edge][I] (activation in the epilogue), h is
// split into terms, phase B (down) produces y[edge][H], and the per-position
// route-ordered combine (k_combine_positions) forms the outputs.
#include <stdint.h>

#include <algorithm>

#include "k3_device.h"
#include "k3_internal.h"
#include "k3_launch.h"

namespace k3 {

typedef int v8i __attribute__((ext_vector_type(8)));
typedef float v4f __attribute__((ext_vector_type(4)));

// ======================================================================
// fp8 E4M3 (OCP, as gfx950's f8f6f4 operands read it) for |y| < 256
// ======================================================================
// Round to nearest even.  Normal codes: exponent field E + 7 for
// y in [2^E, 2^(E+1)), 3 mantissa bits; below 2^-6 the subnormal codes are
// multiples of 2^-9.  The caller keeps |y| < 256, so no code reaches the NaN
// pattern 0x7f (256 itself is 0x78).
__device__ __forceinline__ uint32_t e4m3_rne(float y) {
  const uint32_t sign = (__float_as_uint(y) >> 24) & 0x80u;
  const float a = fabsf(y);
  if (a < 0x1p-6f) return sign | (uint32_t)rintf(a * 512.0f);  // 0..8; 8 = 2^-6
  int e = (int)(__float_as_uint(a) >> 23) - 127;
  uint32_t q = (uint32_t)rintf(a * __uint_as_float((uint32_t)(127 + 3 - e) << 23));  // 8..16
  if (q == 16u) {
    q = 8u;
    ++e;
  }
  return sign | ((uint32_t)(e + 7) << 3) | (q - 8u);
}

__device__ __forceinline__ float e4m3_value(uint32_t b) {
  const uint32_t f = (b >> 3) & 15u, m = b & 7u;
  const float v = f == 0u ? (float)m * 0x1p-9f
                          : (float)(8u + m) * __uint_as_float((uint32_t)(127 + (int)f - 10) << 23);
  return (b & 0x80u) ? -v : v;
}

// ======================================================================
// split activation rows into fp8 terms
// ======================================================================
// Four lanes per 32-element block, eight elements per lane.  Term t of a
// block takes the block's remainder r (r = the row for t = 0): its scale is
// 2^se with se = floor(log2 max|r|) - 7 (so |r| / 2^se < 256), its codes are
// RNE(r / 2^se), and r minus the decoded term (exact: the term is within a
// factor of two of r, or zero) carries to the next term.  A non-finite block
// becomes NaN codes in term 0.
template <typename SrcT>
__device__ __forceinline__ void load8(const SrcT* p, float* v);

template <>
__device__ __forceinline__ void load8<uint16_t>(const uint16_t* p, float* v) {
  const uint4 w = *reinterpret_cast<const uint4*>(p);
  const uint32_t d[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    v[2 * i] = __uint_as_float(d[i] << 16);
    v[2 * i + 1] = __uint_as_float(d[i] & 0xffff0000u);
  }
}

template <>
__device__ __forceinline__ void load8<float>(const float* p, float* v) {
  const float4 a = reinterpret_cast<const float4*>(p)[0];
  const float4 b = reinterpret_cast<const float4*>(p)[1];
  v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
  v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
}

template <int T, typename SrcT>
__global__ __launch_bounds__(256) void k_split_terms(const SrcT* __restrict__ src, int n_rows,
                                                     int K, uint8_t* __restrict__ q,
                                                     uint8_t* __restrict__ qs) {
  const int gb = K >> 5;
  const int idx = blockIdx.x * blockDim.x + threadIdx.x;
  const int blk = idx >> 2, sub = idx & 3;
  const bool active = blk < n_rows * gb;
  const int row = active ? blk / gb : 0;
  const int j = active ? blk - row * gb : 0;
  float v[8];
  if (active) {
    load8<SrcT>(src + (size_t)row * K + 32 * j + 8 * sub, v);
  } else {
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] = 0.0f;
  }
  bool finite = true;
#pragma unroll
  for (int i = 0; i < 8; ++i) finite = finite && isfinite(v[i]);
  // every lane of the block learns whether the block is finite
  int nf = finite ? 0 : 1;
  nf |= __shfl_xor(nf, 1);
  nf |= __shfl_xor(nf, 2);
#pragma unroll
  for (int t = 0; t < T; ++t) {
    float m = 0.0f;
#pragma unroll
    for (int i = 0; i < 8; ++i) m = fmaxf(m, fabsf(v[i]));
    m = fmaxf(m, __shfl_xor(m, 1));
    m = fmaxf(m, __shfl_xor(m, 2));
    const uint32_t mb = __float_as_uint(m);
    const int e = mb >= 0x00800000u ? (int)(mb >> 23) - 127
                                    : (mb == 0u ? -200 : 31 - (int)__clz(mb) - 149);
    const int se = max(e - 7, -127);  // e <= 127, so se <= 120
    const float inv = __uint_as_float((uint32_t)(127 - se) << 23);  // 2^-se, normal
    // 2^se: normal for se >= -126, the subnormal 2^-127 otherwise
    const float fwd = se >= -126 ? __uint_as_float((uint32_t)(127 + se) << 23) : 0x1p-127f;
    uint32_t lo = 0u, hi = 0u;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      uint32_t c;
      if (nf) {
        c = t == 0 ? 0x7fu : 0u;
      } else {
        c = e4m3_rne(v[i] * inv);
        v[i] -= e4m3_value(c) * fwd;
      }
      if (i < 4)
        lo |= c << (8 * i);
      else
        hi |= c << (8 * (i - 4));
    }
    if (active) {
      const size_t o = ((size_t)row * T + t) * K + 32 * j + 8 * sub;
      *reinterpret_cast<uint2*>(q + o) = make_uint2(lo, hi);
      if (sub == 0) qs[((size_t)row * T + t) * gb + j] = (uint8_t)(nf ? 127 : se + 127);
    }
  }
}

// ======================================================================
// unique-expert units on the matrix cores
// ======================================================================
// A unit is (unique expert u, block of 16 NT rows) of one matrix (down) or of
// both gate and up (phase A).  A workgroup is S column-split waves: wave w
// covers K steps [w KS, (w + 1) KS) of every row, KS = K / (128 S).
// Workgroup b takes units b, b + NWG, ... and each wave walks the flattened
// (unit, K-step pair) items with two items in flight: item i + 1 is requested
// before item i is multiplied.  An item takes two adjacent K steps, so the
// two 64-byte halves of each 128-byte line of a weight row are requested
// back to back (one K step per item fetched every line twice: its halves
// were requested a whole item apart and the line was gone from L2 in
// between).  At a unit's last item every wave writes its tiles' partial sums
// to LDS (two slots by unit parity, one barrier per unit) and wave w sums
// tile w (w + S, ...) over the waves in wave order, applies the activation
// (phase A) and stores its tokens' rows.
//
// Every address is in range by construction: units are below U * n_rb,
// rows below the matrix's rows, K steps below K / 128, and lanes whose token
// column is empty read token 0's activation row (their columns are never
// stored).
struct MfmaPlan {
  const uint8_t* uptr[K3_HIP_MAX_EDGES];
  int uoff[K3_HIP_MAX_EDGES + 1];
  int brow[K3_HIP_MAX_EDGES];  // activation row of the i-th grouped edge
  int orow[K3_HIP_MAX_EDGES];  // output row (the edge) of the i-th grouped edge
};

// Loads of one item: KI adjacent K steps from ks.  Scale dwords hold the 4
// block scales of one K step for the lane's row (weights) or token
// (activations); lane group g takes byte g.
// Scale block of a wave's unit: its rows' E8M0 bytes for its K steps, KS
// dwords per row (one per K step), kTiles * 16 * KS dwords in all, loaded as
// dwords by the whole wave at the unit's first item (at most kScaleLoads per
// lane) and parked in the wave's LDS region as [tile][row][K step].
constexpr int kScaleLoads = 16;

template <int kTiles, int KI>
struct MfmaA {  // weights: streamed from HBM, two items in flight
  u32x4 a[kTiles][KI];
  uint32_t sblk[kScaleLoads];  // the unit's scale block (first item of a unit)
};
template <int T, int KI>
struct MfmaB {  // activation terms: L2-resident, one item ahead
  u32x4 b[T][KI][2];  // [term][K step][K runs 16 g.. and 64 + 16 g..]
  uint32_t sb[T][KI];
};

__device__ __forceinline__ v8i a_operand(u32x4 w) {
  v8i r = {(int)w.x, (int)w.y, (int)w.z, (int)w.w, 0, 0, 0, 0};
  return r;
}

__device__ __forceinline__ v8i b_operand(u32x4 lo, u32x4 hi) {
  v8i r = {(int)lo.x, (int)lo.y, (int)lo.z, (int)lo.w, (int)hi.x, (int)hi.y, (int)hi.z, (int)hi.w};
  return r;
}

// Activation terms are re-read by every unit of their expert: ordinary
// (cached) loads, unlike the streamed weight chunks.
__device__ __forceinline__ u32x4 load_b16(const uint8_t* p) { return *(gu32x4*)(p); }

typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef __attribute__((address_space(1))) const u32x2 gu32x2;

// KI scale dwords from p (4 KI-byte aligned): one per K step.
template <int KI>
__device__ __forceinline__ void load_scales(uint32_t (&d)[KI], const uint8_t* p) {
  static_assert(KI == 2 || KI == 4, "two or four K steps per item");
  if constexpr (KI == 2) {
    const u32x2 v = *(gu32x2*)(p);
    d[0] = v.x;
    d[1] = v.y;
  } else {
    const u32x4 v = *(gu32x4*)(p);
    d[0] = v.x;
    d[1] = v.y;
    d[2] = v.z;
    d[3] = v.w;
  }
}

template <bool kGlu, int NT, int T, int KI>
__global__ __launch_bounds__(256, 2) void k_verify_mfma(const Geo g, const Workspace ws,
                                                        const uint8_t* __restrict__ bq,
                                                        const uint8_t* __restrict__ bqs,
                                                        int n_brows, float* __restrict__ out) {
  constexpr int kM = kGlu ? 2 : 1;
  constexpr int kTiles = kM * NT;
  extern __shared__ v4f red[];  // [2][S][kTiles][64] sums, then [S][64 * kScaleLoads] scales
  __shared__ MfmaPlan pl;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int S = blockDim.x >> 6;
  const int r16 = lane & 15, qb = lane >> 4;
  const int K = kGlu ? g.hidden : g.inter;
  const int rows = kGlu ? g.inter : g.hidden;
  const int KS = (K >> 7) / S;  // a multiple of KI (host check)
  const int KP = KS / KI;       // items per wave and unit
  const int n_rb = rows / (16 * NT);
  const size_t rowb = (size_t)K >> 1, srowb = (size_t)K >> 5;
  const uint64_t wp[2] = {kGlu ? g.w1p : g.w2p, g.w3p};
  const uint64_t wsc[2] = {kGlu ? g.w1s : g.w2s, g.w3s};

  const int U = min(ws.plan->n_unique, K3_HIP_MAX_EDGES);
  const int n_edges = min(ws.plan->n_edges, K3_HIP_MAX_EDGES);
  for (int i = threadIdx.x; i < U; i += blockDim.x) pl.uptr[i] = ws.uptr[i];
  for (int i = threadIdx.x; i <= U; i += blockDim.x) pl.uoff[i] = min(max(ws.uoff[i], 0), n_edges);
  for (int i = threadIdx.x; i < n_edges; i += blockDim.x) {
    const int e = min(max(ws.uedges[i], 0), n_edges - 1);
    pl.orow[i] = e;
    pl.brow[i] = min(max(kGlu ? ws.epos[e] : e, 0), n_brows - 1);
  }
  __syncthreads();
  const int n_units = U * n_rb;
  const int NWG = gridDim.x;
  const int b0 = blockIdx.x;
  if (b0 >= n_units) return;  // whole workgroup
  const int iters = (n_units - b0 + NWG - 1) / NWG;
  const int n_items = iters * KP;

  typedef MfmaA<kTiles, KI> ItemA;
  typedef MfmaB<T, KI> ItemB;
  // Loads address a wave-uniform base (scalar registers: the expert's span,
  // the activation terms) plus a 32-bit per-lane offset, so each load needs
  // one VGPR of address instead of two.
  const uint32_t a_lane = (uint32_t)(r16 * rowb) + 16u * qb;  // + row block, tile, K step
  auto load_b = [&](ItemB& it, int i) {
    const int ui = i / KP;
    const int unit = b0 + ui * NWG;
    const int ks = wave * KS + KI * (i - ui * KP);
    const int uid = unit / n_rb;
    const int e0 = pl.uoff[uid], m = pl.uoff[uid + 1] - e0;
    const bool tok = r16 < m;
    const int brow = pl.brow[min(e0 + (tok ? r16 : 0), n_edges - 1)];
    const uint32_t boff = (uint32_t)(brow * T * K) + 128u * ks + 16u * qb;
    const uint32_t bsoff = (uint32_t)(brow * T * (int)srowb) + 4u * ks;
#pragma unroll
    for (int t = 0; t < T; ++t) {
      if (tok) {
#pragma unroll
        for (int k = 0; k < KI; ++k) {
          it.b[t][k][0] = load_b16(bq + (boff + (uint32_t)(t * K + 128 * k)));
          it.b[t][k][1] = load_b16(bq + (boff + (uint32_t)(t * K + 128 * k) + 64u));
        }
        load_scales<KI>(it.sb[t], bqs + (bsoff + (uint32_t)(t * (int)srowb)));
      } else {
#pragma unroll
        for (int k = 0; k < KI; ++k) {
          it.b[t][k][0] = u32x4{0u, 0u, 0u, 0u};
          it.b[t][k][1] = u32x4{0u, 0u, 0u, 0u};
          it.sb[t][k] = 0u;
        }
      }
    }
  };
  // Scale block addressing: dword j*64 + lane of the block is tile
  // idx / (16 KS), row (idx / KS) % 16, K step idx % KS of the wave's range.
  const int n_sdw = kTiles * 16 * KS;  // <= 64 * kScaleLoads (host check)
  auto load_a = [&](ItemA& it, int i) {
    const int ui = i / KP;
    const int unit = b0 + ui * NWG;
    const int kp = i - ui * KP;
    const int ks = wave * KS + KI * kp;
    const int uid = unit / n_rb;
    const int rb = unit - uid * n_rb;
    const uint8_t* span = uniform_ptr(pl.uptr[uid]);
    const uint32_t rbase = (uint32_t)rb * 16u * NT;
    if (kp == 0) {
#pragma unroll
      for (int j = 0; j < kScaleLoads; ++j) {
        const int idx = 64 * j + lane;
        if (64 * j < n_sdw) {
          const int ii = min(idx, n_sdw - 1);
          const int t = ii / (16 * KS), rem = ii - t * 16 * KS;
          const int row = rem / KS, d = rem - row * KS;
          const int mt = t / NT, tt = t - mt * NT;
          it.sblk[j] = load_u32(span + ((uint32_t)wsc[mt] +
                                        (rbase + 16u * tt + row) * (uint32_t)srowb +
                                        4u * (wave * KS + d)));
        }
      }
    }
#pragma unroll
    for (int mt = 0; mt < kM; ++mt) {
#pragma unroll
      for (int t = 0; t < NT; ++t) {
        const uint32_t r = rbase + 16u * t;
        const uint32_t ao = (uint32_t)wp[mt] + r * (uint32_t)rowb + 64u * ks + a_lane;
#pragma unroll
        for (int k = 0; k < KI; ++k) it.a[mt * NT + t][k] = load_chunk(span + (ao + 64u * k));
      }
    }
  };

  v4f acc[kTiles];
  auto epilogue = [&](int ui) {
    const int unit = b0 + ui * NWG;
    const int par = ui & 1;
    v4f* mine = red + (size_t)(par * S + wave) * kTiles * 64;
#pragma unroll
    for (int t = 0; t < kTiles; ++t) mine[t * 64 + lane] = acc[t];
    lds_barrier();
    const int uid = unit / n_rb;
    const int rb = unit - uid * n_rb;
    const int e0 = pl.uoff[uid], m = pl.uoff[uid + 1] - e0;
    if (r16 < m) {
      const int orow = pl.orow[min(e0 + r16, n_edges - 1)];
      const v4f* slot = red + (size_t)(par * S) * kTiles * 64;
      for (int t = wave; t < NT; t += S) {
        v4f s0 = slot[t * 64 + lane];
        for (int w = 1; w < S; ++w) s0 += slot[((size_t)w * kTiles + t) * 64 + lane];
        float4 o;
        if constexpr (kGlu) {
          v4f s1 = slot[(NT + t) * 64 + lane];
          for (int w = 1; w < S; ++w) s1 += slot[((size_t)w * kTiles + NT + t) * 64 + lane];
          o = make_float4(activate(g.act, s0[0], s1[0]), activate(g.act, s0[1], s1[1]),
                          activate(g.act, s0[2], s1[2]), activate(g.act, s0[3], s1[3]));
        } else {
          o = make_float4(s0[0], s0[1], s0[2], s0[3]);
        }
        *reinterpret_cast<float4*>(out + (size_t)orow * rows + (size_t)rb * 16 * NT + 16 * t +
                                   4 * qb) = o;
      }
    }
  };

  const uint32_t sh = 8u * qb;  // this lane group's byte in each scale dword
  uint32_t* sblk_lds = reinterpret_cast<uint32_t*>(red + (size_t)2 * S * kTiles * 64) +
                       (size_t)wave * 64 * kScaleLoads;
  auto compute = [&](const ItemA& ia, const ItemB& ib, int i) {
    const int ui = i / KP;
    const int kp = i - ui * KP;
    if (kp == 0) {
#pragma unroll
      for (int t = 0; t < kTiles; ++t) acc[t] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
      for (int j = 0; j < kScaleLoads; ++j)
        if (64 * j < n_sdw) sblk_lds[64 * j + lane] = ia.sblk[j];
    }
    uint32_t sa_w[kTiles][KI];
#pragma unroll
    for (int t = 0; t < kTiles; ++t) {
      const uint32_t* src = sblk_lds + (t * 16 + r16) * KS + KI * kp;
#pragma unroll
      for (int k = 0; k < KI; ++k) sa_w[t][k] = src[k];
    }
#pragma unroll
    for (int k = 0; k < KI; ++k) {
#pragma unroll
      for (int t = 0; t < kTiles; ++t) {
        const int sa = (int)((sa_w[t][k] >> sh) & 0xffu);
#pragma unroll
        for (int j = 0; j < T; ++j) {
          const int sb = (int)((ib.sb[j][k] >> sh) & 0xffu);
          acc[t] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(
              a_operand(ia.a[t][k]), b_operand(ib.b[j][k][0], ib.b[j][k][1]), acc[t],
              4 /* A: fp4 */, 0 /* B: fp8 e4m3 */, 0, sa, 0, sb);
        }
      }
    }
    if (kp == KP - 1) epilogue(ui);
  };

  // Issue order per item: activation terms of item i + 1, then weights of
  // item i + 2.  Waiting for item i + 1's terms (loads complete in order)
  // then leaves item i + 2's weights in flight, so the weight stream stays
  // two items deep while the terms need one buffer.
  ItemA A0, A1;
  ItemB Bc;
  load_b(Bc, 0);
  load_a(A0, 0);
  load_a(A1, min(1, n_items - 1));
  for (int i = 0;; i += 2) {
    compute(A0, Bc, i);
    if (i + 1 >= n_items) break;
    load_b(Bc, i + 1);
    if (i + 2 < n_items) load_a(A0, i + 2);
    compute(A1, Bc, i + 1);
    if (i + 2 >= n_items) break;
    load_b(Bc, i + 2);
    if (i + 3 < n_items) load_a(A1, i + 3);
  }
}

// ======================================================================
// host side
// ======================================================================
namespace {

#ifndef K3_MFMA_KI
#define K3_MFMA_KI 2
#endif
constexpr int kItemSteps = K3_MFMA_KI;  // K steps per item (2 or 4)
// 16-row tiles per unit: of gate and of up, and of down.  Each keeps two
// items of weights and one of activation terms within the 256 VGPRs of two
// waves per SIMD without spilling (8 KB of weights per item).
template <bool kGlu, int T>
constexpr int unit_tiles() {
  return kGlu ? 2 : 4;
}

// Column-split waves for K = k_elems: the most (up to max_s) that leave every
// wave a whole number of items.
#ifndef K3_MFMA_GLU_WAVES
#define K3_MFMA_GLU_WAVES 4
#endif
#ifndef K3_MFMA_DOWN_WAVES
#define K3_MFMA_DOWN_WAVES 1  // down rows have K = intermediate: longer units per wave
#endif
// Column-split waves for K = k_elems and kTiles tiles per unit: the preferred
// max_s if every wave gets a whole number of items and its scale block fits,
// else the nearest wider split that does, else the nearest narrower; 0 if
// none of 1, 2, 4 does.
int mfma_waves(int k_elems, int k_tiles, int max_s) {
  const int nk = k_elems / 128;
  auto ok = [&](int s) {
    return nk % (kItemSteps * s) == 0 && k_tiles * 16 * (nk / s) <= 64 * kScaleLoads;
  };
  for (int s = max_s; s <= 4; s <<= 1)
    if (ok(s)) return s;
  for (int s = max_s >> 1; s >= 1; s >>= 1)
    if (ok(s)) return s;
  return 0;
}

template <int T, typename SrcT>
int split_launch(const SrcT* src, int n_rows, int K, uint8_t* q, uint8_t* qs, hipStream_t st) {
  const int64_t threads = (int64_t)n_rows * (K / 32) * 4;
  const dim3 grid((unsigned)((threads + 255) / 256)), block(256);
  TimedLaunch tl(KC_SPLIT, st);
  launch_timed(tl, k_split_terms<T, SrcT>, grid, block, 0, st, src, n_rows, K, q, qs);
  return launched(tl, "verify split launch");
}

template <bool kGlu, int T>
int mfma_launch(const Geo& g, int n_edges, const Workspace& ws, const uint8_t* bq,
                const uint8_t* bqs, int n_brows, float* out, hipStream_t st) {
  constexpr int NT = unit_tiles<kGlu, T>();
  constexpr int kTiles = (kGlu ? 2 : 1) * NT;
  const int rows = kGlu ? g.inter : g.hidden;
  const int S = mfma_waves(kGlu ? g.hidden : g.inter, kTiles,
                          kGlu ? K3_MFMA_GLU_WAVES : K3_MFMA_DOWN_WAVES);
  if (S < 1) return fail(K3_HIP_E_INVALID, "verify: no column split fits this geometry");
  const int max_units = n_edges * (rows / (16 * NT));
  // eight resident waves per CU (two per SIMD, the kernel's register budget)
  const int grid = std::max(1, std::min((8 / S) * std::max(1, device_cu_count()), max_units));
  const unsigned lds = (unsigned)(2 * S * kTiles * 64 * sizeof(v4f) +
                                  (size_t)S * 64 * kScaleLoads * sizeof(uint32_t));
  const void* kfn = reinterpret_cast<const void*>(k_verify_mfma<kGlu, NT, T, kItemSteps>);
  if (!lds_fits(kfn, 64 * S, lds))
    return fail(K3_HIP_E_EXEC, "verify: %u B of LDS per workgroup not available", lds);
  TimedLaunch tl(kGlu ? KC_GLU_MFMA : KC_DOWN_MFMA, st);
  launch_timed(tl, k_verify_mfma<kGlu, NT, T, kItemSteps>, dim3(grid), dim3(64 * S), lds, st, g,
               ws, bq, bqs, n_brows, out);
  return launched(tl, kGlu ? "verify gate/up (mfma) launch" : "verify down (mfma) launch");
}

}  // namespace

bool verify_mfma_supported(const Geo& g) {
  // Whole K-step pairs (256 elements) per column wave, whole units of rows.
  constexpr int kGluTiles = 2 * unit_tiles<true, 2>(), kDownTiles = unit_tiles<false, 3>();
  static_assert(unit_tiles<true, 2>() == unit_tiles<true, 3>(), "one gate/up unit shape");
  return g.layout == K3_LAYOUT_RAW_V1 && g.hidden % 128 == 0 && g.inter % 128 == 0 &&
         g.inter % (16 * unit_tiles<true, 2>()) == 0 && g.hidden % (16 * kDownTiles) == 0 &&
         mfma_waves(g.hidden, kGluTiles, K3_MFMA_GLU_WAVES) > 0 &&
         mfma_waves(g.inter, kDownTiles, K3_MFMA_DOWN_WAVES) > 0;
}

int launch_verify_mfma(const Geo& g, int n_edges, int n_positions, const void* x, int x_dtype,
                       void* out, int out_dtype, const Workspace& ws, hipStream_t st) {
  if (!verify_mfma_supported(g))
    return fail(K3_HIP_E_INVALID, "verify: geometry has no matrix-core path");
  if (n_edges < 1 || n_edges > K3_HIP_MAX_EDGES || n_positions < 1 ||
      n_positions > K3_HIP_MAX_POSITIONS)
    return fail(K3_HIP_E_INVALID, "verify: %d edges over %d positions", n_edges, n_positions);
  int rc;
  if (x_dtype == K3_DTYPE_BF16) {
    rc = split_launch<2>(static_cast<const uint16_t*>(x), n_positions, g.hidden, ws.xq, ws.xqs, st);
    if (rc == K3_HIP_OK) rc = mfma_launch<true, 2>(g, n_edges, ws, ws.xq, ws.xqs, n_positions, ws.h, st);
  } else {
    rc = split_launch<3>(static_cast<const float*>(x), n_positions, g.hidden, ws.xq, ws.xqs, st);
    if (rc == K3_HIP_OK) rc = mfma_launch<true, 3>(g, n_edges, ws, ws.xq, ws.xqs, n_positions, ws.h, st);
  }
  if (rc != K3_HIP_OK) return rc;
  rc = split_launch<3>(static_cast<const float*>(ws.h), n_edges, g.inter, ws.hq, ws.hqs, st);
  if (rc != K3_HIP_OK) return rc;
  rc = mfma_launch<false, 3>(g, n_edges, ws, ws.hq, ws.hqs, n_edges, ws.y, st);
  if (rc != K3_HIP_OK) return rc;
  return launch_verify_combine(g, n_positions, out, out_dtype, ws, st);
}

}  // namespace k3
