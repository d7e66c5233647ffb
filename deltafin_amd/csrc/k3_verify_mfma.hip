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
//                  bf16 x in two (exact for most blocks of 32; an element far
//                  below its block's largest can keep a remainder under the
//                  second term's smallest step: at most 4.5e-7 of the block's
//                  largest element over 44,800 N(0,1) blocks), fp32 rows
//                  (fp32 x, h) keep about 12 bits in three.
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
#include "k3_terms.h"

namespace k3 {

typedef int v8i __attribute__((ext_vector_type(8)));
typedef float v4f __attribute__((ext_vector_type(4)));

// ======================================================================
// split activation rows into fp8 terms (k3_terms.h)
// ======================================================================
template <int T, typename SrcT>
__global__ __launch_bounds__(256) void k_split_terms(const SrcT* __restrict__ src, int n_rows,
                                                     int K, uint8_t* __restrict__ q,
                                                     uint8_t* __restrict__ qs) {
  split_terms_at<T, SrcT>(src, n_rows, K, q, qs, (int)(blockIdx.x * blockDim.x + threadIdx.x));
}

// ======================================================================
// unique-expert units on the matrix cores
// ======================================================================
// A unit is (unique expert u, block of 8 NT rows) of one matrix (down) or of
// both gate and up (phase A).  A workgroup is S column-split waves: wave w
// covers K steps [w KS, (w + 1) KS) of every row, KS = K / (128 S).
// Workgroup b takes units b, b + NWG, ... and each wave walks the flattened
// (unit, K-step pair) items: weights two items ahead, activation terms one.
//
// Parity split.  An MFMA row needs its four lanes (l % 16 equal) to hold the
// same weight row, and a load instruction streams fastest when it covers
// whole 128-byte lines.  Each weight row p of a tile of 8 therefore takes two
// MFMA rows, 2p + h, h = 0 for the even K step of the pair and 1 for the odd
// one: lane l (i = l % 16, g = l / 16) loads row i / 2, K step ks + i % 2,
// block g, and one dwordx4 load of a tile covers 8 rows x one full 128-byte
// line (K steps ks, ks + 1).  Two MFMAs per tile and item use that same A
// register, one with the activation terms of step ks (valid in the even
// rows of its result) and one with those of step ks + 1 (valid in the odd
// rows); lane (q, n) then sums rows 4q + 0 / 4q + 1 and 4q + 2 / 4q + 3 of
// the two accumulators into weight rows 2q and 2q + 1 of the tile for token
// n.  The other rows are never read.
//
// At a unit's last item every wave writes its tiles' partial sums to LDS
// (two slots by unit parity, one barrier per unit) and wave w sums tile w
// (w + S, ...) over the waves in wave order, applies the activation (phase A)
// and stores its tokens' rows.
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

// Scale block of a wave's unit: its rows' E8M0 bytes for its K steps, KS
// dwords per row (one per K step), kTiles * 8 * KS dwords in all, loaded as
// dwords by the whole wave at the unit's first item (at most kScaleLoads per
// lane) and parked in the wave's LDS region as [tile][row][K step].
constexpr int kScaleLoads = 16;

template <int kTiles>
struct MfmaA {  // weights: streamed from HBM, two items in flight
  u32x4 a[kTiles];
};
template <int T>
struct MfmaB {  // activation terms of K steps ks, ks + 1: L2-resident, one item ahead
  u32x4 b[T][2][2];  // [term][K step][K runs 16 g.. and 64 + 16 g..]
  uint32_t sb[T][2];
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

template <bool kGlu, int NT, int T>
__global__ __launch_bounds__(256, 2) void k_verify_mfma(const Geo g, const Workspace ws,
                                                        const uint8_t* __restrict__ bq,
                                                        const uint8_t* __restrict__ bqs,
                                                        int n_brows, float* __restrict__ out) {
  constexpr int kM = kGlu ? 2 : 1;
  constexpr int kTiles = kM * NT;
  extern __shared__ float2 red[];  // [2][S][kTiles][64] sums, then [S][64 * kScaleLoads] scales
  __shared__ MfmaPlan pl;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int S = blockDim.x >> 6;
  const int r16 = lane & 15, qb = lane >> 4;
  const int prow = r16 >> 1, par = r16 & 1;  // weight row in the tile, K-step parity
  const int K = kGlu ? g.hidden : g.inter;
  const int rows = kGlu ? g.inter : g.hidden;
  const int KS = (K >> 7) / S;  // even (host check)
  const int KP = KS >> 1;       // items (K-step pairs) per wave and unit
  const int n_rb = rows / (8 * NT);
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

  typedef MfmaA<kTiles> ItemA;
  typedef MfmaB<T> ItemB;
  // Loads address a wave-uniform base (scalar registers: the expert's span,
  // the activation terms) plus a 32-bit per-lane offset, so each load needs
  // one VGPR of address instead of two.
  const uint32_t a_lane = (uint32_t)(prow * rowb) + 64u * par + 16u * qb;  // + row block, tile, K
  auto load_b = [&](ItemB& it, int i) {
    const int ui = i / KP;
    const int unit = b0 + ui * NWG;
    const int ks = wave * KS + 2 * (i - ui * KP);
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
        for (int k = 0; k < 2; ++k) {
          it.b[t][k][0] = load_b16(bq + (boff + (uint32_t)(t * K + 128 * k)));
          it.b[t][k][1] = load_b16(bq + (boff + (uint32_t)(t * K + 128 * k) + 64u));
        }
        const u32x2 sv = *(gu32x2*)(bqs + (bsoff + (uint32_t)(t * (int)srowb)));
        it.sb[t][0] = sv.x;
        it.sb[t][1] = sv.y;
      } else {
#pragma unroll
        for (int k = 0; k < 2; ++k) {
          it.b[t][k][0] = u32x4{0u, 0u, 0u, 0u};
          it.b[t][k][1] = u32x4{0u, 0u, 0u, 0u};
          it.sb[t][k] = 0u;
        }
      }
    }
  };
  // Scale block addressing: dword j*64 + lane of the block is tile
  // idx / (8 KS), row (idx / KS) % 8, K step idx % KS of the wave's range.
  const int n_sdw = kTiles * 8 * KS;  // <= 64 * kScaleLoads (host check)
  // One scale-block buffer: a unit's block is requested three items ahead of
  // the unit's first item and parked in LDS when that item is multiplied;
  // units are at least three items long (host check), so the next unit's
  // block is requested only after that.
  uint32_t sblk[kScaleLoads];
  auto load_s = [&](int i) {  // i: the first item of a unit
    const int ui = i / KP;
    const int unit = b0 + ui * NWG;
    const int uid = unit / n_rb;
    const int rb = unit - uid * n_rb;
    const uint8_t* span = uniform_ptr(pl.uptr[uid]);
    const uint32_t rbase = (uint32_t)rb * 8u * NT;
#pragma unroll
    for (int j = 0; j < kScaleLoads; ++j) {
      if (64 * j < n_sdw) {
        const int ii = min(64 * j + lane, n_sdw - 1);
        const int t = ii / (8 * KS), rem = ii - t * 8 * KS;
        const int row = rem / KS, d = rem - row * KS;
        const int mt = t / NT, tt = t - mt * NT;
        // A 24-bit multiply (rows and scale-row bytes are below 2^24): the
        // plain 32-bit multiply-add becomes v_mad_u64_u32, whose unused high
        // addend half the allocator placed on the previous load's
        // destination, so every load of the block waited for all loads in
        // flight (vmcnt(0)).
        const uint32_t so = (uint32_t)wsc[mt] + __umul24(rbase + 8u * tt + row, (uint32_t)srowb) +
                            4u * (wave * KS + d);
        sblk[j] = load_u32(span + so);
      }
    }
  };
  auto load_a = [&](ItemA& it, int i) {
    const int ui = i / KP;
    const int unit = b0 + ui * NWG;
    const int ks = wave * KS + 2 * (i - ui * KP);
    const int uid = unit / n_rb;
    const int rb = unit - uid * n_rb;
    const uint8_t* span = uniform_ptr(pl.uptr[uid]);
    const uint32_t rbase = (uint32_t)rb * 8u * NT;
#pragma unroll
    for (int mt = 0; mt < kM; ++mt) {
#pragma unroll
      for (int t = 0; t < NT; ++t) {
        const uint32_t r = rbase + 8u * t;
        it.a[mt * NT + t] =
            load_chunk(span + ((uint32_t)wp[mt] + r * (uint32_t)rowb + 64u * ks + a_lane));
      }
    }
  };

  float2 acc[kTiles];  // weight rows 2 qb and 2 qb + 1 of each tile, token r16
  auto epilogue = [&](int ui) {
    const int unit = b0 + ui * NWG;
    const int slot_par = ui & 1;
    float2* mine = red + (size_t)(slot_par * S + wave) * kTiles * 64;
#pragma unroll
    for (int t = 0; t < kTiles; ++t) mine[t * 64 + lane] = acc[t];
    lds_barrier();
    const int uid = unit / n_rb;
    const int rb = unit - uid * n_rb;
    const int e0 = pl.uoff[uid], m = pl.uoff[uid + 1] - e0;
    if (r16 < m) {
      const int orow = pl.orow[min(e0 + r16, n_edges - 1)];
      const float2* slot = red + (size_t)(slot_par * S) * kTiles * 64;
      for (int t = wave; t < NT; t += S) {
        float2 s0 = slot[t * 64 + lane];
        for (int w = 1; w < S; ++w) {
          const float2 v = slot[((size_t)w * kTiles + t) * 64 + lane];
          s0.x += v.x;
          s0.y += v.y;
        }
        float2 o;
        if constexpr (kGlu) {
          float2 s1 = slot[(NT + t) * 64 + lane];
          for (int w = 1; w < S; ++w) {
            const float2 v = slot[((size_t)w * kTiles + NT + t) * 64 + lane];
            s1.x += v.x;
            s1.y += v.y;
          }
          o = make_float2(activate(g.act, s0.x, s1.x), activate(g.act, s0.y, s1.y));
        } else {
          o = s0;
        }
        *reinterpret_cast<float2*>(out + (size_t)orow * rows + (size_t)rb * 8 * NT + 8 * t +
                                   2 * qb) = o;
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
      for (int t = 0; t < kTiles; ++t) acc[t] = make_float2(0.0f, 0.0f);
#pragma unroll
      for (int j = 0; j < kScaleLoads; ++j)
        if (64 * j < n_sdw) sblk_lds[64 * j + lane] = sblk[j];
    }
    // the A scale of this lane: its weight row, K step 2 kp + par, block qb
    const uint32_t* sa_row = sblk_lds + prow * KS + 2 * kp + par;
    // Per tile: the item's two K steps' products, each over all terms, then the
    // valid rows folded into the tile's accumulator (rows 4 qb + 0 and + 2 of
    // the even step's result, + 1 and + 3 of the odd step's).
#pragma unroll
    for (int t = 0; t < kTiles; ++t) {
      const int sa = (int)((sa_row[t * 8 * KS] >> sh) & 0xffu);
      v4f d[2];
#pragma unroll
      for (int k = 0; k < 2; ++k) {
        d[k] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int j = 0; j < T; ++j) {
          const int sb = (int)((ib.sb[j][k] >> sh) & 0xffu);
          d[k] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(
              a_operand(ia.a[t]), b_operand(ib.b[j][k][0], ib.b[j][k][1]), d[k],
              4 /* A: fp4 */, 0 /* B: fp8 e4m3 */, 0, sa, 0, sb);
        }
      }
      acc[t].x += d[0][0] + d[1][1];
      acc[t].y += d[0][2] + d[1][3];
    }
    if (kp == KP - 1) epilogue(ui);
  };

  // Issue order per item (every path issues the same loads after the terms,
  // so the compiler's wait counts stay exact): the scale block of item i + 3
  // when it starts a unit, the activation terms of item i + 1, the weights
  // of item i + 2 (past the end: the last item again).  Waiting for item
  // i + 1's terms then leaves item i + 2's weights in flight, so the weight
  // stream stays two items deep while the terms need one buffer.
  ItemA A0, A1;
  ItemB Bc;
  auto maybe_load_s = [&](int i) {
    if (i < n_items && i - (i / KP) * KP == 0) load_s(i);
  };
  load_s(0);
  load_b(Bc, 0);
  load_a(A0, 0);
  load_a(A1, min(1, n_items - 1));
  for (int i = 0;; i += 2) {
    compute(A0, Bc, i);
    if (i + 1 >= n_items) break;
    maybe_load_s(i + 3);
    load_b(Bc, i + 1);
    load_a(A0, min(i + 2, n_items - 1));
    compute(A1, Bc, i + 1);
    if (i + 2 >= n_items) break;
    maybe_load_s(i + 4);
    load_b(Bc, i + 2);
    load_a(A1, min(i + 3, n_items - 1));
  }
}

// ======================================================================
// host side
// ======================================================================
namespace {

// 8-row tiles per unit: of gate and of up (4: 32 rows each, with bf16 x's
// two terms and with fp32 x's three), and of down (8: 64 rows; the path
// takes hidden sizes that are multiples of 128, so these units always fit).
// Each keeps two items of weights and one of
// activation terms within the 256 VGPRs of two waves per SIMD without
// spilling (fp32 x at 4 tiles: 253, down at 8: 246).  More weight bytes per
// item measured faster: fp32 x at 2 tiles (16 rows each) ran the K3 block's
// 16-position gate/up at 607-634 µs against 465 µs at 4, and down at 7 tiles
// the preset-2 16-position verify's down at 288-289 µs against 266 at 8.
#ifndef K3_MFMA_GLU3_TILES
#define K3_MFMA_GLU3_TILES 4
#endif
template <bool kGlu, int T>
constexpr int glu_tiles() {
  return T == 2 ? 4 : K3_MFMA_GLU3_TILES;
}
#ifndef K3_MFMA_DOWN_TILES
#define K3_MFMA_DOWN_TILES 8
#endif
constexpr int kDownTiles = K3_MFMA_DOWN_TILES;

#ifndef K3_MFMA_GLU_WAVES
#define K3_MFMA_GLU_WAVES 4
#endif
#ifndef K3_MFMA_DOWN_WAVES
#define K3_MFMA_DOWN_WAVES 2  // down rows have K = intermediate: longer units per wave
#endif

// Column-split waves for K = k_elems and kTiles tiles per unit: the preferred
// max_s if every wave gets a whole number of items and its scale block fits,
// else the nearest wider split that does, else the nearest narrower; 0 if
// none of 1, 2, 4 does.
int mfma_waves(int k_elems, int k_tiles, int max_s) {
  const int nk = k_elems / 128;
  auto ok = [&](int s) {  // whole K-step pairs, at least three per unit, scale block fits
    return nk % (2 * s) == 0 && nk / s >= 6 && k_tiles * 8 * (nk / s) <= 64 * kScaleLoads;
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

template <bool kGlu, int NT, int T>
int mfma_launch(const Geo& g, int n_edges, const Workspace& ws, const uint8_t* bq,
                const uint8_t* bqs, int n_brows, float* out, hipStream_t st) {
  constexpr int kTiles = (kGlu ? 2 : 1) * NT;
  const int rows = kGlu ? g.inter : g.hidden;
  const int S = mfma_waves(kGlu ? g.hidden : g.inter, kTiles,
                          kGlu ? K3_MFMA_GLU_WAVES : K3_MFMA_DOWN_WAVES);
  if (S < 1) return fail(K3_HIP_E_INVALID, "verify: no column split fits this geometry");
  const int max_units = n_edges * (rows / (8 * NT));
  // eight resident waves per CU (two per SIMD, the kernel's register budget)
  const int grid = std::max(1, std::min((8 / S) * std::max(1, device_cu_count()), max_units));
  const unsigned lds = (unsigned)(2 * S * kTiles * 64 * sizeof(float2) +
                                  (size_t)S * 64 * kScaleLoads * sizeof(uint32_t));
  const void* kfn = reinterpret_cast<const void*>(k_verify_mfma<kGlu, NT, T>);
  if (!lds_fits(kfn, 64 * S, lds))
    return fail(K3_HIP_E_EXEC, "verify: %u B of LDS per workgroup not available", lds);
  TimedLaunch tl(kGlu ? KC_GLU_MFMA : KC_DOWN_MFMA, st);
  launch_timed(tl, k_verify_mfma<kGlu, NT, T>, dim3(grid), dim3(64 * S), lds, st, g, ws, bq, bqs,
               n_brows, out);
  return launched(tl, kGlu ? "verify gate/up (mfma) launch" : "verify down (mfma) launch");
}

}  // namespace

bool verify_mfma_supported(const Geo& g) {
  // Whole K-step pairs (256 elements) per column wave, whole units of rows.
  return g.layout == K3_LAYOUT_RAW_V1 && g.hidden % 128 == 0 && g.inter % 128 == 0 &&
         g.inter % (8 * glu_tiles<true, 2>()) == 0 && g.inter % (8 * glu_tiles<true, 3>()) == 0 &&
         g.hidden % (8 * kDownTiles) == 0 &&
         mfma_waves(g.hidden, 2 * glu_tiles<true, 2>(), K3_MFMA_GLU_WAVES) > 0 &&
         mfma_waves(g.hidden, 2 * glu_tiles<true, 3>(), K3_MFMA_GLU_WAVES) > 0 &&
         mfma_waves(g.inter, kDownTiles, K3_MFMA_DOWN_WAVES) > 0;
}

int launch_verify_mfma(const Geo& g, int n_edges, int n_positions, const void* x, int x_dtype,
                       void* out, int out_dtype, const Workspace& ws, hipStream_t st,
                       bool x_split_done) {
  if (!verify_mfma_supported(g))
    return fail(K3_HIP_E_INVALID, "verify: geometry has no matrix-core path");
  if (n_edges < 1 || n_edges > K3_HIP_MAX_EDGES || n_positions < 1 ||
      n_positions > K3_HIP_MAX_POSITIONS)
    return fail(K3_HIP_E_INVALID, "verify: %d edges over %d positions", n_edges, n_positions);
  int rc = K3_HIP_OK;
  if (x_dtype == K3_DTYPE_BF16) {
    if (!x_split_done)
      rc = split_launch<2>(static_cast<const uint16_t*>(x), n_positions, g.hidden, ws.xq, ws.xqs,
                           st);
    if (rc == K3_HIP_OK)
      rc = mfma_launch<true, glu_tiles<true, 2>(), 2>(g, n_edges, ws, ws.xq, ws.xqs, n_positions,
                                                       ws.h, st);
  } else {
    if (!x_split_done)
      rc = split_launch<3>(static_cast<const float*>(x), n_positions, g.hidden, ws.xq, ws.xqs,
                           st);
    if (rc == K3_HIP_OK)
      rc = mfma_launch<true, glu_tiles<true, 3>(), 3>(g, n_edges, ws, ws.xq, ws.xqs, n_positions,
                                                       ws.h, st);
  }
  if (rc != K3_HIP_OK) return rc;
  rc = split_launch<3>(static_cast<const float*>(ws.h), n_edges, g.inter, ws.hq, ws.hqs, st);
  if (rc != K3_HIP_OK) return rc;
  rc = mfma_launch<false, kDownTiles, 3>(g, n_edges, ws, ws.hq, ws.hqs, n_edges, ws.y, st);
  if (rc != K3_HIP_OK) return rc;
  return launch_verify_combine(g, n_positions, out, out_dtype, ws, st);
}

}  // namespace k3
