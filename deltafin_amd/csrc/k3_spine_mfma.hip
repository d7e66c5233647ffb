// Spine projections at 3..16 positions on the BF16 matrix cores
// (v_mfma_f32_16x16x32_bf16), for the MoE block's multi-position calls.
//
// Exactness: every fp32 activation is split into three BF16 terms
// (t0 = bf16(x), t1 = bf16(x - t0), t2 = bf16(x - t0 - t1); each remainder is
// exact in fp32), and BF16 x BF16 products are exact in fp32, so the matrix
// cores form the same products as the fp32 FMA kernels and differ only in the
// summation order (plus the ~2^-24 relative remainder of the third term).
//
// Operand layout (measured on gfx950 with a one-hot probe): A lane l holds
// row l % 16, K = 8 (l / 16) .. +7; B lane l holds column l % 16, the same K;
// D lane l holds column l % 16, rows 4 (l / 16) + 0..3.  The B columns are the
// (position, term) pairs n = 3 p + t of up to 16 positions (NB = ceil(3P/16)
// blocks of 16 columns), prepared once per activation by k_split_bf16_terms in
// B-lane order: terms[nb][s][lane] = 8 BF16 (16 bytes) for K = 32 s + 8 (lane
// / 16) .. +7, with two all-zero steps after the last.
//
// Tiles are parity-split (as in the matrix-core verify kernels): MFMA row
// m = 2 i + par holds weight row i's K elements [32 par, 32 par + 32) of a
// 64-element step, so one dwordx4 load of a wave covers 8 weight rows x a
// whole 128-byte line; chain d0 runs against the step's first 32 B elements
// (valid in the even rows), d1 against the second (odd rows), and the epilogue
// adds the two valid rows.  A workgroup owns one 8-row tile and its S waves
// split the K steps; each wave requests weight pieces kAhead steps ahead and
// activation terms kAheadB steps ahead (clamped loads, so every load is
// unconditional and the wait counts stay exact); steps past a wave's range
// read the zero steps of the term buffer.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <algorithm>

#include "k3_device.h"
#include "k3_launch.h"

namespace k3 {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

#ifndef K3_SPINE_MFMA_TILES
#define K3_SPINE_MFMA_TILES 2
#endif
constexpr int kAhead = 8;           // weight KB in flight per wave (steps x tiles)
constexpr int kAheadB = 4;          // activation-term steps in flight per wave
static_assert(kAhead % kAheadB == 0, "the term ring must index statically");

__device__ __forceinline__ uint16_t bf16_rn_bits(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);  // quiet NaN
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

// One thread per (block nb, K32 step s, lane): 8 BF16 terms of column
// n = 16 nb + lane % 16 -> (position n / 3, term n % 3), zero past 3P columns.
// Steps s = cols / 32 and cols / 32 + 1 are zero (the padding steps).
__global__ __launch_bounds__(256) void k_split_bf16_terms(const float* __restrict__ x, int P,
                                                          int cols, int nb_count,
                                                          uint4* __restrict__ terms) {
  const int steps = cols / 32 + 2;
  const int64_t total = (int64_t)nb_count * steps * 64;
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= total) return;
  const int lane = (int)(i % 64);
  const int s = (int)((i / 64) % steps);
  const int nb = (int)(i / (64 * (int64_t)steps));
  const int n = 16 * nb + (lane & 15);
  const int p = n / 3, t = n % 3;
  uint32_t w[4] = {0u, 0u, 0u, 0u};
  if (p < P && s < cols / 32) {
    const float* xp = x + (int64_t)p * cols + 32 * s + 8 * (lane >> 4);
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float v = xp[e];
      const uint16_t b0 = bf16_rn_bits(v);
      const float r1 = v - __uint_as_float((uint32_t)b0 << 16);
      const uint16_t b1 = bf16_rn_bits(r1);
      const float r2 = r1 - __uint_as_float((uint32_t)b1 << 16);
      const uint16_t b = t == 0 ? b0 : t == 1 ? b1 : bf16_rn_bits(r2);
      w[e >> 1] |= (uint32_t)b << (16 * (e & 1));
    }
  }
  terms[i] = make_uint4(w[0], w[1], w[2], w[3]);
}

// TL tiles (8 TL rows) per workgroup: every wave applies each step's terms
// to all TL tiles, so the term loads from L2 are shared by 8 TL weight rows.
template <int NB, int TL>
__global__ __launch_bounds__(256) void k_spine_mfma(const uint8_t* __restrict__ wmat,
                                                    const uint4* __restrict__ terms,
                                                    float* __restrict__ y, int rows, int cols,
                                                    int P, int S, int accumulate) {
  constexpr int kA = kAhead / TL;  // steps of weights in flight (8 / TL KB per tile)
  constexpr int kB = kA < kAheadB ? kA : kAheadB;
  static_assert(kA % kB == 0, "the rings must index statically");
  __shared__ f32x4 part[4][TL][NB][2][64];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int r0 = blockIdx.x * 8 * TL;
  const int steps = cols / 64;                   // 64-element steps of a row
  const int per = (steps + S - 1) / S;           // steps of this wave
  const int k0 = wave * per;
  const int groups = (per + kA - 1) / kA;
  const int tsteps = cols / 32 + 2;              // K32 steps of the term buffer
  const int m = lane & 15;
  const int last = steps - 1;
  const uint8_t* arow[TL];
#pragma unroll
  for (int t = 0; t < TL; ++t) {
    const int row = min(r0 + 8 * t + (m >> 1), rows - 1);
    arow[t] = wmat + (uint64_t)row * cols * 2 + 64 * (m & 1) + 16 * (lane >> 4);
  }

  f32x4 d0[TL][NB], d1[TL][NB];
#pragma unroll
  for (int t = 0; t < TL; ++t)
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) {
      d0[t][nb] = f32x4{0.f, 0.f, 0.f, 0.f};
      d1[t][nb] = f32x4{0.f, 0.f, 0.f, 0.f};
    }
  // A ring: the pieces of steps kA ahead, clamped into the row; B ring: the
  // terms of steps kB ahead (the zero steps past the wave's range).
  u32x4 ring[kA][TL];
  u32x4 bring[kB][NB][2];
  auto a_load = [&](u32x4 (&dst)[TL], int ks) {
#pragma unroll
    for (int t = 0; t < TL; ++t) dst[t] = load_chunk(arow[t] + 128 * (uint64_t)min(ks, last));
  };
  auto b_load = [&](u32x4 (&dst)[NB][2], int idx) {
    const int ks = k0 + idx;
    const int s0 = (idx < per && ks < steps) ? 2 * ks : tsteps - 2;
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) {
      const uint4* tb = terms + ((int64_t)nb * tsteps + s0) * 64 + lane;
      dst[nb][0] = load_chunk(reinterpret_cast<const uint8_t*>(tb));
      dst[nb][1] = load_chunk(reinterpret_cast<const uint8_t*>(tb + 64));
    }
  };
  if (wave < S) {
#pragma unroll
    for (int j = 0; j < kA; ++j) a_load(ring[j], k0 + j);
#pragma unroll
    for (int j = 0; j < kB; ++j) b_load(bring[j], j);
    for (int gi = 0; gi < groups; ++gi) {
#pragma unroll
      for (int j = 0; j < kA; ++j) {
        const int idx = gi * kA + j;              // step index within the wave
        const int ks = k0 + idx;
        u32x4 a[TL];
#pragma unroll
        for (int t = 0; t < TL; ++t) a[t] = ring[j][t];
        u32x4 b[NB][2];
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) {
          b[nb][0] = bring[j % kB][nb][0];
          b[nb][1] = bring[j % kB][nb][1];
        }
        a_load(ring[j], ks + kA);                 // refill kA steps ahead
        b_load(bring[j % kB], idx + kB);
#pragma unroll
        for (int t = 0; t < TL; ++t) {
          const bf16x8 av = __builtin_bit_cast(bf16x8, a[t]);
#pragma unroll
          for (int nb = 0; nb < NB; ++nb) {
            d0[t][nb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                av, __builtin_bit_cast(bf16x8, b[nb][0]), d0[t][nb], 0, 0, 0);
            d1[t][nb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                av, __builtin_bit_cast(bf16x8, b[nb][1]), d1[t][nb], 0, 0, 0);
          }
        }
      }
    }
  }
  // valid rows: weight row 2q from d0[0] + d1[1], row 2q + 1 from d0[2] + d1[3]
#pragma unroll
  for (int t = 0; t < TL; ++t)
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) {
      part[wave][t][nb][0][lane] = d0[t][nb];
      part[wave][t][nb][1][lane] = d1[t][nb];
    }
  __syncthreads();
  for (int o = threadIdx.x; o < 8 * TL * P; o += 256) {
    const int rt = o / P, p = o % P;              // output row rt of the workgroup, position p
    const int t = rt >> 3, r = rt & 7;
    const int q = r >> 1, hi = r & 1;
    float acc = 0.f;
    for (int w = 0; w < S; ++w) {
#pragma unroll
      for (int term = 0; term < 3; ++term) {
        const int n = 3 * p + term;
        const int nb = n >> 4;
        const int ln = 16 * q + (n & 15);
        if (nb < NB) {
          const f32x4 e0 = part[w][t][nb][0][ln], e1 = part[w][t][nb][1][ln];
          acc += hi ? e0[2] + e1[3] : e0[0] + e1[1];
        }
      }
    }
    const int orow = r0 + rt;
    if (orow < rows) {
      float* yp = y + (int64_t)p * rows + orow;
      *yp = accumulate ? *yp + acc : acc;
    }
  }
}

}  // namespace

uint64_t spine_mfma_terms_bytes(int positions, int cols) {
  const int nb = (3 * positions + 15) / 16;
  return (uint64_t)nb * (uint64_t)(cols / 32 + 2) * 64 * 16;
}

bool spine_mfma_supported(int kind, int positions, int rows, int cols) {
  return kind == K3_SPINE_KIND_BF16 && positions >= 1 && positions <= 16 && rows > 0 &&
         cols >= 64 && cols % 64 == 0;
}

int spine_mfma_split(const float* x, int positions, int cols, void* terms, hipStream_t st) {
  const int nb = (3 * positions + 15) / 16;
  const int64_t total = (int64_t)nb * (cols / 32 + 2) * 64;
  TimedLaunch tl(KC_SPLIT, st);
  launch_timed(tl, k_split_bf16_terms, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, st, x,
               positions, cols, nb, static_cast<uint4*>(terms));
  const hipError_t e = hipGetLastError();
  if (e == hipSuccess) return K3_SPINE_OK;
  tl.failed();
  return spine_fail(K3_SPINE_E_RUNTIME, "BF16 term split launch: %s", hipGetErrorString(e));
}

int spine_mfma_gemv(const void* w, const void* terms, float* y, int rows, int cols,
                    int positions, bool accumulate, hipStream_t st) {
  if (!spine_mfma_supported(K3_SPINE_KIND_BF16, positions, rows, cols) ||
      (reinterpret_cast<uintptr_t>(w) & 15) != 0)
    return spine_fail(K3_SPINE_E_UNSUPPORTED, "matrix-core spine: unsupported shape");
  const int steps = cols / 64;
  const int S = steps >= 64 ? 4 : steps >= 16 ? 2 : 1;  // waves splitting K
  const int nb = (3 * positions + 15) / 16;
  constexpr int TL = K3_SPINE_MFMA_TILES;
  const dim3 grid((unsigned)((rows + 8 * TL - 1) / (8 * TL)));
  const auto* wm = static_cast<const uint8_t*>(w);
  const auto* tb = static_cast<const uint4*>(terms);
  TimedLaunch tl(KC_SPINE_MFMA, st);
  switch (nb) {
    case 1: launch_timed(tl, (k_spine_mfma<1, TL>), grid, dim3(256), 0, st, wm, tb, y, rows, cols,
                         positions, S, accumulate ? 1 : 0); break;
    case 2: launch_timed(tl, (k_spine_mfma<2, TL>), grid, dim3(256), 0, st, wm, tb, y, rows, cols,
                         positions, S, accumulate ? 1 : 0); break;
    default: launch_timed(tl, (k_spine_mfma<3, TL>), grid, dim3(256), 0, st, wm, tb, y, rows, cols,
                          positions, S, accumulate ? 1 : 0); break;
  }
  const hipError_t e = hipGetLastError();
  if (e == hipSuccess) return K3_SPINE_OK;
  tl.failed();
  return spine_fail(K3_SPINE_E_RUNTIME, "matrix-core spine launch: %s", hipGetErrorString(e));
}

}  // namespace k3
