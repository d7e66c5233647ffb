// Resident spine projections around the routed experts on gfx950: the exact
// BF16 x FP32 GEMV (replacing native/provider_gate/provider_spine_bf16_cuda.cu:
// 95-165), the row-int8 x FP32 GEMV (at::_weight_int8pack_mm as called by
// provider_moe.cpp:507-516), the BF16 bit decode canary (:282-303) and the
// routed RMS norm (provider_moe.cpp:535-542).
//
// The GEMV is HBM-bound at decode (2 bytes per BF16 weight, 1 per int8 weight,
// one multiply-add per weight and position).  A wave owns R whole rows and
// requests them as 1 KB pieces (16 bytes per lane, the contiguous-row access
// that streams fastest on this part); every piece is requested before any
// arithmetic, so R x NJ pieces per wave are in flight.  The activation of up
// to PG positions sits in LDS, laid out so each ds_read_b128 of a wave reads
// one contiguous KB; the weights stay in registers while the positions are
// walked in groups of PG, so each weight byte is read from HBM once for all
// 1..64 positions.  A row whose byte length is not a whole number of pieces
// has a short last piece: lanes past its end load the row's first 16 bytes
// (in bounds) and replace them by zero weights, so every lane issues the same
// loads and the compiler's wait counts stay exact.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <algorithm>
#include <utility>

#include "k3_device.h"
#include "k3_launch.h"

namespace k3 {
namespace {

constexpr int kSpineThreads = 256;
constexpr int kSpineWaves = kSpineThreads / kWave;
constexpr int kSpineMaxNj = 16;                // pieces per row on the fast path
#ifndef K3_SPINE_LDS_BUDGET
#define K3_SPINE_LDS_BUDGET 65536
#endif
constexpr uint32_t kSpineLdsBudget = K3_SPINE_LDS_BUDGET;  // activation bytes per workgroup
#ifndef K3_SPINE_STREAM_WAVES_PER_CU
#define K3_SPINE_STREAM_WAVES_PER_CU 8
#endif
constexpr int kStreamWavesPerCu = K3_SPINE_STREAM_WAVES_PER_CU;

template <int kKind>
struct SpineElem;
template <>
struct SpineElem<K3_SPINE_KIND_BF16> {
  static constexpr int kPerChunk = 8;  // columns per 16-byte lane chunk
  static constexpr int kBytes = 2;
};
template <>
struct SpineElem<K3_SPINE_KIND_INT8> {
  static constexpr int kPerChunk = 16;
  static constexpr int kBytes = 1;
};

// 16 bytes of BF16 bits -> 8 fp32 values, exactly (bits << 16).
__device__ __forceinline__ void decode_chunk(u32x4 w, float* f, SpineElem<K3_SPINE_KIND_BF16>) {
#pragma unroll
  for (int d = 0; d < 4; ++d) {
    f[2 * d] = __uint_as_float(w[d] << 16);
    f[2 * d + 1] = __uint_as_float(w[d] & 0xffff0000u);
  }
}

// 16 int8 values -> 16 fp32 values, exactly (byte b of each dword, sign-extended).
__device__ __forceinline__ void decode_chunk(u32x4 w, float* f, SpineElem<K3_SPINE_KIND_INT8>) {
#pragma unroll
  for (int d = 0; d < 4; ++d) {
#pragma unroll
    for (int b = 0; b < 4; ++b)
      f[4 * d + b] = (float)((int32_t)(w[d] << (24 - 8 * b)) >> 24);
  }
}

// LDS slot of activation column c: lane l's float4 q of piece j lives at
// ((j * kQ + q) * 64 + l) * 4, so one ds_read_b128 of the wave reads 1 KB.
template <int kKind>
__device__ __forceinline__ int lds_slot(int c) {
  constexpr int kPer = SpineElem<kKind>::kPerChunk;
  constexpr int kQ = kPer / 4;
  const int j = c / (64 * kPer);
  const int in = c - j * 64 * kPer;
  const int l = in / kPer;
  const int q = (in - l * kPer) >> 2;
  return ((j * kQ + q) * 64 + l) * 4 + (c & 3);
}

// Stages positions [p0, p0 + pg) of x into LDS (zero-padded to kPad columns)
// and ends with a barrier; every thread of the workgroup calls it.  With
// norm_w, each staged row is the routed RMS norm of x (rms_norm,
// provider_moe.cpp:535-542): norm_w[c] * (x[c] * r), r = 1 / sqrt(mean(x^2) +
// eps), the sum of squares taken in a fixed order (thread-strided partials,
// wave sums, the waves in order).  x rows and norm_w are 16-byte aligned.
//
// Rows with no padding (cols == kPad) and no norm go straight from memory to
// LDS (global_load_lds_dwordx4): for each (position, piece, quarter) one
// instruction of one wave brings 64 lanes' 16 bytes into the 1 KB that
// ds_read_b128 reads back (lane l's 16 bytes: columns kPer l + 4 q .. + 3 of
// the piece), every one in flight at once and no VGPR held.  The loop below
// takes one memory round trip per float4 per thread (each ~1 µs when x comes
// from L2 or the Infinity Cache: a 16-position router projection spent most
// of its time there).
template <int kKind, int kPad>
__device__ __forceinline__ void stage_x(float* xs, const float* x, int cols, int p0, int pg,
                                        const float* norm_w, float eps, float* red) {
  if (!norm_w && cols == kPad) {
    constexpr int kPer = SpineElem<kKind>::kPerChunk;
    constexpr int kQ = kPer / 4;
    constexpr int kPieces = kPad / (64 * kPer);
    const int lane = threadIdx.x & (kWave - 1);
    const int n = pg * kPieces * kQ;  // one wave instruction each
    for (int idx = (int)(threadIdx.x / kWave); idx < n; idx += kSpineWaves) {
      const int p = idx / (kPieces * kQ);
      const int jq = idx - p * (kPieces * kQ);  // piece j * kQ + quarter q
      const int j = jq / kQ, q = jq - j * kQ;
      const float* src = x + (uint64_t)(p0 + p) * cols + j * 64 * kPer + lane * kPer + 4 * q;
      float* dst = xs + p * kPad + jq * 64 * 4;
      __builtin_amdgcn_global_load_lds(src, (__attribute__((address_space(3))) void*)dst, 16, 0,
                                       0);
    }
    __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): the LDS writes have landed
    __syncthreads();
    return;
  }
  for (int p = 0; p < pg; ++p) {
    const float* xp = x + (uint64_t)(p0 + p) * cols;
    float r = 1.f;
    if (norm_w) {
      float ss = 0.f;
      for (int c = 4 * threadIdx.x; c < cols; c += 4 * kSpineThreads) {
        const float4 v = *reinterpret_cast<const float4*>(xp + c);
        ss = fmaf(v.x, v.x, ss);
        ss = fmaf(v.y, v.y, ss);
        ss = fmaf(v.z, v.z, ss);
        ss = fmaf(v.w, v.w, ss);
      }
      ss = wave_sum(ss);
      if ((threadIdx.x & (kWave - 1)) == 0) red[threadIdx.x / kWave] = ss;
      __syncthreads();
      float tot = red[0];
#pragma unroll
      for (int v = 1; v < kSpineWaves; ++v) tot += red[v];
      r = 1.0f / sqrtf(tot / (float)cols + eps);
      __syncthreads();  // red is reused by the next position
    }
    for (int c = 4 * threadIdx.x; c < kPad; c += 4 * kSpineThreads) {
      float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
      if (c < cols) {
        v = *reinterpret_cast<const float4*>(xp + c);
        if (norm_w) {
          const float4 nw = *reinterpret_cast<const float4*>(norm_w + c);
          v.x = nw.x * (v.x * r);
          v.y = nw.y * (v.y * r);
          v.z = nw.z * (v.z * r);
          v.w = nw.w * (v.w * r);
        }
      }
      *reinterpret_cast<float4*>(xs + p * kPad + lds_slot<kKind>(c)) = v;
    }
  }
  __syncthreads();
}

// kGlu: R = 2 and the wave's two rows are row i of w (gate) and row i of w2
// (up); the output is act(gate . x, up . x) (the shared expert's SiTU, or
// SiLU-GLU), one row per wave.
template <int kKind, int NJ, int R, int PG, bool kGlu = false>
__global__ __launch_bounds__(kSpineThreads, kGlu ? 2 : 4) void k_spine_gemv(
    const uint8_t* __restrict__ w, const float* __restrict__ row_scale,
    const float* __restrict__ x, float* __restrict__ y, int rows, int cols, int positions,
    int tail_lanes, int accumulate, const uint8_t* __restrict__ w2,
    const float* __restrict__ row_scale2, int act, const float* __restrict__ norm_w, float eps) {
  using E = SpineElem<kKind>;
  static_assert(!kGlu || R == 2, "a GLU wave holds one gate row and one up row");
  constexpr int kQ = E::kPerChunk / 4;
  constexpr int kPad = NJ * 64 * E::kPerChunk;  // columns per staged position
  extern __shared__ float4 xs4[];               // [PG][kPad / 4]
  __shared__ float red[kSpineWaves];
  float* xs = reinterpret_cast<float*>(xs4);
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = threadIdx.x / kWave;
  const uint64_t row_bytes = (uint64_t)cols * E::kBytes;
  const int row0 = (blockIdx.x * kSpineWaves + wave) * (kGlu ? 1 : R);
  const bool tail_ok = lane < tail_lanes;

  u32x4 wv[R][NJ];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int row = min(kGlu ? row0 : row0 + r, rows - 1);
    const uint8_t* base = (kGlu && r == 1 ? w2 : w) + (uint64_t)row * row_bytes;
    const uint8_t* rp = base + 16 * lane;
#pragma unroll
    for (int j = 0; j < NJ - 1; ++j) wv[r][j] = load_chunk(rp + 1024 * j);
    wv[r][NJ - 1] = load_chunk(tail_ok ? rp + 1024 * (NJ - 1) : base);
  }

  for (int p0 = 0; p0 < positions; p0 += PG) {
    const int pg = min(PG, positions - p0);
    if (p0) __syncthreads();
    stage_x<kKind, kPad>(xs, x, cols, p0, pg, norm_w, eps, red);

    float acc[R][PG];
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
      for (int p = 0; p < PG; ++p) acc[r][p] = 0.f;
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      // This piece's activation, read once for all R rows; the scheduling
      // fence at the end keeps later pieces' reads and decodes from being
      // hoisted here (they would hold every piece's values in registers).
      float4 xv[PG][kQ];
#pragma unroll
      for (int p = 0; p < PG; ++p) {
        if (p < pg) {
#pragma unroll
          for (int q = 0; q < kQ; ++q) xv[p][q] = xs4[(p * kPad) / 4 + (j * kQ + q) * 64 + lane];
        }
      }
#pragma unroll
      for (int r = 0; r < R; ++r) {
        u32x4 wc = wv[r][j];
        if (j == NJ - 1 && !tail_ok) wc = u32x4{0u, 0u, 0u, 0u};
        // Opaque to the optimiser, so the decode is not hoisted out of the
        // position-group loop (that would keep every decoded piece live).
        asm volatile("" : "+v"(wc));
        float f[E::kPerChunk];
        decode_chunk(wc, f, E{});
#pragma unroll
        for (int p = 0; p < PG; ++p) {
          if (p < pg) {
#pragma unroll
            for (int q = 0; q < kQ; ++q) {
              acc[r][p] = fmaf(f[4 * q + 0], xv[p][q].x, acc[r][p]);
              acc[r][p] = fmaf(f[4 * q + 1], xv[p][q].y, acc[r][p]);
              acc[r][p] = fmaf(f[4 * q + 2], xv[p][q].z, acc[r][p]);
              acc[r][p] = fmaf(f[4 * q + 3], xv[p][q].w, acc[r][p]);
            }
          }
        }
      }
      __builtin_amdgcn_sched_barrier(0);
    }
    if constexpr (kGlu) {
      const int rr = min(row0, rows - 1);
      const float sg = kKind == K3_SPINE_KIND_INT8 ? row_scale[rr] : 1.f;
      const float su = kKind == K3_SPINE_KIND_INT8 ? row_scale2[rr] : 1.f;
#pragma unroll
      for (int p = 0; p < PG; ++p) {
        if (p < pg) {
          float gs = wave_sum(acc[0][p]);
          float us = wave_sum(acc[1][p]);
          if (kKind == K3_SPINE_KIND_INT8) {
            gs *= sg;
            us *= su;
          }
          if (lane == 0 && row0 < rows) y[(uint64_t)(p0 + p) * rows + row0] = activate(act, gs, us);
        }
      }
    } else {
#pragma unroll
      for (int r = 0; r < R; ++r) {
        const int row = row0 + r;
        const float scale = kKind == K3_SPINE_KIND_INT8 ? row_scale[min(row, rows - 1)] : 1.f;
#pragma unroll
        for (int p = 0; p < PG; ++p) {
          if (p < pg) {
            float s = wave_sum(acc[r][p]);
            if (kKind == K3_SPINE_KIND_INT8) s *= scale;
            if (lane == 0 && row < rows) {
              float* yp = y + (uint64_t)(p0 + p) * rows + row;
              *yp = accumulate ? *yp + s : s;
            }
          }
        }
      }
    }
  }
}

// One position group (positions <= PG), persistent waves: the workgroup stages
// the activation once, then each wave walks rows row0, row0 + W, ... (W waves
// in the grid, sized by the host so every wave gets the same number of rows)
// with the next row's pieces requested while the current one is summed.  The
// prefetch past the last row is clamped to row rows - 1 (every wave reads the
// same bytes, served from cache) so that the loads are unconditional.
template <int kKind, int NJ, int PG>
__global__ __launch_bounds__(kSpineThreads, 2) void k_spine_stream(
    const uint8_t* __restrict__ w, const float* __restrict__ row_scale,
    const float* __restrict__ x, float* __restrict__ y, int rows, int cols, int positions,
    int tail_lanes, int accumulate, const float* __restrict__ norm_w, float eps,
    const uint8_t* __restrict__ wb, const float* __restrict__ row_scale_b, float* __restrict__ yb,
    int rows_a) {
  // Rows [0, rows_a) are w's (output y [P][rows_a]); with wb, rows [rows_a,
  // rows) are wb's (output yb [P][rows - rows_a]): two matrices of the same
  // width over the same activation in one launch.  Without wb, rows_a = rows.
  using E = SpineElem<kKind>;
  constexpr int kQ = E::kPerChunk / 4;
  constexpr int kPad = NJ * 64 * E::kPerChunk;
  extern __shared__ float4 xs4[];  // [PG][kPad / 4]
  __shared__ float red[kSpineWaves];
  const int rows_b = rows - rows_a;
  float* xs = reinterpret_cast<float*>(xs4);
  const int lane = threadIdx.x & (kWave - 1);
  const int stride = gridDim.x * kSpineWaves;
  const uint64_t row_bytes = (uint64_t)cols * E::kBytes;
  const bool tail_ok = lane < tail_lanes;

  auto load_row = [&](u32x4* buf, int row) {
    const int r = min(row, rows - 1);
    const uint8_t* base =
        r < rows_a ? w + (uint64_t)r * row_bytes : wb + (uint64_t)(r - rows_a) * row_bytes;
    const uint8_t* rp = base + 16 * lane;
#pragma unroll
    for (int j = 0; j < NJ - 1; ++j) buf[j] = load_chunk(rp + 1024 * j);
    buf[NJ - 1] = load_chunk(tail_ok ? rp + 1024 * (NJ - 1) : base);
  };
  auto sum_row = [&](const u32x4* buf, int row) {
    float acc[PG];
#pragma unroll
    for (int p = 0; p < PG; ++p) acc[p] = 0.f;
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      u32x4 wc = buf[j];
      if (j == NJ - 1 && !tail_ok) wc = u32x4{0u, 0u, 0u, 0u};
      float f[E::kPerChunk];
      decode_chunk(wc, f, E{});
#pragma unroll
      for (int p = 0; p < PG; ++p) {
        if (p < positions) {
#pragma unroll
          for (int q = 0; q < kQ; ++q) {
            const float4 xv = xs4[(p * kPad) / 4 + (j * kQ + q) * 64 + lane];
            acc[p] = fmaf(f[4 * q + 0], xv.x, acc[p]);
            acc[p] = fmaf(f[4 * q + 1], xv.y, acc[p]);
            acc[p] = fmaf(f[4 * q + 2], xv.z, acc[p]);
            acc[p] = fmaf(f[4 * q + 3], xv.w, acc[p]);
          }
        }
      }
    }
    const bool in_a = row < rows_a;
    const float scale = kKind == K3_SPINE_KIND_INT8
                            ? (in_a ? row_scale[row] : row_scale_b[row - rows_a])
                            : 1.f;
#pragma unroll
    for (int p = 0; p < PG; ++p) {
      if (p < positions) {
        float s = wave_sum(acc[p]);
        if (kKind == K3_SPINE_KIND_INT8) s *= scale;
        if (lane == 0) {
          float* yp = in_a ? y + (uint64_t)p * rows_a + row
                           : yb + (uint64_t)p * rows_b + (row - rows_a);
          *yp = accumulate ? *yp + s : s;
        }
      }
    }
  };

  int row = blockIdx.x * kSpineWaves + threadIdx.x / kWave;
  u32x4 a[NJ], b[NJ];
  load_row(a, row);
  stage_x<kKind, kPad>(xs, x, cols, 0, positions, norm_w, eps, red);
  if (row >= rows) return;  // no barrier follows
  for (;;) {
    const int rb = row + stride;
    load_row(b, rb);
    sum_row(a, row);
    if (rb >= rows) break;
    const int ra = rb + stride;
    load_row(a, ra);
    sum_row(b, rb);
    if (ra >= rows) break;
    row = ra;
  }
}

// Any shape and alignment: one wave per row, lanes stride the columns.
template <int kKind>
__global__ __launch_bounds__(kSpineThreads) void k_spine_gemv_generic(
    const uint8_t* __restrict__ w, const float* __restrict__ row_scale,
    const float* __restrict__ x, float* __restrict__ y, int rows, int cols, int positions,
    int accumulate) {
  const int lane = threadIdx.x & (kWave - 1);
  const int row = blockIdx.x * kSpineWaves + threadIdx.x / kWave;
  if (row >= rows) return;
  for (int p = 0; p < positions; ++p) {
    const float* xp = x + (uint64_t)p * cols;
    float acc = 0.f;
    for (int c = lane; c < cols; c += kWave) {
      const uint64_t i = (uint64_t)row * cols + c;
      float wf;
      if (kKind == K3_SPINE_KIND_BF16) {
        wf = __uint_as_float((uint32_t)reinterpret_cast<const uint16_t*>(w)[i] << 16);
      } else {
        wf = (float)reinterpret_cast<const int8_t*>(w)[i];
      }
      acc = fmaf(wf, xp[c], acc);
    }
    float s = wave_sum(acc);
    if (kKind == K3_SPINE_KIND_INT8) s *= row_scale[row];
    if (lane == 0) {
      float* yp = y + (uint64_t)p * rows + row;
      *yp = accumulate ? *yp + s : s;
    }
  }
}

__global__ __launch_bounds__(kSpineThreads) void k_bf16_decode_bits(const uint16_t* __restrict__ in,
                                                                    uint32_t* __restrict__ out,
                                                                    int count) {
  const int i = blockIdx.x * kSpineThreads + threadIdx.x;
  if (i < count) out[i] = (uint32_t)in[i] << 16;
}

// One workgroup per row: sum of squares in a fixed order (lane-strided fp32
// partials, wave sums, then the four waves in order), 1 / sqrt(mean + eps),
// then weight * (x * r) as the reference's ATen ops compose it.
__global__ __launch_bounds__(kSpineThreads) void k_rms_norm(const float* __restrict__ in,
                                                            const float* __restrict__ weight,
                                                            float* __restrict__ out, int cols,
                                                            float eps) {
  __shared__ float part[kSpineWaves];
  const float* xp = in + (uint64_t)blockIdx.x * cols;
  float* op = out + (uint64_t)blockIdx.x * cols;
  float s = 0.f;
  for (int c = threadIdx.x; c < cols; c += kSpineThreads) s = fmaf(xp[c], xp[c], s);
  s = wave_sum(s);
  if ((threadIdx.x & (kWave - 1)) == 0) part[threadIdx.x / kWave] = s;
  __syncthreads();
  float total = part[0];
#pragma unroll
  for (int v = 1; v < kSpineWaves; ++v) total += part[v];
  const float r = 1.0f / sqrtf(total / (float)cols + eps);
  __syncthreads();  // every read of xp above precedes any in-place write below
  for (int c = threadIdx.x; c < cols; c += kSpineThreads) op[c] = weight[c] * (xp[c] * r);
}

// The same for rows of 16-byte aligned float4 (cols % 4 == 0, cols <= 4 *
// kSpineThreads * kNormIter): a thread's float4 (float4 index t + 256 i) and
// their weights are all requested before any is used and kept for the
// scaled store, so a row costs one memory round trip instead of one per
// element per pass.  The sum of squares runs over each thread's float4 in
// index order (x, y, z, w), then wave sums, then the waves in order.
constexpr int kNormIter = 8;

// kTerms: the workgroup of row p also writes the row's three BF16 terms into
// the matrix-core spine's term buffer (k_split_bf16_terms' layout: column
// n = 3 p + t of 16-column block n / 16, 16 bytes per (block, K32 step s,
// lane 16 (k % 32) / 8 + n % 16)), each thread its float4's 8 bytes of each
// term; workgroup 0 also writes the zero columns past 3 P and the two zero
// steps after the last.  The terms are those k_split_bf16_terms forms from
// the stored row.
template <bool kTerms>
__global__ __launch_bounds__(kSpineThreads) void k_rms_norm_vec(const float* __restrict__ in,
                                                                const float* __restrict__ weight,
                                                                float* __restrict__ out, int cols,
                                                                float eps,
                                                                uint8_t* __restrict__ terms,
                                                                int nb_count) {
  __shared__ float part[kSpineWaves];
  const float4* xp = reinterpret_cast<const float4*>(in + (uint64_t)blockIdx.x * cols);
  const float4* wp = reinterpret_cast<const float4*>(weight);
  float4* op = reinterpret_cast<float4*>(out + (uint64_t)blockIdx.x * cols);
  const int n4 = cols >> 2;
  float4 v[kNormIter], nw[kNormIter];
#pragma unroll
  for (int i = 0; i < kNormIter; ++i) {
    const int c = (int)threadIdx.x + kSpineThreads * i;
    v[i] = c < n4 ? xp[c] : make_float4(0.f, 0.f, 0.f, 0.f);
    nw[i] = c < n4 ? wp[c] : make_float4(0.f, 0.f, 0.f, 0.f);
  }
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < kNormIter; ++i) {
    s = fmaf(v[i].x, v[i].x, s);
    s = fmaf(v[i].y, v[i].y, s);
    s = fmaf(v[i].z, v[i].z, s);
    s = fmaf(v[i].w, v[i].w, s);
  }
  s = wave_sum(s);
  if ((threadIdx.x & (kWave - 1)) == 0) part[threadIdx.x / kWave] = s;
  __syncthreads();
  float total = part[0];
#pragma unroll
  for (int w = 1; w < kSpineWaves; ++w) total += part[w];
  const float r = 1.0f / sqrtf(total / (float)cols + eps);
  const int tsteps = cols / 32 + 2;
#pragma unroll
  for (int i = 0; i < kNormIter; ++i) {
    const int c = (int)threadIdx.x + kSpineThreads * i;
    if (c < n4) {
      const float y[4] = {nw[i].x * (v[i].x * r), nw[i].y * (v[i].y * r),
                          nw[i].z * (v[i].z * r), nw[i].w * (v[i].w * r)};
      op[c] = make_float4(y[0], y[1], y[2], y[3]);
      if constexpr (kTerms) {
        uint32_t t[3][2];
#pragma unroll
        for (int e = 0; e < 4; e += 2) {
          uint32_t b[3][2];
#pragma unroll
          for (int o = 0; o < 2; ++o) {
            const float f = y[e + o];
            b[0][o] = f32_to_bf16_bits(f);
            const float r1 = f - __uint_as_float(b[0][o] << 16);
            b[1][o] = f32_to_bf16_bits(r1);
            b[2][o] = f32_to_bf16_bits(r1 - __uint_as_float(b[1][o] << 16));
          }
#pragma unroll
          for (int q = 0; q < 3; ++q) t[q][e >> 1] = b[q][0] | (b[q][1] << 16);
        }
        const int k = 4 * c;  // first K element of the float4
        const int ks = k >> 5, lane16 = 16 * ((k & 31) >> 3), half = (k >> 2) & 1;
#pragma unroll
        for (int q = 0; q < 3; ++q) {
          const int n = 3 * (int)blockIdx.x + q;
          const size_t slot = ((size_t)(n >> 4) * tsteps + ks) * 64 + lane16 + (n & 15);
          *reinterpret_cast<uint2*>(terms + 16 * slot + 8 * half) = make_uint2(t[q][0], t[q][1]);
        }
      }
    }
  }
  if constexpr (kTerms) {
    if (blockIdx.x == 0) {
      // zero columns past 3 P (every step), then the two zero steps (every column)
      const int n0 = 3 * (int)gridDim.x, ncol = 16 * nb_count;
      const int zc = (ncol - n0) * tsteps * 4;
      for (int z = threadIdx.x; z < zc; z += blockDim.x) {
        const int n = n0 + z / (tsteps * 4), rem = z % (tsteps * 4);
        const size_t slot = ((size_t)(n >> 4) * tsteps + rem / 4) * 64 + 16 * (rem % 4) + (n & 15);
        *reinterpret_cast<uint4*>(terms + 16 * slot) = make_uint4(0u, 0u, 0u, 0u);
      }
      for (int z = threadIdx.x; z < nb_count * 2 * 64; z += blockDim.x) {
        const int nb = z / 128, st = cols / 32 + (z / 64) % 2;
        const size_t slot = ((size_t)nb * tsteps + st) * 64 + (z & 63);
        *reinterpret_cast<uint4*>(terms + 16 * slot) = make_uint4(0u, 0u, 0u, 0u);
      }
    }
  }
}

template <int kKind, int NJ>
int spine_fast_launch(const SpineOp& op, int tail_lanes, int pg, int stream_waves,
                      hipStream_t st) {
  // Two rows per wave for short rows (int8 decodes twice the values per
  // piece); a GLU wave always holds its gate and its up row.
  constexpr int R = NJ <= (kKind == K3_SPINE_KIND_BF16 ? 4 : 2) ? 2 : 1;
  constexpr uint32_t kPadBytes = NJ * 64u * SpineElem<kKind>::kPerChunk * 4u;
  const auto* w = static_cast<const uint8_t*>(op.w);
  const auto* w2 = static_cast<const uint8_t*>(op.w2);
  const auto* wb = static_cast<const uint8_t*>(op.wb);
  const int total_rows = op.rows + (op.wb ? op.rows_b : 0);
  const int acc = op.accumulate ? 1 : 0;
  TimedLaunch tl(KC_SPINE, st);
  bool launched_one = false;
  if (op.w2) {
    const dim3 grid((unsigned)((op.rows + kSpineWaves - 1) / kSpineWaves));
    if constexpr (2 * kPadBytes <= kSpineLdsBudget) {
      if (pg == 2) {
        launch_timed(tl, (k_spine_gemv<kKind, NJ, 2, 2, true>), grid, dim3(kSpineThreads),
                     2 * kPadBytes, st, w, op.scales, op.x, op.y, op.rows, op.cols, op.positions,
                     tail_lanes, acc, w2, op.scales2, op.act, op.norm_w, op.eps);
        launched_one = true;
      }
    }
    if (pg == 1) {
      launch_timed(tl, (k_spine_gemv<kKind, NJ, 2, 1, true>), grid, dim3(kSpineThreads),
                   kPadBytes, st, w, op.scales, op.x, op.y, op.rows, op.cols, op.positions,
                   tail_lanes, acc, w2, op.scales2, op.act, op.norm_w, op.eps);
      launched_one = true;
    }
  } else if (op.positions <= pg && stream_waves > 0) {
    // One position group: persistent waves, each with the same row count.
    const dim3 sgrid((unsigned)(stream_waves / kSpineWaves));
    const uint32_t lds = (uint32_t)pg * kPadBytes;
    if constexpr (4 * kPadBytes <= kSpineLdsBudget) {
      if (pg == 4) {
        launch_timed(tl, (k_spine_stream<kKind, NJ, 4>), sgrid, dim3(kSpineThreads), lds, st, w,
                     op.scales, op.x, op.y, total_rows, op.cols, op.positions, tail_lanes, acc,
                     op.norm_w, op.eps, wb, op.scales_b, op.yb, op.rows);
        launched_one = true;
      }
    }
    if constexpr (2 * kPadBytes <= kSpineLdsBudget) {
      if (pg == 2) {
        launch_timed(tl, (k_spine_stream<kKind, NJ, 2>), sgrid, dim3(kSpineThreads), lds, st, w,
                     op.scales, op.x, op.y, total_rows, op.cols, op.positions, tail_lanes, acc,
                     op.norm_w, op.eps, wb, op.scales_b, op.yb, op.rows);
        launched_one = true;
      }
    }
    if (pg == 1) {
      launch_timed(tl, (k_spine_stream<kKind, NJ, 1>), sgrid, dim3(kSpineThreads), lds, st, w,
                   op.scales, op.x, op.y, total_rows, op.cols, op.positions, tail_lanes, acc,
                   op.norm_w, op.eps, wb, op.scales_b, op.yb, op.rows);
      launched_one = true;
    }
  } else {
    const int rows_per_group = kSpineWaves * R;
    const dim3 grid((unsigned)((op.rows + rows_per_group - 1) / rows_per_group));
    // Only the position groups whose activation fits the LDS budget exist.
    if constexpr (4 * kPadBytes <= kSpineLdsBudget) {
      if (pg == 4) {
        launch_timed(tl, (k_spine_gemv<kKind, NJ, R, 4>), grid, dim3(kSpineThreads),
                     4 * kPadBytes, st, w, op.scales, op.x, op.y, op.rows, op.cols, op.positions,
                     tail_lanes, acc, w2, op.scales2, op.act, op.norm_w, op.eps);
        launched_one = true;
      }
    }
    if constexpr (2 * kPadBytes <= kSpineLdsBudget) {
      if (pg == 2) {
        launch_timed(tl, (k_spine_gemv<kKind, NJ, R, 2>), grid, dim3(kSpineThreads),
                     2 * kPadBytes, st, w, op.scales, op.x, op.y, op.rows, op.cols, op.positions,
                     tail_lanes, acc, w2, op.scales2, op.act, op.norm_w, op.eps);
        launched_one = true;
      }
    }
    if (pg == 1) {
      launch_timed(tl, (k_spine_gemv<kKind, NJ, R, 1>), grid, dim3(kSpineThreads), kPadBytes, st,
                   w, op.scales, op.x, op.y, op.rows, op.cols, op.positions, tail_lanes, acc,
                   w2, op.scales2, op.act, op.norm_w, op.eps);
      launched_one = true;
    }
  }
  if (!launched_one) {
    tl.failed();
    return spine_fail(K3_SPINE_E_INVALID, "spine GEMV: no kernel for %d positions per group", pg);
  }
  const hipError_t e = hipGetLastError();
  if (e == hipSuccess) return K3_SPINE_OK;
  tl.failed();
  return spine_fail(K3_SPINE_E_RUNTIME, "spine GEMV launch: %s", hipGetErrorString(e));
}

typedef int (*SpineFastFn)(const SpineOp&, int, int, int, hipStream_t);

template <int kKind, int... NJ>
constexpr SpineFastFn spine_fast_table(int nj, std::integer_sequence<int, NJ...>) {
  SpineFastFn table[] = {nullptr, &spine_fast_launch<kKind, NJ + 1>...};
  return table[nj];
}

int preflight(const char* what) {
  const hipError_t e = hipGetLastError();
  if (e == hipSuccess) return K3_SPINE_OK;
  return spine_fail(K3_SPINE_E_RUNTIME, "%s preflight: %s", what, hipGetErrorString(e));
}

}  // namespace

int spine_gemv_op(int kind, const SpineOp& op, hipStream_t st) {
  const char* what = kind == K3_SPINE_KIND_BF16 ? "RAW_BF16 GEMV" : "row-int8 GEMV";
  if (!op.w || !op.x || !op.y || (kind == K3_SPINE_KIND_INT8 && !op.scales) ||
      (op.w2 && kind == K3_SPINE_KIND_INT8 && !op.scales2))
    return spine_fail(K3_SPINE_E_INVALID, "%s: null input or output pointer", what);
  if (op.rows <= 0 || op.cols <= 0 || op.positions <= 0 ||
      op.positions > K3_SPINE_MAX_POSITIONS)
    return spine_fail(K3_SPINE_E_INVALID,
                      "%s: rows/columns must be positive and positions must be 1..%d", what,
                      K3_SPINE_MAX_POSITIONS);
  if ((uint64_t)op.rows > (uint64_t)INT32_MAX / 2)
    return spine_fail(K3_SPINE_E_INVALID, "%s: too many rows", what);
  if (op.w2 && op.accumulate)
    return spine_fail(K3_SPINE_E_INVALID, "%s: a GLU projection does not accumulate", what);
  if (op.wb && (op.w2 || !op.yb || op.rows_b <= 0 || (kind == K3_SPINE_KIND_INT8 && !op.scales_b) ||
                (uint64_t)op.rows + op.rows_b > (uint64_t)INT32_MAX / 2))
    return spine_fail(K3_SPINE_E_INVALID, "%s: invalid second matrix", what);
  int rc = preflight(what);
  if (rc != K3_SPINE_OK) return rc;
  const auto* w = static_cast<const uint8_t*>(op.w);
  const int esize = kind == K3_SPINE_KIND_BF16 ? 2 : 1;
  const uint64_t row_bytes = (uint64_t)op.cols * esize;
  const int nj = (int)((row_bytes + 1023) / 1024);
  const int per_position = nj * 64 * (16 / esize) * 4;  // staged activation bytes
  const bool aligned =
      (reinterpret_cast<uintptr_t>(w) & 15) == 0 && (reinterpret_cast<uintptr_t>(op.x) & 15) == 0 &&
      (reinterpret_cast<uintptr_t>(op.w2) & 15) == 0 &&
      (reinterpret_cast<uintptr_t>(op.norm_w) & 15) == 0 &&
      (reinterpret_cast<uintptr_t>(op.wb) & 15) == 0 && row_bytes % 16 == 0;
  if (aligned && nj <= kSpineMaxNj && (uint32_t)per_position <= kSpineLdsBudget) {
    // Positions per LDS group: 1, 2 or 4 (the instantiated kernels), at most
    // what the budget holds; 3 positions take one group of 4 (GLU: 1 or 2).
    const int fit = (int)(kSpineLdsBudget / (uint32_t)per_position);
    const int want = op.positions >= 3 ? 4 : op.positions;
    int pg = std::min(want, fit >= 4 ? 4 : fit >= 2 ? 2 : 1);
    if (op.w2 && pg == 4) pg = 2;
    const uint64_t tail_bytes = row_bytes - 1024ull * (nj - 1);
    const int tail_lanes = (int)(tail_bytes / 16);
    // Persistent waves for one position group: about kStreamWavesPerCu per
    // CU, rounded so every wave gets ceil(rows / target) rows, in whole
    // workgroups.
    int stream_waves = 0;
    const int total = op.rows + (op.wb ? op.rows_b : 0);
    if (op.positions <= pg && !op.w2) {
      const int target = std::max(kSpineWaves, std::max(1, device_cu_count()) * kStreamWavesPerCu);
      const int per_wave = (total + target - 1) / target;
      stream_waves = (total + per_wave - 1) / per_wave;
      stream_waves = (stream_waves + kSpineWaves - 1) / kSpineWaves * kSpineWaves;
    } else if (op.wb) {
      return spine_fail(K3_SPINE_E_UNSUPPORTED,
                        "%s: two matrices in one launch need a single position group", what);
    }
    const auto seq = std::make_integer_sequence<int, kSpineMaxNj>{};
    const SpineFastFn fn = kind == K3_SPINE_KIND_BF16
                               ? spine_fast_table<K3_SPINE_KIND_BF16>(nj, seq)
                               : spine_fast_table<K3_SPINE_KIND_INT8>(nj, seq);
    return fn(op, tail_lanes, pg, stream_waves, st);
  }
  if (op.w2 || op.norm_w || op.wb)
    return spine_fail(K3_SPINE_E_UNSUPPORTED,
                      "%s: fused GLU / RMS norm needs 16-byte aligned rows of at most 16 KB", what);
  const dim3 grid((unsigned)((op.rows + kSpineWaves - 1) / kSpineWaves));
  TimedLaunch tl(KC_SPINE, st);
  if (kind == K3_SPINE_KIND_BF16)
    launch_timed(tl, k_spine_gemv_generic<K3_SPINE_KIND_BF16>, grid, dim3(kSpineThreads), 0, st,
                 w, op.scales, op.x, op.y, op.rows, op.cols, op.positions, op.accumulate ? 1 : 0);
  else
    launch_timed(tl, k_spine_gemv_generic<K3_SPINE_KIND_INT8>, grid, dim3(kSpineThreads), 0, st,
                 w, op.scales, op.x, op.y, op.rows, op.cols, op.positions, op.accumulate ? 1 : 0);
  const hipError_t e = hipGetLastError();
  if (e == hipSuccess) return K3_SPINE_OK;
  tl.failed();
  return spine_fail(K3_SPINE_E_RUNTIME, "%s launch: %s", what, hipGetErrorString(e));
}

int spine_gemv(int kind, const void* weights, const float* row_scales, const float* x,
               float* y, int rows, int cols, int positions, bool accumulate, hipStream_t st) {
  SpineOp op{};
  op.w = weights;
  op.scales = row_scales;
  op.x = x;
  op.y = y;
  op.rows = rows;
  op.cols = cols;
  op.positions = positions;
  op.accumulate = accumulate;
  return spine_gemv_op(kind, op, st);
}

int spine_decode_bits(const uint16_t* in, uint32_t* out, int count, hipStream_t st) {
  if (!in || !out || count <= 0)
    return spine_fail(K3_SPINE_E_INVALID, "RAW_BF16 decode: invalid input, output, or count");
  int rc = preflight("RAW_BF16 decode");
  if (rc != K3_SPINE_OK) return rc;
  const int blocks = (int)(((int64_t)count + kSpineThreads - 1) / kSpineThreads);
  hipLaunchKernelGGL(k_bf16_decode_bits, dim3(blocks), dim3(kSpineThreads), 0, st, in, out,
                     count);
  const hipError_t e = hipGetLastError();
  if (e == hipSuccess) return K3_SPINE_OK;
  return spine_fail(K3_SPINE_E_RUNTIME, "RAW_BF16 decode launch: %s", hipGetErrorString(e));
}

int spine_rms_norm(const float* in, const float* weight, float* out, int rows, int cols,
                   float eps, hipStream_t st) {
  if (!in || !weight || !out)
    return spine_fail(K3_SPINE_E_INVALID, "RMS norm: null input, weight or output");
  if (rows <= 0 || cols <= 0)
    return spine_fail(K3_SPINE_E_INVALID, "RMS norm: rows and columns must be positive");
  if (!(eps >= 0.f) || eps == INFINITY)
    return spine_fail(K3_SPINE_E_INVALID, "RMS norm: eps must be finite and non-negative");
  int rc = preflight("RMS norm");
  if (rc != K3_SPINE_OK) return rc;
  TimedLaunch tl(KC_RMS_NORM, st);
  const bool vec = cols % 4 == 0 && cols <= 4 * kSpineThreads * kNormIter &&
                   ((reinterpret_cast<uintptr_t>(in) | reinterpret_cast<uintptr_t>(weight) |
                     reinterpret_cast<uintptr_t>(out)) & 15u) == 0;
  if (vec)
    launch_timed(tl, k_rms_norm_vec<false>, dim3(rows), dim3(kSpineThreads), 0, st, in, weight,
                 out, cols, eps, nullptr, 0);
  else
    launch_timed(tl, k_rms_norm, dim3(rows), dim3(kSpineThreads), 0, st, in, weight, out, cols,
                 eps);
  const hipError_t e = hipGetLastError();
  if (e == hipSuccess) return K3_SPINE_OK;
  tl.failed();
  return spine_fail(K3_SPINE_E_RUNTIME, "RMS norm launch: %s", hipGetErrorString(e));
}

int spine_rms_norm_terms(const float* in, const float* weight, float* out, int rows, int cols,
                         float eps, void* terms, hipStream_t st) {
  if (!in || !weight || !out || !terms || rows <= 0 || rows > 16 || cols < 64 || cols % 64 != 0 ||
      cols > 4 * kSpineThreads * kNormIter || !(eps >= 0.f) || eps == INFINITY ||
      ((reinterpret_cast<uintptr_t>(in) | reinterpret_cast<uintptr_t>(weight) |
        reinterpret_cast<uintptr_t>(out) | reinterpret_cast<uintptr_t>(terms)) & 15u) != 0)
    return K3_SPINE_E_UNSUPPORTED;
  int rc = preflight("RMS norm");
  if (rc != K3_SPINE_OK) return rc;
  TimedLaunch tl(KC_RMS_NORM, st);
  launch_timed(tl, k_rms_norm_vec<true>, dim3(rows), dim3(kSpineThreads), 0, st, in, weight, out,
               cols, eps, static_cast<uint8_t*>(terms), (3 * rows + 15) / 16);
  const hipError_t e = hipGetLastError();
  if (e == hipSuccess) return K3_SPINE_OK;
  tl.failed();
  return spine_fail(K3_SPINE_E_RUNTIME, "RMS norm launch: %s", hipGetErrorString(e));
}

}  // namespace k3
