// Activation rows as fp8 E4M3 terms with E8M0 block scales: the B operand of
// the block-scaled matrix-core verify kernels (k3_verify_mfma.hip), written by
// k_split_terms and, for the activation x, by the verify plan launch's extra
// workgroups (k3_kernels.hip).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace k3 {

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

// Thread idx of a split over n_rows rows of K elements: block idx / 4, lane
// idx % 4 of that block (the four threads of a block are consecutive lanes of
// one wave; every thread of the wave calls this, idx past the end included).
template <int T, typename SrcT>
__device__ __forceinline__ void split_terms_at(const SrcT* __restrict__ src, int n_rows, int K,
                                               uint8_t* __restrict__ q, uint8_t* __restrict__ qs,
                                               int idx) {
  const int gb = K >> 5;
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

}  // namespace k3
