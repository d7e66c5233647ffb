// Device helpers for the gfx950 MXFP4 kernels.
//
// One 16-byte chunk of a packed row holds 32 E2M1 codes (two per byte, the LOW
// nibble is the even column, tools/fused_gemv.c:4-6) and shares one E8M0
// scale byte: a chunk is exactly one scale group.  Codes are decoded with the
// gfx950 hardware converts (v_cvt_scalef32_pk_{bf16,f32}_fp4) at scale 1.0; the
// group's partial dot is then multiplied by the group scale (the
// per-group-then-scale order of tools/metal/moe_mxfp4.metal:95-106).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace k3 {

typedef float v2f __attribute__((ext_vector_type(2)));
typedef __bf16 v2bf __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int kWave = 64;

// E8M0 byte -> fp32 scale.  The byte is the fp32 exponent field exactly as the
// reference CPU decodes it (tools/fused_gemv.c:247-249: s = 0 -> +0.0); a 255
// byte yields NaN so the row is poisoned (tools/cuda_moe_kernels.cu:128-131).
__device__ __forceinline__ float e8m0_scale(uint32_t s) {
  return __uint_as_float(s == 255u ? 0x7fc00000u : (s << 23));
}

__device__ __forceinline__ float bf16_bits_to_f32(uint32_t b) {
  return __uint_as_float(b << 16);
}

// Round-to-nearest-even fp32 -> bf16 bits (NaN stays NaN).
__device__ __forceinline__ uint16_t f32_to_bf16_bits(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

// ---------------------------------------------------------------- chunk dots
// bf16 activations: xv holds 16 dwords, dword i = columns (2i, 2i+1) of the
// chunk as a bf16 pair.  16 converts + 16 dot2 per 32 elements.
__device__ __forceinline__ float chunk_dot_bf16(u32x4 w, const uint32_t* xv) {
  float a0 = 0.0f, a1 = 0.0f;
#define K3_DOT_DWORD(d, base)                                                  \
  {                                                                            \
    v2bf w0 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4((d), 1.0f, 0);         \
    v2bf w1 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4((d), 1.0f, 1);         \
    v2bf w2 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4((d), 1.0f, 2);         \
    v2bf w3 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4((d), 1.0f, 3);         \
    a0 = __builtin_amdgcn_fdot2_f32_bf16(w0, __builtin_bit_cast(v2bf, xv[(base) + 0]), a0, false); \
    a1 = __builtin_amdgcn_fdot2_f32_bf16(w1, __builtin_bit_cast(v2bf, xv[(base) + 1]), a1, false); \
    a0 = __builtin_amdgcn_fdot2_f32_bf16(w2, __builtin_bit_cast(v2bf, xv[(base) + 2]), a0, false); \
    a1 = __builtin_amdgcn_fdot2_f32_bf16(w3, __builtin_bit_cast(v2bf, xv[(base) + 3]), a1, false); \
  }
  K3_DOT_DWORD(w.x, 0)
  K3_DOT_DWORD(w.y, 4)
  K3_DOT_DWORD(w.z, 8)
  K3_DOT_DWORD(w.w, 12)
#undef K3_DOT_DWORD
  return a0 + a1;
}

// fp32 activations: xv holds the chunk's 32 floats.  16 converts + 32 FMA.
__device__ __forceinline__ float chunk_dot_f32(u32x4 w, const float* xv) {
  float a0 = 0.0f, a1 = 0.0f;
#define K3_DOT_DWORD(d, base)                                                  \
  {                                                                            \
    v2f p0 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4((d), 1.0f, 0);           \
    v2f p1 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4((d), 1.0f, 1);           \
    v2f p2 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4((d), 1.0f, 2);           \
    v2f p3 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4((d), 1.0f, 3);           \
    a0 = fmaf(p0.x, xv[(base) + 0], a0);                                        \
    a1 = fmaf(p0.y, xv[(base) + 1], a1);                                        \
    a0 = fmaf(p1.x, xv[(base) + 2], a0);                                        \
    a1 = fmaf(p1.y, xv[(base) + 3], a1);                                        \
    a0 = fmaf(p2.x, xv[(base) + 4], a0);                                        \
    a1 = fmaf(p2.y, xv[(base) + 5], a1);                                        \
    a0 = fmaf(p3.x, xv[(base) + 6], a0);                                        \
    a1 = fmaf(p3.y, xv[(base) + 7], a1);                                        \
  }
  K3_DOT_DWORD(w.x, 0)
  K3_DOT_DWORD(w.y, 8)
  K3_DOT_DWORD(w.z, 16)
  K3_DOT_DWORD(w.w, 24)
#undef K3_DOT_DWORD
  return a0 + a1;
}

// Decode a chunk once into fp32 pairs (for reuse across several activations).
// One chunk against two fp32 activation chunks: each code pair is decoded
// once and feeds both sums (nothing decoded is held beyond its two FMAs).
__device__ __forceinline__ void chunk_dot_f32_x2(u32x4 w, const float* xa, const float* xb,
                                                 float& ra, float& rb) {
  float a0 = 0.0f, a1 = 0.0f, b0 = 0.0f, b1 = 0.0f;
#define K3_DOT2_PAIR(d, sel, base)                                              \
  {                                                                            \
    const v2f q = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4((d), 1.0f, (sel));  \
    a0 = fmaf(q.x, xa[(base) + 0], a0);                                         \
    a1 = fmaf(q.y, xa[(base) + 1], a1);                                         \
    b0 = fmaf(q.x, xb[(base) + 0], b0);                                         \
    b1 = fmaf(q.y, xb[(base) + 1], b1);                                         \
  }
#define K3_DOT2_DWORD(d, base) \
  K3_DOT2_PAIR(d, 0, (base) + 0) \
  K3_DOT2_PAIR(d, 1, (base) + 2) \
  K3_DOT2_PAIR(d, 2, (base) + 4) \
  K3_DOT2_PAIR(d, 3, (base) + 6)
  K3_DOT2_DWORD(w.x, 0)
  K3_DOT2_DWORD(w.y, 8)
  K3_DOT2_DWORD(w.z, 16)
  K3_DOT2_DWORD(w.w, 24)
#undef K3_DOT2_DWORD
#undef K3_DOT2_PAIR
  ra = a0 + a1;
  rb = b0 + b1;
}

__device__ __forceinline__ void chunk_decode_f32(u32x4 w, v2f* out16) {
#define K3_DEC_DWORD(d, base)                                                  \
  out16[(base) + 0] = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4((d), 1.0f, 0);  \
  out16[(base) + 1] = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4((d), 1.0f, 1);  \
  out16[(base) + 2] = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4((d), 1.0f, 2);  \
  out16[(base) + 3] = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4((d), 1.0f, 3);
  K3_DEC_DWORD(w.x, 0)
  K3_DEC_DWORD(w.y, 4)
  K3_DEC_DWORD(w.z, 8)
  K3_DEC_DWORD(w.w, 12)
#undef K3_DEC_DWORD
}

// Decode a chunk once into bf16 pairs.
__device__ __forceinline__ void chunk_decode_bf16(u32x4 w, v2bf* out16) {
#define K3_DEC_DWORD(d, base)                                                  \
  out16[(base) + 0] = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4((d), 1.0f, 0); \
  out16[(base) + 1] = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4((d), 1.0f, 1); \
  out16[(base) + 2] = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4((d), 1.0f, 2); \
  out16[(base) + 3] = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4((d), 1.0f, 3);
  K3_DEC_DWORD(w.x, 0)
  K3_DEC_DWORD(w.y, 4)
  K3_DEC_DWORD(w.z, 8)
  K3_DEC_DWORD(w.w, 12)
#undef K3_DEC_DWORD
}

__device__ __forceinline__ float dot_decoded_f32(const v2f* w16, const float* xv) {
  float a0 = 0.0f, a1 = 0.0f;
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    a0 = fmaf(w16[i].x, xv[2 * i], a0);
    a1 = fmaf(w16[i].y, xv[2 * i + 1], a1);
  }
  return a0 + a1;
}

__device__ __forceinline__ float dot_decoded_bf16(const v2bf* w16, const uint32_t* xv) {
  float a0 = 0.0f, a1 = 0.0f;
#pragma unroll
  for (int i = 0; i < 16; i += 2) {
    a0 = __builtin_amdgcn_fdot2_f32_bf16(w16[i], __builtin_bit_cast(v2bf, xv[i]), a0, false);
    a1 = __builtin_amdgcn_fdot2_f32_bf16(w16[i + 1], __builtin_bit_cast(v2bf, xv[i + 1]), a1, false);
  }
  return a0 + a1;
}

// ---------------------------------------------------------------- reductions
template <int kCtrl>
__device__ __forceinline__ float dpp_f32(float v) {
  return __builtin_bit_cast(
      float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), kCtrl, 0xf, 0xf, false));
}

// Full 64-lane sum; every lane receives the same value (each step adds a
// lane-pair symmetrically, so the order is fixed and lane-independent).
__device__ __forceinline__ float wave_sum(float v) {
  v += dpp_f32<0xB1>(v);   // quad_perm [1,0,3,2]
  v += dpp_f32<0x4E>(v);   // quad_perm [2,3,0,1]
  v += dpp_f32<0x141>(v);  // row_half_mirror
  v += dpp_f32<0x140>(v);  // row_mirror
  v += __shfl_xor(v, 16, kWave);
  v += __shfl_xor(v, 32, kWave);
  return v;
}

// Cross-lane partner exchange for the butterfly below.  Lanes are split by one
// lane bit ("upper" = bit set); a lane's partner has that bit flipped:
//   32: v_permlane32_swap (halves of the wave), 16: v_permlane16_swap (rows),
//   8: row_mirror (lane i <-> 15-i in a row), 4: row_half_mirror (i <-> 7-i),
//   2, 1: quad_perm xor.
// pair_step<o>(lo, hi, upper) returns, in every lane, the sum of the value this
// lane keeps (lo in lower lanes, hi in upper lanes) and the partner's value of
// the same index.
template <int kOff>
__device__ __forceinline__ float pair_step(float lo, float hi, bool upper) {
  if constexpr (kOff == 32 || kOff == 16) {
    // swap(vdst = lo, vsrc = hi): lower lanes get the partner's lo in the
    // second result, upper lanes get the partner's hi in the first.
    const auto r = kOff == 32
                       ? __builtin_amdgcn_permlane32_swap(__float_as_uint(lo), __float_as_uint(hi),
                                                          false, false)
                       : __builtin_amdgcn_permlane16_swap(__float_as_uint(lo), __float_as_uint(hi),
                                                          false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
  } else {
    constexpr int kCtrl = kOff == 8 ? 0x140 : kOff == 4 ? 0x141 : kOff == 2 ? 0x4E : 0xB1;
    const float keep = upper ? hi : lo;
    const float send = upper ? lo : hi;
    return keep + dpp_f32<kCtrl>(send);
  }
}

template <int kOff>
__device__ __forceinline__ float pair_all(float v) {
  return pair_step<kOff>(v, v, false);
}

// Butterfly reduction of N values per lane over the 64 lanes (N a power of two,
// N <= 64).  Afterwards v[0] in lane l holds the wave-wide sum of value
// index l >> (6 - log2 N); every lane of that group holds the same bits.  Each
// halving step costs one exchange per remaining pair, so reducing N values
// takes about N exchanges instead of 6 N.
template <int N>
__device__ __forceinline__ void wave_reduce_multi(float* v, int lane) {
  static_assert(N >= 1 && N <= 64 && (N & (N - 1)) == 0, "N must be a power of two <= 64");
#define K3_HALVE(OFF, CNT)                                                       \
  if constexpr (N >= (CNT)) {                                                    \
    const bool up = (lane & (OFF)) != 0;                                         \
    _Pragma("unroll") for (int i = 0; i < (CNT) / 2; ++i)                        \
      v[i] = pair_step<OFF>(v[i], v[i + (CNT) / 2], up);                         \
  }
  // Step s halves the count with lane bit 5-s; N values need log2 N steps.
  if constexpr (N >= 2) { K3_HALVE(32, N) }
  if constexpr (N >= 4) { K3_HALVE(16, N / 2) }
  if constexpr (N >= 8) { K3_HALVE(8, N / 4) }
  if constexpr (N >= 16) { K3_HALVE(4, N / 8) }
  if constexpr (N >= 32) { K3_HALVE(2, N / 16) }
  if constexpr (N >= 64) { K3_HALVE(1, N / 32) }
#undef K3_HALVE
  // Remaining lane bits: plain all-reduce of the single value.
  if constexpr (N < 2) v[0] = pair_all<32>(v[0]);
  if constexpr (N < 4) v[0] = pair_all<16>(v[0]);
  if constexpr (N < 8) v[0] = pair_all<8>(v[0]);
  if constexpr (N < 16) v[0] = pair_all<4>(v[0]);
  if constexpr (N < 32) v[0] = pair_all<2>(v[0]);
  if constexpr (N < 64) v[0] = pair_all<1>(v[0]);
}

template <int N>
constexpr int log2c() {
  return N <= 1 ? 0 : 1 + log2c<N / 2>();
}

// ---------------------------------------------------------------- activations
// K3 SiTU (provider_moe.cpp:524-533, tools/cuda_moe_kernels.cu:160-177) and
// SiLU-GLU, both in fp32 with the library's IEEE math flags.
__device__ __forceinline__ float activate(int act, float g, float u) {
  const float sig = 1.0f / (1.0f + expf(-g));
  if (act == 1) return g * sig * u;
  return (4.0f * tanhf(g / 4.0f) * sig) * (25.0f * tanhf(u / 25.0f));
}

// ---------------------------------------------------------------- loads
// Global-address-space views: loads through them compile to global_load (vmcnt
// only) rather than flat_load, which would also count against lgkmcnt and make
// every LDS wait drain the in-flight weight loads.
typedef __attribute__((address_space(1))) const u32x4 gu32x4;
typedef __attribute__((address_space(1))) const uint8_t gu8;
typedef __attribute__((address_space(1))) const uint32_t gu32;

__device__ __forceinline__ u32x4 load_chunk(const uint8_t* p) {
  return __builtin_nontemporal_load((gu32x4*)(p));
}

__device__ __forceinline__ uint32_t load_scale(const uint8_t* p) {
  return *(gu8*)(p);
}

__device__ __forceinline__ uint32_t load_u32(const uint8_t* p) {  // p 4-byte aligned
  return *(gu32*)(p);
}

// Buffer-resource loads: a wave-uniform descriptor (base, size), a per-lane
// byte offset and a wave-uniform byte offset in a scalar register, so a run
// of rows needs no per-row address registers.  Offsets past `bytes` read 0.
typedef __amdgpu_buffer_rsrc_t Rsrc;

__device__ __forceinline__ Rsrc make_rsrc(const uint8_t* base, uint32_t bytes) {
  // dword 3 0x00020000: raw 32-bit data format, no swizzle (gfx9 family).
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(base), (short)0, (int)bytes,
                                           0x00020000);
}

__device__ __forceinline__ u32x4 rsrc_load_chunk_nt(Rsrc r, uint32_t lane_off, uint32_t off) {
  return __builtin_amdgcn_raw_buffer_load_b128(r, lane_off, off, 2 /* nt */);
}

__device__ __forceinline__ uint32_t rsrc_load_u32(Rsrc r, uint32_t lane_off, uint32_t off) {
  return __builtin_amdgcn_raw_buffer_load_b32(r, lane_off, off, 0);
}

// The wave-uniform copy of a pointer, in scalar registers (lane 0's value).
// __builtin_amdgcn_readfirstlane returns a signed int, so each half passes
// through uint32_t before widening: a low word >= 2^31 widened from int would
// sign-extend into the high word and form a wild address.
__device__ __forceinline__ const uint8_t* uniform_ptr(const uint8_t* p) {
  const uint64_t v = reinterpret_cast<uint64_t>(p);
  const uint32_t lo = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)v);
  const uint32_t hi = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)(v >> 32));
  return reinterpret_cast<const uint8_t*>(((uint64_t)hi << 32) | (uint64_t)lo);
}

// Workgroup barrier ordering only LDS: outstanding global loads (prefetched
// weight batches) and global stores stay in flight across it.
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

template <typename T>
__device__ __forceinline__ T ld(const T* p) {
  return *p;
}

}  // namespace k3
