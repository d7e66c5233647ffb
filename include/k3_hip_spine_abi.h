#ifndef K3_HIP_SPINE_ABI_H
#define K3_HIP_SPINE_ABI_H
/*
 * Resident "spine" projections on either side of the routed experts, for
 * gfx950 (MI355X).  The reference's MoE block runs them around the expert
 * set (native/provider_gate/provider_moe.cpp:1673-1688 before it:
 * router logits and routed_down; :1997-2014 after it: routed RMS norm,
 * routed_up, shared expert, merge).  Its device kernel for them is the exact
 * RAW_BF16 x FP32 GEMV of native/provider_gate/provider_spine_bf16_cuda.cu;
 * the k3_hip_spine_bf16_* entry points below replace that file's
 * k3_cuda_spine_bf16_* exports one for one (same arguments, statuses and
 * ownership).  The row-int8 projection and the RMS norm have no reference
 * device kernel (the reference runs them through ATen); their entry points
 * follow the ATen calls they replace.
 *
 * Conventions of this surface (as the reference's, :28-40 and :245-280):
 *   - statuses: 0 ok, -1 invalid argument, -2 HIP runtime error,
 *     -3 unsupported device; *_available returns 1 when usable;
 *   - nothing allocates, synchronises, creates a stream or keeps a pointer;
 *     work is enqueued on `stream` (a hipStream_t, NULL = the null stream)
 *     and the caller keeps every buffer alive until that work completes;
 *   - a failed call enqueues nothing; the reason is in
 *     k3_hip_spine_last_error() (thread-local).
 * Every matrix is row-major [rows, columns] and dense; activations are fp32
 * [positions, columns], outputs fp32 [positions, rows], positions 1..64.
 */
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
  K3_SPINE_OK = 0,
  K3_SPINE_E_INVALID = -1,
  K3_SPINE_E_RUNTIME = -2,
  K3_SPINE_E_UNSUPPORTED = -3,
};

#define K3_SPINE_ABI_VERSION 1u
#define K3_SPINE_MAX_POSITIONS 64
#define K3_RMS_EPSILON 1.0e-5f /* the reference's kRmsEpsilon (provider_moe.cpp:87) */

/* Replaces k3_cuda_spine_bf16_abi_version (provider_spine_bf16_cuda.cu:187-189). */
uint32_t k3_hip_spine_bf16_abi_version(void);

/* Replaces k3_cuda_spine_bf16_last_error (:191-193); shared by every
 * k3_hip_spine_* and k3_hip_rms_norm entry point. */
const char* k3_hip_spine_last_error(void);

/* Replaces k3_cuda_spine_bf16_available (:195-251): 1 when `device` is a
 * usable gfx950 (compute_major / compute_minor, when non-null, receive its
 * architecture version, 9 / 5), else a negative status. */
int k3_hip_spine_bf16_available(int device, int* compute_major,
                                int* compute_minor);

/* Replaces k3_cuda_spine_bf16_launch_v1 (:253-278):
 * output[p, r] = sum_c bf16(weights[r, c]) * activation[p, c], every BF16 bit
 * pattern widened exactly (bits << 16) and every product and sum in fp32.
 * weights: uint16 BF16 bits [rows, columns]. */
int k3_hip_spine_bf16_launch_v1(const uint16_t* weights,
                                const float* activation, float* output,
                                int rows, int columns, int positions,
                                void* stream);

/* Replaces k3_cuda_spine_bf16_decode_bits (:282-303): output[i] = the fp32
 * bit pattern of BF16 input[i] (bits << 16), count > 0. */
int k3_hip_spine_bf16_decode_bits(const uint16_t* input, uint32_t* output,
                                  int count, void* stream);

/* Row-int8 projection, the packed-int8 form of the same spine matrices
 * (at::_weight_int8pack_mm(input, quantized, row_scales) in row_int8_linear,
 * provider_moe.cpp:507-516): output[p, r] = row_scales[r] *
 * sum_c quantized[r, c] * activation[p, c], in fp32. */
int k3_hip_spine_int8_launch_v1(const int8_t* quantized,
                                const float* row_scales,
                                const float* activation, float* output,
                                int rows, int columns, int positions,
                                void* stream);

/* Routed RMS norm (rms_norm, provider_moe.cpp:535-542):
 * output[p, c] = weight[c] * (input[p, c] * rsqrt(mean_c(input[p, :]^2) + eps)),
 * fp32 throughout; the reference's eps is 1e-5 (:87).  rows >= 1,
 * columns >= 1; input and output may be the same buffer. */
int k3_hip_rms_norm(const float* input, const float* weight, float* output,
                    int rows, int columns, float eps, void* stream);

#ifdef __cplusplus
}
#endif
#endif /* K3_HIP_SPINE_ABI_H */
