/*
 * CPU oracle for the routed-expert MXFP4 path.  TEST INFRASTRUCTURE ONLY:
 * nothing in the product library links, loads or calls this code.  It is the
 * checker used by tests/, __graft_entry__.smoke() and bench.py's cpu_baseline
 * leg, never the thing measured or shipped.
 *
 * Every function restates the reference algorithm from the mathematics and
 * cites the reference file:line it follows (paths relative to the deltafin
 * source tree).  Pins for each function are listed in oracle/README.md.
 */
#ifndef K3_ORACLE_ORC_H
#define K3_ORACLE_ORC_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum { ORC_ACT_SITU = 0, ORC_ACT_SILU = 1 };

/* E2M1 nibble -> value (tools/fused_gemv.c:243-246). */
double orc_e2m1(uint8_t code);
/* E8M0 byte -> fp32 bits s<<23, widened to double (tools/fused_gemv.c:247-249). */
double orc_e8m0(uint8_t s);

/* fp64-accumulated dequant GEMV y = W x (tools/fused_gemv.c:4-6 layout,
 * :291-319 semantics).  nan_on_255 != 0 reproduces the device reference rule
 * that a 255 scale byte poisons its row with NaN (tools/cuda_moe_kernels.cu:128-131). */
void orc_gemv_f64(const uint8_t *p, const uint8_t *s, const double *x,
                  double *y, int rows, int cols, int nan_on_255);
/* Same, also returning mag[r] = sum_c |W[r,c] x[c]| (condition scale). */
void orc_gemv_f64_mag(const uint8_t *p, const uint8_t *s, const double *x,
                      double *y, double *mag, int rows, int cols);
/* fp32 restatement of the reference lane order: 32 independent FMA chains
 * (lane k <-> column 32g+k) folded by reduce8 and a pairwise horizontal add
 * (tools/fused_gemv.c:282-319, tools/neon_compat_x86.h:75-79).  Bit-exact with
 * the reference CPU kernel for scale bytes in [2, 252]. */
void orc_gemv_f32_lanes(const uint8_t *p, const uint8_t *s, const float *x,
                        float *y, int rows, int cols);

/* Activations in fp64.  SiTU follows provider_moe.cpp:524-533 /
 * tools/fused_gemv_batch.c:171-183; SiLU-GLU is g*sigmoid(g)*u (closed form,
 * no reference implementation). */
double orc_act(int act, double g, double u);

/* Expert span offsets for raw-v1 ordering w1p,w1s,w2p,w2s,w3p,w3s
 * (native/provider_gate/provider_moe.cpp:217-243).  off[7] = {w1p, w1s, w2p,
 * w2s, w3p, w3s, span}. */
void orc_expert_offsets(int hidden, int inter, uint64_t off[7]);

/* One expert FFN in fp64: gate = W1 x, up = W3 x, h = act(gate, up), y = W2 h
 * (tools/fused_gemv_batch.c:465-518 phase order).  h and mag may be NULL;
 * mag[i] = sum_j |W2[i,j] h[j]|. */
void orc_expert_f64(const uint8_t *span, int hidden, int inter, int act,
                    const double *x, double *y, double *h, double *mag);

/* Ordered weighted combine out = sum_e w[e] * expert_e(x) in route order
 * (tools/fused_gemv_batch.c:512-516, provider_moe.cpp:959-968), fp64.
 * mag[i] = sum_e |w[e]| * mag_e[i]. */
void orc_moe_layer_f64(const uint8_t *const *spans, int n_experts,
                       const double *weights, int hidden, int inter, int act,
                       const double *x, double *out, double *mag);

/* Router for the synthetic configs: top-k of n logits, descending value, lower
 * index on ties, then softmax over the k selected values in fp64. */
int orc_topk_softmax(const float *logits, int n, int k, int *ids,
                     double *weights);

/* Counter-based synthetic generator (SplitMix64 finaliser of a keyed
 * counter).  Identical in C, numpy and HIP. */
uint64_t orc_rand_u64(uint64_t seed, uint64_t stream, uint64_t index);
/* Fill packed bytes (uniform) and scales (uniform in [lo, hi]). */
void orc_synth_mxfp4(uint64_t seed, uint64_t stream, uint8_t *packed,
                     uint64_t n_packed, uint8_t *scales, uint64_t n_scales,
                     int scale_lo, int scale_hi);
/* Fill a raw-v1 expert span for (hidden, inter) with the synthetic
 * distribution; stream selects the expert. */
void orc_synth_expert(uint64_t seed, uint64_t expert, int hidden, int inter,
                      uint8_t *span, int scale_lo, int scale_hi);

/* scale4-v2 codec (native/deltafin/src/expert_scale4.rs:114-171): entry i of
 * a scale plane is the 4-bit index value - base, in byte i/2, low nibble for
 * even i.  pack returns -1 when base > 240 or a value lies outside
 * [base, base + 15]; unpack returns -1 when base > 240. */
int orc_scale4_pack(const uint8_t *values, uint64_t n, int base, uint8_t *packed);
int orc_scale4_unpack(const uint8_t *packed, uint64_t n, int base, uint8_t *values);
/* The 8192-byte scale4-v2 header for the K3 geometry (expert_scale4.rs:173-208):
 * identity and lengths, the 32-byte source digest, the three bases, the
 * in-memory payload table, the exponent tables (base + d) << 23 at 128 / 192 /
 * 256 and the on-disk sidecar table at 320.  -1 when a base exceeds 240. */
int orc_scale4_header(const uint8_t *digest32, const uint8_t *bases3, uint8_t *header);

#ifdef __cplusplus
}
#endif

#endif
