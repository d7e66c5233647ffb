/*
 * CPU oracle for the routed-expert MXFP4 path -- TEST INFRASTRUCTURE ONLY.
 * See orc.h.  Built with -ffp-contract=off so every fp32 rounding below is the
 * one written (the fp32 lane restatement depends on explicit fmaf()).
 */
#include "orc.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

/* tools/fused_gemv.c:243-246: codes 0..7 are +{0,.5,1,1.5,2,3,4,6}, bit 3 is
 * the sign (code 8 is -0). */
static const double k_e2m1[16] = {
    0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0,
    -0.0, -0.5, -1.0, -1.5, -2.0, -3.0, -4.0, -6.0,
};

double orc_e2m1(uint8_t code) { return k_e2m1[code & 15u]; }

static float e8m0_f32(uint8_t s) {
    /* tools/fused_gemv.c:247-249: the byte becomes the fp32 exponent field.
     * s = 0 therefore decodes to +0.0 and s = 255 to +inf. */
    union { uint32_t u; float f; } v;
    v.u = (uint32_t)s << 23;
    return v.f;
}

double orc_e8m0(uint8_t s) { return (double)e8m0_f32(s); }

/* Dequantized weight W[r, c] for the row-major layout of tools/fused_gemv.c:4-6:
 * packed [rows, cols/2] with the LOW nibble holding the even column, scales
 * [rows, cols/32]. */
static inline double weight_at(const uint8_t *pp, const uint8_t *sp, int c) {
    const uint8_t byte = pp[c >> 1];
    const uint8_t code = (c & 1) ? (uint8_t)(byte >> 4) : (uint8_t)(byte & 15u);
    return k_e2m1[code] * orc_e8m0(sp[c >> 5]);
}

void orc_gemv_f64_mag(const uint8_t *p, const uint8_t *s, const double *x,
                      double *y, double *mag, int rows, int cols) {
    const size_t cp = (size_t)cols / 2, groups = (size_t)cols / 32;
    for (int r = 0; r < rows; r++) {
        const uint8_t *pp = p + (size_t)r * cp;
        const uint8_t *sp = s + (size_t)r * groups;
        double acc = 0.0, m = 0.0;
        for (int c = 0; c < cols; c++) {
            const double t = weight_at(pp, sp, c) * x[c];
            acc += t;
            m += fabs(t);
        }
        y[r] = acc;
        if (mag) mag[r] = m;
    }
}

void orc_gemv_f64(const uint8_t *p, const uint8_t *s, const double *x,
                  double *y, int rows, int cols, int nan_on_255) {
    orc_gemv_f64_mag(p, s, x, y, NULL, rows, cols);
    if (!nan_on_255) return;
    const size_t groups = (size_t)cols / 32;
    for (int r = 0; r < rows; r++) {
        const uint8_t *sp = s + (size_t)r * groups;
        for (size_t g = 0; g < groups; g++) {
            if (sp[g] == 255u) {
                y[r] = NAN;
                break;
            }
        }
    }
}

void orc_gemv_f32_lanes(const uint8_t *p, const uint8_t *s, const float *x,
                        float *y, int rows, int cols) {
    const size_t cp = (size_t)cols / 2, groups = (size_t)cols / 32;
    for (int r = 0; r < rows; r++) {
        const uint8_t *pp = p + (size_t)r * cp;
        const uint8_t *sp = s + (size_t)r * groups;
        float lane[32];
        for (int k = 0; k < 32; k++) lane[k] = 0.0f;
        for (size_t g = 0; g < groups; g++) {
            const float scale = e8m0_f32(sp[g]);
            for (int k = 0; k < 32; k++) {
                const uint8_t byte = pp[g * 16 + (size_t)(k >> 1)];
                const uint8_t code = (k & 1) ? (uint8_t)(byte >> 4) : (uint8_t)(byte & 15u);
                /* fp32 product of table value and power-of-two scale, exactly as
                 * tools/fused_gemv.c:303-307 forms it, then one rounding per FMA. */
                const float w = (float)k_e2m1[code] * scale;
                lane[k] = fmaf(w, x[g * 32 + (size_t)k], lane[k]);
            }
        }
        /* reduce8 (tools/fused_gemv.c:282-288) over eight 4-lane vectors
         * v_j = lane[4j..4j+3], then the pairwise horizontal add. */
        float b[4][4], c[2][4], d[4];
        for (int i = 0; i < 4; i++) {
            b[0][i] = lane[0 + i] + lane[4 + i];
            b[1][i] = lane[8 + i] + lane[12 + i];
            b[2][i] = lane[16 + i] + lane[20 + i];
            b[3][i] = lane[24 + i] + lane[28 + i];
        }
        for (int i = 0; i < 4; i++) {
            c[0][i] = b[0][i] + b[1][i];
            c[1][i] = b[2][i] + b[3][i];
        }
        for (int i = 0; i < 4; i++) d[i] = c[0][i] + c[1][i];
        y[r] = (d[0] + d[1]) + (d[2] + d[3]);
    }
}

double orc_act(int act, double g, double u) {
    const double sig = 1.0 / (1.0 + exp(-g));
    if (act == ORC_ACT_SILU) return g * sig * u;
    /* SiTU, beta = 4, linear beta = 25 (provider_moe.cpp:524-533). */
    return (4.0 * tanh(g / 4.0) * sig) * (25.0 * tanh(u / 25.0));
}

void orc_expert_offsets(int hidden, int inter, uint64_t off[7]) {
    const uint64_t w13p = (uint64_t)inter * (uint64_t)hidden / 2;
    const uint64_t w13s = (uint64_t)inter * (uint64_t)(hidden / 32);
    const uint64_t w2p = (uint64_t)hidden * (uint64_t)inter / 2;
    const uint64_t w2s = (uint64_t)hidden * (uint64_t)(inter / 32);
    off[0] = 0;
    off[1] = w13p;
    off[2] = off[1] + w13s;
    off[3] = off[2] + w2p;
    off[4] = off[3] + w2s;
    off[5] = off[4] + w13p;
    off[6] = off[5] + w13s;
}

void orc_expert_f64(const uint8_t *span, int hidden, int inter, int act,
                    const double *x, double *y, double *h, double *mag) {
    uint64_t off[7];
    orc_expert_offsets(hidden, inter, off);
    double *gate = (double *)malloc(sizeof(double) * (size_t)inter);
    double *up = (double *)malloc(sizeof(double) * (size_t)inter);
    double *hh = h ? h : (double *)malloc(sizeof(double) * (size_t)inter);
    orc_gemv_f64(span + off[0], span + off[1], x, gate, inter, hidden, 1);
    orc_gemv_f64(span + off[4], span + off[5], x, up, inter, hidden, 1);
    for (int i = 0; i < inter; i++) hh[i] = orc_act(act, gate[i], up[i]);
    orc_gemv_f64_mag(span + off[2], span + off[3], hh, y, mag, hidden, inter);
    free(gate);
    free(up);
    if (!h) free(hh);
}

void orc_moe_layer_f64(const uint8_t *const *spans, int n_experts,
                       const double *weights, int hidden, int inter, int act,
                       const double *x, double *out, double *mag) {
    double *y = (double *)malloc(sizeof(double) * (size_t)hidden);
    double *m = (double *)malloc(sizeof(double) * (size_t)hidden);
    for (int i = 0; i < hidden; i++) {
        out[i] = 0.0;
        if (mag) mag[i] = 0.0;
    }
    for (int e = 0; e < n_experts; e++) {
        orc_expert_f64(spans[e], hidden, inter, act, x, y, NULL, m);
        for (int i = 0; i < hidden; i++) {
            out[i] += weights[e] * y[i];
            if (mag) mag[i] += fabs(weights[e]) * m[i];
        }
    }
    free(y);
    free(m);
}

/* The order the router ranks logits in: NaN as -inf and -0 as +0, so that the
 * order is total (ties then go to the lower index).  The reference does not
 * fix it for NaN: its router takes torch.topk and then rejects a route with a
 * non-finite weight (provider_moe.cpp:570-586, :1673-1683). */
static double rank_value(float v) {
    if (v != v) return -INFINITY;
    return v == 0.0f ? 0.0 : (double)v;
}

int orc_topk_softmax(const float *logits, int n, int k, int *ids,
                     double *weights) {
    if (n <= 0 || k <= 0 || k > n) return -1;
    char *taken = (char *)calloc((size_t)n, 1);
    if (!taken) return -1;
    /* k rounds of argmax: strictly greater wins, so the lower index keeps a tie. */
    for (int j = 0; j < k; j++) {
        int best = -1;
        for (int i = 0; i < n; i++) {
            if (taken[i]) continue;
            if (best < 0 || rank_value(logits[i]) > rank_value(logits[best])) best = i;
        }
        taken[best] = 1;
        ids[j] = best;
    }
    free(taken);
    const double top = rank_value(logits[ids[0]]);
    double sum = 0.0;
    for (int j = 0; j < k; j++) {
        weights[j] = exp(rank_value(logits[ids[j]]) - top);
        sum += weights[j];
    }
    for (int j = 0; j < k; j++) weights[j] /= sum;
    return 0;
}

static inline uint64_t mix64(uint64_t z) {
    z = (z ^ (z >> 30)) * UINT64_C(0xBF58476D1CE4E5B9);
    z = (z ^ (z >> 27)) * UINT64_C(0x94D049BB133111EB);
    return z ^ (z >> 31);
}

uint64_t orc_rand_u64(uint64_t seed, uint64_t stream, uint64_t index) {
    const uint64_t key = mix64(seed ^ mix64(stream ^ UINT64_C(0xD1B54A32D192ED03)));
    return mix64(key + (index + 1) * UINT64_C(0x9E3779B97F4A7C15));
}

void orc_synth_mxfp4(uint64_t seed, uint64_t stream, uint8_t *packed,
                     uint64_t n_packed, uint8_t *scales, uint64_t n_scales,
                     int scale_lo, int scale_hi) {
    /* Packed byte i is byte (i % 8) of draw i / 8 of stream 2*stream, so every
     * nibble is uniform over the 16 codes; scale i is lo + draw i mod (hi-lo+1)
     * of stream 2*stream+1. */
    for (uint64_t i = 0; i < n_packed; i++) {
        const uint64_t v = orc_rand_u64(seed, 2 * stream, i >> 3);
        packed[i] = (uint8_t)(v >> (8 * (i & 7)));
    }
    const uint64_t span = (uint64_t)(scale_hi - scale_lo + 1);
    for (uint64_t i = 0; i < n_scales; i++) {
        const uint64_t v = orc_rand_u64(seed, 2 * stream + 1, i);
        scales[i] = (uint8_t)(scale_lo + (int)(v % span));
    }
}

void orc_synth_expert(uint64_t seed, uint64_t expert, int hidden, int inter,
                      uint8_t *span, int scale_lo, int scale_hi) {
    uint64_t off[7];
    orc_expert_offsets(hidden, inter, off);
    const uint64_t w13p = off[1] - off[0], w13s = off[2] - off[1];
    const uint64_t w2p = off[3] - off[2], w2s = off[4] - off[3];
    /* matrix streams: w1 = 3e, w2 = 3e+1, w3 = 3e+2 */
    orc_synth_mxfp4(seed, 3 * expert + 0, span + off[0], w13p, span + off[1], w13s,
                    scale_lo, scale_hi);
    orc_synth_mxfp4(seed, 3 * expert + 1, span + off[2], w2p, span + off[3], w2s,
                    scale_lo, scale_hi);
    orc_synth_mxfp4(seed, 3 * expert + 2, span + off[4], w13p, span + off[5], w13s,
                    scale_lo, scale_hi);
}

/* ------------------------------------------------------------ scale4-v2 */
int orc_scale4_pack(const uint8_t *values, uint64_t n, int base, uint8_t *packed) {
    if (base < 0 || base > 240) return -1;
    for (uint64_t i = 0; i < (n + 1) / 2; i++) packed[i] = 0;
    for (uint64_t i = 0; i < n; i++) {
        const int d = (int)values[i] - base;
        if (d < 0 || d > 15) return -1;
        packed[i / 2] |= (uint8_t)(d << ((i & 1) * 4));
    }
    return 0;
}

int orc_scale4_unpack(const uint8_t *packed, uint64_t n, int base, uint8_t *values) {
    if (base < 0 || base > 240) return -1;
    for (uint64_t i = 0; i < n; i++)
        values[i] = (uint8_t)(base + ((packed[i / 2] >> ((i & 1) * 4)) & 0x0F));
    return 0;
}

static void put32(uint8_t *p, uint32_t v) {
    for (int i = 0; i < 4; i++) p[i] = (uint8_t)(v >> (8 * i));
}

int orc_scale4_header(const uint8_t *digest32, const uint8_t *bases3, uint8_t *header) {
    /* K3: packed planes 3072 x 3584 / 2 bytes, index planes half a byte per
     * 32-element group. */
    const uint32_t hdr = 8192, packed = 5505024, s4 = 344064 / 2;
    for (int m = 0; m < 3; m++)
        if (bases3[m] > 240) return -1;
    for (int i = 0; i < 8192; i++) header[i] = 0;
    memcpy(header, "K3SC4V2", 8);  /* the terminating zero is the 8th byte */
    put32(header + 8, 2);
    put32(header + 12, hdr);
    put32(header + 16, hdr + 3 * (packed + s4));
    put32(header + 24, 3 * (packed + 344064));
    memcpy(header + 32, digest32, 32);
    memcpy(header + 64, bases3, 3);
    uint32_t off = hdr;
    for (int m = 0; m < 3; m++) {
        put32(header + 72 + 16 * m, off);
        put32(header + 76 + 16 * m, packed);
        off += packed;
        put32(header + 80 + 16 * m, off);
        put32(header + 84 + 16 * m, s4);
        off += s4;
    }
    for (int m = 0; m < 3; m++)
        for (uint32_t d = 0; d < 16; d++)
            put32(header + 128 + 64 * m + 4 * d, ((uint32_t)bases3[m] + d) << 23);
    for (int m = 0; m < 3; m++) {
        put32(header + 320 + 8 * m, hdr + m * s4);
        put32(header + 324 + 8 * m, s4);
    }
    return 0;
}
