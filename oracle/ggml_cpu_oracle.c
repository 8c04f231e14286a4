/*
 * ggml_cpu_oracle.c — CPU reference backend: restated ggml-cpu arithmetic for the ops on
 * GGML-Loader's forward_step path (reference src/model.cpp:1071-1474).
 *
 * TEST INFRASTRUCTURE ONLY (see oracle.h). Built with gcc -O2 -ffp-contract=off -fopenmp.
 *
 * Semantics restated here, per op (upstream ggml is absent from the reference, so these follow
 * ggml-cpu's portable scalar paths; deviations are noted inline):
 *   MUL_MAT   src1 rows are converted to the weight's dot type first (Q4_0/Q8_0 -> Q8_0,
 *             Q4_K -> Q8_K, F16 -> F16, F32 stays), then one block-integer dot per block with a
 *             float block-sum (ggml_vec_dot_*_generic). F16/F32 dots accumulate in double.
 *   RMS_NORM  sum of x*x in double, mean cast to float, scale = 1/sqrtf(mean + eps).
 *   SOFT_MAX  w = x*scale + mask; max; exp(w - max) summed in double; scale by 1/sum.
 *   ROPE      per-position cos/sin cache with theta *= theta_scale iterated in float,
 *             theta_scale = powf(base, -2/n_dims); NORMAL pairs (2i, 2i+1), NEOX (i, i+n_dims/2).
 *   SILU      x / (1 + exp(-x)).
 *   exp/cos/sin are correctly rounded (see exp_cr below).
 *   CPY/CONT  element-wise with f32 -> f16 round-to-nearest-even.
 */
#include "oracle.h"

#include "ggml.h"
#include "ggml-backend-impl.h"
#include "ggml-cpu.h"

#include <math.h>
#include <omp.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

typedef double ggml_float;

/* planted-mistake bits (oracle_set_planted in oracle.h): 0 in every normal use */
static int g_planted = 0;
void oracle_set_planted(int bits) { g_planted = bits; }

/* Transcendentals of the float ops (RoPE cos/sin, softmax and SiLU exp) are the correctly rounded
 * float results: evaluated in double and rounded once. ggml-cpu calls the platform's cosf/sinf/
 * expf, whose last-ulp behaviour differs between libms (glibc's cosf/sinf are off by one ulp on
 * ~1% of RoPE angles; the reference itself targets Android's bionic), so the oracle fixes the
 * platform-independent choice and the HIP backend evaluates the same way. */
static inline float exp_cr(float x) { return (float) exp((double) x); }
static inline float cos_cr(float x) { return (float) cos((double) x); }
static inline float sin_cr(float x) { return (float) sin((double) x); }
static inline float log_cr(float x) { return (float) log((double) x); }
// softplus (ggml's GGML_UNARY_OP_SOFTPLUS): x above 20, else log(1 + exp(x)), in double rounded
// once. No reference source or fixture holds this op: parity unpinned beyond its closed form.
static inline float softplus_cr(float x) { return x > 20.0f ? x : (float) log1p(exp((double) x)); }

/* ------------------------------------------------------------------------------------------ */
/* binary16 — the branch-free formulation of the FP16 library (fp16_ieee_{from,to}_fp32_value),
 * which ggml's own scalar path also uses; an independent formulation from the product's. */

static inline uint32_t fbits(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline float bitsf(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

float oracle_fp16_to_fp32(uint16_t h) {
    const uint32_t w = (uint32_t) h << 16;
    const uint32_t sign = w & 0x80000000u;
    const uint32_t two_w = w + w;
    const uint32_t exp_offset = 0xE0u << 23;
    const float exp_scale = 0x1.0p-112f;
    const float normalized = bitsf((two_w >> 4) + exp_offset) * exp_scale;
    const uint32_t magic_mask = 126u << 23;
    const float magic_bias = 0.5f;
    const float denormalized = bitsf((two_w >> 17) | magic_mask) - magic_bias;
    const uint32_t cutoff = 1u << 27;
    return bitsf(sign | (two_w < cutoff ? fbits(denormalized) : fbits(normalized)));
}

uint16_t oracle_fp32_to_fp16(float f) {
    const float scale_to_inf = 0x1.0p+112f;
    const float scale_to_zero = 0x1.0p-110f;
    float base = (fabsf(f) * scale_to_inf) * scale_to_zero;
    const uint32_t w = fbits(f);
    const uint32_t shl1_w = w + w;
    const uint32_t sign = w & 0x80000000u;
    uint32_t bias = shl1_w & 0xFF000000u;
    if (bias < 0x71000000u) bias = 0x71000000u;
    base = bitsf((bias >> 1) + 0x07800000u) + base;
    const uint32_t bits = fbits(base);
    const uint32_t exp_bits = (bits >> 13) & 0x00007C00u;
    const uint32_t mantissa_bits = bits & 0x00000FFFu;
    const uint32_t nonsign = exp_bits + mantissa_bits;
    return (uint16_t) ((sign >> 16) | (shl1_w > 0xFF000000u ? 0x7E00u : nonsign));
}

#define F16(h) oracle_fp16_to_fp32(h)

/* ------------------------------------------------------------------------------------------ */
/* GGUF block formats (same layouts the reference decodes in moe_stream/dequant.c:39-206)     */

typedef struct { uint16_t d; uint8_t qs[16]; } bq4_0;
typedef struct { uint16_t d; int8_t qs[32]; } bq8_0;
typedef struct { uint16_t d; uint16_t dmin; uint8_t scales[12]; uint8_t qs[128]; } bq4_K;
typedef struct { float d; int8_t qs[256]; int16_t bsums[16]; } bq8_K;
typedef struct { uint16_t d; uint16_t dmin; uint8_t scales[12]; uint8_t qh[32]; uint8_t qs[128]; } bq5_K;
typedef struct { uint8_t ql[128]; uint8_t qh[64]; int8_t scales[16]; uint16_t d; } bq6_K;

_Static_assert(sizeof(bq4_0) == 18, "q4_0");
_Static_assert(sizeof(bq8_0) == 34, "q8_0");
_Static_assert(sizeof(bq4_K) == 144, "q4_K");
_Static_assert(sizeof(bq8_K) == 292, "q8_K");
_Static_assert(sizeof(bq5_K) == 176, "q5_K");
_Static_assert(sizeof(bq6_K) == 210, "q6_K");

/* ggml's nearest_int: round half to even through the float mantissa, |v| < 2^22 */
static inline int nearest_int(float v) {
    float t = v + 12582912.f;
    int32_t i;
    memcpy(&i, &t, 4);
    return (i & 0x007fffff) - 0x00400000;
}

/* moe_stream/dequant.c:132-141 (get_scale_min_k4) */
static inline void scale_min_k4(int j, const uint8_t * q, uint8_t * d, uint8_t * m) {
    if (j < 4) {
        *d = q[j] & 63;
        *m = q[j + 4] & 63;
    } else {
        *d = (uint8_t) ((q[j + 4] & 0xF) | ((q[j - 4] >> 6) << 4));
        *m = (uint8_t) ((q[j + 4] >> 4) | ((q[j] >> 6) << 4));
    }
}

void oracle_quantize_q4_0(const float * x, void * vy, int64_t k) {
    bq4_0 * y = (bq4_0 *) vy;
    for (int64_t i = 0; i < k / 32; i++) {
        float amax = 0.0f, max = 0.0f;
        for (int j = 0; j < 32; j++) {
            const float v = x[i * 32 + j];
            if (amax < fabsf(v)) { amax = fabsf(v); max = v; }
        }
        const float d = max / -8;
        const float id = d ? 1.0f / d : 0.0f;
        y[i].d = oracle_fp32_to_fp16(d);
        for (int j = 0; j < 16; ++j) {
            const float x0 = x[i * 32 + j] * id;
            const float x1 = x[i * 32 + 16 + j] * id;
            const float half = g_planted & 8 ? 8.0f : 8.5f;
            const int8_t a = (int8_t) (x0 + half);
            const int8_t b = (int8_t) (x1 + half);
            const uint8_t xi0 = (uint8_t) (a < 15 ? a : 15);
            const uint8_t xi1 = (uint8_t) (b < 15 ? b : 15);
            y[i].qs[j] = (uint8_t) (xi0 | (xi1 << 4));
        }
    }
}

void oracle_quantize_q8_0(const float * x, void * vy, int64_t k) {
    bq8_0 * y = (bq8_0 *) vy;
    for (int64_t i = 0; i < k / 32; i++) {
        float amax = 0.0f;
        for (int j = 0; j < 32; j++) {
            const float v = fabsf(x[i * 32 + j]);
            amax = amax > v ? amax : v;
        }
        const float d = amax / ((1 << 7) - 1);
        const float id = d ? 1.0f / d : 0.0f;
        y[i].d = oracle_fp32_to_fp16(d);
        for (int j = 0; j < 32; ++j) y[i].qs[j] = (int8_t) roundf(x[i * 32 + j] * id);
    }
}

void oracle_quantize_q8_K(const float * x, void * vy, int64_t k) {
    bq8_K * y = (bq8_K *) vy;
    for (int64_t i = 0; i < k / 256; i++) {
        const float * xb = x + i * 256;
        float max = 0, amax = 0;
        for (int j = 0; j < 256; ++j) {
            const float ax = fabsf(xb[j]);
            if (ax > amax) { amax = ax; max = xb[j]; }
        }
        memset(&y[i], 0, sizeof(bq8_K));
        if (!amax) continue;
        const float iscale = -127.f / max;
        for (int j = 0; j < 256; ++j) {
            const int v = nearest_int(iscale * xb[j]);
            y[i].qs[j] = (int8_t) (v < 127 ? v : 127);
        }
        for (int j = 0; j < 16; ++j) {
            int sum = 0;
            for (int ii = 0; ii < 16; ++ii) sum += y[i].qs[j * 16 + ii];
            y[i].bsums[j] = (int16_t) sum;
        }
        y[i].d = 1 / iscale;
    }
}

/* ggml's make_qkx2_quants: weighted least-squares asymmetric grid fit with a scale search */
static float make_qkx2_quants(int n, int nmax, const float * x, const float * weights, uint8_t * L,
                              float * the_min, uint8_t * Laux, float rmin, float rdelta, int nstep) {
    float min = x[0], max = x[0];
    float sum_w = weights[0];
    float sum_x = sum_w * x[0];
    for (int i = 1; i < n; ++i) {
        if (x[i] < min) min = x[i];
        if (x[i] > max) max = x[i];
        const float w = weights[i];
        sum_w += w;
        sum_x += w * x[i];
    }
    if (min > 0) min = 0;
    if (max == min) {
        for (int i = 0; i < n; ++i) L[i] = 0;
        *the_min = -min;
        return 0.f;
    }
    if (g_planted & 16) nstep = -1;
    float iscale = nmax / (max - min);
    float scale = 1 / iscale;
    float best_error = 0;
    for (int i = 0; i < n; ++i) {
        int l = nearest_int(iscale * (x[i] - min));
        L[i] = (uint8_t) (l < 0 ? 0 : (l > nmax ? nmax : l));
        float diff = scale * L[i] + min - x[i];
        diff = diff * diff;
        best_error += weights[i] * diff;
    }
    for (int is = 0; is <= nstep; ++is) {
        iscale = (rmin + rdelta * is + nmax) / (max - min);
        float sum_l = 0, sum_l2 = 0, sum_xl = 0;
        for (int i = 0; i < n; ++i) {
            int l = nearest_int(iscale * (x[i] - min));
            l = l < 0 ? 0 : (l > nmax ? nmax : l);
            Laux[i] = (uint8_t) l;
            const float w = weights[i];
            sum_l += w * l;
            sum_l2 += w * l * l;
            sum_xl += w * l * x[i];
        }
        const float D = sum_w * sum_l2 - sum_l * sum_l;
        if (D > 0) {
            float this_scale = (sum_w * sum_xl - sum_x * sum_l) / D;
            float this_min = (sum_l2 * sum_x - sum_l * sum_xl) / D;
            if (this_min > 0) {
                this_min = 0;
                this_scale = sum_xl / sum_l2;
            }
            float cur_error = 0;
            for (int i = 0; i < n; ++i) {
                float diff = this_scale * Laux[i] + this_min - x[i];
                diff = diff * diff;
                cur_error += weights[i] * diff;
            }
            if (cur_error < best_error) {
                for (int i = 0; i < n; ++i) L[i] = Laux[i];
                best_error = cur_error;
                scale = this_scale;
                min = this_min;
            }
        }
    }
    *the_min = -min;
    return scale;
}

/* exported for the tests: one sub-block's grid fit, exactly as oracle_quantize_q4_K calls it */
float oracle_make_qkx2_quants(int n, int nmax, const float * x, const float * weights, uint8_t * L, float * the_min,
                              float rmin, float rdelta, int nstep) {
    uint8_t Laux[256];
    if (n > 256) return -1.f;
    return make_qkx2_quants(n, nmax, x, weights, L, the_min, Laux, rmin, rdelta, nstep);
}

void oracle_quantize_q4_K(const float * x, void * vy, int64_t k) {
    bq4_K * y = (bq4_K *) vy;
    uint8_t L[256], Laux[32];
    float weights[32], mins[8], scales[8];
    for (int64_t i = 0; i < k / 256; i++) {
        const float * xb = x + i * 256;
        float max_scale = 0, max_min = 0;
        for (int j = 0; j < 8; ++j) {
            float sum_x2 = 0;
            for (int l = 0; l < 32; ++l) sum_x2 += xb[32 * j + l] * xb[32 * j + l];
            const float av_x = sqrtf(sum_x2 / 32);
            for (int l = 0; l < 32; ++l) weights[l] = g_planted & 32 ? 1.0f : av_x + fabsf(xb[32 * j + l]);
            scales[j] = make_qkx2_quants(32, 15, xb + 32 * j, weights, L + 32 * j, &mins[j], Laux, -1.f, 0.1f, 20);
            if (scales[j] > max_scale) max_scale = scales[j];
            if (mins[j] > max_min) max_min = mins[j];
        }
        const float inv_scale = max_scale > 0 ? 63.f / max_scale : 0.f;
        const float inv_min = max_min > 0 ? 63.f / max_min : 0.f;
        for (int j = 0; j < 8; ++j) {
            uint8_t ls = (uint8_t) nearest_int(inv_scale * scales[j]);
            uint8_t lm = (uint8_t) nearest_int(inv_min * mins[j]);
            ls = ls < 63 ? ls : 63;
            lm = lm < 63 ? lm : 63;
            if (j < 4) {
                y[i].scales[j] = ls;
                y[i].scales[j + 4] = lm;
            } else {
                y[i].scales[j + 4] = (uint8_t) ((ls & 0xF) | ((lm & 0xF) << 4));
                y[i].scales[j - 4] |= (uint8_t) ((ls >> 4) << 6);
                y[i].scales[j - 0] |= (uint8_t) ((lm >> 4) << 6);
            }
        }
        y[i].d = oracle_fp32_to_fp16(max_scale / 63.f);
        y[i].dmin = oracle_fp32_to_fp16(max_min / 63.f);
        for (int j = 0; j < 8; ++j) {
            uint8_t sc, m;
            scale_min_k4(j, y[i].scales, &sc, &m);
            const float d = F16(y[i].d) * sc;
            if (!d) continue;
            const float dm = F16(y[i].dmin) * m;
            for (int ii = 0; ii < 32; ++ii) {
                int l = nearest_int((xb[32 * j + ii] + dm) / d);
                l = l < 0 ? 0 : (l > 15 ? 15 : l);
                L[32 * j + ii] = (uint8_t) l;
            }
        }
        uint8_t * q = y[i].qs;
        for (int j = 0; j < 256; j += 64) {
            for (int l = 0; l < 32; ++l) q[l] = (uint8_t) (L[j + l] | (L[j + l + 32] << 4));
            q += 32;
        }
    }
}

/* The 6-bit scale and min codes of eight sub-blocks packed into 12 bytes (the layout
   scale_min_k4 reads back), from the float scales and mins and their maxima. */
static void pack_scale_min_k4(const float * scales, const float * mins, float max_scale, float max_min, uint8_t * out) {
    const float inv_scale = max_scale > 0 ? 63.f / max_scale : 0.f;
    const float inv_min = max_min > 0 ? 63.f / max_min : 0.f;
    memset(out, 0, 12);
    for (int j = 0; j < 8; ++j) {
        uint8_t ls = (uint8_t) nearest_int(inv_scale * scales[j]);
        uint8_t lm = (uint8_t) nearest_int(inv_min * mins[j]);
        ls = ls < 63 ? ls : 63;
        lm = lm < 63 ? lm : 63;
        if (j < 4) {
            out[j] = ls;
            out[j + 4] = lm;
        } else {
            out[j + 4] = (uint8_t) ((ls & 0xF) | ((lm & 0xF) << 4));
            out[j - 4] |= (uint8_t) ((ls >> 4) << 6);
            out[j - 0] |= (uint8_t) ((lm >> 4) << 6);
        }
    }
}

/* ggml's quantize_row_q5_K_ref: as Q4_K with 5-bit codes (0..31), the grid search of each
   sub-block over 16 rescalings starting at -0.5; the fifth bit of element l of sub-block j goes
   to bit j of qh[l]. */
void oracle_quantize_q5_K(const float * x, void * vy, int64_t k) {
    bq5_K * y = (bq5_K *) vy;
    uint8_t L[256], Laux[32];
    float weights[32], mins[8], scales[8];
    for (int64_t i = 0; i < k / 256; i++) {
        const float * xb = x + i * 256;
        float max_scale = 0, max_min = 0;
        for (int j = 0; j < 8; ++j) {
            float sum_x2 = 0;
            for (int l = 0; l < 32; ++l) sum_x2 += xb[32 * j + l] * xb[32 * j + l];
            const float av_x = sqrtf(sum_x2 / 32);
            for (int l = 0; l < 32; ++l) weights[l] = av_x + fabsf(xb[32 * j + l]);
            scales[j] = make_qkx2_quants(32, 31, xb + 32 * j, weights, L + 32 * j, &mins[j], Laux, -0.5f, 0.1f, 15);
            if (scales[j] > max_scale) max_scale = scales[j];
            if (mins[j] > max_min) max_min = mins[j];
        }
        pack_scale_min_k4(scales, mins, max_scale, max_min, y[i].scales);
        y[i].d = oracle_fp32_to_fp16(max_scale / 63.f);
        y[i].dmin = oracle_fp32_to_fp16(max_min / 63.f);
        for (int j = 0; j < 8; ++j) {
            uint8_t sc, m;
            scale_min_k4(j, y[i].scales, &sc, &m);
            const float d = F16(y[i].d) * sc;
            if (!d) continue;
            const float dm = F16(y[i].dmin) * m;
            for (int ii = 0; ii < 32; ++ii) {
                int l = nearest_int((xb[32 * j + ii] + dm) / d);
                L[32 * j + ii] = (uint8_t) (l < 0 ? 0 : (l > 31 ? 31 : l));
            }
        }
        memset(y[i].qh, 0, 32);
        for (int j = 0; j < 4; ++j) {                   /* sub-blocks 2j (low nibbles), 2j + 1 (high) */
            for (int l = 0; l < 32; ++l) {
                const int a = L[64 * j + l], b = L[64 * j + 32 + l];
                y[i].qs[32 * j + l] = (uint8_t) ((a & 15) | ((b & 15) << 4));
                y[i].qh[l] |= (uint8_t) (((a >> 4) << (2 * j)) | ((b >> 4) << (2 * j + 1)));
            }
        }
    }
}

/* ggml's make_qx_quants with rmse_type 1 (weights x^2): symmetric codes -nmax..nmax-1 around the
   element of largest magnitude, then 18 rescalings (nmax + 0.1 is) / max, is = -9..9, kept when
   they raise sum(w x l)^2 / sum(w l^2). Returns the scale; L gets codes + nmax. */
static float make_qx_quants(int n, int nmax, const float * x, int8_t * L) {
    float max = 0, amax = 0;
    for (int i = 0; i < n; ++i) {
        const float ax = fabsf(x[i]);
        if (ax > amax) { amax = ax; max = x[i]; }
    }
    if (amax < 1e-15f) {
        for (int i = 0; i < n; ++i) L[i] = 0;
        return 0.f;
    }
    float iscale = -nmax / max;
    float sumlx = 0, suml2 = 0;
    for (int i = 0; i < n; ++i) {
        int l = nearest_int(iscale * x[i]);
        l = l < -nmax ? -nmax : (l > nmax - 1 ? nmax - 1 : l);
        L[i] = (int8_t) (l + nmax);
        const float w = x[i] * x[i];
        sumlx += w * x[i] * l;
        suml2 += w * l * l;
    }
    float scale = suml2 ? sumlx / suml2 : 0.0f;
    float best = scale * sumlx;
    if (g_planted & 256) return scale;
    for (int is = -9; is <= 9; ++is) {
        if (is == 0) continue;
        iscale = -(nmax + 0.1f * is) / max;
        sumlx = suml2 = 0;
        for (int i = 0; i < n; ++i) {
            int l = nearest_int(iscale * x[i]);
            l = l < -nmax ? -nmax : (l > nmax - 1 ? nmax - 1 : l);
            const float w = x[i] * x[i];
            sumlx += w * x[i] * l;
            suml2 += w * l * l;
        }
        if (suml2 > 0 && sumlx * sumlx > best * suml2) {
            for (int i = 0; i < n; ++i) {
                int l = nearest_int(iscale * x[i]);
                L[i] = (int8_t) (nmax + (l < -nmax ? -nmax : (l > nmax - 1 ? nmax - 1 : l)));
            }
            scale = sumlx / suml2;
            best = scale * sumlx;
        }
    }
    return scale;
}

float oracle_make_qx_quants(int n, int nmax, const float * x, int8_t * L) {
    return n > 256 ? -1.f : make_qx_quants(n, nmax, x, L);
}

/* ggml's quantize_row_q6_K_ref: 16 sub-blocks of 16 with signed 8-bit scales (the largest-magnitude
   sub-block scale maps to -128), 6-bit codes (-32..31, stored + 32) re-rounded under the decoded
   scales; element 32 g + l of each 128-half in the low (g < 2) or high nibble of ql, bits 2g, 2g+1
   of qh[l]. */
void oracle_quantize_q6_K(const float * x, void * vy, int64_t k) {
    bq6_K * y = (bq6_K *) vy;
    int8_t L[256];
    float scales[16];
    for (int64_t i = 0; i < k / 256; i++) {
        const float * xb = x + i * 256;
        float max_scale = 0, max_abs_scale = 0;
        for (int ib = 0; ib < 16; ++ib) {
            const float sc = make_qx_quants(16, 32, xb + 16 * ib, L + 16 * ib);
            scales[ib] = sc;
            if (fabsf(sc) > max_abs_scale) { max_abs_scale = fabsf(sc); max_scale = sc; }
        }
        memset(&y[i], 0, sizeof(bq6_K));
        if (max_abs_scale < 1e-15f) continue;
        const float iscale = -128.f / max_scale;
        y[i].d = oracle_fp32_to_fp16(1 / iscale);
        for (int ib = 0; ib < 16; ++ib) {
            const int v = nearest_int(iscale * scales[ib]);
            y[i].scales[ib] = (int8_t) (v < 127 ? v : 127);
        }
        for (int j = 0; j < 16; ++j) {
            const float d = F16(y[i].d) * y[i].scales[j];
            if (!d) continue;
            for (int ii = 0; ii < 16; ++ii) {
                int l = nearest_int(xb[16 * j + ii] / d);
                l = l < -32 ? -32 : (l > 31 ? 31 : l);
                L[16 * j + ii] = (int8_t) (l + 32);
            }
        }
        for (int h = 0; h < 2; ++h) {
            const int8_t * Lh = L + 128 * h;
            uint8_t * ql = y[i].ql + 64 * h;
            uint8_t * qh = y[i].qh + 32 * h;
            for (int l = 0; l < 32; ++l) {
                const int q0 = Lh[l], q1 = Lh[l + 32], q2 = Lh[l + 64], q3 = Lh[l + 96];
                ql[l] = (uint8_t) ((q0 & 15) | ((q2 & 15) << 4));
                ql[l + 32] = (uint8_t) ((q1 & 15) | ((q3 & 15) << 4));
                qh[l] = (uint8_t) ((q0 >> 4) | ((q1 >> 4) << 2) | ((q2 >> 4) << 4) | ((q3 >> 4) << 6));
            }
        }
    }
}

/* moe_stream/dequant.c:143-171 (dequant_q4_K), :237-244 (dequant_q8_0); Q4_0 by its layout */
int oracle_dequantize(int type, const void * vx, float * y, int64_t k) {
    switch (type) {
        case GGML_TYPE_F32: memcpy(y, vx, (size_t) k * 4); return 1;
        case GGML_TYPE_F16: {
            const uint16_t * x = (const uint16_t *) vx;
            for (int64_t i = 0; i < k; i++) y[i] = F16(x[i]);
            return 1;
        }
        case GGML_TYPE_BF16: {
            const uint16_t * x = (const uint16_t *) vx;
            for (int64_t i = 0; i < k; i++) y[i] = bitsf((uint32_t) x[i] << 16);
            return 1;
        }
        case GGML_TYPE_Q4_0: {
            const bq4_0 * x = (const bq4_0 *) vx;
            for (int64_t i = 0; i < k / 32; i++) {
                const float d = F16(x[i].d);
                for (int j = 0; j < 16; ++j) {
                    const int x0 = (x[i].qs[j] & 0x0F) - 8;
                    const int x1 = (x[i].qs[j] >> 4) - 8;
                    y[i * 32 + j] = x0 * d;
                    y[i * 32 + j + 16] = x1 * d;
                }
            }
            return 1;
        }
        case GGML_TYPE_Q8_0: {
            const bq8_0 * x = (const bq8_0 *) vx;
            for (int64_t i = 0; i < k / 32; i++) {
                const float d = F16(x[i].d);
                for (int j = 0; j < 32; ++j) y[i * 32 + j] = d * (float) x[i].qs[j];
            }
            return 1;
        }
        case GGML_TYPE_Q4_K: {
            const bq4_K * x = (const bq4_K *) vx;
            for (int64_t i = 0; i < k / 256; i++) {
                const float d = F16(x[i].d);
                const float dmin = F16(x[i].dmin);
                const uint8_t * q = x[i].qs;
                int is = 0;
                for (int j = 0; j < 256; j += 64) {
                    uint8_t s, m;
                    scale_min_k4(is + 0, x[i].scales, &s, &m);
                    const float d1 = d * s, m1 = dmin * m;
                    scale_min_k4(is + 1, x[i].scales, &s, &m);
                    const float d2 = d * s, m2 = dmin * m;
                    for (int l = 0; l < 32; ++l) *y++ = d1 * (float) (q[l] & 0x0F) - m1;
                    for (int l = 0; l < 32; ++l) *y++ = d2 * (float) (q[l] >> 4) - m2;
                    q += 32;
                    is += 2;
                }
            }
            return 1;
        }
        case GGML_TYPE_Q5_K: {      /* moe_stream/dequant.c:135-168 */
            const bq5_K * x = (const bq5_K *) vx;
            for (int64_t i = 0; i < k / 256; i++) {
                const float d = F16(x[i].d), dmin = F16(x[i].dmin);
                for (int j = 0; j < 4; ++j) {
                    uint8_t sa, ma, sb, mb;
                    scale_min_k4(2 * j, x[i].scales, &sa, &ma);
                    scale_min_k4(2 * j + 1, x[i].scales, &sb, &mb);
                    const float da = d * sa, mna = dmin * ma, db = d * sb, mnb = dmin * mb;
                    for (int l = 0; l < 32; ++l) {
                        const int hi = (x[i].qh[l] >> (2 * j)) & 1;
                        *y++ = da * (float) ((x[i].qs[32 * j + l] & 0x0F) + 16 * hi) - mna;
                    }
                    for (int l = 0; l < 32; ++l) {
                        const int hi = (x[i].qh[l] >> (2 * j + 1)) & 1;
                        *y++ = db * (float) ((x[i].qs[32 * j + l] >> 4) + 16 * hi) - mnb;
                    }
                }
            }
            return 1;
        }
        case GGML_TYPE_Q6_K: {      /* moe_stream/dequant.c:170-197 */
            const bq6_K * x = (const bq6_K *) vx;
            for (int64_t i = 0; i < k / 256; i++) {
                const float d = F16(x[i].d);
                for (int h = 0; h < 2; ++h) {
                    const uint8_t * ql = x[i].ql + 64 * h;
                    const uint8_t * qh = x[i].qh + 32 * h;
                    const int8_t * sc = x[i].scales + 8 * h;
                    for (int g = 0; g < 4; ++g) {       /* element 32 g + l of the half */
                        for (int l = 0; l < 32; ++l) {
                            const int lo = (ql[l + 32 * (g & 1)] >> (4 * (g >> 1))) & 0xF;
                            const int q = (lo | (((qh[l] >> (2 * g)) & 3) << 4)) - 32;
                            y[128 * h + 32 * g + l] = d * (float) sc[2 * g + l / 16] * (float) q;
                        }
                    }
                }
                y += 256;
            }
            return 1;
        }
        default: return 0;
    }
}

/* ------------------------------------------------------------------------------------------ */
/* block dots (ggml_vec_dot_*_generic)                                                        */

/* Experiment hook (tests/exactness_experiment.py only): the order in which the Q4_0 / Q8_0 dots
   add their block terms. 0 (the default, and the oracle's definition) is ggml-cpu's generic order,
   sumf += term block by block. 1 is a 32-lane wave reduction: lane l adds blocks l, l + 32, ... in
   order, then the lanes are added pairwise (l + 16 into l, then l + 8, ... 1). The block terms
   themselves are the same floats in both. */
static int g_block_sum_order = 0;
void oracle_set_block_sum_order(int mode) { g_block_sum_order = mode; }

/* Test hook (tests/test_ref_qwen.py only): plants a known attention mistake so that a test can show
   its fixture catches it. 0, the default, plants nothing. Bit 1: a query head h reads KV head
   h % n_head_kv instead of h / (n_head / n_head_kv) (mul_mat's and flash_attn_ext's head
   broadcast). Bit 2: rope rotates the other pairing (NEOX's (i, i + n_dims/2) and NORMAL's
   (2i, 2i + 1) exchanged). Bit 4: soft_max and flash_attn_ext drop the scale (1/sqrt(head_dim)). */

static float sum_block_terms(const float * t, int64_t n) {
    if (g_block_sum_order == 0) {
        float s = 0;
        for (int64_t i = 0; i < n; i++) s += t[i];
        return s;
    }
    float p[32] = { 0 };
    for (int64_t i = 0; i < n; i++) p[i % 32] += t[i];
    for (int o = 16; o >= 1; o >>= 1) {
        for (int l = 0; l < o; l++) p[l] = p[l] + p[l + o];
    }
    return p[0];
}

float oracle_vec_dot_q4_0_q8_0(int64_t n, const void * vx, const void * vy) {
    const bq4_0 * x = (const bq4_0 *) vx;
    const bq8_0 * y = (const bq8_0 *) vy;
    if (g_block_sum_order != 0) {
        float * t = (float *) malloc((size_t) (n / 32) * sizeof(float));
        for (int64_t ib = 0; ib < n / 32; ++ib) {
            int sumi = 0;
            for (int j = 0; j < 16; ++j) sumi += ((x[ib].qs[j] & 0x0F) - 8) * y[ib].qs[j] + ((x[ib].qs[j] >> 4) - 8) * y[ib].qs[j + 16];
            t[ib] = sumi * F16(x[ib].d) * F16(y[ib].d);
        }
        const float s = sum_block_terms(t, n / 32);
        free(t);
        return s;
    }
    float sumf = 0;
    for (int64_t ib = 0; ib < n / 32; ++ib) {
        int sumi0 = 0, sumi1 = 0;
        for (int j = 0; j < 16; ++j) {
            const int v0 = (x[ib].qs[j] & 0x0F) - 8;
            const int v1 = (x[ib].qs[j] >> 4) - 8;
            sumi0 += v0 * y[ib].qs[j];
            sumi1 += v1 * y[ib].qs[j + 16];
        }
        const int sumi = sumi0 + sumi1;
        sumf += sumi * F16(x[ib].d) * F16(y[ib].d);
    }
    return sumf;
}

float oracle_vec_dot_q8_0_q8_0(int64_t n, const void * vx, const void * vy) {
    const bq8_0 * x = (const bq8_0 *) vx;
    const bq8_0 * y = (const bq8_0 *) vy;
    if (g_block_sum_order != 0) {
        float * t = (float *) malloc((size_t) (n / 32) * sizeof(float));
        for (int64_t ib = 0; ib < n / 32; ++ib) {
            int sumi = 0;
            for (int j = 0; j < 32; j++) sumi += x[ib].qs[j] * y[ib].qs[j];
            t[ib] = sumi * (F16(x[ib].d) * F16(y[ib].d));
        }
        const float s = sum_block_terms(t, n / 32);
        free(t);
        return s;
    }
    float sumf = 0;
    for (int64_t ib = 0; ib < n / 32; ++ib) {
        int sumi = 0;
        for (int j = 0; j < 32; j++) sumi += x[ib].qs[j] * y[ib].qs[j];
        sumf += sumi * (F16(x[ib].d) * F16(y[ib].d));
    }
    return sumf;
}

float oracle_vec_dot_q4_K_q8_K(int64_t n, const void * vx, const void * vy) {
    const bq4_K * x = (const bq4_K *) vx;
    const bq8_K * y = (const bq8_K *) vy;
    float sums[8] = { 0 };
    float sumf = 0;
    for (int64_t i = 0; i < n / 256; ++i) {
        /* 8 sub-blocks of 32: integer dot of the 4-bit quants with the Q8_K quants, scaled by
           the 6-bit sub-block scale; the mins act through the 16-wise sums bsums */
        int32_t aux32[8] = { 0 };
        int sumi_min = 0;
        uint8_t sc[8], mn[8];
        for (int j = 0; j < 8; j++) scale_min_k4(j, x[i].scales, &sc[j], &mn[j]);
        for (int j = 0; j < 16; ++j) sumi_min += y[i].bsums[j] * mn[j / 2];
        for (int j = 0; j < 8; ++j) {
            const uint8_t * q4 = x[i].qs + 32 * (j / 2);
            const int8_t * q8 = y[i].qs + 32 * j;
            /* the running 8-lane accumulators of the generic kernel: lane l gets elements l, l+8, l+16, l+24 */
            for (int l = 0; l < 32; ++l) {
                const int a = (j & 1) ? (q4[l] >> 4) : (q4[l] & 0xF);
                aux32[l & 7] += (int32_t) sc[j] * (int32_t) (int16_t) (q8[l] * a);
            }
        }
        const float d = F16(x[i].d) * y[i].d;
        for (int l = 0; l < 8; ++l) sums[l] += d * aux32[l];
        const float dmin = F16(x[i].dmin) * y[i].d;
        sumf -= dmin * sumi_min;
    }
    for (int l = 0; l < 8; ++l) sumf += sums[l];
    return sumf;
}

/* ggml_vec_dot_q5_K_q8_K_generic: the Q4_K kernel with the fifth bit of each code */
float oracle_vec_dot_q5_K_q8_K(int64_t n, const void * vx, const void * vy) {
    const bq5_K * x = (const bq5_K *) vx;
    const bq8_K * y = (const bq8_K *) vy;
    float sums[8] = { 0 };
    float sumf = 0;
    for (int64_t i = 0; i < n / 256; ++i) {
        int32_t aux32[8] = { 0 };
        int sumi_min = 0;
        uint8_t sc[8], mn[8];
        for (int j = 0; j < 8; j++) scale_min_k4(j, x[i].scales, &sc[j], &mn[j]);
        for (int j = 0; j < 16; ++j) sumi_min += y[i].bsums[j] * mn[j / 2];
        for (int j = 0; j < 8; ++j) {
            const uint8_t * q4 = x[i].qs + 32 * (j / 2);
            const int8_t * q8 = y[i].qs + 32 * j;
            for (int l = 0; l < 32; ++l) {
                const int a = ((j & 1) ? (q4[l] >> 4) : (q4[l] & 0xF)) + 16 * ((x[i].qh[l] >> j) & 1);
                aux32[l & 7] += (int32_t) sc[j] * (int32_t) (int16_t) (q8[l] * a);
            }
        }
        const float d = F16(x[i].d) * y[i].d;
        for (int l = 0; l < 8; ++l) sums[l] += d * aux32[l];
        const float dmin = F16(x[i].dmin) * y[i].d;
        sumf -= dmin * sumi_min;
    }
    for (int l = 0; l < 8; ++l) sumf += sums[l];
    return sumf;
}

/* ggml_vec_dot_q6_K_q8_K_generic: 16 sub-blocks of 16 with signed scales, codes - 32, no mins */
float oracle_vec_dot_q6_K_q8_K(int64_t n, const void * vx, const void * vy) {
    const bq6_K * x = (const bq6_K *) vx;
    const bq8_K * y = (const bq8_K *) vy;
    float sums[8] = { 0 };
    float sumf = 0;
    for (int64_t i = 0; i < n / 256; ++i) {
        int8_t a[256];
        for (int h = 0; h < 2; ++h) {
            const uint8_t * ql = x[i].ql + 64 * h;
            const uint8_t * qh = x[i].qh + 32 * h;
            for (int g = 0; g < 4; ++g) {
                for (int l = 0; l < 32; ++l) {
                    const int lo = (ql[l + 32 * (g & 1)] >> (4 * (g >> 1))) & 0xF;
                    a[128 * h + 32 * g + l] = (int8_t) ((lo | (((qh[l] >> (2 * g)) & 3) << 4)) - 32);
                }
            }
        }
        int32_t aux32[8] = { 0 };
        for (int j = 0; j < 16; ++j) {
            const int scale = x[i].scales[j];
            for (int e = 16 * j; e < 16 * j + 16; ++e) aux32[e & 7] += scale * (int32_t) (int16_t) (y[i].qs[e] * a[e]);
        }
        const float d = F16(x[i].d) * y[i].d;
        for (int l = 0; l < 8; ++l) sums[l] += d * aux32[l];
    }
    for (int l = 0; l < 8; ++l) sumf += sums[l];
    return sumf;
}

static float vec_dot_f16(int64_t n, const uint16_t * x, const uint16_t * y) {
    ggml_float sumf = 0.0;
    for (int64_t i = 0; i < n; ++i) sumf += (ggml_float) (F16(x[i]) * F16(y[i]));
    return (float) sumf;
}

static float vec_dot_f32(int64_t n, const float * x, const float * y) {
    ggml_float sumf = 0.0;
    for (int64_t i = 0; i < n; ++i) sumf += (ggml_float) (x[i] * y[i]);
    return (float) sumf;
}

/* ------------------------------------------------------------------------------------------ */
/* dot-type conversion of an activation row                                                   */

static int dot_type_of(int wtype) {
    switch (wtype) {
        case GGML_TYPE_Q4_0: case GGML_TYPE_Q8_0: return GGML_TYPE_Q8_0;
        case GGML_TYPE_Q4_K: case GGML_TYPE_Q5_K: case GGML_TYPE_Q6_K: return GGML_TYPE_Q8_K;
        case GGML_TYPE_F16: return GGML_TYPE_F16;
        case GGML_TYPE_BF16: return GGML_TYPE_BF16;
        case GGML_TYPE_F32: return GGML_TYPE_F32;
        default: return -1;
    }
}

static size_t dot_row_size(int dtype, int64_t k) {
    switch (dtype) {
        case GGML_TYPE_Q8_0: return (size_t) (k / 32) * sizeof(bq8_0);
        case GGML_TYPE_Q8_K: return (size_t) (k / 256) * sizeof(bq8_K);
        case GGML_TYPE_F16: case GGML_TYPE_BF16: return (size_t) k * 2;
        default: return (size_t) k * 4;
    }
}

static void to_dot_type(int dtype, const float * x, void * y, int64_t k) {
    switch (dtype) {
        case GGML_TYPE_Q8_0: oracle_quantize_q8_0(x, y, k); break;
        case GGML_TYPE_Q8_K: oracle_quantize_q8_K(x, y, k); break;
        case GGML_TYPE_F16: for (int64_t i = 0; i < k; i++) ((uint16_t *) y)[i] = oracle_fp32_to_fp16(x[i]); break;
        case GGML_TYPE_BF16: {
            for (int64_t i = 0; i < k; i++) {
                uint32_t u = fbits(x[i]);
                ((uint16_t *) y)[i] = (uint16_t) ((u + (0x7fffu + ((u >> 16) & 1u))) >> 16);
            }
            break;
        }
        default: memcpy(y, x, (size_t) k * 4); break;
    }
}

static float row_dot(int wtype, const void * w, const void * xd, int64_t k) {
    switch (wtype) {
        case GGML_TYPE_Q4_0: return oracle_vec_dot_q4_0_q8_0(k, w, xd);
        case GGML_TYPE_Q8_0: return oracle_vec_dot_q8_0_q8_0(k, w, xd);
        case GGML_TYPE_Q4_K: return oracle_vec_dot_q4_K_q8_K(k, w, xd);
        case GGML_TYPE_Q5_K: return oracle_vec_dot_q5_K_q8_K(k, w, xd);
        case GGML_TYPE_Q6_K: return oracle_vec_dot_q6_K_q8_K(k, w, xd);
        case GGML_TYPE_F16: return vec_dot_f16(k, (const uint16_t *) w, (const uint16_t *) xd);
        case GGML_TYPE_BF16: {
            ggml_float s = 0.0;
            const uint16_t * a = (const uint16_t *) w;
            const uint16_t * b = (const uint16_t *) xd;
            for (int64_t i = 0; i < k; i++) s += (ggml_float) (bitsf((uint32_t) a[i] << 16) * bitsf((uint32_t) b[i] << 16));
            return (float) s;
        }
        default: return vec_dot_f32(k, (const float *) w, (const float *) xd);
    }
}

static size_t weight_row_size(int wtype, int64_t k) {
    switch (wtype) {
        case GGML_TYPE_Q4_0: return (size_t) (k / 32) * 18;
        case GGML_TYPE_Q8_0: return (size_t) (k / 32) * 34;
        case GGML_TYPE_Q4_K: return (size_t) (k / 256) * 144;
        case GGML_TYPE_Q5_K: return (size_t) (k / 256) * 176;
        case GGML_TYPE_Q6_K: return (size_t) (k / 256) * 210;
        case GGML_TYPE_F16: case GGML_TYPE_BF16: return (size_t) k * 2;
        default: return (size_t) k * 4;
    }
}

void oracle_gemv(int type, const void * w, int64_t nrows, int64_t k, const float * x, float * y, int n_threads) {
    const int dt = dot_type_of(type);
    void * xd = malloc(dot_row_size(dt, k) + 64);
    to_dot_type(dt, x, xd, k);
    const size_t rs = weight_row_size(type, k);
    #pragma omp parallel for num_threads(n_threads > 0 ? n_threads : 1) schedule(static)
    for (int64_t r = 0; r < nrows; r++) y[r] = row_dot(type, (const char *) w + r * rs, xd, k);
    free(xd);
}

/* ------------------------------------------------------------------------------------------ */
/* RoPE (ggml_rope_ext; YaRN blend only when ext_factor != 0)                                  */

static float yarn_ramp(float low, float high, int i0) {
    const float y = (i0 / 2 - low) / fmaxf(0.001f, high - low);
    return 1 - fminf(1, fmaxf(0, y));
}

static void rope_yarn(float theta_extrap, float freq_scale, const float corr_dims[2], int64_t i0, float ext_factor,
                      float mscale, float * cos_theta, float * sin_theta) {
    const float theta_interp = freq_scale * theta_extrap;
    float theta = theta_interp;
    if (ext_factor != 0.0f) {
        const float ramp_mix = yarn_ramp(corr_dims[0], corr_dims[1], (int) i0) * ext_factor;
        theta = g_planted & 64 ? theta_extrap * (1 - ramp_mix) + theta_interp * ramp_mix
                               : theta_interp * (1 - ramp_mix) + theta_extrap * ramp_mix;
        mscale *= 1.0f + 0.1f * log_cr(1.0f / freq_scale);
    }
    *cos_theta = cos_cr(theta) * mscale;
    *sin_theta = sin_cr(theta) * mscale;
}

static void corr_dims_of(int n_dims, int n_ctx_orig, float freq_base, float beta_fast, float beta_slow, float dims[2]) {
    const float start = floorf(n_dims * logf(n_ctx_orig / (beta_fast * 2 * (float) M_PI)) / (2 * logf(freq_base)));
    const float end = ceilf(n_dims * logf(n_ctx_orig / (beta_slow * 2 * (float) M_PI)) / (2 * logf(freq_base)));
    dims[0] = fmaxf(0, start);
    dims[1] = fminf((float) (n_dims - 1), end);
}

static void rope_cache(int32_t pos, float freq_scale, const float * freq_factors, const float corr_dims[2], int64_t ne0,
                       float ext_factor, float mscale, float theta_scale, float * cache) {
    float theta = (float) pos;
    for (int64_t i0 = 0; i0 < ne0; i0 += 2) {
        const float ff = freq_factors ? freq_factors[i0 / 2] : 1.0f;
        rope_yarn(g_planted & 128 ? theta * ff : theta / ff, freq_scale, corr_dims, i0, ext_factor, mscale,
                  &cache[i0 + 0], &cache[i0 + 1]);
        theta *= theta_scale;
    }
}

static void rope_apply(float * dst, const float * src, int64_t ne0, int n_dims, int mode, const float * cache) {
    if (mode & GGML_ROPE_TYPE_NEOX) {
        for (int64_t i0 = 0; i0 < n_dims; i0 += 2) {
            const int64_t ic = i0 / 2;
            const float c = cache[i0 + 0], s = cache[i0 + 1];
            const float x0 = src[ic], x1 = src[ic + n_dims / 2];
            dst[ic] = x0 * c - x1 * s;
            dst[ic + n_dims / 2] = x0 * s + x1 * c;
        }
    } else {
        for (int64_t i0 = 0; i0 < n_dims; i0 += 2) {
            const float c = cache[i0 + 0], s = cache[i0 + 1];
            const float x0 = src[i0], x1 = src[i0 + 1];
            dst[i0] = x0 * c - x1 * s;
            dst[i0 + 1] = x0 * s + x1 * c;
        }
    }
    for (int64_t i0 = n_dims; i0 < ne0; i0++) dst[i0] = src[i0];
}

void oracle_rope(float * dst, const float * src, int64_t ne0, int n_dims, int mode, int32_t pos,
                 float freq_base, float freq_scale, float ext_factor, float attn_factor,
                 float beta_fast, float beta_slow, int n_ctx_orig, const float * freq_factors) {
    float * cache = (float *) malloc((size_t) (ne0 + 2) * sizeof(float));
    float corr[2];
    corr_dims_of(n_dims, n_ctx_orig, freq_base, beta_fast, beta_slow, corr);
    const float theta_scale = powf(freq_base, -2.0f / n_dims);
    rope_cache(pos, freq_scale, freq_factors, corr, ne0, ext_factor, attn_factor, theta_scale, cache);
    rope_apply(dst, src, ne0, n_dims, mode, cache);
    free(cache);
}

/* ------------------------------------------------------------------------------------------ */
/* MoE routing, restating moe_route (qwen_model.c:551-606) with sc_softmax (compute_backend.c:68-86) */

void oracle_moe_route(const float * logits, int n_expert, int top_k, int32_t * ids, float * w) {
    float * p = (float *) malloc((size_t) n_expert * sizeof(float));
    memcpy(p, logits, (size_t) n_expert * sizeof(float));
    float mx = p[0];
    for (int i = 1; i < n_expert; i++) if (p[i] > mx) mx = p[i];
    float sum = 0.0f;
    for (int i = 0; i < n_expert; i++) { p[i] = expf(p[i] - mx); sum += p[i]; }
    const float inv = 1.0f / sum;
    for (int i = 0; i < n_expert; i++) p[i] *= inv;
    int bi[64];
    float bw[64];
    for (int k = 0; k < top_k; k++) { bi[k] = -1; bw[k] = -1.0f; }
    for (int e = 0; e < n_expert; e++) {
        const float v = p[e];
        if (v <= bw[top_k - 1]) continue;
        int j = top_k - 1;
        while (j > 0 && bw[j - 1] < v) { bw[j] = bw[j - 1]; bi[j] = bi[j - 1]; j--; }
        bw[j] = v;
        bi[j] = e;
    }
    float s = 0.0f;
    for (int k = 0; k < top_k; k++) s += bw[k];
    if (s > 0.0f) for (int k = 0; k < top_k; k++) bw[k] /= s;
    for (int k = 0; k < top_k; k++) { ids[k] = bi[k]; w[k] = bw[k]; }
    free(p);
}

/* ------------------------------------------------------------------------------------------ */
/* Token sampler, restating sample() (model.cpp:1675-1728) and argmax() (model.cpp:1659-1666). The
   weighted draw restates libstdc++'s std::discrete_distribution (GCC 11, bits/random.tcc:
   param_type::_M_initialize and operator()): weights widened to double, divided by their double
   sum, partial sums in order with the last set to 1, then the first partial sum not below u, where
   u is the std::generate_canonical<double, 53> value the generator would have produced (the
   caller supplies it); with fewer than two weights the result is 0 and no u is used. Logits order
   by value, then ascending id among equal values (std::partial_sort leaves that order open);
   a NaN orders and weighs as -inf. */

static const float * g_sample_keys;

static int sample_cmp(const void * a, const void * b) {
    const int32_t ia = *(const int32_t *) a, ib = *(const int32_t *) b;
    const float va = g_sample_keys[ia], vb = g_sample_keys[ib];
    if (va > vb) return -1;
    if (va < vb) return 1;
    return ia < ib ? -1 : (ia > ib);
}

int32_t oracle_sample(const float * logits, int64_t n, const int32_t * recent, int64_t n_recent, float temp,
                      int32_t top_k, float top_p, float repeat_penalty, int32_t repeat_last_n, double u,
                      int32_t * used_draw) {
    float * l = (float *) malloc((size_t) n * sizeof(float));
    memcpy(l, logits, (size_t) n * sizeof(float));
    *used_draw = 0;
    /* model.cpp:1678-1687 */
    if (repeat_penalty != 1.0f && n_recent > 0) {
        const size_t nr = (size_t) n_recent;
        const size_t start = nr > (size_t) repeat_last_n ? nr - (size_t) repeat_last_n : 0;
        for (size_t i = start; i < nr; i++) {
            const int32_t id = recent[i];
            if (id < 0 || (int64_t) id >= n) continue;
            l[id] = l[id] > 0.0f ? l[id] / repeat_penalty : l[id] * repeat_penalty;
        }
    }
    /* model.cpp:1689-1691, 1659-1666 */
    if (temp <= 0.0f) {
        int32_t best = 0;
        float bv = l[0];
        for (int64_t i = 1; i < n; i++) {
            if (l[i] > bv) { bv = l[i]; best = (int32_t) i; }
        }
        free(l);
        return best;
    }
    for (int64_t i = 0; i < n; i++) if (isnan(l[i])) l[i] = -INFINITY;
    int32_t * ids = (int32_t *) malloc((size_t) n * sizeof(int32_t));
    for (int64_t i = 0; i < n; i++) ids[i] = (int32_t) i;
    /* model.cpp:1693-1698 */
    const int64_t k = (top_k > 0 && (int64_t) top_k < n) ? top_k : n;
    g_sample_keys = l;
    qsort(ids, (size_t) n, sizeof(int32_t), sample_cmp);
    const float max_logit = l[ids[0]];
    if (!isfinite(max_logit)) {
        free(ids);
        free(l);
        return -1;
    }
    /* model.cpp:1700-1707 */
    float * probs = (float *) malloc((size_t) k * sizeof(float));
    float sum = 0.0f;
    for (int64_t i = 0; i < k; i++) {
        probs[i] = exp_cr((l[ids[i]] - max_logit) / temp);
        sum += probs[i];
    }
    for (int64_t i = 0; i < k; i++) probs[i] /= sum;
    /* model.cpp:1711-1724 */
    int64_t cutoff = k;
    if (top_p < 1.0f) {
        float cum = 0.0f;
        for (int64_t i = 0; i < k; i++) {
            cum += probs[i];
            if (cum >= top_p) { cutoff = i + 1; break; }
        }
        float s = 0.0f;
        for (int64_t i = 0; i < cutoff; i++) s += probs[i];
        for (int64_t i = 0; i < cutoff; i++) probs[i] /= s;
    }
    /* model.cpp:1726-1727 with discrete_distribution */
    int64_t idx = 0;
    if (cutoff >= 2) {
        double sd = 0.0;
        for (int64_t i = 0; i < cutoff; i++) sd += (double) probs[i];
        double cp = 0.0;
        idx = cutoff - 1;
        for (int64_t i = 0; i < cutoff - 1; i++) {
            cp += (double) probs[i] / sd;
            if (!(cp < u)) { idx = i; break; }
        }
        *used_draw = 1;
    }
    const int32_t tok = ids[idx];
    free(probs);
    free(ids);
    free(l);
    return tok;
}

/* ------------------------------------------------------------------------------------------ */
/* graph executor                                                                              */

#define ELEM(t, i0, i1, i2, i3) ((char *) (t)->data + (i0) * (t)->nb[0] + (i1) * (t)->nb[1] + (i2) * (t)->nb[2] + (i3) * (t)->nb[3])

static float load_f(const struct ggml_tensor * t, const char * p) {
    switch (t->type) {
        case GGML_TYPE_F32: { float v; memcpy(&v, p, 4); return v; }
        case GGML_TYPE_F16: { uint16_t h; memcpy(&h, p, 2); return F16(h); }
        case GGML_TYPE_BF16: { uint16_t h; memcpy(&h, p, 2); return bitsf((uint32_t) h << 16); }
        case GGML_TYPE_I32: { int32_t v; memcpy(&v, p, 4); return (float) v; }
        default: fprintf(stderr, "oracle: load of type %s\n", ggml_type_name(t->type)); abort();
    }
}

static void store_f(const struct ggml_tensor * t, char * p, float v) {
    switch (t->type) {
        case GGML_TYPE_F32: memcpy(p, &v, 4); break;
        case GGML_TYPE_F16: { uint16_t h = oracle_fp32_to_fp16(v); memcpy(p, &h, 2); break; }
        case GGML_TYPE_BF16: {
            uint32_t u = fbits(v);
            uint16_t h = (uint16_t) ((u + (0x7fffu + ((u >> 16) & 1u))) >> 16);
            memcpy(p, &h, 2);
            break;
        }
        case GGML_TYPE_I32: { int32_t i = (int32_t) v; memcpy(p, &i, 4); break; }
        default: fprintf(stderr, "oracle: store of type %s\n", ggml_type_name(t->type)); abort();
    }
}

typedef struct {
    int n_threads;
    ggml_backend_eval_callback cb;
    void * cb_user;
} cpu_ctx;

static void op_dup(struct ggml_tensor * dst, const struct ggml_tensor * src, int nth) {
    /* element-wise copy in row-major order of src into row-major order of dst (shapes may differ
       when nelements match: cont_2d etc.) */
    const int64_t n = ggml_nelements(src);
    if (ggml_is_quantized(src->type) || ggml_is_quantized(dst->type)) {
        if (src->type == dst->type && ggml_is_contiguous(src) && ggml_is_contiguous(dst)) {
            memcpy(dst->data, src->data, ggml_nbytes(src));
            return;
        }
        fprintf(stderr, "oracle: unsupported quantized copy %s -> %s\n", ggml_type_name(src->type), ggml_type_name(dst->type));
        abort();
    }
    #pragma omp parallel for num_threads(nth) schedule(static)
    for (int64_t i = 0; i < n; i++) {
        int64_t r = i;
        const int64_t s0 = r % src->ne[0]; r /= src->ne[0];
        const int64_t s1 = r % src->ne[1]; r /= src->ne[1];
        const int64_t s2 = r % src->ne[2]; r /= src->ne[2];
        const int64_t s3 = r;
        r = i;
        const int64_t d0 = r % dst->ne[0]; r /= dst->ne[0];
        const int64_t d1 = r % dst->ne[1]; r /= dst->ne[1];
        const int64_t d2 = r % dst->ne[2]; r /= dst->ne[2];
        const int64_t d3 = r;
        const char * sp = ELEM(src, s0, s1, s2, s3);
        char * dp = ELEM(dst, d0, d1, d2, d3);
        if (src->type == dst->type) memcpy(dp, sp, ggml_type_size(src->type));
        else store_f(dst, dp, load_f(src, sp));
    }
}

static void op_get_rows(struct ggml_tensor * dst, const struct ggml_tensor * a, const struct ggml_tensor * b, int nth) {
    const int64_t ne00 = a->ne[0];
    #pragma omp parallel for collapse(3) num_threads(nth) schedule(static)
    for (int64_t i12 = 0; i12 < b->ne[2]; i12++)
    for (int64_t i11 = 0; i11 < b->ne[1]; i11++)
    for (int64_t i10 = 0; i10 < b->ne[0]; i10++) {
        int32_t row;
        memcpy(&row, ELEM(b, i10, i11, i12, 0), 4);
        const char * src = (const char *) a->data + row * a->nb[1] + i11 * a->nb[2] + i12 * a->nb[3];
        float * out = (float *) ELEM(dst, 0, i10, i11, i12);
        if (a->type == GGML_TYPE_I32) { memcpy(out, src, (size_t) ne00 * 4); continue; }
        if (!oracle_dequantize(a->type, src, out, ne00)) { fprintf(stderr, "oracle: get_rows type\n"); abort(); }
    }
}

static void op_rms_norm(struct ggml_tensor * dst, const struct ggml_tensor * a, int nth) {
    float eps;
    memcpy(&eps, dst->op_params, 4);
    const int64_t ne00 = a->ne[0];
    #pragma omp parallel for collapse(3) num_threads(nth) schedule(static)
    for (int64_t i3 = 0; i3 < a->ne[3]; i3++)
    for (int64_t i2 = 0; i2 < a->ne[2]; i2++)
    for (int64_t i1 = 0; i1 < a->ne[1]; i1++) {
        const float * x = (const float *) ELEM(a, 0, i1, i2, i3);
        float * y = (float *) ELEM(dst, 0, i1, i2, i3);
        ggml_float sum = 0.0;
        for (int64_t i0 = 0; i0 < ne00; i0++) sum += (ggml_float) (x[i0] * x[i0]);
        const float mean = (float) (sum / ne00);
        const float scale = 1.0f / sqrtf(mean + eps);
        for (int64_t i0 = 0; i0 < ne00; i0++) y[i0] = x[i0] * scale;
    }
}

static void op_binary(struct ggml_tensor * dst, const struct ggml_tensor * a, const struct ggml_tensor * b, int nth) {
    const enum ggml_op op = dst->op;
    #pragma omp parallel for collapse(3) num_threads(nth) schedule(static)
    for (int64_t i3 = 0; i3 < a->ne[3]; i3++)
    for (int64_t i2 = 0; i2 < a->ne[2]; i2++)
    for (int64_t i1 = 0; i1 < a->ne[1]; i1++) {
        for (int64_t i0 = 0; i0 < a->ne[0]; i0++) {
            const float x = load_f(a, ELEM(a, i0, i1, i2, i3));
            const float y = load_f(b, ELEM(b, i0 % b->ne[0], i1 % b->ne[1], i2 % b->ne[2], i3 % b->ne[3]));
            store_f(dst, ELEM(dst, i0, i1, i2, i3), op == GGML_OP_ADD ? x + y : op == GGML_OP_MUL ? x * y : op == GGML_OP_SUB ? x - y : x / y);
        }
    }
}

static void op_unary(struct ggml_tensor * dst, const struct ggml_tensor * a, int nth) {
    const int kind = dst->op == GGML_OP_UNARY ? dst->op_params[0] : -1;
    float s = 1.0f;
    if (dst->op == GGML_OP_SCALE) memcpy(&s, dst->op_params, 4);
    #pragma omp parallel for collapse(3) num_threads(nth) schedule(static)
    for (int64_t i3 = 0; i3 < a->ne[3]; i3++)
    for (int64_t i2 = 0; i2 < a->ne[2]; i2++)
    for (int64_t i1 = 0; i1 < a->ne[1]; i1++) {
        for (int64_t i0 = 0; i0 < a->ne[0]; i0++) {
            const float x = load_f(a, ELEM(a, i0, i1, i2, i3));
            float y;
            if (dst->op == GGML_OP_SCALE) y = x * s;
            else if (dst->op == GGML_OP_SQR) y = x * x;
            else if (kind == GGML_UNARY_OP_SILU) y = x / (1.0f + exp_cr(-x));
            else if (kind == GGML_UNARY_OP_RELU) y = x > 0.f ? x : 0.f;
            else if (kind == GGML_UNARY_OP_SIGMOID) y = 1.0f / (1.0f + exp_cr(-x));
            else if (kind == GGML_UNARY_OP_ABS) y = fabsf(x);
            else if (kind == GGML_UNARY_OP_SOFTPLUS) y = softplus_cr(x);
            else { fprintf(stderr, "oracle: unary op %d\n", kind); abort(); }
            store_f(dst, ELEM(dst, i0, i1, i2, i3), y);
        }
    }
}

// ggml_l2_norm (upstream ggml-cpu's l2_norm: the row's sum of f32 squares in double, then
// scale = 1 / max(sqrtf(sum), eps), y = x * scale)
static void op_l2_norm(struct ggml_tensor * dst, const struct ggml_tensor * a, int nth) {
    float eps;
    memcpy(&eps, dst->op_params, 4);
    #pragma omp parallel for collapse(3) num_threads(nth) schedule(static)
    for (int64_t i3 = 0; i3 < a->ne[3]; i3++)
    for (int64_t i2 = 0; i2 < a->ne[2]; i2++)
    for (int64_t i1 = 0; i1 < a->ne[1]; i1++) {
        ggml_float sum = 0.0;
        for (int64_t i0 = 0; i0 < a->ne[0]; i0++) {
            const float x = load_f(a, ELEM(a, i0, i1, i2, i3));
            sum += (ggml_float) (x * x);
        }
        const float scale = 1.0f / fmaxf(sqrtf((float) sum), eps);
        for (int64_t i0 = 0; i0 < a->ne[0]; i0++) {
            store_f(dst, ELEM(dst, i0, i1, i2, i3), load_f(a, ELEM(a, i0, i1, i2, i3)) * scale);
        }
    }
}

// ggml_concat: element i of dim `dim` comes from a while i < a->ne[dim], else from b
static void op_concat(struct ggml_tensor * dst, const struct ggml_tensor * a, const struct ggml_tensor * b) {
    const int dim = dst->op_params[0];
    const size_t es = ggml_type_size(dst->type);
    for (int64_t i3 = 0; i3 < dst->ne[3]; i3++)
    for (int64_t i2 = 0; i2 < dst->ne[2]; i2++)
    for (int64_t i1 = 0; i1 < dst->ne[1]; i1++)
    for (int64_t i0 = 0; i0 < dst->ne[0]; i0++) {
        int64_t ix[4] = { i0, i1, i2, i3 };
        const struct ggml_tensor * s = a;
        if (ix[dim] >= a->ne[dim]) { ix[dim] -= a->ne[dim]; s = b; }
        memcpy(ELEM(dst, i0, i1, i2, i3), ELEM(s, ix[0], ix[1], ix[2], ix[3]), es);
    }
}

// ggml_swiglu_split: silu(a) * b with the silu and mul ops' roundings
static void op_glu(struct ggml_tensor * dst, const struct ggml_tensor * a, const struct ggml_tensor * b, int nth) {
    if (dst->op_params[0] != GGML_GLU_OP_SWIGLU) { fprintf(stderr, "oracle: glu op %d\n", dst->op_params[0]); abort(); }
    #pragma omp parallel for collapse(3) num_threads(nth) schedule(static)
    for (int64_t i3 = 0; i3 < a->ne[3]; i3++)
    for (int64_t i2 = 0; i2 < a->ne[2]; i2++)
    for (int64_t i1 = 0; i1 < a->ne[1]; i1++) {
        for (int64_t i0 = 0; i0 < a->ne[0]; i0++) {
            const float x = load_f(a, ELEM(a, i0, i1, i2, i3));
            const float g = load_f(b, ELEM(b, i0, i1, i2, i3));
            const float sl = x / (1.0f + exp_cr(-x));
            store_f(dst, ELEM(dst, i0, i1, i2, i3), sl * g);
        }
    }
}

static void op_soft_max(struct ggml_tensor * dst, const struct ggml_tensor * a, const struct ggml_tensor * mask, int nth) {
    float scale, max_bias;
    memcpy(&scale, &dst->op_params[0], 4);
    memcpy(&max_bias, &dst->op_params[1], 4);
    if (g_planted & 4) scale = 1.0f;
    const int64_t nc = a->ne[0];
    const uint32_t n_head = (uint32_t) a->ne[2];
    const uint32_t n_head_log2 = n_head ? 1u << (uint32_t) floor(log2((double) n_head)) : 1u;
    const float m0 = powf(2.0f, -(max_bias) / n_head_log2);
    const float m1 = powf(2.0f, -(max_bias / 2.0f) / n_head_log2);
    #pragma omp parallel for collapse(3) num_threads(nth) schedule(static)
    for (int64_t i3 = 0; i3 < a->ne[3]; i3++)
    for (int64_t i2 = 0; i2 < a->ne[2]; i2++)
    for (int64_t i1 = 0; i1 < a->ne[1]; i1++) {
        float * wp = (float *) malloc((size_t) nc * sizeof(float));
        const float * sp = (const float *) ELEM(a, 0, i1, i2, i3);
        float * dp = (float *) ELEM(dst, 0, i1, i2, i3);
        const uint32_t h = (uint32_t) i2;
        const float slope = max_bias > 0.0f ? (h < n_head_log2 ? powf(m0, h + 1) : powf(m1, 2 * (h - n_head_log2) + 1)) : 1.0f;
        for (int64_t i = 0; i < nc; i++) wp[i] = sp[i] * scale;
        if (mask) {
            const char * mrow = (const char *) mask->data + i1 * mask->nb[1] + (i2 % mask->ne[2]) * mask->nb[2] + (i3 % mask->ne[3]) * mask->nb[3];
            for (int64_t i = 0; i < nc; i++) wp[i] += slope * load_f(mask, mrow + i * mask->nb[0]);
        }
        float max = -INFINITY;
        for (int64_t i = 0; i < nc; i++) max = max > wp[i] ? max : wp[i];
        ggml_float sum = 0.0;
        for (int64_t i = 0; i < nc; i++) {
            const float v = exp_cr(wp[i] - max);
            sum += (ggml_float) v;
            dp[i] = v;
        }
        sum = 1.0 / sum;
        const float fs = (float) sum;
        for (int64_t i = 0; i < nc; i++) dp[i] *= fs;
        free(wp);
    }
}

static void op_rope(struct ggml_tensor * dst, const struct ggml_tensor * a, const struct ggml_tensor * pos,
                    const struct ggml_tensor * ff, int nth) {
    const int n_dims = dst->op_params[1];
    const int mode = dst->op_params[2];
    const int n_ctx_orig = dst->op_params[4];
    float freq_base, freq_scale, ext_factor, attn_factor, beta_fast, beta_slow;
    memcpy(&freq_base, dst->op_params + 5, 4);
    memcpy(&freq_scale, dst->op_params + 6, 4);
    memcpy(&ext_factor, dst->op_params + 7, 4);
    memcpy(&attn_factor, dst->op_params + 8, 4);
    memcpy(&beta_fast, dst->op_params + 9, 4);
    memcpy(&beta_slow, dst->op_params + 10, 4);
    float corr[2];
    corr_dims_of(n_dims, n_ctx_orig, freq_base, beta_fast, beta_slow, corr);
    const float theta_scale = powf(freq_base, -2.0f / n_dims);
    const int64_t ne0 = a->ne[0];
    const float * factors = ff ? (const float *) ff->data : NULL;
    #pragma omp parallel for collapse(2) num_threads(nth) schedule(static)
    for (int64_t i3 = 0; i3 < a->ne[3]; i3++)
    for (int64_t i2 = 0; i2 < a->ne[2]; i2++) {
        float * cache = (float *) malloc((size_t) (ne0 + 2) * sizeof(float));
        float * tmp = (float *) malloc((size_t) ne0 * sizeof(float));
        const int32_t p = ((const int32_t *) pos->data)[i2];
        rope_cache(p, freq_scale, factors, corr, ne0, ext_factor, attn_factor, theta_scale, cache);
        for (int64_t i1 = 0; i1 < a->ne[1]; i1++) {
            for (int64_t i0 = 0; i0 < ne0; i0++) tmp[i0] = load_f(a, ELEM(a, i0, i1, i2, i3));
            float * out = (float *) malloc((size_t) ne0 * sizeof(float));
            rope_apply(out, tmp, ne0, n_dims, g_planted & 2 ? mode ^ GGML_ROPE_TYPE_NEOX : mode, cache);
            for (int64_t i0 = 0; i0 < ne0; i0++) store_f(dst, ELEM(dst, i0, i1, i2, i3), out[i0]);
            free(out);
        }
        free(cache);
        free(tmp);
    }
}

/* dst[i01, i11, i12, i13] = src0[:, i01, i12/r2, i13/r3] . src1[:, i11, i12, i13] */
/* Q4_0 / Q8_0 weights against many Q8_0 columns, tiled (16 rows x 64 columns): the block scales
   of the tile's rows and of every column are converted from fp16 once instead of once per dot.
   Each output is oracle_vec_dot_q4_0_q8_0 / _q8_0_q8_0's value: the same integer block sums and
   the same float expression per block, added in block order. */
static void mul_mat_q_tiled(struct ggml_tensor * dst, const struct ggml_tensor * src0, const struct ggml_tensor * src1,
                            const char * wdata, size_t drs, int nth) {
    const int wt = src0->type;
    const int64_t K = src0->ne[0], nb = K / 32, nr = src0->ne[1];
    const int64_t n1 = src1->ne[1], n2 = src1->ne[2], n3 = src1->ne[3];
    const int64_t r2 = n2 / src0->ne[2], r3 = n3 / src0->ne[3];
    const int64_t ncols = n1 * n2 * n3;
    const int64_t TR = 16, TC = 64;
    const int64_t nrt = (nr + TR - 1) / TR, nct = (ncols + TC - 1) / TC;
    float * xs = (float *) malloc((size_t) (ncols * nb) * sizeof(float));
    for (int64_t c = 0; c < ncols; c++) {
        const bq8_0 * y = (const bq8_0 *) (wdata + drs * (size_t) c);
        for (int64_t ib = 0; ib < nb; ib++) xs[c * nb + ib] = F16(y[ib].d);
    }
    #pragma omp parallel for collapse(2) num_threads(nth) schedule(static)
    for (int64_t rt = 0; rt < nrt; rt++)
    for (int64_t ct = 0; ct < nct; ct++) {
        float ws[16 * 512];
        const int64_t r0 = rt * TR, r1 = r0 + TR < nr ? r0 + TR : nr;
        const int64_t c0 = ct * TC, c1 = c0 + TC < ncols ? c0 + TC : ncols;
        const int fits = nb <= 512;
        for (int64_t c = c0; c < c1; c++) {
            const int64_t i11 = c % n1, i12 = (c / n1) % n2, i13 = c / (n1 * n2);
            const char * base = (const char *) src0->data + (i12 / r2) * src0->nb[2] + (i13 / r3) * src0->nb[3];
            if (fits && (c == c0 || (c % (n1 * n2)) == 0 || ((c / n1) % n2) != (((c - 1) / n1) % n2))) {
                for (int64_t i01 = r0; i01 < r1; i01++) {
                    const char * w = base + i01 * src0->nb[1];
                    for (int64_t ib = 0; ib < nb; ib++) {
                        const uint16_t d = wt == GGML_TYPE_Q4_0 ? ((const bq4_0 *) w)[ib].d : ((const bq8_0 *) w)[ib].d;
                        ws[(i01 - r0) * nb + ib] = F16(d);
                    }
                }
            }
            const bq8_0 * y = (const bq8_0 *) (wdata + drs * (size_t) c);
            const float * yd = xs + c * nb;
            for (int64_t i01 = r0; i01 < r1; i01++) {
                const char * w = base + i01 * src0->nb[1];
                float sumf = 0;
                if (!fits) {
                    sumf = wt == GGML_TYPE_Q4_0 ? oracle_vec_dot_q4_0_q8_0(K, w, y) : oracle_vec_dot_q8_0_q8_0(K, w, y);
                } else if (wt == GGML_TYPE_Q4_0) {
                    const bq4_0 * x = (const bq4_0 *) w;
                    const float * wd = ws + (i01 - r0) * nb;
                    for (int64_t ib = 0; ib < nb; ++ib) {
                        int sumi0 = 0, sumi1 = 0;
                        for (int j = 0; j < 16; ++j) {
                            const int v0 = (x[ib].qs[j] & 0x0F) - 8;
                            const int v1 = (x[ib].qs[j] >> 4) - 8;
                            sumi0 += v0 * y[ib].qs[j];
                            sumi1 += v1 * y[ib].qs[j + 16];
                        }
                        const int sumi = sumi0 + sumi1;
                        sumf += sumi * wd[ib] * yd[ib];
                    }
                } else {
                    const bq8_0 * x = (const bq8_0 *) w;
                    const float * wd = ws + (i01 - r0) * nb;
                    for (int64_t ib = 0; ib < nb; ++ib) {
                        int sumi = 0;
                        for (int j = 0; j < 32; j++) sumi += x[ib].qs[j] * y[ib].qs[j];
                        sumf += sumi * (wd[ib] * yd[ib]);
                    }
                }
                *(float *) ELEM(dst, i01, i11, i12, i13) = sumf;
            }
        }
    }
    free(xs);
}

static void op_mul_mat(struct ggml_tensor * dst, const struct ggml_tensor * src0, const struct ggml_tensor * src1, int nth) {
    const int wt = src0->type;
    const int dt = dot_type_of(wt);
    if (dt < 0) { fprintf(stderr, "oracle: mul_mat weight type %s\n", ggml_type_name(src0->type)); abort(); }
    if (src0->nb[0] != ggml_type_size(src0->type)) { fprintf(stderr, "oracle: mul_mat src0 rows not contiguous\n"); abort(); }
    const int64_t K = src0->ne[0];
    const int64_t n1 = src1->ne[1], n2 = src1->ne[2], n3 = src1->ne[3];
    const int64_t r2 = n2 / src0->ne[2], r3 = n3 / src0->ne[3];
    const size_t drs = dot_row_size(dt, K);
    const int64_t ncols = n1 * n2 * n3;
    char * wdata = (char *) malloc(drs * (size_t) ncols + 64);
    #pragma omp parallel for num_threads(nth) schedule(static)
    for (int64_t c = 0; c < ncols; c++) {
        const int64_t i11 = c % n1, i12 = (c / n1) % n2, i13 = c / (n1 * n2);
        float * row = (float *) malloc((size_t) K * sizeof(float));
        for (int64_t i = 0; i < K; i++) row[i] = load_f(src1, ELEM(src1, i, i11, i12, i13));
        to_dot_type(dt, row, wdata + drs * (size_t) c, K);
        free(row);
    }
    const int64_t nr = src0->ne[1];
    // tiles of 16 weight rows x 64 columns, so a tile's rows stay in cache across its columns
    // (each output is the same row_dot either way)
    const int64_t TR = 16, TC = 64;
    const int64_t nrt = (nr + TR - 1) / TR, nct = (ncols + TC - 1) / TC;
    if ((wt == GGML_TYPE_Q4_0 || wt == GGML_TYPE_Q8_0) && ncols >= 8 && g_block_sum_order == 0) {
        mul_mat_q_tiled(dst, src0, src1, wdata, drs, nth);
        free(wdata);
        return;
    }
    #pragma omp parallel for collapse(2) num_threads(nth) schedule(static)
    for (int64_t rt = 0; rt < nrt; rt++)
    for (int64_t ct = 0; ct < nct; ct++) {
        for (int64_t c = ct * TC; c < ncols && c < (ct + 1) * TC; c++) {
            const int64_t i11 = c % n1, i12 = (c / n1) % n2, i13 = c / (n1 * n2);
            for (int64_t i01 = rt * TR; i01 < nr && i01 < (rt + 1) * TR; i01++) {
                const int64_t i02 = g_planted & 1 ? i12 % src0->ne[2] : i12 / r2;
                const char * w = (const char *) src0->data + i01 * src0->nb[1] + i02 * src0->nb[2] + (i13 / r3) * src0->nb[3];
                *(float *) ELEM(dst, i01, i11, i12, i13) = row_dot(wt, w, wdata + drs * (size_t) c, K);
            }
        }
    }
    free(wdata);
}

/* dst[:, e, t] = as[:, :, ids[e, t]] . b[:, e % b->ne[1], t] */
static void op_mul_mat_id(struct ggml_tensor * dst, const struct ggml_tensor * as, const struct ggml_tensor * b,
                          const struct ggml_tensor * ids, int nth) {
    const int wt = as->type;
    const int dt = dot_type_of(wt);
    const int64_t K = as->ne[0], N = as->ne[1];
    const int64_t n_used = ids->ne[0], n_tok = ids->ne[1];
    const size_t drs = dot_row_size(dt, K);
    char * wdata = (char *) malloc(drs * (size_t) (b->ne[1] * b->ne[2]) + 64);
    for (int64_t t = 0; t < b->ne[2]; t++)
    for (int64_t j = 0; j < b->ne[1]; j++) {
        float * row = (float *) malloc((size_t) K * sizeof(float));
        for (int64_t i = 0; i < K; i++) row[i] = load_f(b, ELEM(b, i, j, t, 0));
        to_dot_type(dt, row, wdata + drs * (size_t) (t * b->ne[1] + j), K);
        free(row);
    }
    #pragma omp parallel for collapse(3) num_threads(nth) schedule(static)
    for (int64_t t = 0; t < n_tok; t++)
    for (int64_t e = 0; e < n_used; e++)
    for (int64_t r = 0; r < N; r++) {
        int32_t ex;
        memcpy(&ex, ELEM(ids, e, t, 0, 0), 4);
        if (ex < 0 || ex >= as->ne[2]) { fprintf(stderr, "oracle: expert id %d out of range\n", ex); abort(); }
        const char * w = (const char *) as->data + r * as->nb[1] + ex * as->nb[2];
        const char * x = wdata + drs * (size_t) (t * b->ne[1] + (e % b->ne[1]));
        *(float *) ELEM(dst, r, e, t, 0) = row_dot(wt, w, x, K);
    }
    free(wdata);
}

/* flash attention: per (query, head) online softmax over the keys; K dot in F16 like MUL_MAT;
   V accumulated in f32 (upstream accumulates F16 V in F16 in some versions: deviation noted) */
static void op_flash_attn(struct ggml_tensor * dst, const struct ggml_tensor * q, const struct ggml_tensor * k,
                          const struct ggml_tensor * v, const struct ggml_tensor * mask, int nth) {
    float scale, max_bias, softcap;
    memcpy(&scale, &dst->op_params[0], 4);
    memcpy(&max_bias, &dst->op_params[1], 4);
    memcpy(&softcap, &dst->op_params[2], 4);
    if (g_planted & 4) scale = 1.0f;
    const int64_t D = q->ne[0], DV = v->ne[0], n_kv = k->ne[1];
    const int64_t rk2 = q->ne[2] / k->ne[2], rv2 = q->ne[2] / v->ne[2];
    #pragma omp parallel for collapse(3) num_threads(nth) schedule(static)
    for (int64_t iq3 = 0; iq3 < q->ne[3]; iq3++)
    for (int64_t iq2 = 0; iq2 < q->ne[2]; iq2++)
    for (int64_t iq1 = 0; iq1 < q->ne[1]; iq1++) {
        uint16_t * q16 = (uint16_t *) malloc((size_t) D * 2);
        float * acc = (float *) calloc((size_t) DV, sizeof(float));
        for (int64_t i = 0; i < D; i++) q16[i] = oracle_fp32_to_fp16(load_f(q, ELEM(q, i, iq1, iq2, iq3)));
        float M = -INFINITY, S = 0.0f;
        for (int64_t ic = 0; ic < n_kv; ic++) {
            const float mv = mask ? load_f(mask, (const char *) mask->data + ic * mask->nb[0] + iq1 * mask->nb[1]) : 0.0f;
            if (mv == -INFINITY) continue;
            ggml_float s = 0.0;
            for (int64_t i = 0; i < D; i++) s += (ggml_float) (load_f(k, ELEM(k, i, ic, g_planted & 1 ? iq2 % k->ne[2] : iq2 / rk2, iq3)) * F16(q16[i]));
            float sf = (float) s * scale;
            if (softcap != 0.0f) sf = softcap * tanhf(sf / softcap);
            sf += mv;
            const float Mold = M;
            float ms = 1.0f, vs = 1.0f;
            if (sf > M) {
                M = sf;
                ms = exp_cr(Mold - M);
                for (int64_t i = 0; i < DV; i++) acc[i] *= ms;
            } else {
                vs = exp_cr(sf - M);
            }
            for (int64_t i = 0; i < DV; i++) acc[i] += load_f(v, ELEM(v, i, ic, g_planted & 1 ? iq2 % v->ne[2] : iq2 / rv2, iq3)) * vs;
            S = S * ms + vs;
        }
        const float inv = S == 0.0f ? 0.0f : 1.0f / S;
        for (int64_t i = 0; i < DV; i++) *(float *) ELEM(dst, i, iq2, iq1, iq3) = acc[i] * inv;
        free(q16);
        free(acc);
    }
}

static void op_argmax(struct ggml_tensor * dst, const struct ggml_tensor * a) {
    for (int64_t r = 0; r < a->ne[1]; r++) {
        const float * x = (const float *) ELEM(a, 0, r, 0, 0);
        int32_t best = 0;
        float bv = x[0];
        for (int64_t i = 1; i < a->ne[0]; i++) if (x[i] > bv) { bv = x[i]; best = (int32_t) i; }
        ((int32_t *) dst->data)[r] = best;
    }
}

/* sum of each row, accumulated in double (ggml's generic ggml_vec_sum_f32) */
static void op_sum_rows(struct ggml_tensor * dst, const struct ggml_tensor * a) {
    for (int64_t i3 = 0; i3 < a->ne[3]; i3++)
    for (int64_t i2 = 0; i2 < a->ne[2]; i2++)
    for (int64_t i1 = 0; i1 < a->ne[1]; i1++) {
        ggml_float sum = 0.0;
        for (int64_t i0 = 0; i0 < a->ne[0]; i0++) sum += (ggml_float) load_f(a, ELEM(a, i0, i1, i2, i3));
        store_f(dst, ELEM(dst, 0, i1, i2, i3), (float) sum);
    }
}

/* indices that sort each row, equal values in ascending index order: the tie rule of the router's
   top-k insertion (qwen_model.c:577-590, an earlier expert wins). Insertion sort: stable. */
static void op_argsort(struct ggml_tensor * dst, const struct ggml_tensor * a) {
    const int desc = dst->op_params[0] == GGML_SORT_ORDER_DESC;
    const int64_t n = a->ne[0];
    for (int64_t i3 = 0; i3 < a->ne[3]; i3++)
    for (int64_t i2 = 0; i2 < a->ne[2]; i2++)
    for (int64_t i1 = 0; i1 < a->ne[1]; i1++) {
        int32_t * out = (int32_t *) ELEM(dst, 0, i1, i2, i3);
        for (int64_t i = 0; i < n; i++) {
            const float v = load_f(a, ELEM(a, i, i1, i2, i3));
            int64_t j = i;
            while (j > 0) {
                const float u = load_f(a, ELEM(a, out[j - 1], i1, i2, i3));
                if (desc ? !(u < v) : !(u > v)) break;
                out[j] = out[j - 1];
                j--;
            }
            out[j] = (int32_t) i;
        }
    }
}

static void compute_node(struct ggml_tensor * t, int nth) {
    switch (t->op) {
        case GGML_OP_NONE: case GGML_OP_RESHAPE: case GGML_OP_VIEW: case GGML_OP_PERMUTE: case GGML_OP_TRANSPOSE:
            return;
        case GGML_OP_DUP: case GGML_OP_CONT: op_dup(t, t->src[0], nth); return;
        case GGML_OP_CPY: op_dup(t, t->src[0], nth); return;
        case GGML_OP_GET_ROWS: op_get_rows(t, t->src[0], t->src[1], nth); return;
        case GGML_OP_RMS_NORM: op_rms_norm(t, t->src[0], nth); return;
        case GGML_OP_ADD: case GGML_OP_MUL: case GGML_OP_DIV: case GGML_OP_SUB: op_binary(t, t->src[0], t->src[1], nth); return;
        case GGML_OP_L2_NORM: op_l2_norm(t, t->src[0], nth); return;
        case GGML_OP_CONCAT: op_concat(t, t->src[0], t->src[1]); return;
        case GGML_OP_GLU: op_glu(t, t->src[0], t->src[1], nth); return;
        case GGML_OP_SUM_ROWS: op_sum_rows(t, t->src[0]); return;
        case GGML_OP_ARGSORT: op_argsort(t, t->src[0]); return;
        case GGML_OP_SCALE: case GGML_OP_SQR: case GGML_OP_UNARY: op_unary(t, t->src[0], nth); return;
        case GGML_OP_SOFT_MAX: op_soft_max(t, t->src[0], t->src[1], nth); return;
        case GGML_OP_ROPE: op_rope(t, t->src[0], t->src[1], t->src[2], nth); return;
        case GGML_OP_MUL_MAT: op_mul_mat(t, t->src[0], t->src[1], nth); return;
        case GGML_OP_MUL_MAT_ID: op_mul_mat_id(t, t->src[0], t->src[1], t->src[2], nth); return;
        case GGML_OP_FLASH_ATTN_EXT: op_flash_attn(t, t->src[0], t->src[1], t->src[2], t->src[3], nth); return;
        case GGML_OP_ARGMAX: op_argmax(t, t->src[0]); return;
        default:
            fprintf(stderr, "oracle: unsupported op %s\n", ggml_op_name(t->op));
            abort();
    }
}

/* ------------------------------------------------------------------------------------------ */
/* the "CPU" ggml backend (host buffers)                                                       */

static const char * cpu_buft_name(ggml_backend_buffer_type_t b) { (void) b; return "CPU"; }
static size_t cpu_buft_align(ggml_backend_buffer_type_t b) { (void) b; return 64; }
static bool cpu_buft_is_host(ggml_backend_buffer_type_t b) { (void) b; return true; }

static void cpu_buf_free(ggml_backend_buffer_t b) { free(b->context); }
static void * cpu_buf_base(ggml_backend_buffer_t b) { return b->context; }
static void cpu_buf_set(ggml_backend_buffer_t b, struct ggml_tensor * t, const void * data, size_t off, size_t size) {
    (void) b; memcpy((char *) t->data + off, data, size);
}
static void cpu_buf_get(ggml_backend_buffer_t b, const struct ggml_tensor * t, void * data, size_t off, size_t size) {
    (void) b; memcpy(data, (const char *) t->data + off, size);
}
static void cpu_buf_memset(ggml_backend_buffer_t b, struct ggml_tensor * t, uint8_t v, size_t off, size_t size) {
    (void) b; memset((char *) t->data + off, v, size);
}
static void cpu_buf_clear(ggml_backend_buffer_t b, uint8_t v) { memset(b->context, v, b->size); }

static ggml_backend_buffer_t cpu_buft_alloc(ggml_backend_buffer_type_t buft, size_t size) {
    void * p = aligned_alloc(64, GGML_PAD(size ? size : 64, 64));
    if (!p) return NULL;
    struct ggml_backend_buffer_i iface = {
        cpu_buf_free, cpu_buf_base, NULL, cpu_buf_set, cpu_buf_get, cpu_buf_memset, cpu_buf_clear,
    };
    return ggml_backend_buffer_init(buft, iface, p, size);
}

static struct ggml_backend_buffer_type g_cpu_buft = {
    { cpu_buft_name, cpu_buft_alloc, cpu_buft_align, NULL, cpu_buft_is_host, NULL },
    NULL,
};

static const char * cpu_name(ggml_backend_t b) { (void) b; return "CPU"; }
static void cpu_free(ggml_backend_t b) { free(b->context); free(b); }
static ggml_backend_buffer_type_t cpu_default_buft(ggml_backend_t b) { (void) b; return &g_cpu_buft; }
static enum ggml_status cpu_graph_compute(ggml_backend_t b, struct ggml_cgraph * g) {
    cpu_ctx * c = (cpu_ctx *) b->context;
    for (int i = 0; i < g->n_nodes; i++) {
        compute_node(g->nodes[i], c->n_threads);
        if (c->cb && !c->cb(g->nodes[i], false, c->cb_user)) c->cb = NULL;
    }
    return GGML_STATUS_SUCCESS;
}

static void cpu_set_eval_callback(ggml_backend_t b, ggml_backend_eval_callback cb, void * user) {
    cpu_ctx * c = (cpu_ctx *) b->context;
    c->cb = cb;
    c->cb_user = user;
}

ggml_backend_t ggml_backend_cpu_init(void) {
    ggml_backend_t b = (ggml_backend_t) calloc(1, sizeof(struct ggml_backend));
    cpu_ctx * c = (cpu_ctx *) calloc(1, sizeof(cpu_ctx));
    c->n_threads = 8; /* the reference's default thread count (model.h:308-310) */
    b->iface.get_name = cpu_name;
    b->iface.free = cpu_free;
    b->iface.get_default_buffer_type = cpu_default_buft;
    b->iface.graph_compute = cpu_graph_compute;
    b->iface.synchronize = NULL;
    b->iface.set_eval_callback = cpu_set_eval_callback;
    b->context = c;
    return b;
}

bool ggml_backend_is_cpu(ggml_backend_t backend) { return backend && backend->iface.get_name == cpu_name; }

void ggml_backend_cpu_set_n_threads(ggml_backend_t backend, int n_threads) {
    if (!ggml_backend_is_cpu(backend)) return;
    ((cpu_ctx *) backend->context)->n_threads = n_threads > 0 ? n_threads : 1;
}

/* params: the thread count as a decimal string (init_backend("cpu", n_threads) passes it) */
static ggml_backend_t cpu_init_by_name(const char * params) {
    ggml_backend_t b = ggml_backend_cpu_init();
    if (params && atoi(params) > 0) ggml_backend_cpu_set_n_threads(b, atoi(params));
    return b;
}

__attribute__((constructor)) static void oracle_register(void) { ggml_backend_register("CPU", cpu_init_by_name); }
