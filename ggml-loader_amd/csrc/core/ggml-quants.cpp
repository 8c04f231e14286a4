// ggml-quants.cpp — GGUF block formats: reference quantizers and row decoders.
//
// Block layouts are fixed by the GGUF format (the reference decodes the same layouts in
// src/moe_stream/dequant.c:39-206):
//   Q4_0  18 B / 32 w : fp16 d, u8 qs[16]; w[j] = (lo4(qs[j]) - 8) d, w[j+16] = (hi4(qs[j]) - 8) d
//   Q8_0  34 B / 32 w : fp16 d, i8 qs[32]; w[j] = qs[j] d
//   Q4_K 144 B / 256 w: fp16 d, fp16 dmin, u8 scales[12] (8 x 6-bit scale + 8 x 6-bit min),
//                       u8 qs[128]; w = d sc_j q - dmin m_j per 32-weight sub-block j
//   Q8_K 292 B / 256 w: f32 d, i8 qs[256], i16 bsums[16] (sum of each 16 quants)
// The quantizers restate ggml's published reference quantizers (quantize_row_*_ref), which are
// what "quantized with ggml's own quantize_row_q4_0" in the benchmark configs means. This file
// is compiled with -ffp-contract=off so its float operation order is the written one.
#include "ggml.h"

#include <cmath>
#include <cstring>
#include <cstdio>
#include <cstdlib>

namespace {

struct blk_q4_0 { ggml_fp16_t d; uint8_t qs[16]; };
struct blk_q8_0 { ggml_fp16_t d; int8_t qs[32]; };
struct blk_q4_K { ggml_fp16_t d; ggml_fp16_t dmin; uint8_t scales[12]; uint8_t qs[128]; };
struct blk_q8_K { float d; int8_t qs[256]; int16_t bsums[16]; };
static_assert(sizeof(blk_q4_0) == 18, "q4_0 block");
static_assert(sizeof(blk_q8_0) == 34, "q8_0 block");
static_assert(sizeof(blk_q4_K) == 144, "q4_K block");
static_assert(sizeof(blk_q8_K) == 292, "q8_K block");

// round-half-to-even for |v| < 2^22 via the float mantissa (the value ggml's nearest_int gives)
inline int round_half_even(float v) {
    float t = v + 12582912.0f; // 1.5 * 2^23
    int32_t i;
    memcpy(&i, &t, 4);
    return (i & 0x007fffff) - 0x00400000;
}

// 6-bit scale/min pair j of a Q4_K block (j = 0..7)
inline void q4k_scale_min(int j, const uint8_t * s, uint8_t * sc, uint8_t * mn) {
    if (j < 4) {
        *sc = s[j] & 63;
        *mn = s[j + 4] & 63;
    } else {
        *sc = (uint8_t) ((s[j + 4] & 0x0f) | ((s[j - 4] >> 6) << 4));
        *mn = (uint8_t) ((s[j + 4] >> 4) | ((s[j] >> 6) << 4));
    }
}

// Weighted least-squares fit of an asymmetric 4-bit (nmax=15) grid to n values, searching the
// scale over nstep+1 candidates around nmax/(max-min). Returns the scale; *neg_min receives
// -min (>= 0). Restatement of ggml's make_qkx2_quants.
float fit_scale_min(int n, int nmax, const float * x, const float * w, uint8_t * L, float * neg_min,
                    uint8_t * Laux, float rmin, float rdelta, int nstep) {
    float mn = x[0], mx = x[0];
    float sum_w = w[0];
    float sum_x = sum_w * x[0];
    for (int i = 1; i < n; ++i) {
        if (x[i] < mn) mn = x[i];
        if (x[i] > mx) mx = x[i];
        sum_w += w[i];
        sum_x += w[i] * x[i];
    }
    if (mn > 0) mn = 0;
    if (mx == mn) {
        for (int i = 0; i < n; ++i) L[i] = 0;
        *neg_min = -mn;
        return 0.f;
    }
    float iscale = nmax / (mx - mn);
    float scale = 1 / iscale;
    float best = 0;
    for (int i = 0; i < n; ++i) {
        int l = round_half_even(iscale * (x[i] - mn));
        l = l < 0 ? 0 : (l > nmax ? nmax : l);
        L[i] = (uint8_t) l;
        float diff = scale * L[i] + mn - x[i];
        best += w[i] * (diff * diff);
    }
    for (int is = 0; is <= nstep; ++is) {
        iscale = (rmin + rdelta * is + nmax) / (mx - mn);
        float sum_l = 0, sum_l2 = 0, sum_xl = 0;
        for (int i = 0; i < n; ++i) {
            int l = round_half_even(iscale * (x[i] - mn));
            l = l < 0 ? 0 : (l > nmax ? nmax : l);
            Laux[i] = (uint8_t) l;
            sum_l += w[i] * l;
            sum_l2 += w[i] * l * l;
            sum_xl += w[i] * l * x[i];
        }
        float D = sum_w * sum_l2 - sum_l * sum_l;
        if (D > 0) {
            float this_scale = (sum_w * sum_xl - sum_x * sum_l) / D;
            float this_min = (sum_l2 * sum_x - sum_l * sum_xl) / D;
            if (this_min > 0) {
                this_min = 0;
                this_scale = sum_xl / sum_l2;
            }
            float err = 0;
            for (int i = 0; i < n; ++i) {
                float diff = this_scale * Laux[i] + this_min - x[i];
                err += w[i] * (diff * diff);
            }
            if (err < best) {
                for (int i = 0; i < n; ++i) L[i] = Laux[i];
                best = err;
                scale = this_scale;
                mn = this_min;
            }
        }
    }
    *neg_min = -mn;
    return scale;
}

} // namespace

extern "C" {

void quantize_row_q4_0_ref(const float * x, void * vy, int64_t k) {
    blk_q4_0 * y = (blk_q4_0 *) vy;
    const int64_t nb = k / 32;
    for (int64_t i = 0; i < nb; i++) {
        const float * xb = x + i * 32;
        float amax = 0.0f, vmax = 0.0f; // signed value with the largest magnitude (first wins)
        for (int j = 0; j < 32; j++) {
            if (amax < fabsf(xb[j])) { amax = fabsf(xb[j]); vmax = xb[j]; }
        }
        const float d = vmax / -8;
        const float id = d ? 1.0f / d : 0.0f;
        y[i].d = ggml_fp32_to_fp16(d);
        for (int j = 0; j < 16; ++j) {
            const float x0 = xb[j] * id;
            const float x1 = xb[16 + j] * id;
            int q0 = (int8_t) (x0 + 8.5f);
            int q1 = (int8_t) (x1 + 8.5f);
            q0 = q0 < 15 ? q0 : 15;
            q1 = q1 < 15 ? q1 : 15;
            y[i].qs[j] = (uint8_t) (q0 | (q1 << 4));
        }
    }
}

void quantize_row_q8_0_ref(const float * x, void * vy, int64_t k) {
    blk_q8_0 * y = (blk_q8_0 *) vy;
    const int64_t nb = k / 32;
    for (int64_t i = 0; i < nb; i++) {
        const float * xb = x + i * 32;
        float amax = 0.0f;
        for (int j = 0; j < 32; j++) amax = fmaxf(amax, fabsf(xb[j]));
        const float d = amax / 127;
        const float id = d ? 1.0f / d : 0.0f;
        y[i].d = ggml_fp32_to_fp16(d);
        for (int j = 0; j < 32; ++j) y[i].qs[j] = (int8_t) roundf(xb[j] * id);
    }
}

void quantize_row_q8_K_ref(const float * x, void * vy, int64_t k) {
    blk_q8_K * y = (blk_q8_K *) vy;
    const int64_t nb = k / QK_K;
    for (int64_t i = 0; i < nb; i++) {
        const float * xb = x + i * QK_K;
        float amax = 0, vmax = 0;
        for (int j = 0; j < QK_K; ++j) {
            const float ax = fabsf(xb[j]);
            if (ax > amax) { amax = ax; vmax = xb[j]; }
        }
        if (!amax) {
            y[i].d = 0;
            memset(y[i].qs, 0, QK_K);
            memset(y[i].bsums, 0, sizeof(y[i].bsums));
            continue;
        }
        const float iscale = -127.f / vmax;
        for (int j = 0; j < QK_K; ++j) {
            const int v = round_half_even(iscale * xb[j]);
            y[i].qs[j] = (int8_t) (v < 127 ? v : 127);
        }
        for (int j = 0; j < QK_K / 16; ++j) {
            int s = 0;
            for (int l = 0; l < 16; ++l) s += y[i].qs[j * 16 + l];
            y[i].bsums[j] = (int16_t) s;
        }
        y[i].d = 1 / iscale;
    }
}

void quantize_row_q4_K_ref(const float * x, void * vy, int64_t k) {
    blk_q4_K * y = (blk_q4_K *) vy;
    const int64_t nb = k / QK_K;
    uint8_t L[QK_K];
    uint8_t Laux[32];
    float weights[32];
    float mins[QK_K / 32];
    float scales[QK_K / 32];
    for (int64_t i = 0; i < nb; i++) {
        const float * xb = x + i * QK_K;
        float max_scale = 0, max_min = 0;
        for (int j = 0; j < QK_K / 32; ++j) {
            float sum_x2 = 0;
            for (int l = 0; l < 32; ++l) sum_x2 += xb[32 * j + l] * xb[32 * j + l];
            const float av_x = sqrtf(sum_x2 / 32);
            for (int l = 0; l < 32; ++l) weights[l] = av_x + fabsf(xb[32 * j + l]);
            scales[j] = fit_scale_min(32, 15, xb + 32 * j, weights, L + 32 * j, &mins[j], Laux, -1.f, 0.1f, 20);
            if (scales[j] > max_scale) max_scale = scales[j];
            if (mins[j] > max_min) max_min = mins[j];
        }
        const float inv_scale = max_scale > 0 ? 63.f / max_scale : 0.f;
        const float inv_min = max_min > 0 ? 63.f / max_min : 0.f;
        memset(y[i].scales, 0, 12);
        for (int j = 0; j < QK_K / 32; ++j) {
            uint8_t ls = (uint8_t) round_half_even(inv_scale * scales[j]);
            uint8_t lm = (uint8_t) round_half_even(inv_min * mins[j]);
            ls = ls < 63 ? ls : 63;
            lm = lm < 63 ? lm : 63;
            if (j < 4) {
                y[i].scales[j] = ls;
                y[i].scales[j + 4] = lm;
            } else {
                y[i].scales[j + 4] = (uint8_t) ((ls & 0xf) | ((lm & 0xf) << 4));
                y[i].scales[j - 4] |= (uint8_t) ((ls >> 4) << 6);
                y[i].scales[j - 0] |= (uint8_t) ((lm >> 4) << 6);
            }
        }
        y[i].d = ggml_fp32_to_fp16(max_scale / 63.f);
        y[i].dmin = ggml_fp32_to_fp16(max_min / 63.f);
        for (int j = 0; j < QK_K / 32; ++j) {
            uint8_t sc, m;
            q4k_scale_min(j, y[i].scales, &sc, &m);
            const float d = ggml_fp16_to_fp32(y[i].d) * sc;
            if (!d) continue;
            const float dm = ggml_fp16_to_fp32(y[i].dmin) * m;
            for (int ii = 0; ii < 32; ++ii) {
                int l = round_half_even((xb[32 * j + ii] + dm) / d);
                l = l < 0 ? 0 : (l > 15 ? 15 : l);
                L[32 * j + ii] = (uint8_t) l;
            }
        }
        uint8_t * q = y[i].qs;
        for (int j = 0; j < QK_K; j += 64) {
            for (int l = 0; l < 32; ++l) q[l] = (uint8_t) (L[j + l] | (L[j + l + 32] << 4));
            q += 32;
        }
    }
}

void dequantize_row_q4_0(const void * vx, float * y, int64_t k) {
    const blk_q4_0 * x = (const blk_q4_0 *) vx;
    for (int64_t i = 0; i < k / 32; i++) {
        const float d = ggml_fp16_to_fp32(x[i].d);
        for (int j = 0; j < 16; ++j) {
            const int x0 = (x[i].qs[j] & 0x0f) - 8;
            const int x1 = (x[i].qs[j] >> 4) - 8;
            y[i * 32 + j] = x0 * d;
            y[i * 32 + j + 16] = x1 * d;
        }
    }
}

void dequantize_row_q8_0(const void * vx, float * y, int64_t k) {
    const blk_q8_0 * x = (const blk_q8_0 *) vx;
    for (int64_t i = 0; i < k / 32; i++) {
        const float d = ggml_fp16_to_fp32(x[i].d);
        for (int j = 0; j < 32; ++j) y[i * 32 + j] = x[i].qs[j] * d;
    }
}

void dequantize_row_q4_K(const void * vx, float * y, int64_t k) {
    const blk_q4_K * x = (const blk_q4_K *) vx;
    for (int64_t i = 0; i < k / QK_K; i++) {
        const float d = ggml_fp16_to_fp32(x[i].d);
        const float dmin = ggml_fp16_to_fp32(x[i].dmin);
        const uint8_t * q = x[i].qs;
        int is = 0;
        for (int j = 0; j < QK_K; j += 64) {
            uint8_t sc, m;
            q4k_scale_min(is + 0, x[i].scales, &sc, &m);
            const float d1 = d * sc, m1 = dmin * m;
            q4k_scale_min(is + 1, x[i].scales, &sc, &m);
            const float d2 = d * sc, m2 = dmin * m;
            for (int l = 0; l < 32; ++l) *y++ = d1 * (q[l] & 0xf) - m1;
            for (int l = 0; l < 32; ++l) *y++ = d2 * (q[l] >> 4) - m2;
            q += 32;
            is += 2;
        }
    }
}

bool ggml_dequantize_row(enum ggml_type type, const void * x, float * y, int64_t k) {
    switch (type) {
        case GGML_TYPE_F32: memcpy(y, x, (size_t) k * 4); return true;
        case GGML_TYPE_F16: ggml_fp16_to_fp32_row((const ggml_fp16_t *) x, y, k); return true;
        case GGML_TYPE_BF16: for (int64_t i = 0; i < k; i++) y[i] = ggml_bf16_to_fp32(((const ggml_bf16_t *) x)[i]); return true;
        case GGML_TYPE_Q4_0: dequantize_row_q4_0(x, y, k); return true;
        case GGML_TYPE_Q8_0: dequantize_row_q8_0(x, y, k); return true;
        case GGML_TYPE_Q4_K: dequantize_row_q4_K(x, y, k); return true;
        default: return false;
    }
}

size_t ggml_quantize_chunk(enum ggml_type type, const float * src, void * dst, int64_t start,
                           int64_t nrows, int64_t n_per_row, const float * imatrix) {
    (void) imatrix; // importance weighting is not used by the synthetic models
    if (start % n_per_row != 0) {
        fprintf(stderr, "ggml_quantize_chunk: start %lld is not row aligned\n", (long long) start);
        abort();
    }
    const size_t row_size = ggml_row_size(type, n_per_row);
    char * out = (char *) dst + (start / n_per_row) * row_size;
    const float * in = src + start;
    for (int64_t r = 0; r < nrows; r++) {
        const float * xr = in + r * n_per_row;
        void * yr = out + r * row_size;
        switch (type) {
            case GGML_TYPE_Q4_0: quantize_row_q4_0_ref(xr, yr, n_per_row); break;
            case GGML_TYPE_Q8_0: quantize_row_q8_0_ref(xr, yr, n_per_row); break;
            case GGML_TYPE_Q4_K: quantize_row_q4_K_ref(xr, yr, n_per_row); break;
            case GGML_TYPE_Q8_K: quantize_row_q8_K_ref(xr, yr, n_per_row); break;
            case GGML_TYPE_F16: ggml_fp32_to_fp16_row(xr, (ggml_fp16_t *) yr, n_per_row); break;
            case GGML_TYPE_F32: memcpy(yr, xr, (size_t) n_per_row * 4); break;
            default:
                fprintf(stderr, "ggml_quantize_chunk: unsupported type %s\n", ggml_type_name(type));
                abort();
        }
    }
    return (size_t) nrows * row_size;
}

} // extern "C"
