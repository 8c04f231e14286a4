// ggml-quants.cpp — GGUF block formats: reference quantizers and row decoders.
//
// Block layouts are fixed by the GGUF format (the reference decodes the same layouts in
// src/moe_stream/dequant.c:39-206):
//   Q4_0  18 B / 32 w : fp16 d, u8 qs[16]; w[j] = (lo4(qs[j]) - 8) d, w[j+16] = (hi4(qs[j]) - 8) d
//   Q8_0  34 B / 32 w : fp16 d, i8 qs[32]; w[j] = qs[j] d
//   Q4_K 144 B / 256 w: fp16 d, fp16 dmin, u8 scales[12] (8 x 6-bit scale + 8 x 6-bit min),
//                       u8 qs[128]; w = d sc_j q - dmin m_j per 32-weight sub-block j
//   Q5_K 176 B / 256 w: fp16 d, fp16 dmin, u8 scales[12] (as Q4_K), u8 qh[32] (bit j of qh[l]: the
//                       fifth bit of element l of sub-block j), u8 qs[128] (low nibbles as Q4_K)
//   Q6_K 210 B / 256 w: u8 ql[128], u8 qh[64], i8 scales[16], fp16 d; per 128-weight half h and
//                       element 32 g + l of it: q = nibble (g >> 1) of ql[64 h + 32 (g & 1) + l] |
//                       bits 2g..2g+1 of qh[32 h + l] << 4; w = d scales[8 h + 2 g + l / 16] (q - 32)
//   Q8_K 292 B / 256 w: f32 d, i8 qs[256], i16 bsums[16] (sum of each 16 quants)
// The quantizers restate ggml's published reference quantizers (quantize_row_*_ref), which are
// what "quantized with ggml's own quantize_row_q4_0" in the benchmark configs means. This file
// is compiled with -ffp-contract=off so its float operation order is the written one.
#include "ggml.h"

#include <algorithm>
#include <cmath>
#include <cstring>
#include <cstdio>
#include <cstdlib>

namespace {

struct blk_q4_0 { ggml_fp16_t d; uint8_t qs[16]; };
struct blk_q8_0 { ggml_fp16_t d; int8_t qs[32]; };
struct blk_q4_K { ggml_fp16_t d; ggml_fp16_t dmin; uint8_t scales[12]; uint8_t qs[128]; };
struct blk_q8_K { float d; int8_t qs[256]; int16_t bsums[16]; };
struct blk_q5_K { ggml_fp16_t d; ggml_fp16_t dmin; uint8_t scales[12]; uint8_t qh[32]; uint8_t qs[128]; };
struct blk_q6_K { uint8_t ql[128]; uint8_t qh[64]; int8_t scales[16]; ggml_fp16_t d; };
static_assert(sizeof(blk_q5_K) == 176, "q5_K block");
static_assert(sizeof(blk_q6_K) == 210, "q6_K block");
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

// The 8 sub-block scales and mins of a Q4_K / Q5_K block as 6-bit codes relative to their
// maxima, packed into the 12 scale bytes (the layout q4k_scale_min reads).
void pack_k4_scales(const float * scales, const float * mins, float max_scale, float max_min, uint8_t * dst) {
    const float inv_scale = max_scale > 0 ? 63.f / max_scale : 0.f;
    const float inv_min = max_min > 0 ? 63.f / max_min : 0.f;
    memset(dst, 0, 12);
    for (int j = 0; j < QK_K / 32; ++j) {
        const int ls = std::min(63, round_half_even(inv_scale * scales[j]));
        const int lm = std::min(63, round_half_even(inv_min * mins[j]));
        if (j < 4) {
            dst[j] = (uint8_t) ls;
            dst[j + 4] = (uint8_t) lm;
        } else {
            dst[j + 4] = (uint8_t) ((ls & 0xf) | ((lm & 0xf) << 4));
            dst[j - 4] |= (uint8_t) ((ls >> 4) << 6);
            dst[j] |= (uint8_t) ((lm >> 4) << 6);
        }
    }
}

// Symmetric fit of codes -nmax..nmax-1 to n values with squared weights x^2, searching the scale
// over 18 rescalings (nmax + 0.1 is) of the largest-magnitude value (is = -9..9, 0 skipped): the
// one with the largest sum(w x l)^2 / sum(w l^2) wins. Codes + nmax land in L. Restatement of
// ggml's make_qx_quants (rmse_type 1, no importance weights).
float fit_symmetric(int n, int nmax, const float * x, int8_t * L) {
    int imax = 0;
    for (int i = 1; i < n; ++i) if (fabsf(x[i]) > fabsf(x[imax])) imax = i;
    const float vmax = x[imax];
    if (fabsf(vmax) < 1e-15f) {
        memset(L, 0, (size_t) n);
        return 0.f;
    }
    auto code = [&](float iscale, int i) { return std::max(-nmax, std::min(nmax - 1, round_half_even(iscale * x[i]))); };
    auto moments = [&](float iscale, float & sxl, float & sl2) {
        sxl = 0; sl2 = 0;
        for (int i = 0; i < n; ++i) {
            const int l = code(iscale, i);
            const float w = x[i] * x[i];
            sxl += w * x[i] * l;
            sl2 += w * l * l;
        }
    };
    float iscale = -nmax / vmax;
    float sxl, sl2;
    moments(iscale, sxl, sl2);
    for (int i = 0; i < n; ++i) L[i] = (int8_t) (code(iscale, i) + nmax);
    float scale = sl2 ? sxl / sl2 : 0.0f;
    float best = scale * sxl;
    for (int is = -9; is <= 9; ++is) {
        if (is == 0) continue;
        iscale = -(nmax + 0.1f * is) / vmax;
        moments(iscale, sxl, sl2);
        if (sl2 > 0 && sxl * sxl > best * sl2) {
            for (int i = 0; i < n; ++i) L[i] = (int8_t) (code(iscale, i) + nmax);
            scale = sxl / sl2;
            best = scale * sxl;
        }
    }
    return scale;
}

// fifth bit j (0/1) of element l of a Q5_K block
inline int q5k_hbit(const blk_q5_K & b, int j, int l) { return (b.qh[l] >> j) & 1; }

// 6-bit code of element e (0..255) of a Q6_K block, before the -32
inline int q6k_code(const blk_q6_K & b, int e) {
    const int h = e / 128, g = (e % 128) / 32, l = e % 32;
    const int lo = (b.ql[64 * h + 32 * (g & 1) + l] >> (4 * (g >> 1))) & 0xf;
    const int hi = (b.qh[32 * h + l] >> (2 * g)) & 3;
    return lo | (hi << 4);
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

// ggml's quantize_row_q5_K_ref: Q4_K's scheme with 5-bit codes (0..31) and a scale search of 16
// rescalings starting at -0.5
void quantize_row_q5_K_ref(const float * x, void * vy, int64_t k) {
    blk_q5_K * y = (blk_q5_K *) vy;
    uint8_t L[QK_K], Laux[32];
    float weights[32], mins[QK_K / 32], scales[QK_K / 32];
    for (int64_t i = 0; i < k / QK_K; i++) {
        const float * xb = x + i * QK_K;
        float max_scale = 0, max_min = 0;
        for (int j = 0; j < QK_K / 32; ++j) {
            const float * xs = xb + 32 * j;
            float sum_x2 = 0;
            for (int l = 0; l < 32; ++l) sum_x2 += xs[l] * xs[l];
            const float av_x = sqrtf(sum_x2 / 32);
            for (int l = 0; l < 32; ++l) weights[l] = av_x + fabsf(xs[l]);
            scales[j] = fit_scale_min(32, 31, xs, weights, L + 32 * j, &mins[j], Laux, -0.5f, 0.1f, 15);
            max_scale = std::max(max_scale, scales[j]);
            max_min = std::max(max_min, mins[j]);
        }
        pack_k4_scales(scales, mins, max_scale, max_min, y[i].scales);
        y[i].d = ggml_fp32_to_fp16(max_scale / 63.f);
        y[i].dmin = ggml_fp32_to_fp16(max_min / 63.f);
        for (int j = 0; j < QK_K / 32; ++j) {
            uint8_t sc, m;
            q4k_scale_min(j, y[i].scales, &sc, &m);
            const float d = ggml_fp16_to_fp32(y[i].d) * sc;
            if (!d) continue;
            const float dm = ggml_fp16_to_fp32(y[i].dmin) * m;
            for (int l = 0; l < 32; ++l) L[32 * j + l] = (uint8_t) std::max(0, std::min(31, round_half_even((xb[32 * j + l] + dm) / d)));
        }
        memset(y[i].qh, 0, sizeof(y[i].qh));
        for (int j = 0; j < QK_K / 32; ++j) {       // sub-block j: nibble j % 2 of qs[32 (j / 2) + l]
            for (int l = 0; l < 32; ++l) {
                const int q = L[32 * j + l];
                uint8_t & dst = y[i].qs[32 * (j / 2) + l];
                dst = (j & 1) ? (uint8_t) ((dst & 0x0f) | ((q & 15) << 4)) : (uint8_t) (q & 15);
                y[i].qh[l] |= (uint8_t) ((q >> 4) << j);
            }
        }
    }
}

// ggml's quantize_row_q6_K_ref: 16 sub-blocks of 16 fitted symmetrically (codes -32..31), the
// sub-block scales as signed 8-bit codes of the largest-magnitude one (-> -128), the codes
// re-rounded under the decoded scales
void quantize_row_q6_K_ref(const float * x, void * vy, int64_t k) {
    blk_q6_K * y = (blk_q6_K *) vy;
    int8_t L[QK_K];
    float scales[QK_K / 16];
    for (int64_t i = 0; i < k / QK_K; i++) {
        const float * xb = x + i * QK_K;
        float max_scale = 0, max_abs = 0;
        for (int j = 0; j < QK_K / 16; ++j) {
            scales[j] = fit_symmetric(16, 32, xb + 16 * j, L + 16 * j);
            if (fabsf(scales[j]) > max_abs) {
                max_abs = fabsf(scales[j]);
                max_scale = scales[j];
            }
        }
        memset(&y[i], 0, sizeof(blk_q6_K));
        if (max_abs < 1e-15f) continue;
        const float iscale = -128.f / max_scale;
        y[i].d = ggml_fp32_to_fp16(1 / iscale);
        for (int j = 0; j < QK_K / 16; ++j) y[i].scales[j] = (int8_t) std::min(127, round_half_even(iscale * scales[j]));
        for (int j = 0; j < QK_K / 16; ++j) {
            const float d = ggml_fp16_to_fp32(y[i].d) * y[i].scales[j];
            if (!d) continue;
            for (int l = 0; l < 16; ++l) L[16 * j + l] = (int8_t) (std::max(-32, std::min(31, round_half_even(xb[16 * j + l] / d))) + 32);
        }
        for (int e = 0; e < QK_K; ++e) {            // the code of element e into its nibble and bit pair
            const int h = e / 128, g = (e % 128) / 32, l = e % 32, q = L[e];
            y[i].ql[64 * h + 32 * (g & 1) + l] |= (uint8_t) ((q & 15) << (4 * (g >> 1)));
            y[i].qh[32 * h + l] |= (uint8_t) ((q >> 4) << (2 * g));
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

void dequantize_row_q5_K(const void * vx, float * y, int64_t k) {
    const blk_q5_K * x = (const blk_q5_K *) vx;
    for (int64_t i = 0; i < k / QK_K; i++) {
        const float d = ggml_fp16_to_fp32(x[i].d), dmin = ggml_fp16_to_fp32(x[i].dmin);
        for (int j = 0; j < QK_K / 32; ++j) {
            uint8_t sc, m;
            q4k_scale_min(j, x[i].scales, &sc, &m);
            const float dj = d * sc, mj = dmin * m;
            for (int l = 0; l < 32; ++l) {
                const uint8_t b = x[i].qs[32 * (j / 2) + l];
                const int q = ((j & 1) ? (b >> 4) : (b & 0xf)) + 16 * q5k_hbit(x[i], j, l);
                *y++ = dj * q - mj;
            }
        }
    }
}

void dequantize_row_q6_K(const void * vx, float * y, int64_t k) {
    const blk_q6_K * x = (const blk_q6_K *) vx;
    for (int64_t i = 0; i < k / QK_K; i++) {
        const float d = ggml_fp16_to_fp32(x[i].d);
        for (int e = 0; e < QK_K; ++e) {
            const int h = e / 128, g = (e % 128) / 32, l = e % 32;
            *y++ = d * x[i].scales[8 * h + 2 * g + l / 16] * (q6k_code(x[i], e) - 32);
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
        case GGML_TYPE_Q5_K: dequantize_row_q5_K(x, y, k); return true;
        case GGML_TYPE_Q6_K: dequantize_row_q6_K(x, y, k); return true;
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
            case GGML_TYPE_Q5_K: quantize_row_q5_K_ref(xr, yr, n_per_row); break;
            case GGML_TYPE_Q6_K: quantize_row_q6_K_ref(xr, yr, n_per_row); break;
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
