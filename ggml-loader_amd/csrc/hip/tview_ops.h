// tview_ops.h — device helpers over strided tensor views: element addressing, typed loads and
// stores (with ggml's conversions), and the RoPE rotation of one element.
#pragma once

#include "kernels.h"

#include "ggml.h"

__device__ __forceinline__ float ld(const char * p, int type) {
    switch (type) {
        case GGML_TYPE_F32: return *(const float *) p;
        case GGML_TYPE_F16: return __half2float(*(const __half *) p);
        case GGML_TYPE_BF16: return __uint_as_float(((uint32_t) *(const uint16_t *) p) << 16);
        case GGML_TYPE_I32: return (float) *(const int32_t *) p;
        default: return 0.0f;
    }
}

__device__ __forceinline__ void st(char * p, int type, float v) {
    switch (type) {
        case GGML_TYPE_F32: *(float *) p = v; break;
        case GGML_TYPE_F16: *(__half *) p = __float2half_rn(as_f32(v)); break;
        case GGML_TYPE_BF16: {
            uint32_t u = __float_as_uint(as_f32(v));
            if ((u & 0x7fffffffu) > 0x7f800000u) u = (u >> 16) | 64u;
            else u = (u + (0x7fffu + ((u >> 16) & 1u))) >> 16;
            *(uint16_t *) p = (uint16_t) u;
            break;
        }
        case GGML_TYPE_I32: *(int32_t *) p = (int32_t) v; break;
        default: break;
    }
}

struct idx4 { int64_t i0, i1, i2, i3; };

__device__ __forceinline__ idx4 unflatten(int64_t i, const int64_t ne[4]) {
    idx4 r;
    r.i0 = i % ne[0]; i /= ne[0];
    r.i1 = i % ne[1]; i /= ne[1];
    r.i2 = i % ne[2]; i /= ne[2];
    r.i3 = i;
    return r;
}

__device__ __forceinline__ char * at(const tview & t, int64_t i0, int64_t i1, int64_t i2, int64_t i3) {
    return t.data + i0 * t.nb[0] + i1 * t.nb[1] + i2 * t.nb[2] + i3 * t.nb[3];
}

// ---------------------------------------------------------------------------------------------
// RoPE

__device__ __forceinline__ void rope_cs(float theta_extrap, const rope_params & p, int i0, float & c, float & s) {
    const float theta_interp = p.freq_scale * theta_extrap;
    float theta = theta_interp;
    float mscale = p.attn_factor;
    if (p.ext_factor != 0.0f) {
        const float y = (i0 / 2 - p.corr_dims[0]) / fmaxf(0.001f, p.corr_dims[1] - p.corr_dims[0]);
        const float ramp = 1 - fminf(1, fmaxf(0, y));
        const float ramp_mix = ramp * p.ext_factor;
        theta = theta_interp * (1 - ramp_mix) + theta_extrap * ramp_mix;
        mscale *= 1.0f + 0.1f * log_cr(1.0f / p.freq_scale);
    }
    float sv, cv;
    sincos_cr(theta, sv, cv);
    c = cv * mscale;
    s = sv * mscale;
}

// the (cos, sin) of rotation pair ip at position pos, as the RoPE kernel forms them (theta by
// repeated multiplication, the same scaling)
__device__ __forceinline__ void rope_pair_cs(const rope_params & p, const float * ff, int32_t pos, int ip, float & c, float & s) {
    float theta = (float) pos;
    for (int k = 0; k < ip; k++) theta *= p.theta_scale;
    const float f = ff ? ff[ip] : 1.0f;
    rope_cs(theta / f, p, 2 * ip, c, s);
}

// element d of a row rotated with the (cos, sin) cs[ip] of its pair; val(e) gives element e of the
// row before the rotation
template <typename F>
__device__ __forceinline__ float rope_value_with(const rope_params & p, int d, const float2 * cs, F val) {
    if (d >= p.n_dims) return val(d);
    const bool neox = (p.mode & GGML_ROPE_TYPE_NEOX) != 0;
    const int ip = neox ? d % (p.n_dims / 2) : d / 2;
    const int a0 = neox ? ip : 2 * ip, a1 = neox ? ip + p.n_dims / 2 : 2 * ip + 1;
    const float x0 = val(a0), x1 = val(a1);
    const float c = cs[ip].x, sn = cs[ip].y;
    return d == a0 ? x0 * c - x1 * sn : x0 * sn + x1 * c;
}

// element d of row (i1, i2, i3) of J.src rotated with the (cos, sin) cs[ip] of its pair
__device__ __forceinline__ float rope_value_cs(const rope_job & J, int64_t i1, int64_t i2, int64_t i3, int d, const float2 * cs) {
    return rope_value_with(J.p, d, cs, [&](int e) { return *(const float *) at(J.src, e, i1, i2, i3); });
}

// the same for a row normalized first (qk_norm), with its scale already formed
__device__ __forceinline__ float rope_value_norm_cs(const rope_params & p, const qk_norm & N, int64_t head, int64_t tok,
                                                    float scale, int d, const float2 * cs) {
    const float * xr = N.x + head * N.nb1 + tok * N.nb2;
    return rope_value_with(p, d, cs, [&](int e) { return (xr[e] * scale) * N.w[e]; });
}

// element d of row (i1, i2, i3) of J.src rotated as ggml's RoPE does (the arithmetic of one pair of
// the RoPE kernel: theta by repeated multiplication, the same cos/sin and products)
__device__ __forceinline__ float rope_value(const rope_job & J, int64_t i1, int64_t i2, int64_t i3, int d) {
    const rope_params & p = J.p;
    if (d >= p.n_dims) return *(const float *) at(J.src, d, i1, i2, i3);
    const bool neox = (p.mode & GGML_ROPE_TYPE_NEOX) != 0;
    const int ip = neox ? d % (p.n_dims / 2) : d / 2;
    const int i0 = 2 * ip;
    float theta = (float) J.pos[i2];
    for (int k = 0; k < ip; k++) theta *= p.theta_scale;
    const float f = J.ff ? J.ff[ip] : 1.0f;
    float c, sn;
    rope_cs(theta / f, p, i0, c, sn);
    const int a0 = neox ? ip : i0, a1 = neox ? ip + p.n_dims / 2 : i0 + 1;
    const float x0 = *(const float *) at(J.src, a0, i1, i2, i3);
    const float x1 = *(const float *) at(J.src, a1, i1, i2, i3);
    return d == a0 ? x0 * c - x1 * sn : x0 * sn + x1 * c;
}
