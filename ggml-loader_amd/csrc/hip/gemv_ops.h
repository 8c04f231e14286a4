// gemv_ops.h — device helpers shared by the GEMV kernels (one column per workgroup in k_gemv.hip,
// several columns per workgroup in k_gemv_mc.hip): launch arguments, the integer block dots of
// Q4_0 / Q8_0 / Q4_K against Q8_0 / Q8_K activations, and the block-ordered float sum.
#pragma once

#include "kernels.h"

#include "ggml.h"

// Grid rows: the matrices' rows one after another, each matrix starting on a workgroup boundary
// (row_begin[i] is a multiple of rows_per_block), so every workgroup reads a single matrix and
// selects it with uniform (scalar) arithmetic. Rows past a matrix's n_rows are padding.
struct gemv_kargs {
    gemv_launch L;
    int total_rows;
    int row_begin[GEMV_MAX_MATS + 1];
    int rows_per_block;
};

__device__ __forceinline__ int find_mat(const gemv_kargs & a, int row) {
    int m = 0;
#pragma unroll
    for (int i = 1; i < GEMV_MAX_MATS; i++) if (i < a.L.n_mats && row >= a.row_begin[i]) m = i;
    return m;
}

// sum(q * x) over one Q4_0 block with q in 0..15 (the -8 offset is applied through the block sum)
__device__ __forceinline__ int dot_q4_0_block(const uint4 q, const int4 xa, const int4 xb) {
    int s = 0;
    s = dot4((int) (q.x & 0x0F0F0F0Fu), xa.x, s);
    s = dot4((int) (q.y & 0x0F0F0F0Fu), xa.y, s);
    s = dot4((int) (q.z & 0x0F0F0F0Fu), xa.z, s);
    s = dot4((int) (q.w & 0x0F0F0F0Fu), xa.w, s);
    s = dot4((int) ((q.x >> 4) & 0x0F0F0F0Fu), xb.x, s);
    s = dot4((int) ((q.y >> 4) & 0x0F0F0F0Fu), xb.y, s);
    s = dot4((int) ((q.z >> 4) & 0x0F0F0F0Fu), xb.z, s);
    s = dot4((int) ((q.w >> 4) & 0x0F0F0F0Fu), xb.w, s);
    return s;
}

__device__ __forceinline__ int dot_q8_0_block(const uint4 qa, const uint4 qb, const int4 xa, const int4 xb) {
    int s = 0;
    s = dot4((int) qa.x, xa.x, s);
    s = dot4((int) qa.y, xa.y, s);
    s = dot4((int) qa.z, xa.z, s);
    s = dot4((int) qa.w, xa.w, s);
    s = dot4((int) qb.x, xb.x, s);
    s = dot4((int) qb.y, xb.y, s);
    s = dot4((int) qb.z, xb.z, s);
    s = dot4((int) qb.w, xb.w, s);
    return s;
}

// byte i (0..11) of the 12 Q4_K scale bytes held in three dwords
__device__ __forceinline__ int sbyte(uint32_t w0, uint32_t w1, uint32_t w2, int i) {
    const uint32_t w = i < 4 ? w0 : (i < 8 ? w1 : w2);
    return (int) ((w >> (8 * (i & 3))) & 0xff);
}

// 6-bit scale/min j (0..7) of a Q4_K block (moe_stream/dequant.c:132-141 layout)
__device__ __forceinline__ void q4k_sc_m(uint32_t w0, uint32_t w1, uint32_t w2, int j, int & sc, int & m) {
    if (j < 4) {
        sc = sbyte(w0, w1, w2, j) & 63;
        m = sbyte(w0, w1, w2, j + 4) & 63;
    } else {
        sc = (sbyte(w0, w1, w2, j + 4) & 0x0F) | ((sbyte(w0, w1, w2, j - 4) >> 6) << 4);
        m = (sbyte(w0, w1, w2, j + 4) >> 4) | ((sbyte(w0, w1, w2, j) >> 6) << 4);
    }
}

// 4x4 byte transpose: t_b = { byte b of a, byte b of b, byte b of c, byte b of d } (v_perm_b32:
// selector bytes 0-3 pick from the second operand, 4-7 from the first)
__device__ __forceinline__ void transpose4(uint32_t a, uint32_t b, uint32_t c, uint32_t d, uint32_t t[4]) {
    const uint32_t p0 = __builtin_amdgcn_perm(b, a, 0x05010400u), p1 = __builtin_amdgcn_perm(b, a, 0x07030602u);
    const uint32_t q0 = __builtin_amdgcn_perm(d, c, 0x05010400u), q1 = __builtin_amdgcn_perm(d, c, 0x07030602u);
    t[0] = __builtin_amdgcn_perm(q0, p0, 0x05040100u);
    t[1] = __builtin_amdgcn_perm(q0, p0, 0x07060302u);
    t[2] = __builtin_amdgcn_perm(q1, p1, 0x05040100u);
    t[3] = __builtin_amdgcn_perm(q1, p1, 0x07060302u);
}

// The 32 bytes of a sub-block rearranged so that dword l holds elements l, l+8, l+16, l+24 (the
// elements ggml's generic q4_K x q8_K dot accumulates into aux32[l]); in place, 8 dwords.
__device__ __forceinline__ void q4k_group_by_l(uint32_t * w) {
    uint32_t t[8];
    transpose4(w[0], w[2], w[4], w[6], t);
    transpose4(w[1], w[3], w[5], w[7], t + 4);
#pragma unroll
    for (int l = 0; l < 8; l++) w[l] = t[l];
}

// n 32-byte sub-blocks of an int8 activation in LDS grouped by l in place, one thread per sub-block
__device__ __forceinline__ void group_by_l_lds(int8_t * xq, int n) {
    for (int sbk = threadIdx.x; sbk < n; sbk += blockDim.x) {
        uint4 * p = (uint4 *) (xq + sbk * 32);
        const uint4 lo4 = p[0], hi4 = p[1];
        uint32_t w8[8] = { lo4.x, lo4.y, lo4.z, lo4.w, hi4.x, hi4.y, hi4.z, hi4.w };
        q4k_group_by_l(w8);
        p[0] = make_uint4(w8[0], w8[1], w8[2], w8[3]);
        p[1] = make_uint4(w8[4], w8[5], w8[6], w8[7]);
    }
}

// One Q4_K unit u = (super-block u/4, sub-block pair p = u%4) of a weight row, ready for dots: the
// two sub-blocks' 6-bit scales and mins and their 32 quant bytes grouped by l (q4k_group_by_l;
// low nibbles: sub-block 2p, high nibbles: 2p + 1). hdr is the block's first 16 bytes (d, dmin,
// scales), qa/qb the pair's 32 quant bytes.
struct q4k_unit {
    int sc_a, m_a, sc_b, m_b;
    uint32_t q[8];
};

__device__ __forceinline__ q4k_unit q4k_prepare(const uint4 hdr, const uint4 qa, const uint4 qb, int p) {
    q4k_unit U;
    q4k_sc_m(hdr.y, hdr.z, hdr.w, 2 * p, U.sc_a, U.m_a);
    q4k_sc_m(hdr.y, hdr.z, hdr.w, 2 * p + 1, U.sc_b, U.m_b);
    U.q[0] = qa.x; U.q[1] = qa.y; U.q[2] = qa.z; U.q[3] = qa.w;
    U.q[4] = qb.x; U.q[5] = qb.y; U.q[6] = qb.z; U.q[7] = qb.w;
    q4k_group_by_l(U.q);
    return U;
}

// Per-lane integer partials of a unit against one activation column: aux[l] = sum over the pair's
// 64 elements e with e%8 == l of sc_sub * q4 * q8, mins = the pair's share of sum(bsums * m).
// (ggml's generic q4_K x q8_K kernel accumulates exactly these integers.) xa/xb: the two
// sub-blocks' activations grouped by l, so each aux[l] takes one v_dot4 per sub-block; xbs: the
// super-block's 16 bsums.
__device__ __forceinline__ void q4k_unit_dot(const q4k_unit & U, int p, const int * xa, const int * xb,
                                             const int16_t * xbs, int aux[8], int & mins) {
#pragma unroll
    for (int l = 0; l < 8; l++) {
        const int lo = (int) (U.q[l] & 0x0F0F0F0Fu), hi = (int) ((U.q[l] >> 4) & 0x0F0F0F0Fu);
        aux[l] = U.sc_a * dot4(lo, xa[l], 0) + U.sc_b * dot4(hi, xb[l], 0);
    }
    mins = U.m_a * ((int) xbs[4 * p] + (int) xbs[4 * p + 1]) + U.m_b * ((int) xbs[4 * p + 2] + (int) xbs[4 * p + 3]);
}

// A Q5_K unit (sub-block pair p): the Q4_K unit's nibbles (U, from the block's header and the
// pair's 32 bytes of qs) with each code's fifth bit, bit 2p (low nibbles: sub-block 2p) or 2p + 1
// (high nibbles) of qh[l] for element position l; the 32 qh bytes (h0, h1) grouped by l as the
// nibbles are. Codes 0..31 fit a signed byte, so the dots are Q4_K's; the mins term is Q4_K's too.
// The integers are those of ggml's generic q5_K x q8_K kernel.
__device__ __forceinline__ void q5k_unit_dot(const q4k_unit & U, uint4 h0, uint4 h1, int p, const int * xa, const int * xb,
                                             const int16_t * xbs, int aux[8], int & mins) {
    uint32_t h[8] = { h0.x, h0.y, h0.z, h0.w, h1.x, h1.y, h1.z, h1.w };
    q4k_group_by_l(h);
#pragma unroll
    for (int l = 0; l < 8; l++) {
        const int lo = (int) ((U.q[l] & 0x0F0F0F0Fu) | (((h[l] >> (2 * p)) & 0x01010101u) << 4));
        const int hi = (int) (((U.q[l] >> 4) & 0x0F0F0F0Fu) | (((h[l] >> (2 * p + 1)) & 0x01010101u) << 4));
        aux[l] = U.sc_a * dot4(lo, xa[l], 0) + U.sc_b * dot4(hi, xb[l], 0);
    }
    mins = U.m_a * ((int) xbs[4 * p] + (int) xbs[4 * p + 1]) + U.m_b * ((int) xbs[4 * p + 2] + (int) xbs[4 * p + 3]);
}

// A Q6_K unit u = (super-block u/4, p = u%4): elements 64p .. 64p + 63, the 32-runs A (group
// g = 2 (p & 1) of half p >> 1) and B (group g + 1). Their codes: nibble p & 1 of ql bytes 0..31
// (A) and 32..63 (B) of the half (ql[0..3], 64 bytes), with bits 2g, 2g + 1 (A) and 2g + 2, 2g + 3
// (B) of the half's 32 qh bytes (h0, h1) as bits 4-5; minus 32 as signed bytes. Each run's first
// and second 16 elements have their own int8 scale (sc4: the unit's four scales, bytes 4p .. 4p +
// 3 of the block's). Grouped by l, a dword holds elements l, l + 8 (first 16) and l + 16, l + 24
// (second 16), so one v_dot4 per scale takes the dword with the other two bytes masked off. No
// mins. aux[l] is the integer ggml's generic q6_K x q8_K kernel accumulates.
__device__ __forceinline__ void q6k_unit_dot(const uint4 (&ql)[4], uint4 h0, uint4 h1, uint32_t sc4, int p,
                                             const int * xa, const int * xb, int aux[8]) {
    uint32_t a[8] = { ql[0].x, ql[0].y, ql[0].z, ql[0].w, ql[1].x, ql[1].y, ql[1].z, ql[1].w };
    uint32_t b[8] = { ql[2].x, ql[2].y, ql[2].z, ql[2].w, ql[3].x, ql[3].y, ql[3].z, ql[3].w };
    uint32_t h[8] = { h0.x, h0.y, h0.z, h0.w, h1.x, h1.y, h1.z, h1.w };
    q4k_group_by_l(a);
    q4k_group_by_l(b);
    q4k_group_by_l(h);
    const int nib = 4 * (p & 1), ga = 4 * (p & 1);
    const int s0 = (int) (int8_t) (sc4 & 0xff), s1 = (int) (int8_t) ((sc4 >> 8) & 0xff);
    const int s2 = (int) (int8_t) ((sc4 >> 16) & 0xff), s3 = (int) (int8_t) (sc4 >> 24);
#pragma unroll
    for (int l = 0; l < 8; l++) {
        const uint32_t qa = ((a[l] >> nib) & 0x0F0F0F0Fu) | (((h[l] >> ga) & 0x03030303u) << 4);
        const uint32_t qb = ((b[l] >> nib) & 0x0F0F0F0Fu) | (((h[l] >> (ga + 2)) & 0x03030303u) << 4);
        // q - 32 per byte without borrows: bytes 0x80..0xBF minus 0x20 stay positive, then flip bit 7
        const int wa = (int) (((qa | 0x80808080u) - 0x20202020u) ^ 0x80808080u);
        const int wb = (int) (((qb | 0x80808080u) - 0x20202020u) ^ 0x80808080u);
        aux[l] = s0 * dot4(wa & 0x0000FFFF, xa[l], 0) + s1 * dot4(wa & (int) 0xFFFF0000u, xa[l], 0) +
                 s2 * dot4(wb & 0x0000FFFF, xb[l], 0) + s3 * dot4(wb & (int) 0xFFFF0000u, xb[l], 0);
    }
}

// floats between the term rows of two Q4_0/Q8_0 chains: 4 more than the terms, so the 16-byte
// reads of consecutive chains (one lane each) start on different LDS banks
__host__ __device__ constexpr int gemv_term_stride(int nb) { return nb + 4; }

// The float sum of a chain's block terms in block order (ggml-cpu's sumf += term), 32 terms per
// step with the next step's LDS reads in flight during the adds.
__device__ __forceinline__ float ordered_sum(const float * terms, int nb) {
    float acc = 0.0f;
    if ((nb & 31) == 0) {
        const float4 * t4 = (const float4 *) terms;
        const int n32 = nb / 32;
        float4 cur[8], nxt[8];
#pragma unroll
        for (int k = 0; k < 8; k++) cur[k] = t4[k];
        for (int b = 0; b < n32; b++) {
            if (b + 1 < n32) {
#pragma unroll
                for (int k = 0; k < 8; k++) nxt[k] = t4[(b + 1) * 8 + k];
            }
#pragma unroll
            for (int k = 0; k < 8; k++) acc = acc + cur[k].x + cur[k].y + cur[k].z + cur[k].w;
#pragma unroll
            for (int k = 0; k < 8; k++) cur[k] = nxt[k];
        }
    } else if ((nb & 3) == 0) {
        const float4 * t4 = (const float4 *) terms;
        for (int b4 = 0; b4 < nb / 4; b4++) {
            const float4 v = t4[b4];
            acc = acc + v.x + v.y + v.z + v.w;
        }
    } else {
        for (int b = 0; b < nb; b++) acc = acc + terms[b];
    }
    return acc;
}

