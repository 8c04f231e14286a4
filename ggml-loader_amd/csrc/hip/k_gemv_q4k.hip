// k_gemv_q4k.hip — single-column GEMV for Q4_K weights (the batch-1 decode path of Q4_K models).
//
// y[c][r] = W[r] . x[c] (+ add[c][r]) in ggml-cpu's arithmetic: x quantized to Q8_K
// (quantize_row_q8_K), per 256-element super-block the integers of the generic q4_K x q8_K kernel
// (aux32[l] = the sum over the super-block's elements e with e % 8 == l of scale * q4 * q8, and
// the mins sum over the 16-element bsums), then its float chains in super-block order:
// sums[l] += d * aux32[l], sumf -= dmin * summs, and sumf + sums[0] + ... + sums[7] at the end.
//
// Taken for SwiGLU pairs and rows up to 2048 elements (see gemv_q4k_supported); the multi-unit
// kernel of k_gemv.hip runs the rest.
//
// Mapping: a unit is 64 weights (sub-block pair p of a super-block): its 16-byte block header and
// the pair's 32 quant bytes. LPR lanes per row (a multiple of 4); lane l takes units l, l + LPR,
// ... (ITS of them), so the 4 units of a super-block sit on 4 consecutive lanes, whose integers
// are added by DPP (exact). Every weight load of a lane is issued at entry. After each slice of
// LPR units, each quad's 9 float terms go to LDS and lanes of the row advance the 9 chains (one
// chain per lane) over the slice's super-blocks in order, while later slices are in flight.
//
// The activation is staged in LDS as Q8_K with each 32-element sub-block's bytes grouped by l
// (byte k of word l is element l + 8k), so one dot4 covers 4 elements of one accumulator:
//   PRO 0  already quantized (xq / xd / xbs in ggml's layout): copied and regrouped
//   PRO 1  rms_norm(x) * w computed here (ggml's rms_norm -> mul -> quantize_row_q8_K roundings):
//          float4 chunks of x, CPT per thread; a wave quantizes one 256-element super-block (the
//          first value of largest magnitude by a DPP max and a ballot, bsums by DPP)
//   PRO 2  x quantized as is (the quantization ggml-cpu applies inside mul_mat)
#include "kernels.h"
#include "gemv_ops.h"

#include "ggml.h"

namespace {

constexpr int Q4K_MAX_WAVES = 16;
constexpr int Q4K_BS_PER = 4;      // 16-element sums of a pre-quantized column per thread (K / 16 <= 4 threads)

__host__ __device__ constexpr int q4k_term_stride(int lpr) { return (lpr / 4) * 9 + 1; }

// dynamic LDS: [terms: rows_pb * NCH][TS] floats | [fin: rows_pb * NCH * 9] floats |
// [xq: K] | [xd: K/256] | [xbs: K/16 int16] | [red: 16 doubles]
struct q4k_lds {
    float *   terms;
    float *   fin;
    int8_t *  xq;
    float *   xd;
    int16_t * xbs;
    double *  red;
};

__host__ __device__ inline size_t q4k_lds_bytes(int lpr, int rows_pb, int nch, int K) {
    size_t b = (size_t) rows_pb * nch * (q4k_term_stride(lpr) + 9) * 4;
    b = (b + 15) & ~(size_t) 15;
    b += (size_t) K + (size_t) (K / 256) * 4 + (size_t) (K / 16) * 2;
    b = (b + 15) & ~(size_t) 15;
    b += Q4K_MAX_WAVES * 8;
    return b;
}

__device__ __forceinline__ q4k_lds q4k_layout(uint8_t * smem, int lpr, int rows_pb, int nch, int K) {
    q4k_lds s;
    s.terms = (float *) smem;
    s.fin = s.terms + rows_pb * nch * q4k_term_stride(lpr);
    size_t off = ((size_t) rows_pb * nch * (q4k_term_stride(lpr) + 9) * 4 + 15) & ~(size_t) 15;
    s.xq = (int8_t *) (smem + off);
    off += (size_t) K;
    s.xd = (float *) (smem + off);
    off += (size_t) (K / 256) * 4;
    s.xbs = (int16_t *) (smem + off);
    off += (size_t) (K / 16) * 2;
    off = (off + 15) & ~(size_t) 15;
    s.red = (double *) (smem + off);
    return s;
}

// the maximum over the wave (uniform)
__device__ __forceinline__ float wave_max_dpp(float v) {
    v = fmaxf(v, dpp_f<0xB1>(v));
    v = fmaxf(v, dpp_f<0x4E>(v));
    v = fmaxf(v, dpp_f<0x141>(v));
    v = fmaxf(v, dpp_f<0x140>(v));
    return fmaxf(fmaxf(lane_f(v, 0), lane_f(v, 16)), fmaxf(lane_f(v, 32), lane_f(v, 48)));
}

// Q8_K quantization of one super-block held by a whole wave, 4 consecutive values per lane
// (element 4 * lane + e), into the grouped LDS layout: quantize_row_q8_K_ref's iscale = -127 / max
// (max = the first value of largest magnitude), q = min(127, nearest_int(iscale * v)), d = 1 /
// iscale, bsums over 16 elements.
__device__ __forceinline__ void q8k_quant_wave(float v0, float v1, float v2, float v3, int sb, const q4k_lds & s) {
    const int lane = threadIdx.x % WAVE;
    float ax = fabsf(v0), val = v0;
    if (fabsf(v1) > ax) { ax = fabsf(v1); val = v1; }
    if (fabsf(v2) > ax) { ax = fabsf(v2); val = v2; }
    if (fabsf(v3) > ax) { ax = fabsf(v3); val = v3; }
    const float amax = wave_max_dpp(ax);
    // the first lane holding the largest magnitude (its own first such value is the block's first)
    const uint64_t hit = __ballot(ax == amax);
    const int wl = __ffsll((unsigned long long) hit) - 1;
    const float mx = lane_f(val, wl);
    const float iscale = amax != 0.0f ? -127.f / mx : 0.0f;
    int q[4];
    const float v[4] = { v0, v1, v2, v3 };
#pragma unroll
    for (int e = 0; e < 4; e++) {
        const int qv = amax != 0.0f ? round_half_even(iscale * v[e]) : 0;
        q[e] = qv < 127 ? qv : 127;
    }
    int bs = q[0] + q[1] + q[2] + q[3];
    bs += dpp_i<0xB1>(bs);
    bs += dpp_i<0x4E>(bs);
    // element i = 4 * lane + e of the super-block: sub-block i / 32, accumulator (i % 32) % 8,
    // byte (i % 32) / 8 of that accumulator's word
    int8_t * sub = s.xq + sb * 256 + (lane / 8) * 32;
    const int k = (lane % 8) / 2, l0 = 4 * (lane % 2);
#pragma unroll
    for (int e = 0; e < 4; e++) sub[(l0 + e) * 4 + k] = (int8_t) q[e];
    if ((lane % 4) == 0) s.xbs[sb * 16 + lane / 4] = (int16_t) bs;
    if (lane == 0) s.xd[sb] = amax != 0.0f ? 1 / iscale : 0.0f;
}

template <int LPR, int ITS, bool SWIGLU, int PRO, int CPT, int MAXT, bool ROUTE = false>
__global__ __launch_bounds__(MAXT) void gemv_q4k_kernel(const gemv_kargs a) {
    prefetch_kernargs<sizeof(gemv_kargs)>();
    extern __shared__ __align__(16) uint8_t smem[];
    constexpr int RPW = WAVE / LPR;
    constexpr int NCH = SWIGLU ? 2 : 1;
    constexpr int QPR = LPR / 4;                        // super-blocks per slice
    constexpr int TS = q4k_term_stride(LPR);
    constexpr int CPL = (9 * NCH + LPR - 1) / LPR;      // chains per lane
    const gemv_launch & L = a.L;
    const int t = threadIdx.x, nt = blockDim.x;
    const int lane = t % WAVE, wave = t / WAVE;
    const int g = lane / LPR, l = lane % LPR;
    const int rows_pb = a.rows_per_block;
    const int rib = wave * RPW + g;
    const int row = blockIdx.x * rows_pb + rib;
    const int col = blockIdx.y;
    const int K = L.K, nsb = K / 256, units = K / 64, nc = K / 4;
    const int mi = SWIGLU ? 0 : find_mat(a, blockIdx.x * rows_pb);   // uniform: the workgroup's matrix
    const int lrow = SWIGLU ? row : row - a.row_begin[mi];
    const bool valid = row < a.total_rows && lrow < L.m[mi].n_rows;
    const q4k_lds s = q4k_layout(smem, LPR, rows_pb, NCH, K);

    // mul_mat_id: the expert of this column and its activation column
    int xcol = col;
    int64_t erow = 0;
    if constexpr (ROUTE) {
        // one token, column = slot: the routing runs here, in every workgroup, before any load
        // that needs the expert (256 threads, at most 256 experts)
        __shared__ float r_p[256];
        __shared__ int r_ids[MOE_ROUTE_MAX_K];
        __shared__ int r_cnt[256];
        __shared__ __align__(16) uint64_t r_key[256];   // read as 16-byte pairs
        __shared__ float r_red[4];
        __shared__ double r_sum[4];
        const int E = L.n_experts;
        const float lg = L.route_logits[min(t, E - 1)];
        moe_route_256(t < E ? lg * L.route_scale : -INFINITY, E, L.n_slots, r_p, r_ids, r_cnt, r_key, r_red, r_sum);
        // the ids and weights the down projection and the weighted slot sum read (later launches)
        if (blockIdx.x == 0 && col == 0 && t == 0) moe_route_store(r_p, r_ids, L.n_slots, (int32_t *) L.ids, L.route_w);
        xcol = col % L.x_cols;
        erow = (int64_t) r_ids[col] * L.expert_rows;
    } else if (L.ids) {
        const int tk = col / L.n_slots, sl = col % L.n_slots;
        xcol = tk * L.x_cols + sl % L.x_cols;
        const int e = min(max(L.ids[(int64_t) tk * L.ids_stride + sl], 0), L.n_experts - 1);
        erow = (int64_t) e * L.expert_rows;
    }

    // ---- activation loads (before the weights): CPT float4 chunks of x and the norm weight, or
    // the pre-quantized column's 32-byte sub-blocks (two per thread at most) ----
    float4 xv[CPT], wv[CPT];
    int4 pa[2], pb[2];
    int16_t bsv[Q4K_BS_PER];
    float xdv = 0.0f;
    if constexpr (PRO != 0) {
        const float4 * x4 = (const float4 *) (L.norm.x + (int64_t) xcol * L.norm.x_stride);
        const float4 * w4 = (const float4 *) (PRO == 1 && L.norm.w ? L.norm.w : L.norm.x);
#pragma unroll
        for (int k = 0; k < CPT; k++) {
            const int c = min(t + k * nt, nc - 1);
            xv[k] = x4[c];
            if (PRO == 1) wv[k] = w4[c];
        }
    } else {
        const int8_t * xq = L.xq + (int64_t) xcol * K;
#pragma unroll
        for (int k = 0; k < 2; k++) {
            const int sub = min(t + k * nt, K / 32 - 1);
            pa[k] = *(const int4 *) (xq + sub * 32);
            pb[k] = *(const int4 *) (xq + sub * 32 + 16);
        }
        // the column's 16-element sums and super-block scales too (unconditional, at clamped
        // indices): loaded in a loop after the weights, each would wait for every weight load
        const int16_t * gbs = L.xbs + (int64_t) xcol * (K / 16);
#pragma unroll
        for (int k = 0; k < Q4K_BS_PER; k++) bsv[k] = gbs[min(t + k * nt, K / 16 - 1)];
        xdv = L.xd[(int64_t) xcol * nsb + min(t, nsb - 1)];
    }

    // ---- every weight load of this lane (row and unit clamped into the matrix), issued after the
    // activation's (the empty asm keeps the compiler from moving any of those behind them:
    // waiting for one would then wait for the weights) ----
    asm volatile("" ::: "memory");
    uint4 hd[NCH][ITS], qa[NCH][ITS], qb[NCH][ITS];
    const int64_t row_bytes = (int64_t) nsb * Q4_K_BYTES;
#pragma unroll
    for (int ch = 0; ch < NCH; ch++) {
        const gemv_mat & wm = L.m[SWIGLU ? ch : mi];
        const uint8_t * wrow = wm.w + (erow + min(lrow, wm.n_rows - 1)) * row_bytes;
#pragma unroll
        for (int it = 0; it < ITS; it++) {
            const int u = min(l + it * LPR, units - 1);
            const uint8_t * blk = wrow + (int64_t) (u >> 2) * Q4_K_BYTES;
            hd[ch][it] = *(const uint4 *) blk;
            qa[ch][it] = *(const uint4 *) (blk + 16 + 32 * (u & 3));
            qb[ch][it] = *(const uint4 *) (blk + 32 + 32 * (u & 3));
        }
    }

    // ---- the activation into LDS ----
    if constexpr (PRO == 0) {
        const int nsub = K / 32;
#pragma unroll
        for (int k = 0; k < Q4K_BS_PER; k++) {
            if (t + k * nt < K / 16) s.xbs[t + k * nt] = bsv[k];
        }
        if (t < nsb) s.xd[t] = xdv;
#pragma unroll
        for (int k = 0; k < 2; k++) {
            const int sub = t + k * nt;
            uint32_t w8[8] = { (uint32_t) pa[k].x, (uint32_t) pa[k].y, (uint32_t) pa[k].z, (uint32_t) pa[k].w,
                               (uint32_t) pb[k].x, (uint32_t) pb[k].y, (uint32_t) pb[k].z, (uint32_t) pb[k].w };
            q4k_group_by_l(w8);
            if (sub < nsub) {
                uint4 * d = (uint4 *) (s.xq + sub * 32);
                d[0] = make_uint4(w8[0], w8[1], w8[2], w8[3]);
                d[1] = make_uint4(w8[4], w8[5], w8[6], w8[7]);
            }
        }
    } else {
        float scale = 1.0f;
        if constexpr (PRO == 1) {
            double ss = 0.0;
#pragma unroll
            for (int k = 0; k < CPT; k++) {
                if (t + k * nt < nc) {
                    ss += (double) (xv[k].x * xv[k].x);
                    ss += (double) (xv[k].y * xv[k].y);
                    ss += (double) (xv[k].z * xv[k].z);
                    ss += (double) (xv[k].w * xv[k].w);
                }
            }
            ss = wave_sum_d_dpp(ss);
            if (lane == 0) s.red[wave] = ss;
            __syncthreads();
            double tot = 0.0;
            for (int w = 0; w < nt / WAVE; w++) tot += s.red[w];
            const float mean = (float) (tot / (double) K);
            scale = 1.0f / sqrtf(mean + L.norm.eps);
        }
#pragma unroll
        for (int k = 0; k < CPT; k++) {
            // chunk c = t + k * nt: elements 4c .. 4c + 3; a wave holds one whole super-block
            // (nt and nc are multiples of 64), so the test below is uniform across the wave
            if (k * nt + wave * WAVE < nc) {
                float v0 = xv[k].x, v1 = xv[k].y, v2 = xv[k].z, v3 = xv[k].w;
                if (PRO == 1) {
                    v0 = v0 * scale; v1 = v1 * scale; v2 = v2 * scale; v3 = v3 * scale;
                    if (L.norm.w) { v0 = v0 * wv[k].x; v1 = v1 * wv[k].y; v2 = v2 * wv[k].z; v3 = v3 * wv[k].w; }
                }
                q8k_quant_wave(v0, v1, v2, v3, (k * nt + wave * WAVE) / 64, s);
            }
        }
    }
    __syncthreads();

    // ---- dots and the ordered chains, one slice at a time ----
    float * tr = s.terms + rib * NCH * TS;
    float acc[CPL];
#pragma unroll
    for (int j = 0; j < CPL; j++) acc[j] = 0.0f;
#pragma unroll
    for (int it = 0; it < ITS; it++) {
        const int u = l + it * LPR;
        const int sb = min(u, units - 1) >> 2, p = u & 3;
        const bool has = u < units;
        const int * xs = (const int *) (s.xq + sb * 256 + 64 * p);
        int xa[8], xb[8];
#pragma unroll
        for (int k = 0; k < 8; k++) { xa[k] = xs[k]; xb[k] = xs[8 + k]; }
        const float yd = s.xd[sb];
#pragma unroll
        for (int ch = 0; ch < NCH; ch++) {
            int aux[8], mins = 0;
            q4k_unit_dot(q4k_prepare(hd[ch][it], qa[ch][it], qb[ch][it], p), p, xa, xb, s.xbs + sb * 16, aux, mins);
            if (!has) {
#pragma unroll
                for (int k = 0; k < 8; k++) aux[k] = 0;
                mins = 0;
            }
            // the super-block's 4 units sit on lanes 4q .. 4q + 3: their integers added (exact)
#pragma unroll
            for (int k = 0; k < 8; k++) {
                aux[k] += dpp_i<0xB1>(aux[k]);
                aux[k] += dpp_i<0x4E>(aux[k]);
            }
            mins += dpp_i<0xB1>(mins);
            mins += dpp_i<0x4E>(mins);
            const uint32_t dd = hd[ch][it].x;
            const float d = __half2float(__ushort_as_half((unsigned short) (dd & 0xffff))) * yd;
            const float dmin = __half2float(__ushort_as_half((unsigned short) (dd >> 16))) * yd;
            // lane p of the quad stores the terms of accumulators 2p, 2p + 1 (and p = 0 the mins term)
            float t0 = 0.0f, t1 = 0.0f;
#pragma unroll
            for (int k = 0; k < 8; k++) {
                if (k == 2 * p) t0 = d * (float) aux[k];
                if (k == 2 * p + 1) t1 = d * (float) aux[k];
            }
            float * tq = tr + ch * TS + (l / 4) * 9;
            tq[2 * p] = t0;
            tq[2 * p + 1] = t1;
            if (p == 0) tq[8] = dmin * (float) mins;
        }
        // the slice's terms were written by lanes of this wave: a wave-level ordering point
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        const int nq = min(QPR, nsb - it * QPR);     // super-blocks of this slice
#pragma unroll
        for (int j = 0; j < CPL; j++) {
            const int c = l + j * LPR;                 // chain c: accumulator c % 9 of matrix c / 9
            if (c < 9 * NCH) {
                const float * tc = tr + (c / 9) * TS + (c % 9);
                if (c % 9 < 8) {
                    for (int q = 0; q < nq; q++) acc[j] = acc[j] + tc[q * 9];
                } else {
                    for (int q = 0; q < nq; q++) acc[j] = acc[j] - tc[q * 9];
                }
            }
        }
        if (it + 1 < ITS) {
            // the next slice overwrites the terms: every lane's reads of this one come first
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
            __builtin_amdgcn_wave_barrier();
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        }
    }
    // sumf (the mins chain) + sums[0] + ... + sums[7], on the row's first lane
    float * fr = s.fin + rib * NCH * 9;
#pragma unroll
    for (int j = 0; j < CPL; j++) {
        const int c = l + j * LPR;
        if (c < 9 * NCH) fr[c] = acc[j];
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    float res[NCH];
#pragma unroll
    for (int ch = 0; ch < NCH; ch++) {
        float f = fr[ch * 9 + 8];
#pragma unroll
        for (int k = 0; k < 8; k++) f = f + fr[ch * 9 + k];
        res[ch] = f;
    }
    if (!valid || l != 0) return;
    if constexpr (SWIGLU) {
        // act = silu(gate) * up (two roundings, as the silu and mul ops)
        const float gv = res[0], uv = res[1];
        const float sl = gv / (1.0f + exp_cr(-gv));
        L.m[0].y[(int64_t) col * L.m[0].y_stride + row] = sl * uv;
    } else {
        const gemv_mat & m = L.m[mi];
        float v = res[0];
        if (m.add) v = v + m.add[(int64_t) col * m.add_stride + lrow];
        m.y[(int64_t) col * m.y_stride + lrow] = v;
    }
}

// ---- host: shapes ----

struct q4k_shape {
    int lpr, its, waves, cpt;
};

template <int LPR, int ITS, bool SWIGLU, int PRO, int CPT>
void q4k_launch_t(const gemv_kargs & ka, int waves, size_t lds, hipStream_t st) {
    const dim3 grid((ka.total_rows + ka.rows_per_block - 1) / ka.rows_per_block, ka.L.ncols);
    const dim3 block(waves * WAVE);
    if (waves <= 4) return launch((gemv_q4k_kernel<LPR, ITS, SWIGLU, PRO, CPT, 256>), grid, block, lds, st, ka);
    if (waves <= 8) return launch((gemv_q4k_kernel<LPR, ITS, SWIGLU, PRO, CPT, 512>), grid, block, lds, st, ka);
    launch((gemv_q4k_kernel<LPR, ITS, SWIGLU, PRO, CPT, 1024>), grid, block, lds, st, ka);
}

template <int LPR, int ITS, bool SWIGLU>
void q4k_launch_its(const gemv_kargs & ka, int pro, int waves, int cpt, size_t lds, hipStream_t st) {
    if constexpr (SWIGLU) {
        if (ka.L.route_logits) {
            const dim3 grid((ka.total_rows + ka.rows_per_block - 1) / ka.rows_per_block, ka.L.ncols);
            if (waves != 4 || (pro != 0 && (pro != 2 || cpt > 2))) HIP_ABORT("gemv q4_K: routing inside the launch needs 256 threads and an unnormalized column");
            if (pro == 0) return launch((gemv_q4k_kernel<LPR, ITS, true, 0, 1, 256, true>), grid, dim3(256), lds, st, ka);
            return launch((gemv_q4k_kernel<LPR, ITS, true, 2, 2, 256, true>), grid, dim3(256), lds, st, ka);
        }
    }
    if (pro == 0) return q4k_launch_t<LPR, ITS, SWIGLU, 0, 1>(ka, waves, lds, st);
    if (pro == 1) {
        if (cpt <= 2) return q4k_launch_t<LPR, ITS, SWIGLU, 1, 2>(ka, waves, lds, st);
        return q4k_launch_t<LPR, ITS, SWIGLU, 1, 3>(ka, waves, lds, st);
    }
    if (cpt <= 2) return q4k_launch_t<LPR, ITS, SWIGLU, 2, 2>(ka, waves, lds, st);
    q4k_launch_t<LPR, ITS, SWIGLU, 2, 3>(ka, waves, lds, st);
}

template <bool SWIGLU>
void q4k_dispatch(const gemv_kargs & ka, const q4k_shape & sh, int pro, size_t lds, hipStream_t st) {
#define Q4K_CASE(LPR_, ITS_) \
    if (sh.lpr == LPR_ && sh.its == ITS_) return q4k_launch_its<LPR_, ITS_, SWIGLU>(ka, pro, sh.waves, sh.cpt, lds, st);
    Q4K_CASE(16, 1) Q4K_CASE(16, 2) Q4K_CASE(16, 3)
    Q4K_CASE(32, 2) Q4K_CASE(32, 3)
    if constexpr (!SWIGLU) {
        Q4K_CASE(32, 4) Q4K_CASE(32, 5)
        Q4K_CASE(64, 3) Q4K_CASE(64, 4) Q4K_CASE(64, 5) Q4K_CASE(64, 6)
    }
#undef Q4K_CASE
    HIP_ABORT("gemv q4_K: no kernel for %d lanes per row x %d units", sh.lpr, sh.its);
}

// lanes per row and units per lane: 16 lanes for rows of up to 48 units (3 per lane), 32 for up
// to 160 units (96 with SwiGLU: both matrices' weights stay in registers), 64 beyond (384 units)
bool q4k_shape_of(int units, bool swiglu, q4k_shape & sh) {
    if (units <= 48) { sh.lpr = 16; sh.its = (units + 15) / 16; }
    else if (units <= (swiglu ? 96 : 160)) { sh.lpr = 32; sh.its = (units + 31) / 32; }
    else if (!swiglu && units <= 384) { sh.lpr = 64; sh.its = (units + 63) / 64; }
    else return false;
    return true;
}

// threads for the prologue's float4 chunks, at most 2 (3 past 512 threads) per thread
bool q4k_prologue_of(int pro, int K, q4k_shape & sh) {
    sh.waves = 4;
    sh.cpt = 1;
    if (pro == 0) return true;
    const int nc = K / 4;
    sh.waves = std::max(4, (nc + 2 * WAVE - 1) / (2 * WAVE));
    if (sh.waves > Q4K_MAX_WAVES) sh.waves = Q4K_MAX_WAVES;
    sh.cpt = (nc + sh.waves * WAVE - 1) / (sh.waves * WAVE);
    return sh.cpt <= 3;
}

}  // namespace

bool gemv_q4k_enabled() {
    static const bool on = !getenv("GGML_HIP_NO_Q4K_GEMV");
    return on;
}

bool gemv_q4k_supported(const gemv_launch & L) {
    if (L.type != GGML_TYPE_Q4_K || L.K % 256 || L.out_q.qs || L.norm.f64) return false;
    // taken where it measured faster than the multi-unit kernel of k_gemv.hip (C3: gate/up + SwiGLU
    // 15.9 against 17.6 us; C5: QKV 7.7 against 8.8, expert down 6.3 against 8.5): SwiGLU pairs of
    // a plain GEMV and rows of at most 2048 elements. Longer single rows (C3's QKV, O, down and the
    // LM head) measured slower here: their prologue needs workgroups of many rows, hence few of them.
    if (!(L.swiglu && !L.ids) && L.K > 2048) return false;
    if (L.norm.x && L.norm.x_stride % 4) return false;
    q4k_shape sh{};
    if (!q4k_shape_of(L.K / 64, L.swiglu, sh)) return false;
    const int pro = !L.norm.x ? 0 : L.norm.rms ? 1 : 2;
    if (!q4k_prologue_of(pro, L.K, sh)) return false;
    if (pro == 0 && L.K / 32 > 2 * sh.waves * WAVE) return false;
    // the routing inside the launch: one token's slots, 256 threads, at most 256 experts, the
    // column pre-quantized or quantized as is
    if (L.route_logits && !(L.swiglu && L.ids && (pro == 0 || (pro == 2 && sh.cpt <= 2)) && sh.waves == 4 &&
                            L.ncols == L.n_slots && L.x_cols >= 1 &&
                            L.n_experts >= 1 && L.n_experts <= 256 && L.n_slots >= 1 && L.n_slots <= MOE_ROUTE_MAX_K &&
                            L.n_slots <= L.n_experts && L.route_w)) return false;
    const int rows_pb = sh.waves * (WAVE / sh.lpr);
    return q4k_lds_bytes(sh.lpr, rows_pb, L.swiglu ? 2 : 1, L.K) <= 64 * 1024;
}

void launch_gemv_q4k(const gemv_launch & L, hipStream_t st) {
    if (!gemv_q4k_supported(L)) HIP_ABORT("gemv q4_K: unsupported launch (K=%d)", L.K);
    gemv_kargs ka;
    ka.L = L;
    const int pro = !L.norm.x ? 0 : L.norm.rms ? 1 : 2;
    q4k_shape sh{};
    q4k_shape_of(L.K / 64, L.swiglu, sh);
    q4k_prologue_of(pro, L.K, sh);
    ka.rows_per_block = sh.waves * (WAVE / sh.lpr);
    const int nthr = sh.waves * WAVE;
    if (pro == 0 && (L.K / 32 > 2 * nthr || L.K / 16 > Q4K_BS_PER * nthr || L.K / 256 > nthr))
        HIP_ABORT("gemv q4_K: a pre-quantized column of K=%d needs more than %d threads", L.K, nthr);
    if (L.swiglu) {
        if (L.n_mats != 2 || L.m[0].n_rows != L.m[1].n_rows) HIP_ABORT("gemv: swiglu needs two equal matrices");
        for (int i = 0; i <= GEMV_MAX_MATS; i++) ka.row_begin[i] = 0;
        ka.total_rows = L.m[0].n_rows;
    } else {
        // every matrix starts on a workgroup boundary
        int r = 0;
        for (int i = 0; i < L.n_mats; i++) {
            ka.row_begin[i] = r;
            r += (L.m[i].n_rows + ka.rows_per_block - 1) / ka.rows_per_block * ka.rows_per_block;
        }
        for (int i = L.n_mats; i <= GEMV_MAX_MATS; i++) ka.row_begin[i] = r;
        ka.total_rows = r;
    }
    const size_t lds = q4k_lds_bytes(sh.lpr, ka.rows_per_block, L.swiglu ? 2 : 1, L.K);
    if (L.swiglu) q4k_dispatch<true>(ka, sh, pro, lds, st);
    else q4k_dispatch<false>(ka, sh, pro, lds, st);
}
