// k_gemv.hip — quantized matrix-vector kernels (the decode hot path) and their helpers:
// weight plane repacking, activation quantization (ggml Q8_0 / Q8_K semantics) and the
// Q4_0 / Q8_0 / Q4_K integer-dot GEMVs.
//
// GEMV mapping: a wavefront owns 64/LPR rows; LPR lanes split a row's blocks (lane l takes blocks
// l, l+LPR, ...), so one load instruction moves LPR consecutive 16-byte block payloads per row.
// Each lane decodes its blocks in registers, does the integer dot with v_dot4_i32_i8 against the
// quantized activation, scales by the block scales, and the LPR partials are combined with
// cross-lane shuffles. Rows of up to four matrices (e.g. Q, K and V, or gate and up) are
// concatenated in one grid so one launch streams all of them.
#include "kernels.h"

#include "ggml.h"

// ---------------------------------------------------------------------------------------------
// weight plane repack

__global__ void repack_q_kernel(int qs_bytes, int blk_bytes, const uint8_t * __restrict__ raw,
                                uint8_t * __restrict__ qs, __half * __restrict__ d, int64_t nblocks, int64_t first) {
    const int64_t b = (int64_t) blockIdx.x * blockDim.x + threadIdx.x;
    if (b >= nblocks) return;
    const uint8_t * src = raw + b * blk_bytes;
    uint8_t * dq = qs + (first + b) * qs_bytes;
    d[first + b] = __ushort_as_half((unsigned short) (src[0] | (src[1] << 8)));
    for (int i = 0; i < qs_bytes; i++) dq[i] = src[2 + i];
}

__global__ void unpack_q_kernel(int qs_bytes, int blk_bytes, uint8_t * __restrict__ raw,
                                const uint8_t * __restrict__ qs, const __half * __restrict__ d, int64_t nblocks, int64_t first) {
    const int64_t b = (int64_t) blockIdx.x * blockDim.x + threadIdx.x;
    if (b >= nblocks) return;
    uint8_t * dst = raw + b * blk_bytes;
    const unsigned short h = __half_as_ushort(d[first + b]);
    dst[0] = (uint8_t) (h & 0xff);
    dst[1] = (uint8_t) (h >> 8);
    const uint8_t * sq = qs + (first + b) * qs_bytes;
    for (int i = 0; i < qs_bytes; i++) dst[2 + i] = sq[i];
}

static void qs_geometry(int type, int & qs_bytes, int & blk_bytes) {
    if (type == GGML_TYPE_Q4_0) { qs_bytes = Q4_0_QS; blk_bytes = 18; return; }
    if (type == GGML_TYPE_Q8_0) { qs_bytes = Q8_0_QS; blk_bytes = 34; return; }
    HIP_ABORT("repack: unsupported type %d", type);
}

void launch_repack_q(int type, const uint8_t * raw, uint8_t * qs_plane, __half * d_plane,
                     int64_t nblocks, int64_t first_block, hipStream_t st) {
    if (nblocks <= 0) return;
    int qsb, bb;
    qs_geometry(type, qsb, bb);
    const int threads = 256;
    const int64_t grid = (nblocks + threads - 1) / threads;
    hipLaunchKernelGGL(repack_q_kernel, dim3((unsigned) grid), dim3(threads), 0, st, qsb, bb, raw, qs_plane, d_plane, nblocks, first_block);
    HIP_CHECK(hipGetLastError());
}

void launch_unpack_q(int type, uint8_t * raw, const uint8_t * qs_plane, const __half * d_plane,
                     int64_t nblocks, int64_t first_block, hipStream_t st) {
    if (nblocks <= 0) return;
    int qsb, bb;
    qs_geometry(type, qsb, bb);
    const int threads = 256;
    const int64_t grid = (nblocks + threads - 1) / threads;
    hipLaunchKernelGGL(unpack_q_kernel, dim3((unsigned) grid), dim3(threads), 0, st, qsb, bb, raw, qs_plane, d_plane, nblocks, first_block);
    HIP_CHECK(hipGetLastError());
}

// ---------------------------------------------------------------------------------------------
// activation quantization

// Q8_0 (ggml quantize_row_q8_0_ref): d = amax/127, q = roundf(x * (d ? 1/d : 0)), d stored as
// fp16. One 32-lane half-wave per block. grid: (ceil(nblk/8), ncols), 256 threads.
__global__ void quantize_q8_kernel(const float * __restrict__ x, int64_t x_col_stride, int64_t K,
                                   int8_t * __restrict__ qs, float * __restrict__ d, int32_t * __restrict__ s) {
    const int64_t nblk = K / 32;
    const int64_t c = blockIdx.y;
    const int64_t blk = (int64_t) blockIdx.x * 8 + threadIdx.x / 32;
    const int j = threadIdx.x % 32;
    const bool ok = blk < nblk;
    const float v = ok ? x[c * x_col_stride + blk * 32 + j] : 0.0f;
    const float amax = group_max<32>(fabsf(v));
    const float dd = amax / 127;
    const float id = dd ? 1.0f / dd : 0.0f;
    const int q = (int) roundf(v * id);
    const float qsum = group_sum<32>((float) q);
    if (ok) {
        qs[c * K + blk * 32 + j] = (int8_t) q;
        if (j == 0) {
            d[c * nblk + blk] = __half2float(__float2half_rn(dd));
            s[c * nblk + blk] = (int32_t) qsum;
        }
    }
}

void launch_quantize_q8(const float * x, int64_t x_col_stride, int64_t K, int64_t ncols, q8_act out, hipStream_t st) {
    const int64_t nblk = K / 32;
    dim3 grid((unsigned) ((nblk + 7) / 8), (unsigned) ncols);
    hipLaunchKernelGGL(quantize_q8_kernel, grid, dim3(256), 0, st, x, x_col_stride, K, out.qs, out.d, out.s);
    HIP_CHECK(hipGetLastError());
}

// Q8_K (ggml quantize_row_q8_K_ref): max = the value of largest magnitude (first one on ties),
// iscale = -127/max, q = min(127, nearest_int(iscale*x)), d = 1/iscale, bsums over 16s.
// One 256-thread block per (super-block, column).
__global__ void quantize_q8k_kernel(const float * __restrict__ x, int64_t x_col_stride, int64_t K,
                                    int8_t * __restrict__ qs, float * __restrict__ d, int16_t * __restrict__ bsums) {
    __shared__ float s_ax[4];
    __shared__ int s_idx[4];
    __shared__ float s_val[4];
    __shared__ int s_q[256];
    const int64_t nsb = K / 256;
    const int64_t c = blockIdx.y;
    const int64_t sb = blockIdx.x;
    const int t = threadIdx.x;
    const float v = x[c * x_col_stride + sb * 256 + t];
    // argmax of |v| with the lowest index winning ties
    float ax = fabsf(v);
    int idx = t;
    float val = v;
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        const float ax2 = __shfl_xor(ax, o, WAVE);
        const int idx2 = __shfl_xor(idx, o, WAVE);
        const float val2 = __shfl_xor(val, o, WAVE);
        if (ax2 > ax || (ax2 == ax && idx2 < idx)) { ax = ax2; idx = idx2; val = val2; }
    }
    if ((t % 64) == 0) { s_ax[t / 64] = ax; s_idx[t / 64] = idx; s_val[t / 64] = val; }
    __syncthreads();
    float bax = s_ax[0], bval = s_val[0];
    int bidx = s_idx[0];
    for (int w = 1; w < 4; w++) {
        if (s_ax[w] > bax || (s_ax[w] == bax && s_idx[w] < bidx)) { bax = s_ax[w]; bidx = s_idx[w]; bval = s_val[w]; }
    }
    int q = 0;
    if (bax != 0.0f) {
        const float iscale = -127.f / bval;
        q = round_half_even(iscale * v);
        q = q < 127 ? q : 127;
        if (t == 0) d[c * nsb + sb] = 1 / iscale;
    } else if (t == 0) {
        d[c * nsb + sb] = 0.0f;
    }
    qs[c * K + sb * 256 + t] = (int8_t) q;
    s_q[t] = q;
    __syncthreads();
    if (t < 16) {
        int sum = 0;
        for (int i = 0; i < 16; i++) sum += s_q[t * 16 + i];
        bsums[c * (K / 16) + sb * 16 + t] = (int16_t) sum;
    }
}

void launch_quantize_q8k(const float * x, int64_t x_col_stride, int64_t K, int64_t ncols, q8k_act out, hipStream_t st) {
    dim3 grid((unsigned) (K / 256), (unsigned) ncols);
    hipLaunchKernelGGL(quantize_q8k_kernel, grid, dim3(256), 0, st, x, x_col_stride, K, out.qs, out.d, out.bsums);
    HIP_CHECK(hipGetLastError());
}

// ---------------------------------------------------------------------------------------------
// GEMV kernels

struct gemv_kargs {
    gemv_launch L;
    int total_rows;
    int row_begin[GEMV_MAX_MATS + 1];
};

__device__ __forceinline__ int find_mat(const gemv_kargs & a, int row) {
    int m = 0;
#pragma unroll
    for (int i = 1; i < GEMV_MAX_MATS; i++) if (i < a.L.n_mats && row >= a.row_begin[i]) m = i;
    return m;
}

// integer dot of one Q4_0 block payload (16 bytes of nibbles) with 32 int8 activations;
// returns sum(q * x) with q in 0..15 (the -8 offset is applied by the caller via the block sum)
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

// 6-bit scale/min j (0..7) of a Q4_K block from its 12 scale bytes held in 3 dwords
__device__ __forceinline__ void q4k_sc_m(const uint32_t s[3], int j, int & sc, int & m) {
    const uint8_t * b = (const uint8_t *) s;
    if (j < 4) {
        sc = b[j] & 63;
        m = b[j + 4] & 63;
    } else {
        sc = (b[j + 4] & 0x0F) | ((b[j - 4] >> 6) << 4);
        m = (b[j + 4] >> 4) | ((b[j] >> 6) << 4);
    }
}

// partial dot of Q4_K unit u (sub-blocks 2p, 2p+1 of super-block sb) with the Q8_K activation
__device__ __forceinline__ float q4k_unit(const uint8_t * __restrict__ wrow, int u, const int8_t * __restrict__ xq,
                                          const float * __restrict__ xd, const int16_t * __restrict__ xbs) {
    const int sb = u >> 2, p = u & 3;
    const uint8_t * blk = wrow + (int64_t) sb * Q4_K_BYTES;
    const uint4 hdr = *(const uint4 *) blk;
    const uint4 qa = *(const uint4 *) (blk + 16 + 32 * p);
    const uint4 qb = *(const uint4 *) (blk + 32 + 32 * p);
    const int8_t * xp = xq + (int64_t) sb * 256 + 64 * p;
    const int4 x0 = *(const int4 *) (xp + 0);
    const int4 x1 = *(const int4 *) (xp + 16);
    const int4 x2 = *(const int4 *) (xp + 32);
    const int4 x3 = *(const int4 *) (xp + 48);
    int lo = 0, hi = 0;
    lo = dot4((int) (qa.x & 0x0F0F0F0Fu), x0.x, lo);
    lo = dot4((int) (qa.y & 0x0F0F0F0Fu), x0.y, lo);
    lo = dot4((int) (qa.z & 0x0F0F0F0Fu), x0.z, lo);
    lo = dot4((int) (qa.w & 0x0F0F0F0Fu), x0.w, lo);
    lo = dot4((int) (qb.x & 0x0F0F0F0Fu), x1.x, lo);
    lo = dot4((int) (qb.y & 0x0F0F0F0Fu), x1.y, lo);
    lo = dot4((int) (qb.z & 0x0F0F0F0Fu), x1.z, lo);
    lo = dot4((int) (qb.w & 0x0F0F0F0Fu), x1.w, lo);
    hi = dot4((int) ((qa.x >> 4) & 0x0F0F0F0Fu), x2.x, hi);
    hi = dot4((int) ((qa.y >> 4) & 0x0F0F0F0Fu), x2.y, hi);
    hi = dot4((int) ((qa.z >> 4) & 0x0F0F0F0Fu), x2.z, hi);
    hi = dot4((int) ((qa.w >> 4) & 0x0F0F0F0Fu), x2.w, hi);
    hi = dot4((int) ((qb.x >> 4) & 0x0F0F0F0Fu), x3.x, hi);
    hi = dot4((int) ((qb.y >> 4) & 0x0F0F0F0Fu), x3.y, hi);
    hi = dot4((int) ((qb.z >> 4) & 0x0F0F0F0Fu), x3.z, hi);
    hi = dot4((int) ((qb.w >> 4) & 0x0F0F0F0Fu), x3.w, hi);
    const uint32_t sc3[3] = { hdr.y, hdr.z, hdr.w };
    int sc_a, m_a, sc_b, m_b;
    q4k_sc_m(sc3, 2 * p, sc_a, m_a);
    q4k_sc_m(sc3, 2 * p + 1, sc_b, m_b);
    const int16_t * bs = xbs + (int64_t) sb * 16 + 4 * p;
    const int msum = m_a * ((int) bs[0] + (int) bs[1]) + m_b * ((int) bs[2] + (int) bs[3]);
    const float dw = __half2float(__ushort_as_half((unsigned short) (hdr.x & 0xffff)));
    const float dmin = __half2float(__ushort_as_half((unsigned short) (hdr.x >> 16)));
    const float dx = xd[sb];
    return (dw * dx) * (float) (sc_a * lo + sc_b * hi) - (dmin * dx) * (float) msum;
}

template <int TYPE, int LPR, int NCOLS, bool SWIGLU>
__global__ __launch_bounds__(512) void gemv_kernel(const gemv_kargs a) {
    constexpr int RPW = WAVE / LPR;
    const int lane = threadIdx.x % WAVE;
    const int wave = threadIdx.x / WAVE;
    const int waves = blockDim.x / WAVE;
    const int g = lane / LPR;
    const int l = lane % LPR;
    const int row = (blockIdx.x * waves + wave) * RPW + g;
    const int col0 = blockIdx.y * NCOLS;
    const gemv_launch & L = a.L;
    const int ncols = min(NCOLS, L.ncols - col0);
    const bool valid = row < a.total_rows;
    const int mi = SWIGLU ? 0 : find_mat(a, valid ? row : 0);
    const int lrow = SWIGLU ? row : row - a.row_begin[mi];
    const int K = L.K;

    float acc[NCOLS];
    float acc2[NCOLS];
#pragma unroll
    for (int c = 0; c < NCOLS; c++) { acc[c] = 0.0f; acc2[c] = 0.0f; }

    if (valid) {
        if (TYPE == GGML_TYPE_Q4_0 || TYPE == GGML_TYPE_Q8_0) {
            constexpr int QS = TYPE == GGML_TYPE_Q4_0 ? Q4_0_QS : Q8_0_QS;
            const int nb = K / 32;
            const uint8_t * wq = L.m[mi].w + (int64_t) lrow * nb * QS;
            const __half * wd = L.m[mi].wd + (int64_t) lrow * nb;
            const uint8_t * wq2 = SWIGLU ? L.m[1].w + (int64_t) lrow * nb * QS : nullptr;
            const __half * wd2 = SWIGLU ? L.m[1].wd + (int64_t) lrow * nb : nullptr;
#pragma unroll 4
            for (int b = l; b < nb; b += LPR) {
                uint4 qa = *(const uint4 *) (wq + (int64_t) b * QS);
                uint4 qb = qa;
                if (TYPE == GGML_TYPE_Q8_0) qb = *(const uint4 *) (wq + (int64_t) b * QS + 16);
                const float dw = __half2float(wd[b]);
                uint4 ra = qa, rb = qb;
                float dw2 = 0.0f;
                if (SWIGLU) {
                    ra = *(const uint4 *) (wq2 + (int64_t) b * QS);
                    rb = ra;
                    if (TYPE == GGML_TYPE_Q8_0) rb = *(const uint4 *) (wq2 + (int64_t) b * QS + 16);
                    dw2 = __half2float(wd2[b]);
                }
#pragma unroll
                for (int c = 0; c < NCOLS; c++) {
                    if (c < ncols) {
                        const int64_t col = col0 + c;
                        const int8_t * xp = L.xq + col * K + (int64_t) b * 32;
                        const int4 xa = *(const int4 *) xp;
                        const int4 xb = *(const int4 *) (xp + 16);
                        const float dx = L.xd[col * nb + b];
                        if (TYPE == GGML_TYPE_Q4_0) {
                            const int xs8 = 8 * L.xs[col * nb + b];
                            const int sumi = dot_q4_0_block(qa, xa, xb) - xs8;
                            acc[c] += (float) sumi * dw * dx;
                            if (SWIGLU) {
                                const int sumi2 = dot_q4_0_block(ra, xa, xb) - xs8;
                                acc2[c] += (float) sumi2 * dw2 * dx;
                            }
                        } else {
                            const int sumi = dot_q8_0_block(qa, qb, xa, xb);
                            acc[c] += (float) sumi * (dw * dx);
                            if (SWIGLU) {
                                const int sumi2 = dot_q8_0_block(ra, rb, xa, xb);
                                acc2[c] += (float) sumi2 * (dw2 * dx);
                            }
                        }
                    }
                }
            }
        } else { // Q4_K
            const int units = K / 64;
            const int64_t row_bytes = (int64_t) (K / 256) * Q4_K_BYTES;
            const uint8_t * wrow = L.m[mi].w + (int64_t) lrow * row_bytes;
            const uint8_t * wrow2 = SWIGLU ? L.m[1].w + (int64_t) lrow * row_bytes : nullptr;
#pragma unroll 2
            for (int u = l; u < units; u += LPR) {
#pragma unroll
                for (int c = 0; c < NCOLS; c++) {
                    if (c < ncols) {
                        const int64_t col = col0 + c;
                        const int8_t * xq = L.xq + col * K;
                        const float * xd = L.xd + col * (K / 256);
                        const int16_t * xbs = L.xbs + col * (K / 16);
                        acc[c] += q4k_unit(wrow, u, xq, xd, xbs);
                        if (SWIGLU) acc2[c] += q4k_unit(wrow2, u, xq, xd, xbs);
                    }
                }
            }
        }
    }

#pragma unroll
    for (int c = 0; c < NCOLS; c++) {
        acc[c] = group_sum<LPR>(acc[c]);
        if (SWIGLU) acc2[c] = group_sum<LPR>(acc2[c]);
    }

    if (!SWIGLU) {
        if (valid && l == 0) {
            const gemv_mat & m = L.m[mi];
#pragma unroll
            for (int c = 0; c < NCOLS; c++) {
                if (c < ncols) {
                    const int64_t col = col0 + c;
                    float v = acc[c];
                    if (m.add) v += m.add[col * m.add_stride + lrow];
                    m.y[col * m.y_stride + lrow] = v;
                }
            }
        }
        return;
    }

    // SwiGLU epilogue: act = silu(gate) * up; optional Q8_0 quantization of 32-row groups
    // (rows per block is a multiple of 32 and n_rows % 32 == 0 when act_q is requested)
    __shared__ float s_act[NCOLS][512 / 4];
    const int rows_per_block = waves * RPW;
    const int row_in_block = wave * RPW + g;
#pragma unroll
    for (int c = 0; c < NCOLS; c++) {
        const float gv = acc[c], uv = acc2[c];
        const float act = gv / (1.0f + expf(-gv)) * uv;
        if (valid && l == 0 && c < ncols) {
            L.m[0].y[(int64_t) (col0 + c) * L.m[0].y_stride + lrow] = act;
        }
        if (l == 0) s_act[c][row_in_block] = act;
    }
    if (L.act_q.qs == nullptr) return;
    __syncthreads();
    // one 32-lane half-wave per (column, 32-row block)
    const int n_qblk = rows_per_block / 32;
    const int half = threadIdx.x / 32;
    const int j = threadIdx.x % 32;
    const int64_t nb_out = a.total_rows / 32;
    for (int task = half; task < NCOLS * n_qblk; task += blockDim.x / 32) {
        const int c = task / n_qblk, qb = task % n_qblk;
        const int out_row = blockIdx.x * rows_per_block + qb * 32 + j;
        const bool ok = c < ncols && out_row < a.total_rows;
        const float v = ok ? s_act[c][qb * 32 + j] : 0.0f;
        const float amax = group_max<32>(fabsf(v));
        const float dd = amax / 127;
        const float id = dd ? 1.0f / dd : 0.0f;
        const int q = (int) roundf(v * id);
        const float qsum = group_sum<32>((float) q);
        if (ok) {
            const int64_t col = col0 + c;
            L.act_q.qs[col * a.total_rows + out_row] = (int8_t) q;
            if (j == 0) {
                L.act_q.d[col * nb_out + out_row / 32] = __half2float(__float2half_rn(dd));
                L.act_q.s[col * nb_out + out_row / 32] = (int32_t) qsum;
            }
        }
    }
}

template <int TYPE, int LPR, int NCOLS, bool SWIGLU>
static void launch_gemv_t(const gemv_kargs & ka, int waves, hipStream_t st) {
    constexpr int RPW = WAVE / LPR;
    const int rows_per_block = waves * RPW;
    const int grid_x = (ka.total_rows + rows_per_block - 1) / rows_per_block;
    const int grid_y = (ka.L.ncols + NCOLS - 1) / NCOLS;
    hipLaunchKernelGGL((gemv_kernel<TYPE, LPR, NCOLS, SWIGLU>), dim3(grid_x, grid_y), dim3(waves * WAVE), 0, st, ka);
    HIP_CHECK(hipGetLastError());
}

template <int TYPE, int LPR>
static void launch_gemv_cols(const gemv_kargs & ka, int waves, hipStream_t st) {
    const int nc = ka.L.ncols;
    if (ka.L.swiglu) {
        if (nc == 1) launch_gemv_t<TYPE, LPR, 1, true>(ka, waves, st);
        else if (nc == 2) launch_gemv_t<TYPE, LPR, 2, true>(ka, waves, st);
        else if (nc <= 4) launch_gemv_t<TYPE, LPR, 4, true>(ka, waves, st);
        else launch_gemv_t<TYPE, LPR, 8, true>(ka, waves, st);
    } else {
        if (nc == 1) launch_gemv_t<TYPE, LPR, 1, false>(ka, waves, st);
        else if (nc == 2) launch_gemv_t<TYPE, LPR, 2, false>(ka, waves, st);
        else if (nc <= 4) launch_gemv_t<TYPE, LPR, 4, false>(ka, waves, st);
        else launch_gemv_t<TYPE, LPR, 8, false>(ka, waves, st);
    }
}

void launch_gemv(const gemv_launch & L, hipStream_t st) {
    gemv_kargs ka;
    ka.L = L;
    int r = 0;
    for (int i = 0; i < L.n_mats; i++) {
        ka.row_begin[i] = r;
        r += L.m[i].n_rows;
    }
    for (int i = L.n_mats; i <= GEMV_MAX_MATS; i++) ka.row_begin[i] = r;
    ka.total_rows = L.swiglu ? L.m[0].n_rows : r;
    if (L.swiglu && (L.n_mats != 2 || L.m[0].n_rows != L.m[1].n_rows)) HIP_ABORT("gemv: swiglu needs two equal matrices");
    if (L.swiglu && L.act_q.qs && (ka.total_rows % 32 != 0)) HIP_ABORT("gemv: quantized swiglu output needs rows %% 32 == 0");
    // 8 waves x (64/LPR) rows: a multiple of 32 rows per block, as the swiglu quantization needs
    const int waves = 8;
    switch (L.type) {
        case GGML_TYPE_Q4_0:
            if (L.K % 32) HIP_ABORT("gemv q4_0: K %% 32");
            launch_gemv_cols<GGML_TYPE_Q4_0, 16>(ka, waves, st);
            break;
        case GGML_TYPE_Q8_0:
            if (L.K % 32) HIP_ABORT("gemv q8_0: K %% 32");
            launch_gemv_cols<GGML_TYPE_Q8_0, 16>(ka, waves, st);
            break;
        case GGML_TYPE_Q4_K:
            if (L.K % 256) HIP_ABORT("gemv q4_K: K %% 256");
            launch_gemv_cols<GGML_TYPE_Q4_K, 8>(ka, waves, st);
            break;
        default:
            HIP_ABORT("gemv: unsupported weight type %d", L.type);
    }
}
