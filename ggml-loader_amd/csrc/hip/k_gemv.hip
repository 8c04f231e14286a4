// k_gemv.hip — quantized matrix-vector kernels (the decode hot path) and their helpers:
// weight plane repacking, activation quantization (ggml Q8_0 / Q8_K semantics) and the
// Q4_0 / Q8_0 / Q4_K integer-dot GEMVs.
//
// GEMV mapping: a wavefront owns 64/LPR rows; LPR lanes split a row's blocks (lane l takes blocks
// l, l+LPR, ...), so one load instruction moves LPR consecutive 16-byte block payloads per row,
// and every lane issues all of its weight loads before the first use. The column's quantized
// activation is staged once per workgroup in LDS. Each lane decodes its blocks in registers and
// does the integer dot with v_dot4_i32_i8; the per-block float terms go to LDS and one lane per
// row adds them in block order — the float summation order of ggml-cpu's scalar dot kernels, so
// the GEMV result is the same float as the CPU reference's (the integer parts are exact in any
// order). Rows of up to four matrices (Q, K and V, or gate and up) are concatenated in one grid
// so one launch streams all of them; grid.y runs over the activation columns.
#include "kernels.h"
#include "gemv_ops.h"

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

// Q6_K GGUF blocks <-> the four planes (q6k_planes), one thread per block
__global__ void repack_q6k_kernel(const uint8_t * __restrict__ raw, q6k_planes p, int64_t nblocks, int64_t first) {
    const int64_t b = (int64_t) blockIdx.x * blockDim.x + threadIdx.x;
    if (b >= nblocks) return;
    const uint8_t * src = raw + b * 210;
    const int64_t o = first + b;
    for (int i = 0; i < 128; i++) p.ql[o * 128 + i] = src[i];
    for (int i = 0; i < 64; i++) p.qh[o * 64 + i] = src[128 + i];
    for (int i = 0; i < 16; i++) p.sc[o * 16 + i] = (int8_t) src[192 + i];
    p.d[o] = __ushort_as_half((unsigned short) (src[208] | (src[209] << 8)));
}

__global__ void unpack_q6k_kernel(uint8_t * __restrict__ raw, q6k_planes p, int64_t nblocks, int64_t first) {
    const int64_t b = (int64_t) blockIdx.x * blockDim.x + threadIdx.x;
    if (b >= nblocks) return;
    uint8_t * dst = raw + b * 210;
    const int64_t o = first + b;
    for (int i = 0; i < 128; i++) dst[i] = p.ql[o * 128 + i];
    for (int i = 0; i < 64; i++) dst[128 + i] = p.qh[o * 64 + i];
    for (int i = 0; i < 16; i++) dst[192 + i] = (uint8_t) p.sc[o * 16 + i];
    const unsigned short h = __half_as_ushort(p.d[o]);
    dst[208] = (uint8_t) (h & 0xff);
    dst[209] = (uint8_t) (h >> 8);
}

void launch_repack_q6k(const uint8_t * raw, q6k_planes p, int64_t nblocks, int64_t first_block, hipStream_t st) {
    if (nblocks <= 0) return;
    launch(repack_q6k_kernel, dim3((unsigned) ((nblocks + 255) / 256)), dim3(256), 0, st, raw, p, nblocks, first_block);
}

void launch_unpack_q6k(uint8_t * raw, q6k_planes p, int64_t nblocks, int64_t first_block, hipStream_t st) {
    if (nblocks <= 0) return;
    launch(unpack_q6k_kernel, dim3((unsigned) ((nblocks + 255) / 256)), dim3(256), 0, st, raw, p, nblocks, first_block);
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
    launch(repack_q_kernel, dim3((unsigned) grid), dim3(threads), 0, st, qsb, bb, raw, qs_plane, d_plane, nblocks, first_block);
}

void launch_unpack_q(int type, uint8_t * raw, const uint8_t * qs_plane, const __half * d_plane,
                     int64_t nblocks, int64_t first_block, hipStream_t st) {
    if (nblocks <= 0) return;
    int qsb, bb;
    qs_geometry(type, qsb, bb);
    const int threads = 256;
    const int64_t grid = (nblocks + threads - 1) / threads;
    launch(unpack_q_kernel, dim3((unsigned) grid), dim3(threads), 0, st, qsb, bb, raw, qs_plane, d_plane, nblocks, first_block);
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
    launch(quantize_q8_kernel, grid, dim3(256), 0, st, x, x_col_stride, K, out.qs, out.d, out.s);
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
    launch(quantize_q8k_kernel, grid, dim3(256), 0, st, x, x_col_stride, K, out.qs, out.d, out.bsums);
}

// ---------------------------------------------------------------------------------------------
// GEMV kernels

// dynamic LDS layout: [staged activation][terms]
struct gemv_lds {
    int8_t * xq;
    float * xd;
    int32_t * xs;      // q8
    int16_t * xbs;     // q8K
    float * terms;     // [rows_per_block * n_chain][T] (T = nb for Q4_0/Q8_0, 9 * nsb for Q4_K)
};

template <int TYPE>
__host__ __device__ inline size_t gemv_lds_bytes(int K, int rows_per_block, int n_chain) {
    if (TYPE == GGML_TYPE_Q4_K) {
        const int nsb = K / 256;
        return (size_t) K + (size_t) nsb * 4 + (size_t) (K / 16) * 2 + 16 + (size_t) rows_per_block * n_chain * nsb * 9 * 4;
    }
    const int nb = K / 32;
    return (size_t) K + (size_t) nb * 8 + (size_t) rows_per_block * n_chain * gemv_term_stride(nb) * 4;
}

template <int TYPE>
__device__ __forceinline__ gemv_lds lds_layout(uint8_t * smem, int K) {
    gemv_lds s;
    s.xq = (int8_t *) smem;
    s.xs = nullptr;
    s.xbs = nullptr;
    if (TYPE == GGML_TYPE_Q4_K) {
        const int nsb = K / 256;
        s.xd = (float *) (smem + K);
        s.xbs = (int16_t *) (smem + K + nsb * 4);
        s.terms = (float *) (smem + ((K + nsb * 4 + (K / 16) * 2 + 15) & ~15));
    } else {
        const int nb = K / 32;
        s.xd = (float *) (smem + K);
        s.xs = (int32_t *) (smem + K + nb * 4);
        s.terms = (float *) (smem + K + nb * 8);
    }
    return s;
}

__device__ __forceinline__ int pack4(int a, int b, int c, int d) {
    return (a & 0xff) | ((b & 0xff) << 8) | ((c & 0xff) << 16) | (d << 24);
}

// Quantizes chunk c (C = 32 or 16 values in v, already in their final float form) of the staged
// column into LDS with ggml's quantize_row_q8_0 (Q4_0/Q8_0 weights) or quantize_row_q8_K (Q4_K)
// roundings. A Q8_0 block is one thread's chunk; a Q8_K super-block is the chunks of 16
// consecutive lanes, which must all call this together (has = the chunk exists).
template <int TYPE, int C>
__device__ __forceinline__ void quant_chunk(const float (&v)[C], int c, bool has, const gemv_lds & s) {
    if (TYPE != GGML_TYPE_Q4_K) {
        if (!has) return;
        float amax = 0.0f;
#pragma unroll
        for (int e = 0; e < C; e++) amax = fmaxf(amax, fabsf(v[e]));
        const float dd = amax / 127;
        const float id = dd ? 1.0f / dd : 0.0f;
        int q[C];
        int sum = 0;
#pragma unroll
        for (int e = 0; e < C; e++) {
            q[e] = (int) roundf(v[e] * id);
            sum += q[e];
        }
        int4 * dst = (int4 *) (s.xq + c * C);
        dst[0] = make_int4(pack4(q[0], q[1], q[2], q[3]), pack4(q[4], q[5], q[6], q[7]),
                           pack4(q[8], q[9], q[10], q[11]), pack4(q[12], q[13], q[14], q[15]));
        dst[1] = make_int4(pack4(q[16], q[17], q[18], q[19]), pack4(q[20], q[21], q[22], q[23]),
                           pack4(q[24], q[25], q[26], q[27]), pack4(q[28], q[29], q[30], q[31]));
        s.xd[c] = __half2float(__float2half_rn(dd));
        s.xs[c] = sum;
    } else {
        // the super-block's value of largest magnitude, the first one on ties
        float ax = -1.0f, val = 0.0f;
        int idx = 0;
        if (has) {
#pragma unroll
            for (int e = 0; e < C; e++) {
                const float a = fabsf(v[e]);
                if (a > ax) { ax = a; idx = c * C + e; val = v[e]; }
            }
        }
        // across the super-block's 16 lanes: quad lanes xor 1, xor 2, then the mirrored lane of the
        // half row and of the row (the combine is a total order, so the pairing does not matter)
        auto take = [&](float ax2, int idx2, float val2) {
            if (ax2 > ax || (ax2 == ax && idx2 < idx)) { ax = ax2; idx = idx2; val = val2; }
        };
        take(dpp_f<0xB1>(ax), dpp_i<0xB1>(idx), dpp_f<0xB1>(val));
        take(dpp_f<0x4E>(ax), dpp_i<0x4E>(idx), dpp_f<0x4E>(val));
        take(dpp_f<0x141>(ax), dpp_i<0x141>(idx), dpp_f<0x141>(val));
        take(dpp_f<0x140>(ax), dpp_i<0x140>(idx), dpp_f<0x140>(val));
        if (!has) return;
        int q[C];
        int bsum = 0;
        const float iscale = ax != 0.0f ? -127.f / val : 0.0f;
#pragma unroll
        for (int e = 0; e < C; e++) {
            const int qv = ax != 0.0f ? round_half_even(iscale * v[e]) : 0;
            q[e] = qv < 127 ? qv : 127;
            bsum += q[e];
        }
        *(int4 *) (s.xq + c * C) = make_int4(pack4(q[0], q[1], q[2], q[3]), pack4(q[4], q[5], q[6], q[7]),
                                             pack4(q[8], q[9], q[10], q[11]), pack4(q[12], q[13], q[14], q[15]));
        s.xbs[c] = (int16_t) bsum;
        if ((c % 16) == 0) s.xd[c / 16] = ax != 0.0f ? 1 / iscale : 0.0f;
    }
}

template <int C>
__device__ __forceinline__ void load_chunk(float (&v)[C], const float * p) {
#pragma unroll
    for (int k = 0; k < C / 4; k++) {
        const float4 f = ((const float4 *) p)[k];
        v[4 * k] = f.x; v[4 * k + 1] = f.y; v[4 * k + 2] = f.z; v[4 * k + 3] = f.w;
    }
}

// The activation prologue: x of column col quantized straight into the LDS staging area, as
// rms_norm(x) * w (rms set: ggml's rms_norm -> mul -> quantize chain, same roundings; one chunk per
// thread, so only the sum of squares is reduced over the workgroup) or as x itself (the quantize
// that ggml-cpu applies to a mul_mat's activation; several chunks per thread).
//
// Loads complete in issue order, so the prologue's loads go out before the weight stream: the
// prologue then computes while the weights are in flight instead of after they arrive. The first
// 32 values per thread (one Q8_0 block, or two Q8_K groups in the quantize-only mode) are loaded by
// prologue_load into registers, and so is one more chunk in the quantize-only mode (in the
// registers that hold the norm weights in the rms mode); further chunks are loaded when they are
// quantized, after the weights (each such load waits for every weight load).
constexpr int PRO_REGS = 32;
// threads of every gemv_kernel and act_quant_kernel workgroup: a constant, so that the prologue's
// addresses need no load of the launch's workgroup size ahead of the weight loads
constexpr int GEMV_NT = 256;

// 16 doubles at p (16-byte aligned) into r as raw bits (double e: r[2e] its low word, r[2e + 1]
// its high word), converted only when they are quantized
__device__ __forceinline__ void load_chunk_f64(float (&r)[PRO_REGS], const double * p) {
#pragma unroll
    for (int k = 0; k < 8; k++) {
        const double2 d = ((const double2 *) p)[k];
        r[4 * k] = __int_as_float(__double2loint(d.x));
        r[4 * k + 1] = __int_as_float(__double2hiint(d.x));
        r[4 * k + 2] = __int_as_float(__double2loint(d.y));
        r[4 * k + 3] = __int_as_float(__double2hiint(d.y));
    }
}

__device__ __forceinline__ void chunk_from_f64(float (&v)[16], const float (&r)[PRO_REGS]) {
#pragma unroll
    for (int e = 0; e < 16; e++) v[e] = (float) __hiloint2double(__float_as_int(r[2 * e + 1]), __float_as_int(r[2 * e]));
}

// F64: the column holds doubles (gemv_norm::f64; Q8_K layout only), each rounded to float and
// quantized as is: chunk t's 16 doubles are loaded into xv and, for rows of more than GEMV_NT
// chunks, chunk t + GEMV_NT's into wv (raw); later chunks when they are quantized.
template <int TYPE, bool PRO, bool F64 = false>
__device__ __forceinline__ void prologue_load(const gemv_launch & L, int col, float (&xv)[PRO_REGS], float (&wv)[PRO_REGS]) {
    // Every load here is unconditional (indices clamped; a thread past the end loads the last
    // chunk again and never uses it), so none of them sits in a branch that the compiler would
    // close with a wait before the weight loads are issued.
    constexpr int C = TYPE == GGML_TYPE_Q4_K ? 16 : 32;
    const int t = threadIdx.x;
#pragma unroll
    for (int e = 0; e < PRO_REGS; e++) { xv[e] = 0.0f; wv[e] = 1.0f; }
    if constexpr (!PRO) {
        // an already quantized column: its quants (xv, 4 x 16 bytes per thread) and, for Q8_0, the
        // block scales and sums (wv[0..1], wv[2..3]); for Q8_K the super-block scale (wv[0]) and
        // two dwords of the 16-element sums (wv[1..2]). Ahead of the weights as well.
        const int K = L.K;
        const int8_t * xq = L.xq + (int64_t) col * K;
#pragma unroll
        for (int k = 0; k < 4; k++) {
            const int i = min(t + k * GEMV_NT, K / 16 - 1);
            const int4 v = *(const int4 *) (xq + i * 16);
            xv[4 * k] = __int_as_float(v.x); xv[4 * k + 1] = __int_as_float(v.y);
            xv[4 * k + 2] = __int_as_float(v.z); xv[4 * k + 3] = __int_as_float(v.w);
        }
        if constexpr (TYPE != GGML_TYPE_Q4_K) {
            const int nb = K / 32;
#pragma unroll
            for (int k = 0; k < 2; k++) {
                const int i = min(t + k * GEMV_NT, nb - 1);
                wv[k] = L.xd[(int64_t) col * nb + i];
                wv[2 + k] = __int_as_float(L.xs[(int64_t) col * nb + i]);
            }
        } else {
            const int nsb = K / 256;
            wv[0] = L.xd[(int64_t) col * nsb + min(t, nsb - 1)];
            const int * bs = (const int *) (L.xbs + (int64_t) col * (K / 16));
#pragma unroll
            for (int k = 0; k < 2; k++) wv[1 + k] = __int_as_float(bs[min(t + k * GEMV_NT, K / 32 - 1)]);
        }
        return;
    } else if constexpr (F64) {
        static_assert(TYPE == GGML_TYPE_Q4_K, "double-valued columns are quantized to Q8_K");
        const int nchunk = L.K / C;
        const double * xcol = (const double *) L.norm.x + (int64_t) col * L.norm.x_stride;
        load_chunk_f64(xv, xcol + (int64_t) min(t, nchunk - 1) * C);
        // (uniform: rows of at most GEMV_NT chunks have no second one)
        if (nchunk > GEMV_NT) load_chunk_f64(wv, xcol + (int64_t) min(t + GEMV_NT, nchunk - 1) * C);
    } else {
        const int nchunk = L.K / C;
        const float * xcol = L.norm.x + (int64_t) col * L.norm.x_stride;
        load_chunk(*reinterpret_cast<float (*)[C]>(&xv[0]), xcol + (int64_t) min(t, nchunk - 1) * C);
        // wv: the norm weights (rms mode) or, in the quantize-only mode, the chunk after the ones
        // xv holds (one unconditional load either way; unused in the rms mode without weights)
        const bool wload = L.norm.rms && L.norm.w;
        load_chunk(*reinterpret_cast<float (*)[C]>(&wv[0]),
                   wload ? L.norm.w + (int64_t) min(t, nchunk - 1) * C
                         : xcol + (int64_t) min(t + (PRO_REGS / C) * GEMV_NT, nchunk - 1) * C);
        if (C * 2 == PRO_REGS) {
            // the quantize-only mode's second chunk; loaded (and left unused) in the rms mode too, so
            // that no branch joins before the weight loads (the join would wait for these loads)
            load_chunk(*reinterpret_cast<float (*)[C]>(&xv[PRO_REGS - C]), xcol + (int64_t) min(t + GEMV_NT, nchunk - 1) * C);
        }
    }
}

template <int TYPE, bool F64 = false>
__device__ __forceinline__ void prologue_finish(const gemv_launch & L, int col, float (&xv)[PRO_REGS], const float (&wv)[PRO_REGS],
                                                const gemv_lds & s, double * s_red) {
    constexpr int C = TYPE == GGML_TYPE_Q4_K ? 16 : 32;
    const int K = L.K;
    const int nchunk = K / C;
    const int t = threadIdx.x;
    if constexpr (F64) {
        float v[16];
        chunk_from_f64(v, xv);
        quant_chunk<TYPE, 16>(v, t, t < nchunk, s);
        if (nchunk > GEMV_NT) {
            chunk_from_f64(v, wv);
            quant_chunk<TYPE, 16>(v, GEMV_NT + t, GEMV_NT + t < nchunk, s);
        }
        const double * xcol = (const double *) L.norm.x + (int64_t) col * L.norm.x_stride;
        for (int c0 = 2 * GEMV_NT; c0 < nchunk; c0 += GEMV_NT) {
            const int c = c0 + t;
            const bool has = c < nchunk;
#pragma unroll
            for (int e = 0; e < 16; e++) v[e] = 0.0f;
            if (has) {
#pragma unroll
                for (int k = 0; k < 8; k++) {
                    const double2 d = ((const double2 *) (xcol + (int64_t) c * 16))[k];
                    v[2 * k] = (float) d.x;
                    v[2 * k + 1] = (float) d.y;
                }
            }
            quant_chunk<TYPE, 16>(v, c, has, s);
        }
        return;
    }
    float (&x0)[C] = *reinterpret_cast<float (*)[C]>(&xv[0]);
    if (!L.norm.rms) {
        quant_chunk<TYPE, C>(x0, t, t < nchunk, s);
        int c0 = GEMV_NT;
        if (C * 2 == PRO_REGS) {
            quant_chunk<TYPE, C>(*reinterpret_cast<float (*)[C]>(&xv[PRO_REGS - C]), c0 + t, c0 + t < nchunk, s);
            c0 += GEMV_NT;
        }
        quant_chunk<TYPE, C>(*reinterpret_cast<const float (*)[C]>(&wv[0]), c0 + t, c0 + t < nchunk, s);
        c0 += GEMV_NT;
        const float * xcol = L.norm.x + (int64_t) col * L.norm.x_stride;
        for (; c0 < nchunk; c0 += GEMV_NT) {
            const int c = c0 + t;
            const bool has = c < nchunk;
            float v[C];
#pragma unroll
            for (int e = 0; e < C; e++) v[e] = 0.0f;
            if (has) load_chunk(v, xcol + (int64_t) c * C);
            quant_chunk<TYPE, C>(v, c, has, s);
        }
        return;
    }
    const int lane = t % WAVE, wave = t / WAVE;
    double ss = 0.0;
    if (t < nchunk) {
#pragma unroll
        for (int e = 0; e < C; e++) ss += (double) (x0[e] * x0[e]);
    }
    ss = wave_sum_d(ss);
    if (lane == 0) s_red[wave] = ss;
    __syncthreads();
    double total = 0.0;
    for (int w = 0; w < GEMV_NT / WAVE; w++) total += s_red[w];
    const float mean = (float) (total / (double) K);
    const float scale = 1.0f / sqrtf(mean + L.norm.eps);
#pragma unroll
    for (int e = 0; e < C; e++) {
        x0[e] = x0[e] * scale;
        if (L.norm.w) x0[e] = x0[e] * wv[e];
    }
    quant_chunk<TYPE, C>(x0, t, t < nchunk, s);
}

// the quantized activation column in LDS: finished by the prologue, or copied
template <int TYPE, bool PRO, bool F64 = false>
__device__ __forceinline__ void stage_x(const gemv_launch & L, int col, const gemv_lds & s, double * s_red,
                                        float (&xv)[PRO_REGS], const float (&wv)[PRO_REGS]) {
    const int K = L.K;
    if constexpr (PRO) {
        prologue_finish<TYPE, F64>(L, col, xv, wv, s, s_red);
    } else if constexpr (TYPE == GGML_TYPE_Q4_K) {
        // from the registers prologue_load filled; a row longer than they cover (K > 64 * GEMV_NT)
        // copies the rest here
        // The stores are unconditional: a thread past the end stores the last element it loaded
        // (the index was clamped) over that same element. A guarded store would let the compiler
        // sink its load behind the weight loads, where waiting for it waits for all of them.
        const int nsb = K / 256, nt = GEMV_NT;
#pragma unroll
        for (int k = 0; k < 4; k++) {
            const int i = min((int) threadIdx.x + k * nt, K / 16 - 1);
            *(int4 *) (s.xq + i * 16) = make_int4(__float_as_int(xv[4 * k]), __float_as_int(xv[4 * k + 1]),
                                                  __float_as_int(xv[4 * k + 2]), __float_as_int(xv[4 * k + 3]));
        }
        for (int i = (threadIdx.x + 4 * nt) * 16; i < K; i += nt * 16) *(int4 *) (s.xq + i) = *(const int4 *) (L.xq + (int64_t) col * K + i);
        s.xd[min((int) threadIdx.x, nsb - 1)] = wv[0];
        for (int i = threadIdx.x + nt; i < nsb; i += nt) s.xd[i] = L.xd[(int64_t) col * nsb + i];
        int * sbs = (int *) s.xbs;
        const int * gbs = (const int *) (L.xbs + (int64_t) col * (K / 16));
#pragma unroll
        for (int k = 0; k < 2; k++) sbs[min((int) threadIdx.x + k * nt, K / 32 - 1)] = __float_as_int(wv[1 + k]);
        for (int i = threadIdx.x + 2 * nt; i < K / 32; i += nt) sbs[i] = gbs[i];
    } else {
        // from the registers prologue_load filled (K <= 64 * GEMV_NT, nb <= 2 * GEMV_NT), with
        // unconditional stores as in the Q8_K copy above
        const int nb = K / 32;
#pragma unroll
        for (int k = 0; k < 4; k++) {
            const int i = min((int) (threadIdx.x + k * GEMV_NT), K / 16 - 1);
            *(int4 *) (s.xq + i * 16) = make_int4(__float_as_int(xv[4 * k]), __float_as_int(xv[4 * k + 1]),
                                                  __float_as_int(xv[4 * k + 2]), __float_as_int(xv[4 * k + 3]));
        }
#pragma unroll
        for (int k = 0; k < 2; k++) {
            const int i = min((int) (threadIdx.x + k * GEMV_NT), nb - 1);
            s.xd[i] = wv[k];
            s.xs[i] = __float_as_int(wv[2 + k]);
        }
    }
    __syncthreads();
}

// The prologue run once per column into global memory, for consumers too wide to redo it in every
// workgroup (the LM head): same arithmetic, so the GEMV that copies the result computes the same floats.
template <int TYPE>
__global__ __launch_bounds__(GEMV_NT) void act_quant_kernel(const gemv_launch L, q8_act q8, q8k_act q8k) {
    prefetch_kernargs<sizeof(gemv_launch) + sizeof(q8_act) + sizeof(q8k_act)>();
    extern __shared__ __align__(16) uint8_t smem[];
    __shared__ double s_red[GEMV_NT / WAVE];
    const int col = blockIdx.x;
    const int K = L.K;
    const gemv_lds s = lds_layout<TYPE>(smem, K);
    float xv[PRO_REGS], wv[PRO_REGS];
    prologue_load<TYPE, true>(L, col, xv, wv);
    prologue_finish<TYPE>(L, col, xv, wv, s, s_red);
    __syncthreads();
    int8_t * qs = (TYPE == GGML_TYPE_Q4_K ? q8k.qs : q8.qs) + (int64_t) col * K;
    for (int i = threadIdx.x * 16; i < K; i += GEMV_NT * 16) *(int4 *) (qs + i) = *(const int4 *) (s.xq + i);
    if (TYPE == GGML_TYPE_Q4_K) {
        for (int i = threadIdx.x; i < K / 256; i += GEMV_NT) q8k.d[(int64_t) col * (K / 256) + i] = s.xd[i];
        for (int i = threadIdx.x; i < K / 16; i += GEMV_NT) q8k.bsums[(int64_t) col * (K / 16) + i] = s.xbs[i];
    } else {
        for (int i = threadIdx.x; i < K / 32; i += GEMV_NT) {
            q8.d[(int64_t) col * (K / 32) + i] = s.xd[i];
            q8.s[(int64_t) col * (K / 32) + i] = s.xs[i];
        }
    }
}

// moe_wsum_kernel's weighted sum of the k expert rows (+ residual) for one token per workgroup,
// written out as that kernel writes it, then the next rms_norm * w of the row quantized to Q8_K
// with act_quant_kernel's arithmetic (thread t holds elements 16t .. 16t + 15, its chunk): the
// launch that produces the residual stream also produces the next projection's quantized input.
__global__ __launch_bounds__(GEMV_NT) void wsum_norm_q8k_kernel(const moe_wsum M, const float * nw, float eps, q8k_act q8k) {
    prefetch_kernargs<sizeof(moe_wsum)>();
    extern __shared__ __align__(16) uint8_t smem[];
    __shared__ double s_red[GEMV_NT / WAVE];
    __shared__ __align__(16) float s_x[16 * GEMV_NT];
    const int K = (int) M.n_embd, tok = blockIdx.x, t = threadIdx.x;
    const int lane = t % WAVE, wave = t / WAVE, nchunk = K / 16, nv = K / 4;
    const int c = min(t, nchunk - 1);                 // clamped, unused past the row
    const gemv_lds s = lds_layout<GGML_TYPE_Q4_K>(smem, K);
    const float4 * e = (const float4 *) (M.e + (int64_t) tok * M.e_nb2);
    const float * w = M.w + (int64_t) tok * M.w_nb2;
    // the sum: float4 columns v0 + t and v0 + GEMV_NT + t of the row per thread (every thread, loads
    // coalesced), the slots in order with each product rounded, as the mul and add chain; then the
    // residual. The row goes out and into LDS, where each thread picks its 16-element chunk up.
    for (int v0 = 0; v0 < nv; v0 += 2 * GEMV_NT) {
        const int va = min(v0 + t, nv - 1), vb = min(v0 + GEMV_NT + t, nv - 1);   // clamped, unused past the row
        float4 xa = make_float4(0.0f, 0.0f, 0.0f, 0.0f), xb = xa;
        for (int s0 = 0; s0 < M.k; s0 += 8) {
            float4 ea[8], eb[8];
            float wv[8];
#pragma unroll
            for (int j = 0; j < 8; j++) {
                const int sl = min(s0 + j, M.k - 1);  // clamped, unused past k
                wv[j] = w[sl * M.w_nb1];
                ea[j] = e[sl * (M.e_nb1 / 4) + va];
                eb[j] = e[sl * (M.e_nb1 / 4) + vb];
            }
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int j = 0; j < 8; j++) {
                if (s0 + j < M.k) {
                    const float4 pa = make_float4(ea[j].x * wv[j], ea[j].y * wv[j], ea[j].z * wv[j], ea[j].w * wv[j]);
                    const float4 pb = make_float4(eb[j].x * wv[j], eb[j].y * wv[j], eb[j].z * wv[j], eb[j].w * wv[j]);
                    if (s0 + j == 0) {
                        xa = pa;
                        xb = pb;
                    } else {
                        xa = make_float4(xa.x + pa.x, xa.y + pa.y, xa.z + pa.z, xa.w + pa.w);
                        xb = make_float4(xb.x + pb.x, xb.y + pb.y, xb.z + pb.z, xb.w + pb.w);
                    }
                }
            }
        }
        if (M.res) {
            const float4 * r = (const float4 *) (M.res + (int64_t) tok * M.res_nb1);
            const float4 ra = r[va], rb = r[vb];
            xa = make_float4(xa.x + ra.x, xa.y + ra.y, xa.z + ra.z, xa.w + ra.w);
            xb = make_float4(xb.x + rb.x, xb.y + rb.y, xb.z + rb.z, xb.w + rb.w);
        }
        float4 * o = (float4 *) (M.out + (int64_t) tok * M.out_nb1);
        if (v0 + t < nv) {
            o[va] = xa;
            ((float4 *) s_x)[va] = xa;
        }
        if (v0 + GEMV_NT + t < nv) {
            o[vb] = xb;
            ((float4 *) s_x)[vb] = xb;
        }
    }
    __syncthreads();
    float x0[16];
#pragma unroll
    for (int q = 0; q < 4; q++) {
        const float4 v = ((const float4 *) s_x)[c * 4 + q];
        x0[4 * q] = v.x; x0[4 * q + 1] = v.y; x0[4 * q + 2] = v.z; x0[4 * q + 3] = v.w;
    }
    // rms_norm * w and Q8_K: the steps of prologue_finish's rms mode
    double ss = 0.0;
    if (t < nchunk) {
#pragma unroll
        for (int i = 0; i < 16; i++) ss += (double) (x0[i] * x0[i]);
    }
    ss = wave_sum_d(ss);
    if (lane == 0) s_red[wave] = ss;
    __syncthreads();
    double total = 0.0;
    for (int w8 = 0; w8 < GEMV_NT / WAVE; w8++) total += s_red[w8];
    const float mean = (float) (total / (double) K);
    const float scale = 1.0f / sqrtf(mean + eps);
    const float4 * w4 = (const float4 *) (nw + c * 16);
#pragma unroll
    for (int q = 0; q < 4; q++) {
        const float4 g = w4[q];
        x0[4 * q] = x0[4 * q] * scale; x0[4 * q] = x0[4 * q] * g.x;
        x0[4 * q + 1] = x0[4 * q + 1] * scale; x0[4 * q + 1] = x0[4 * q + 1] * g.y;
        x0[4 * q + 2] = x0[4 * q + 2] * scale; x0[4 * q + 2] = x0[4 * q + 2] * g.z;
        x0[4 * q + 3] = x0[4 * q + 3] * scale; x0[4 * q + 3] = x0[4 * q + 3] * g.w;
    }
    quant_chunk<GGML_TYPE_Q4_K, 16>(x0, t, t < nchunk, s);
    __syncthreads();
    int8_t * qs = q8k.qs + (int64_t) tok * K;
    for (int i = t * 16; i < K; i += GEMV_NT * 16) *(int4 *) (qs + i) = *(const int4 *) (s.xq + i);
    for (int i = t; i < K / 256; i += GEMV_NT) q8k.d[(int64_t) tok * (K / 256) + i] = s.xd[i];
    for (int i = t; i < K / 16; i += GEMV_NT) q8k.bsums[(int64_t) tok * (K / 16) + i] = s.xbs[i];
}

bool wsum_norm_q8k_supported(const moe_wsum & M, const float * nw) {
    const int64_t K = M.n_embd;
    return K % 256 == 0 && K <= 16 * GEMV_NT && M.k >= 1 && M.n_tok >= 1 && ((uintptr_t) M.e | (uintptr_t) M.out | (uintptr_t) nw) % 16 == 0 &&
           (!M.res || ((uintptr_t) M.res % 16 == 0 && M.res_nb1 % 4 == 0)) && M.e_nb1 % 4 == 0 && M.e_nb2 % 4 == 0 && M.out_nb1 % 4 == 0;
}

void launch_wsum_norm_q8k(const moe_wsum & M, const float * nw, float eps, q8k_act q8k, hipStream_t st) {
    const int64_t K = M.n_embd;
    if (!wsum_norm_q8k_supported(M, nw)) HIP_ABORT("wsum_norm_q8k: unsupported rows (n_embd %lld)", (long long) K);
    launch(wsum_norm_q8k_kernel, dim3((unsigned) M.n_tok), dim3(GEMV_NT), gemv_lds_bytes<GGML_TYPE_Q4_K>((int) K, 0, 0), st, M, nw, eps,
           q8k);
}

void launch_act_quant(const gemv_launch & L, const q8_act & q8, const q8k_act & q8k, hipStream_t st) {
    if (!L.norm.x || L.K > act_quant_max_k(L.type, L.norm.rms != 0)) HIP_ABORT("act_quant: K=%d unsupported", L.K);
    switch (L.type) {
        case GGML_TYPE_Q4_0: case GGML_TYPE_Q8_0:
            launch(act_quant_kernel<GGML_TYPE_Q4_0>, dim3(L.ncols), dim3(GEMV_NT), gemv_lds_bytes<GGML_TYPE_Q4_0>(L.K, 0, 0), st, L, q8, q8k);
            break;
        case GGML_TYPE_Q4_K: case GGML_TYPE_Q5_K: case GGML_TYPE_Q6_K:   // Q8_K activations
            launch(act_quant_kernel<GGML_TYPE_Q4_K>, dim3(L.ncols), dim3(GEMV_NT), gemv_lds_bytes<GGML_TYPE_Q4_K>(L.K, 0, 0), st, L, q8, q8k);
            break;
        default:
            HIP_ABORT("act_quant: unsupported weight type %d", L.type);
    }
}

template <int TYPE, int LPR, bool SWIGLU, int ITS, bool PRO, bool F64 = false>
__global__ __launch_bounds__(512) void gemv_kernel(const gemv_kargs a) {
    prefetch_kernargs<sizeof(gemv_kargs)>();
    extern __shared__ __align__(16) uint8_t smem[];
    constexpr int RPW = WAVE / LPR;
    constexpr int NCH = SWIGLU ? 2 : 1;          // gate and up chains
    const int lane = threadIdx.x % WAVE;
    const int wave = threadIdx.x / WAVE;
    const int g = lane / LPR;
    const int l = lane % LPR;
    const int rows_pb = a.rows_per_block;
    const int rib = wave * RPW + g;               // row in block
    const int row = blockIdx.x * rows_pb + rib;
    const int col = blockIdx.y;
    const gemv_launch & L = a.L;
    const int K = L.K;
    const int mi = SWIGLU ? 0 : find_mat(a, blockIdx.x * rows_pb);   // uniform: the workgroup's matrix
    const int lrow = SWIGLU ? row : row - a.row_begin[mi];
    const bool valid = row < a.total_rows && lrow < L.m[mi].n_rows;

    constexpr int AT = is_kquant(TYPE) ? GGML_TYPE_Q4_K : TYPE;   // the activation's layout: Q8_K or Q8_0
    const gemv_lds s = lds_layout<AT>(smem, K);
    __shared__ double s_red[512 / WAVE];

    // mul_mat_id: the expert of this column and its activation column
    int xcol = col;
    int64_t erow = 0;
    if (L.ids) {
        const int t = col / L.n_slots, sl = col % L.n_slots;
        xcol = t * L.x_cols + sl % L.x_cols;
        const int e = min(max(L.ids[(int64_t) t * L.ids_stride + sl], 0), L.n_experts - 1);
        erow = (int64_t) e * L.expert_rows;
    }

    // ---- per-block terms ----
    if (TYPE == GGML_TYPE_Q4_0 || TYPE == GGML_TYPE_Q8_0) {
        constexpr int QS = TYPE == GGML_TYPE_Q4_0 ? Q4_0_QS : Q8_0_QS;
        constexpr int MAXIT = ITS;   // blocks per lane (nb <= ITS * LPR)
        const int nb = K / 32;
        // prologue loads, then every weight load of this lane, then the prologue's arithmetic: the
        // weight stream is in flight while the column is normalized and quantized
        float xv[PRO_REGS], wv[PRO_REGS];
        prologue_load<TYPE, PRO>(L, xcol, xv, wv);
        // Straight-line loads (row and block clamped into the matrix; the extra lanes' values are
        // never used) so they all issue back to back; the fp16 scales stay raw until the dots.
        uint4 qa[NCH][MAXIT], qb[NCH][MAXIT];
        uint32_t dwb[NCH][MAXIT];
#pragma unroll
        for (int ch = 0; ch < NCH; ch++) {
            const gemv_mat & wm = L.m[SWIGLU ? ch : mi];
            const int64_t wr = erow + min(lrow, wm.n_rows - 1);
            const uint8_t * wq = wm.w + wr * nb * QS;
            const unsigned short * wd = (const unsigned short *) wm.wd + wr * nb;
#pragma unroll
            for (int it = 0; it < MAXIT; it++) {
                const int b = min(l + it * LPR, nb - 1);
                qa[ch][it] = *(const uint4 *) (wq + (int64_t) b * QS);
                if (TYPE == GGML_TYPE_Q8_0) qb[ch][it] = *(const uint4 *) (wq + (int64_t) b * QS + 16);
                dwb[ch][it] = wd[b];
            }
        }
        stage_x<TYPE, PRO>(L, xcol, s, s_red, xv, wv);
#pragma unroll
        for (int ch = 0; ch < NCH; ch++) {
            if (!valid) break;
            float * terms = s.terms + (rib * NCH + ch) * gemv_term_stride(nb);
#pragma unroll
            for (int it = 0; it < MAXIT; it++) {
                const int b = l + it * LPR;
                if (b < nb) {
                    const int4 xa = *(const int4 *) (s.xq + b * 32);
                    const int4 xb = *(const int4 *) (s.xq + b * 32 + 16);
                    const float dx = s.xd[b];
                    const float dw = __half2float(__ushort_as_half((unsigned short) dwb[ch][it]));
                    float t;
                    if (TYPE == GGML_TYPE_Q4_0) {
                        const int sumi = dot_q4_0_block(qa[ch][it], xa, xb) - 8 * s.xs[b];
                        t = ((float) sumi * dw) * dx;           // ggml: sumi*d_x*d_y
                    } else {
                        const int sumi = dot_q8_0_block(qa[ch][it], qb[ch][it], xa, xb);
                        t = (float) sumi * (dw * dx);           // ggml: sumi*(d_x*d_y)
                    }
                    terms[b] = t;
                }
            }
        }
    } else { // K-quants: per (super-block, l) products d*aux32[l] and dmin*mins
        // as above: the prologue's loads, then every weight load of this lane (ITS units of 64
        // weights; unit and row clamped into the matrix), then the prologue's arithmetic while the
        // weights are in flight. A unit's 16-byte pieces: Q4_K the block header and the pair's 32
        // quant bytes; Q5_K those and the block's 32 qh bytes; Q6_K (planes) the half's 64 ql and 32
        // qh bytes, plus its four scales and the block's d.
        float xv[PRO_REGS], wv[PRO_REGS];
        prologue_load<AT, PRO, F64>(L, xcol, xv, wv);
        // (the double-valued column's loads are many: kept ahead of the weights' so that waiting
        // for them does not wait for any weight load)
        if constexpr (F64) asm volatile("" ::: "memory");
        const int units = K / 64, nsb = K / 256;
        constexpr int NW = TYPE == GGML_TYPE_Q4_K ? 3 : TYPE == GGML_TYPE_Q5_K ? 5 : 6;
        constexpr int BB = TYPE == GGML_TYPE_Q4_K ? Q4_K_BYTES : Q5_K_BYTES;
        uint4 wq[NCH][ITS][NW];
        uint32_t wsc[NCH][ITS], wdd[NCH][ITS];
#pragma unroll
        for (int ch = 0; ch < NCH; ch++) {
            const gemv_mat & wm = L.m[SWIGLU ? ch : mi];
            const int64_t wr = erow + min(lrow, wm.n_rows - 1);
#pragma unroll
            for (int it = 0; it < ITS; it++) {
                const int u = min(l + it * LPR, units - 1);
                const int sb = u >> 2, p = u & 3;
                if constexpr (TYPE == GGML_TYPE_Q6_K) {
                    const int64_t b = wr * nsb + sb;
                    const uint4 * ql = (const uint4 *) (wm.w + b * 128 + 64 * (p >> 1));
                    const uint4 * qh = (const uint4 *) (wm.wqh + b * 64 + 32 * (p >> 1));
                    wq[ch][it][0] = ql[0]; wq[ch][it][1] = ql[1]; wq[ch][it][2] = ql[2]; wq[ch][it][3] = ql[3];
                    wq[ch][it][4] = qh[0]; wq[ch][it][5] = qh[1];
                    wsc[ch][it] = *(const uint32_t *) (wm.wsc + b * 16 + 4 * p);
                    wdd[ch][it] = ((const unsigned short *) wm.wd)[b];
                } else {
                    const uint8_t * blk = wm.w + (wr * nsb + sb) * BB;
                    wq[ch][it][0] = *(const uint4 *) blk;
                    const int qoff = TYPE == GGML_TYPE_Q4_K ? 16 : 48;
                    wq[ch][it][1] = *(const uint4 *) (blk + qoff + 32 * p);
                    wq[ch][it][2] = *(const uint4 *) (blk + qoff + 16 + 32 * p);
                    if constexpr (TYPE == GGML_TYPE_Q5_K) {
                        wq[ch][it][3] = *(const uint4 *) (blk + 16);
                        wq[ch][it][4] = *(const uint4 *) (blk + 32);
                    }
                }
            }
        }
        // a double-valued column stays raw until every weight load is out (converted earlier, its
        // registers would be reused, and the reuse waits for the loads)
        if constexpr (F64) __builtin_amdgcn_sched_barrier(0);
        stage_x<AT, PRO, F64>(L, xcol, s, s_red, xv, wv);
        // the staged activation's sub-blocks grouped by l
        group_by_l_lds(s.xq, K / 32);
        __syncthreads();
#pragma unroll
        for (int ch = 0; ch < NCH; ch++) {
            float * terms = s.terms + (rib * NCH + ch) * nsb * 9;
#pragma unroll
            for (int it = 0; it < ITS; it++) {
                if (it * LPR >= units) break;       // uniform across the workgroup
                const int u = l + it * LPR;
                const int sb = u >> 2, p = u & 3;
                const bool has = valid && u < units;
                int aux[8], mins = 0;
#pragma unroll
                for (int k = 0; k < 8; k++) aux[k] = 0;
                if (has) {
                    const int * xs = (const int *) (s.xq + sb * 256 + 64 * p);
                    const uint4 (&w)[NW] = wq[ch][it];
                    if constexpr (TYPE == GGML_TYPE_Q4_K) {
                        q4k_unit_dot(q4k_prepare(w[0], w[1], w[2], p), p, xs, xs + 8, s.xbs + sb * 16, aux, mins);
                    } else if constexpr (TYPE == GGML_TYPE_Q5_K) {
                        q5k_unit_dot(q4k_prepare(w[0], w[1], w[2], p), w[3], w[4], p, xs, xs + 8, s.xbs + sb * 16, aux, mins);
                    } else {
                        const uint4 ql[4] = { w[0], w[1], w[2], w[3] };
                        q6k_unit_dot(ql, w[4], w[5], wsc[ch][it], p, xs, xs + 8, aux);
                    }
                }
                // the 4 units of a super-block sit on 4 consecutive lanes: combine (exact integers)
#pragma unroll
                for (int k = 0; k < 8; k++) {
                    aux[k] += dpp_i<0xB1>(aux[k]);   // quad lanes xor 1
                    aux[k] += dpp_i<0x4E>(aux[k]);   // quad lanes xor 2
                }
                mins += dpp_i<0xB1>(mins);
                mins += dpp_i<0x4E>(mins);
                if (has) {
                    const float yd = s.xd[sb];
                    // Q4_K/Q5_K: d and dmin from the block header; Q6_K: d from its plane, no mins
                    // (a zero mins term leaves ggml's sumf = 0 + sums[0] + ... unchanged)
                    const uint32_t dd = TYPE == GGML_TYPE_Q6_K ? wdd[ch][it] : wq[ch][it][0].x;
                    const float d = __half2float(__ushort_as_half((unsigned short) (dd & 0xffff))) * yd;
                    const float dmin = TYPE == GGML_TYPE_Q6_K ? 0.0f : __half2float(__ushort_as_half((unsigned short) (dd >> 16))) * yd;
                    // this lane stores the products for l = 2p, 2p+1 (static register indexing)
                    float t0 = 0.0f, t1 = 0.0f;
#pragma unroll
                    for (int k = 0; k < 8; k++) {
                        if (k == 2 * p) t0 = d * (float) aux[k];
                        if (k == 2 * p + 1) t1 = d * (float) aux[k];
                    }
                    float * tt = terms + sb * 9;
                    tt[2 * p] = t0;
                    tt[2 * p + 1] = t1;
                    if (p == 0) tt[8] = TYPE == GGML_TYPE_Q6_K ? 0.0f : dmin * (float) mins;
                }
            }
        }
    }
    if constexpr (TYPE == GGML_TYPE_Q4_0 || TYPE == GGML_TYPE_Q8_0) {
        // ---- ordered sums: every chain of the workgroup on its own lane of wave 0 (lane = row *
        // NCH + chain), so one wave instruction advances all of them ----
        __syncthreads();
        if (wave != 0) return;
        const int nb = K / 32;
        const int r = lane / NCH, ch = lane % NCH;
        const int rrow = blockIdx.x * rows_pb + r;
        const bool has = r < rows_pb && rrow < a.total_rows && (SWIGLU || rrow - a.row_begin[mi] < L.m[mi].n_rows);
        float acc = 0.0f;
        if (has) acc = ordered_sum(s.terms + (r * NCH + ch) * gemv_term_stride(nb), nb);
        if constexpr (SWIGLU) {
            // act = silu(gate) * up (two roundings, as the silu and mul ops); up sits on the next lane
            const float uv = __shfl_down(acc, 1, WAVE);
            if (has && ch == 0) {
                const float sl = acc / (1.0f + exp_cr(-acc));
                L.m[0].y[(int64_t) col * L.m[0].y_stride + rrow] = sl * uv;
            }
        } else if (has) {
            const int rl = rrow - a.row_begin[mi];
            const gemv_mat & m = L.m[mi];
            float v = acc;
            if (m.add) v = v + m.add[(int64_t) col * m.add_stride + rl];
            m.y[(int64_t) col * m.y_stride + rl] = v;
        }
        return;
    }

    // a K-quant row's terms were written by lanes of its own wave: a wave-level ordering point suffices
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");

    // ---- ordered sums, one lane per chain ----
    float res[NCH];
#pragma unroll
    for (int ch = 0; ch < NCH; ch++) res[ch] = 0.0f;
    {
        const int nsb = K / 256;
        // lanes 0..8 of a group: l < 8 -> sums[l] chain, l == 8 -> the mins chain (per ch)
        float v = 0.0f;
        const int ch = l / 9, k = l % 9;
        if (ch < NCH && valid) {
            const float * terms = s.terms + (rib * NCH + ch) * nsb * 9;
            if (k < 8) {
                for (int i = 0; i < nsb; i++) v = v + terms[i * 9 + k];
            } else {
                for (int i = 0; i < nsb; i++) v = v - terms[i * 9 + 8];
            }
        }
        // sumf (the mins chain) then += sums[0..7] in order
#pragma unroll
        for (int c = 0; c < NCH; c++) {
            float f = __shfl(v, g * LPR + c * 9 + 8, WAVE);
#pragma unroll
            for (int kk = 0; kk < 8; kk++) f = f + __shfl(v, g * LPR + c * 9 + kk, WAVE);
            res[c] = f;
        }
    }

    if (!SWIGLU) {
        if (valid && l == 0) {
            const gemv_mat & m = L.m[mi];
            float v = res[0];
            if (m.add) v = v + m.add[(int64_t) col * m.add_stride + lrow];
            m.y[(int64_t) col * m.y_stride + lrow] = v;
        }
        return;
    }

    // SwiGLU epilogue: act = silu(gate) * up (two roundings, as the silu and mul ops)
    const float gv = res[0], uv = res[NCH - 1];
    const float sl = gv / (1.0f + exp_cr(-gv));
    const float act = sl * uv;
    if (valid && l == 0) L.m[0].y[(int64_t) col * L.m[0].y_stride + lrow] = act;
}

template <int TYPE, int LPR, bool SWIGLU, int ITS>
static void launch_gemv_its(gemv_kargs & ka, int waves, hipStream_t st) {
    constexpr int RPW = WAVE / LPR;
    if (waves * WAVE != GEMV_NT) HIP_ABORT("gemv: %d-thread workgroups (the kernel assumes %d)", waves * WAVE, GEMV_NT);
    ka.rows_per_block = waves * RPW;
    if (!SWIGLU) {
        // every matrix starts on a workgroup boundary
        int r = 0;
        for (int i = 0; i < ka.L.n_mats; i++) {
            ka.row_begin[i] = r;
            r += (ka.L.m[i].n_rows + ka.rows_per_block - 1) / ka.rows_per_block * ka.rows_per_block;
        }
        for (int i = ka.L.n_mats; i <= GEMV_MAX_MATS; i++) ka.row_begin[i] = r;
        ka.total_rows = r;
    }
    const int grid_x = (ka.total_rows + ka.rows_per_block - 1) / ka.rows_per_block;
    constexpr int AT = is_kquant(TYPE) ? GGML_TYPE_Q4_K : TYPE;
    const size_t lds = gemv_lds_bytes<AT>(ka.L.K, ka.rows_per_block, SWIGLU ? 2 : 1);
    if (!is_kquant(TYPE) && ka.rows_per_block * (SWIGLU ? 2 : 1) > WAVE) {
        HIP_ABORT("gemv: %d chains per workgroup exceed one wave", ka.rows_per_block * (SWIGLU ? 2 : 1));
    }
    if (lds > 160 * 1024) HIP_ABORT("gemv: K=%d needs %zu bytes of LDS", ka.L.K, lds);
    if (ka.L.norm.x && ka.L.norm.f64) {
        if constexpr (is_kquant(TYPE) && !SWIGLU) {
            return launch((gemv_kernel<TYPE, LPR, SWIGLU, ITS, true, true>), dim3(grid_x, ka.L.ncols), dim3(waves * WAVE), lds, st, ka);
        }
        HIP_ABORT("gemv: a double-valued column needs K-quant weights without SwiGLU");
    }
    if (ka.L.norm.x) launch((gemv_kernel<TYPE, LPR, SWIGLU, ITS, true>), dim3(grid_x, ka.L.ncols), dim3(waves * WAVE), lds, st, ka);
    else launch((gemv_kernel<TYPE, LPR, SWIGLU, ITS, false>), dim3(grid_x, ka.L.ncols), dim3(waves * WAVE), lds, st, ka);
}

// ITS = weight blocks per lane for Q4_0/Q8_0, held in registers from the up-front loads. The ladder
// stops where the registers of both SwiGLU chains would spill (12) and at 16 for a single chain.
// largest K-quant units (64 weights) per lane held in registers: 3, 5 or 6 16-byte pieces per
// unit (Q4_K, Q5_K, Q6_K), per chain
template <int TYPE, bool SWIGLU>
constexpr int kq_max_its() {
    return TYPE == GGML_TYPE_Q4_K ? (SWIGLU ? 4 : 10) : TYPE == GGML_TYPE_Q5_K ? (SWIGLU ? 3 : 6) : (SWIGLU ? 2 : 4);
}

template <int TYPE, int LPR, bool SWIGLU>
static void launch_gemv_t(gemv_kargs & ka, int waves, hipStream_t st) {
    if constexpr (is_kquant(TYPE) && TYPE != GGML_TYPE_Q4_K) {
        // Q5_K / Q6_K: units of 64 weights per lane, up to kq_max_its
        const int its = (ka.L.K / 64 + LPR - 1) / LPR;
        constexpr int MAXI = kq_max_its<TYPE, SWIGLU>();
        if (its > MAXI) HIP_ABORT("gemv type %d: K=%d needs %d units per lane (at most %d)", TYPE, ka.L.K, its, MAXI);
        if (its <= 1) launch_gemv_its<TYPE, LPR, SWIGLU, 1>(ka, waves, st);
        else if (its <= 2) launch_gemv_its<TYPE, LPR, SWIGLU, 2>(ka, waves, st);
        else if constexpr (MAXI >= 3) {
            if (its <= 3) launch_gemv_its<TYPE, LPR, SWIGLU, 3>(ka, waves, st);
            else if constexpr (MAXI >= 4) {
                if (its <= 4) launch_gemv_its<TYPE, LPR, SWIGLU, 4>(ka, waves, st);
                else if constexpr (MAXI >= 6) launch_gemv_its<TYPE, LPR, SWIGLU, 6>(ka, waves, st);
            }
        }
    } else if constexpr (TYPE == GGML_TYPE_Q4_K) {
        // units of 64 weights per lane
        const int its = (ka.L.K / 64 + LPR - 1) / LPR;
        if (its <= 1) launch_gemv_its<TYPE, LPR, SWIGLU, 1>(ka, waves, st);
        else if (its <= 2) launch_gemv_its<TYPE, LPR, SWIGLU, 2>(ka, waves, st);
        else if (its <= 3) launch_gemv_its<TYPE, LPR, SWIGLU, 3>(ka, waves, st);
        else if (its <= 4) launch_gemv_its<TYPE, LPR, SWIGLU, 4>(ka, waves, st);
        else if constexpr (!SWIGLU) {
            if (its <= 6) launch_gemv_its<TYPE, LPR, SWIGLU, 6>(ka, waves, st);
            else if (its <= 8) launch_gemv_its<TYPE, LPR, SWIGLU, 8>(ka, waves, st);
            else if (its <= 10) launch_gemv_its<TYPE, LPR, SWIGLU, 10>(ka, waves, st);
            else HIP_ABORT("gemv q4_K: K=%d is too long", ka.L.K);
        } else {
            HIP_ABORT("gemv q4_K: SwiGLU launch with K=%d exceeds %d", ka.L.K, gemv_swiglu_max_k(TYPE));
        }
    } else {
        const int its = (ka.L.K / 32 + LPR - 1) / LPR;
        if (its <= 1) launch_gemv_its<TYPE, LPR, SWIGLU, 1>(ka, waves, st);
        else if (its <= 2) launch_gemv_its<TYPE, LPR, SWIGLU, 2>(ka, waves, st);
        else if (its <= 4) launch_gemv_its<TYPE, LPR, SWIGLU, 4>(ka, waves, st);
        else if (its <= 6) launch_gemv_its<TYPE, LPR, SWIGLU, 6>(ka, waves, st);
        else if (its <= 8) launch_gemv_its<TYPE, LPR, SWIGLU, 8>(ka, waves, st);
        else if constexpr (!SWIGLU) {
            if (its <= 12) launch_gemv_its<TYPE, LPR, SWIGLU, 12>(ka, waves, st);
            else if (its <= 16) launch_gemv_its<TYPE, LPR, SWIGLU, 16>(ka, waves, st);
            else HIP_ABORT("gemv: K=%d is too long", ka.L.K);
        } else if constexpr (TYPE == GGML_TYPE_Q4_0) {
            if (its <= 12) launch_gemv_its<TYPE, LPR, SWIGLU, 12>(ka, waves, st);
            else HIP_ABORT("gemv: SwiGLU launch with K=%d exceeds %d", ka.L.K, gemv_swiglu_max_k(TYPE));
        } else {
            HIP_ABORT("gemv: SwiGLU launch with K=%d exceeds %d", ka.L.K, gemv_swiglu_max_k(TYPE));
        }
    }
}

// Lanes per row for a single-chain Q4_0/Q8_0 launch of 4-wave workgroups: the fewest (longest
// register-resident run of blocks per lane) that still gives about two workgroups per CU, so short
// matrices (the o-projection, the down projection) spread over the whole chip.
template <int TYPE, bool SWIGLU>
static void launch_gemv_lanes(gemv_kargs & ka, hipStream_t st) {
    constexpr int WAVES = 4, TARGET_BLOCKS = 512;
    const int rows = ka.total_rows, K = ka.L.K;
    // workgroups of the launch: row blocks times the grid's columns (mul_mat_id: token x slot)
    const auto blocks = [&](int lpr) { return (rows + WAVES * (WAVE / lpr) - 1) / (WAVES * (WAVE / lpr)) * ka.L.ncols; };
    const int k16 = SWIGLU ? gemv_swiglu_max_k(TYPE) : 8192;     // longest K of 16 lanes per row
    if (K <= k16 && blocks(16) >= TARGET_BLOCKS) launch_gemv_t<TYPE, 16, SWIGLU>(ka, WAVES, st);
    else if (K <= 2 * k16 && blocks(32) >= TARGET_BLOCKS) launch_gemv_t<TYPE, 32, SWIGLU>(ka, WAVES, st);
    else launch_gemv_t<TYPE, 64, SWIGLU>(ka, WAVES, st);
}

// Lanes per row for Q4_K launches of 4-wave workgroups, as above: at most 4 units (256 weights)
// per lane when the rows still fill about two workgroups per CU. A SwiGLU launch uses at least 32
// lanes per row: its ordered sums put the 9 chains of each of the two matrices on a row's lanes.
template <bool SWIGLU>
static void launch_gemv_q4k_lanes(gemv_kargs & ka, hipStream_t st) {
    constexpr int WAVES = 4, TARGET_BLOCKS = 512;
    const int rows = ka.total_rows, units = ka.L.K / 64;
    const auto blocks = [&](int lpr) { return (rows + WAVES * (WAVE / lpr) - 1) / (WAVES * (WAVE / lpr)) * ka.L.ncols; };
    if constexpr (!SWIGLU) {
        if (units <= 16 * 4 && blocks(16) >= TARGET_BLOCKS) return launch_gemv_t<GGML_TYPE_Q4_K, 16, SWIGLU>(ka, WAVES, st);
    }
    if (units <= 32 * 4 && blocks(32) >= TARGET_BLOCKS) launch_gemv_t<GGML_TYPE_Q4_K, 32, SWIGLU>(ka, WAVES, st);
    else launch_gemv_t<GGML_TYPE_Q4_K, 64, SWIGLU>(ka, WAVES, st);
}

// Lanes per row for Q5_K / Q6_K launches of 4-wave workgroups: the fewest that keep a lane's units
// within kq_max_its and still give about two workgroups per CU (SwiGLU: at least 32, as for Q4_K)
template <int TYPE, bool SWIGLU>
static void launch_gemv_kq_lanes(gemv_kargs & ka, hipStream_t st) {
    constexpr int WAVES = 4, TARGET_BLOCKS = 512, MAXI = kq_max_its<TYPE, SWIGLU>();
    const int rows = ka.total_rows, units = ka.L.K / 64;
    const auto blocks = [&](int lpr) { return (rows + WAVES * (WAVE / lpr) - 1) / (WAVES * (WAVE / lpr)) * ka.L.ncols; };
    if constexpr (!SWIGLU) {
        if (units <= 16 * MAXI && blocks(16) >= TARGET_BLOCKS) return launch_gemv_t<TYPE, 16, SWIGLU>(ka, WAVES, st);
    }
    if (units <= 32 * MAXI && blocks(32) >= TARGET_BLOCKS) launch_gemv_t<TYPE, 32, SWIGLU>(ka, WAVES, st);
    else launch_gemv_t<TYPE, 64, SWIGLU>(ka, WAVES, st);
}

bool gemv_f64_input_supported(const gemv_launch & L) {
    if (L.swiglu || L.ids || L.ncols != 1 || L.out_q.qs) return false;
    if (L.type == GGML_TYPE_Q4_0 || L.type == GGML_TYPE_Q8_0) return gemv_q_supported(L) && L.K <= gemv_prologue_max_k(L.type, false);
    return is_kquant(L.type) && L.K % 256 == 0 && L.K <= act_quant_max_k(L.type, false);
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
    if (L.ids && (L.n_slots < 1 || L.x_cols < 1 || L.n_experts < 1 || L.ncols % L.n_slots)) HIP_ABORT("gemv: bad mul_mat_id geometry");
    if (L.norm.f64 && (!L.norm.x || L.norm.rms || L.swiglu || L.ids || L.norm.x_stride % 2 || !gemv_f64_input_supported(L)))
        HIP_ABORT("gemv: a double-valued column is quantized as is, for a plain Q4_0 / Q8_0 / K-quant launch");
    if (L.norm.x) {
        const int max_k = act_quant_max_k(L.type, L.norm.rms != 0);
        if (L.K > max_k) HIP_ABORT("gemv: the activation prologue handles K <= %d (K=%d)", max_k, L.K);
        if (((uintptr_t) L.norm.x | (uintptr_t) L.norm.w) % 16 || L.norm.x_stride % 4) HIP_ABORT("gemv: RMSNorm prologue operands must be 16-byte aligned");
    }
    if (L.route_logits) {
        // only the single-column Q4_K kernel routes inside the launch
        if (!gemv_q4k_supported(L)) HIP_ABORT("gemv: routing inside the launch unsupported for this launch");
        return launch_gemv_q4k(L, st);
    }
    if (gemv_q_supported(L)) return launch_gemv_q(L, st);
    if (gemv_q4k_enabled() && gemv_q4k_supported(L)) return launch_gemv_q4k(L, st);
    if (L.out_q.qs) HIP_ABORT("gemv: quantized SwiGLU output needs the Q4_0 / Q8_0 kernel");
    switch (L.type) {
        case GGML_TYPE_Q4_0:
            if (L.K % 32 || L.K > GEMV_MAX_K) HIP_ABORT("gemv q4_0: K=%d unsupported", L.K);
            if (L.swiglu) launch_gemv_lanes<GGML_TYPE_Q4_0, true>(ka, st);
            else launch_gemv_lanes<GGML_TYPE_Q4_0, false>(ka, st);
            break;
        case GGML_TYPE_Q8_0:
            if (L.K % 32 || L.K > GEMV_MAX_K) HIP_ABORT("gemv q8_0: K=%d unsupported", L.K);
            if (L.swiglu) launch_gemv_lanes<GGML_TYPE_Q8_0, true>(ka, st);
            else launch_gemv_lanes<GGML_TYPE_Q8_0, false>(ka, st);
            break;
        case GGML_TYPE_Q4_K:
            if (L.K % 256 || L.K / 64 > 640) HIP_ABORT("gemv q4_K: K=%d unsupported", L.K);
            if (L.swiglu) launch_gemv_q4k_lanes<true>(ka, st);
            else launch_gemv_q4k_lanes<false>(ka, st);
            break;
        case GGML_TYPE_Q5_K:
            if (L.K % 256 || L.K / 64 > 64 * kq_max_its<GGML_TYPE_Q5_K, false>()) HIP_ABORT("gemv q5_K: K=%d unsupported", L.K);
            if (L.swiglu) launch_gemv_kq_lanes<GGML_TYPE_Q5_K, true>(ka, st);
            else launch_gemv_kq_lanes<GGML_TYPE_Q5_K, false>(ka, st);
            break;
        case GGML_TYPE_Q6_K:
            if (L.K % 256 || L.K / 64 > 64 * kq_max_its<GGML_TYPE_Q6_K, false>()) HIP_ABORT("gemv q6_K: K=%d unsupported", L.K);
            if (L.swiglu) launch_gemv_kq_lanes<GGML_TYPE_Q6_K, true>(ka, st);
            else launch_gemv_kq_lanes<GGML_TYPE_Q6_K, false>(ka, st);
            break;
        default:
            HIP_ABORT("gemv: unsupported weight type %d", L.type);
    }
}
