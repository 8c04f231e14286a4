// k_gemm.hip — the prefill GEMM: Q4_0 / Q8_0 weights times Q8_0-quantized activation columns on
// the matrix cores.
//
// ggml-cpu computes every output of a quantized mul_mat as a float sum over the weight row's
// 32-element blocks, in block order, of an exact integer block dot scaled by the two fp16 block
// scales: Q8_0 sumf += sumi * (d_w * d_x), Q4_0 sumf += (sumi * d_w) * d_x. The integer quants are
// staged as int8 (Q4_0 nibbles as nibble - 8), so one v_mfma_i32_16x16x32_i8 yields the exact
// block dots of a tile of 16 weight rows x 16 activation columns, and the kernel adds the scaled
// terms (the block dot converted to float, exactly: it is below 2^24 in magnitude) to f32
// accumulators in block order: every output is the same float as the GEMV's and the CPU
// reference's. The per-term float work (a conversion, two multiplies, one add) runs on the VALU
// and bounds the kernel, not the MFMA rate.
//
// Tiling: a workgroup is 2 x 2 waves; a wave owns WTM x WTN MFMA tiles. Each pipeline stage moves
// KB blocks of the workgroup's weight rows and activation columns from global memory (16-byte
// loads, consecutive threads on consecutive bytes) into LDS as int8 rows (Q4_0 unpacked on the
// way) and the fp16 weight scales as floats; the next stage's loads are in flight while the
// current stage is reduced, with one barrier per stage. In a tile, lane l reads weight row l%16
// and activation column l%16, k-slice 8(l/16)..8(l/16)+7 of the block (one 8-byte LDS read each;
// rows are 8 bytes longer than their blocks, so the 16 rows of a read fall on distinct banks), and
// receives the results of rows 4(l/16)..4(l/16)+3 of column l%16. Workgroups are numbered so that
// the column tiles of one row tile run on one XCD and share its L2.
//
// Q4_K, Q5_K and Q6_K weights run on gemm_k_kernel (below) against Q8_K activation columns.
#include "kernels.h"
#include "gemv_ops.h"

#include "ggml.h"

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef int i32x4 __attribute__((ext_vector_type(4)));

namespace {

// 4 int8 (one dword) -> 4 f16 in two dwords: bytes biased by 128 are placed under the f16 exponent
// of 1024 (0x64xx = 1024 + byte), then 1152 is subtracted, both exact
__device__ __forceinline__ void i8x4_to_f16(uint32_t v, uint32_t & lo, uint32_t & hi) {
    const uint32_t u = v ^ 0x80808080u;
    lo = __builtin_amdgcn_perm(0x64646464u, u, 0x04010400u);
    hi = __builtin_amdgcn_perm(0x64646464u, u, 0x04030402u);
    const __half2 bias = __halves2half2(__ushort_as_half(0xE480), __ushort_as_half(0xE480));   // -1152
    lo = __builtin_bit_cast(uint32_t, __hadd2(__builtin_bit_cast(__half2, lo), bias));
    hi = __builtin_bit_cast(uint32_t, __hadd2(__builtin_bit_cast(__half2, hi), bias));
}

// one Q4_0 block's 16 bytes -> its 32 weights as int8 of value nibble - 8 (low nibbles are elements
// 0-15, high 16-31), 8 bytes per store: per byte n in 0..15, ((n | 0x80) - 8) ^ 0x80 = n - 8 with no
// borrow between bytes
__device__ __forceinline__ void store_q4x32_i8(int8_t * dst, const uint4 & a) {
    const uint32_t w[4] = { a.x, a.y, a.z, a.w };
    uint32_t lo[4], hi[4];
#pragma unroll
    for (int k = 0; k < 4; k++) {
        lo[k] = (((w[k] & 0x0F0F0F0Fu) | 0x80808080u) - 0x08080808u) ^ 0x80808080u;
        hi[k] = ((((w[k] >> 4) & 0x0F0F0F0Fu) | 0x80808080u) - 0x08080808u) ^ 0x80808080u;
    }
    uint2 * d = (uint2 *) dst;
    d[0] = make_uint2(lo[0], lo[1]); d[1] = make_uint2(lo[2], lo[3]);
    d[2] = make_uint2(hi[0], hi[1]); d[3] = make_uint2(hi[2], hi[3]);
}

// 32 int8 (two 16-byte loads) to an 8-byte aligned LDS row
__device__ __forceinline__ void store_i8x32_raw(int8_t * dst, const uint4 & a, const uint4 & b) {
    uint2 * d = (uint2 *) dst;
    d[0] = make_uint2(a.x, a.y); d[1] = make_uint2(a.z, a.w);
    d[2] = make_uint2(b.x, b.y); d[3] = make_uint2(b.z, b.w);
}

template <int TYPE, int WTM, int WTN, int KB>
struct gemm_cfg {
    static constexpr int QB = TYPE == GGML_TYPE_Q4_0 ? Q4_0_QS : Q8_0_QS;
    static constexpr int BM = 32 * WTM, BN = 32 * WTN;
    static constexpr int ROW = KB * 32 + 8;                               // int8 per LDS row (8-byte pad)
    static constexpr int UA = (BM * KB + 255) / 256, UB = (BN * KB + 255) / 256;   // staged blocks per thread
    static constexpr int A_BYTES = BM * ROW, B_BYTES = BN * ROW;
    static constexpr size_t LDS = 2 * ((size_t) (A_BYTES + B_BYTES) + (size_t) KB * (BM + BN) * 4);
};

template <int TYPE, int WTM, int WTN, int KB>
__global__ __launch_bounds__(256, WTM == 1 ? 4 : 1) void gemm_q_kernel(const gemm_launch G) {
    prefetch_kernargs<sizeof(gemm_launch)>();
    using C = gemm_cfg<TYPE, WTM, WTN, KB>;
    constexpr int QB = C::QB, BM = C::BM, BN = C::BN, ROW = C::ROW;
    extern __shared__ __align__(16) uint8_t g_lds[];
    int8_t * sA = (int8_t *) g_lds;                           // [2][BM][ROW]
    int8_t * sB = sA + 2 * C::A_BYTES;                        // [2][BN][ROW]
    float * sdw = (float *) (sB + 2 * C::B_BYTES);            // [2][KB][BM]
    float * sdx = sdw + 2 * KB * BM;                          // [2][KB][BN]

    const int64_t M = G.n_rows, N = G.ncols, K = G.K, nb = K / 32;
    const int tid = threadIdx.x, lane = tid % WAVE, wave = tid / WAVE;
    const int q = lane / 16, c = lane % 16;

    const int64_t n_ct = (N + BN - 1) / BN, tiles = ((M + BM - 1) / BM) * n_ct;
    int64_t t = blockIdx.x;
    if (tiles % 8 == 0) t = (int64_t) (blockIdx.x % 8) * (tiles / 8) + blockIdx.x / 8;
    const int64_t m0 = (t / n_ct) * BM, n0 = (t % n_ct) * BN;
    const int wr = (wave / 2) * 16 * WTM, wc = (wave % 2) * 16 * WTN;   // wave's tile origin in the workgroup tile

    // staging: unit u = (row or column, block of the stage); rows / columns past the end repeat the last one
    uint4 ra[C::UA][2], rb[C::UB][2];
    __half rd[C::UA];
    float rx[C::UB];
    auto load = [&](int64_t b0) {
#pragma unroll
        for (int k = 0; k < C::UA; k++) {
            const int u = tid + 256 * k;
            if (u < BM * KB) {
                const int64_t row = min(m0 + u / KB, M - 1);
                const int64_t blk = row * nb + b0 + u % KB;
                const uint4 * p = (const uint4 *) (G.w + blk * QB);
                ra[k][0] = p[0];
                if constexpr (QB == 32) ra[k][1] = p[1];
                rd[k] = G.wd[blk];
            }
        }
#pragma unroll
        for (int k = 0; k < C::UB; k++) {
            const int u = tid + 256 * k;
            if (u < BN * KB) {
                const int64_t col = min(n0 + u / KB, N - 1);
                const uint4 * p = (const uint4 *) (G.xq + col * K + (b0 + u % KB) * 32);
                rb[k][0] = p[0];
                rb[k][1] = p[1];
                rx[k] = G.xd[col * nb + b0 + u % KB];
            }
        }
    };
    auto store = [&](int buf) {
#pragma unroll
        for (int k = 0; k < C::UA; k++) {
            const int u = tid + 256 * k;
            if (u < BM * KB) {
                const int r = u / KB, kb = u % KB;
                int8_t * dst = sA + buf * C::A_BYTES + r * ROW + kb * 32;
                if constexpr (QB == 32) store_i8x32_raw(dst, ra[k][0], ra[k][1]);
                else store_q4x32_i8(dst, ra[k][0]);
                sdw[(buf * KB + kb) * BM + r] = __half2float(rd[k]);
            }
        }
#pragma unroll
        for (int k = 0; k < C::UB; k++) {
            const int u = tid + 256 * k;
            if (u < BN * KB) {
                const int cc = u / KB, kb = u % KB;
                store_i8x32_raw(sB + buf * C::B_BYTES + cc * ROW + kb * 32, rb[k][0], rb[k][1]);
                sdx[(buf * KB + kb) * BN + cc] = rx[k];
            }
        }
    };

    float acc[WTM][WTN][4];
#pragma unroll
    for (int i = 0; i < WTM; i++)
#pragma unroll
        for (int j = 0; j < WTN; j++)
#pragma unroll
            for (int r = 0; r < 4; r++) acc[i][j][r] = 0.0f;

    // Stage s's loads are issued before stage s - 1's dots and stored to LDS at the top of
    // iteration s, so the previous stage's MFMAs and epilogue cover their latency (stored at the end
    // of the iteration, the compiler would move the stores and their wait ahead of the epilogue).
    // One barrier per stage: a stage's stores go to the buffer that the stage before last read, and
    // every wave passed the last barrier after that.
    const int64_t n_stages = nb / KB;
    load(0);
    for (int64_t s = 0; s < n_stages; s++) {
        const int buf = (int) (s & 1);
        store(buf);
        __syncthreads();
        if (s + 1 < n_stages) load((s + 1) * KB);
        const int8_t * A = sA + buf * C::A_BYTES;
        const int8_t * B = sB + buf * C::B_BYTES;
#pragma unroll
        for (int kb = 0; kb < KB; kb++) {
            long a[WTM], b[WTN];
            f32x4 dw[WTM];
            float dx[WTN];
#pragma unroll
            for (int i = 0; i < WTM; i++) {
                a[i] = *(const long *) (A + (wr + 16 * i + c) * ROW + kb * 32 + 8 * q);
                dw[i] = *(const f32x4 *) (sdw + (buf * KB + kb) * BM + wr + 16 * i + 4 * q);
            }
#pragma unroll
            for (int j = 0; j < WTN; j++) {
                b[j] = *(const long *) (B + (wc + 16 * j + c) * ROW + kb * 32 + 8 * q);
                dx[j] = sdx[(buf * KB + kb) * BN + wc + 16 * j + c];
            }
#pragma unroll
            for (int i = 0; i < WTM; i++)
#pragma unroll
                for (int j = 0; j < WTN; j++) {
                    const i32x4 si = __builtin_amdgcn_mfma_i32_16x16x32_i8(a[i], b[j], i32x4{ 0, 0, 0, 0 }, 0, 0, 0);
#pragma unroll
                    for (int r = 0; r < 4; r++) {
                        const float sv = (float) si[r];
                        if constexpr (TYPE == GGML_TYPE_Q8_0) {
                            const float dd = dw[i][r] * dx[j];
                            acc[i][j][r] += sv * dd;
                        } else {
                            acc[i][j][r] += (sv * dw[i][r]) * dx[j];
                        }
                    }
                }
        }
    }

#pragma unroll
    for (int j = 0; j < WTN; j++) {
        const int64_t col = n0 + wc + 16 * j + c;
        if (col >= N) continue;
#pragma unroll
        for (int i = 0; i < WTM; i++) {
            const int64_t r0 = m0 + wr + 16 * i + 4 * q;
            if (r0 >= M) continue;
            float v[4] = { acc[i][j][0], acc[i][j][1], acc[i][j][2], acc[i][j][3] };
            if (G.add) {
                const float * ap = G.add + col * G.add_stride + r0;
                for (int r = 0; r < 4; r++) if (r0 + r < M) v[r] = v[r] + ap[r];
            }
            float * yp = G.y + col * G.y_stride + r0;
            if (r0 + 3 < M) {
                *(float4 *) yp = make_float4(v[0], v[1], v[2], v[3]);
            } else {
                for (int r = 0; r < 4; r++) if (r0 + r < M) yp[r] = v[r];
            }
        }
    }
}

// ---------------------------------------------------------------------------------------------
// K-quants x Q8_K. ggml-cpu's generic q4_K / q5_K / q6_K x q8_K dots (ggml-cpu/arch-fallback: the
// oracle's oracle_vec_dot_q{4,5,6}_K_q8_K) keep eight float accumulators per output, one per
// element index mod 8: for every 256-element super-block, aux32[l] = sum over the 32 elements
// e = 8k + l of sc[sub-block of e] * q[e] * q8[e] (an exact integer), sums[l] += (d_w * d_x) *
// aux32[l]; Q4_K and Q5_K subtract their mins as sumf -= (dmin_w * d_x) * sum_j bsums[j] * m[j / 2];
// the output is sumf + sums[0] + ... + sums[7].
// Staged in LDS as f16 in the order p = 32 l + k, each l-slice of a super-block is one contiguous
// 32-element run, so one v_mfma_f32_16x16x32_f16 per slice yields aux32[l] for a 16 x 16 tile: the
// weight operand is sc * q, exact in f16 for Q4_K (at most 63 * 15 = 945) and Q5_K (63 * 31 =
// 1953), and every product and partial sum is an integer of magnitude at most 2^24. Q6_K's
// sc * (q - 32) reaches 4096 in magnitude, and above 2048 f16 holds only even integers: it is
// staged as two f16 parts, hi = sc * (q - 32) rounded to f16 and lo = the remainder (-1, 0 or 1,
// exact from one fused multiply-add), and aux32[l] = mfma(hi) + mfma(lo): two exact integers whose
// sum, aux32[l] itself, is at most 32 * 4096 * 127 < 2^24. The mins term is one
// v_mfma_f32_16x16x16_f16 of the mins (each repeated for its two 16-element halves) against the 16
// bsums (|bsum| <= 16 * 127, exact in f16). Per output the kernel holds the 9 accumulators in
// registers and adds them in ggml's order, so every output is the GEMV's and the CPU reference's
// float. A stage is one super-block of the workgroup's rows and columns; the next stage's global
// loads are in flight while the current one is reduced.

// 4 nibbles (0..15 in the byte lanes of n) -> 4 f16 of value nibble * sc, exact
__device__ __forceinline__ void u4x4_scaled(uint32_t n, __half2 sc, uint32_t & lo, uint32_t & hi) {
    lo = __builtin_amdgcn_perm(0x64646464u, n, 0x04010400u);
    hi = __builtin_amdgcn_perm(0x64646464u, n, 0x04030402u);
    const __half2 bias = __halves2half2(__ushort_as_half(0xE400), __ushort_as_half(0xE400));   // -1024
    lo = __builtin_bit_cast(uint32_t, __hmul2(__hadd2(__builtin_bit_cast(__half2, lo), bias), sc));
    hi = __builtin_bit_cast(uint32_t, __hmul2(__hadd2(__builtin_bit_cast(__half2, hi), bias), sc));
}

// 4 biased 6-bit quants (q in 0..63 in the byte lanes of n) times the scales sa (lanes 0, 1) and sb
// (lanes 2, 3) as two f16 parts: hi = sc * (q - 32) rounded to f16, lo = sc * (q - 32) - hi exactly
// (one fused multiply-add; -1, 0 or 1)
__device__ __forceinline__ void q6x4_split(uint32_t n, __half2 sa, __half2 sb, uint32_t & h0, uint32_t & h1,
                                           uint32_t & l0, uint32_t & l1) {
    const __half2 bias = __halves2half2(__ushort_as_half(0xE420), __ushort_as_half(0xE420));   // -1056
    const __half2 qa = __hadd2(__builtin_bit_cast(__half2, __builtin_amdgcn_perm(0x64646464u, n, 0x04010400u)), bias);
    const __half2 qb = __hadd2(__builtin_bit_cast(__half2, __builtin_amdgcn_perm(0x64646464u, n, 0x04030402u)), bias);
    const __half2 ha = __hmul2(qa, sa), hb = __hmul2(qb, sb);
    h0 = __builtin_bit_cast(uint32_t, ha);
    h1 = __builtin_bit_cast(uint32_t, hb);
    l0 = __builtin_bit_cast(uint32_t, __hfma2(qa, sa, __hneg2(ha)));
    l1 = __builtin_bit_cast(uint32_t, __hfma2(qb, sb, __hneg2(hb)));
}

// int8 byte b of v as an f16 pair (exact)
__device__ __forceinline__ __half2 sbyte_h2(uint32_t v, int b) {
    const __half h = __short2half_rn((short) (int8_t) (v >> (8 * b)));
    return __halves2half2(h, h);
}

typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));

template <int TYPE, int WTM, int WTN>
struct gemm_k_cfg {
    static constexpr bool Q6 = TYPE == GGML_TYPE_Q6_K;
    static constexpr bool MINS = !Q6;
    static constexpr int BLK = TYPE == GGML_TYPE_Q4_K ? 144 : 176;        // Q4_K / Q5_K block bytes (GGUF layout)
    static constexpr int BM = 32 * WTM, BN = 32 * WTN;
    static constexpr int ROW = 256 + 8;                                    // f16 per LDS row (16-byte pad)
    static constexpr int UPR = Q6 ? 2 : 4;                                 // staging units per weight row and super-block
    static constexpr int UA = (BM * UPR + 255) / 256, UB = (BN * 4 + 255) / 256;
    static constexpr int A_PARTS = Q6 ? 2 : 1;
    static constexpr size_t LDS = (size_t) (A_PARTS * BM + BN) * ROW * 2 + (MINS ? (size_t) (BM + BN) * 16 * 2 : 0) +
                                  (size_t) ((MINS ? 2 : 1) * BM + BN) * 4;
};

template <int TYPE, int WTM, int WTN>
__global__ __launch_bounds__(256, 2) void gemm_k_kernel(const gemm_launch G) {
    prefetch_kernargs<sizeof(gemm_launch)>();
    using C = gemm_k_cfg<TYPE, WTM, WTN>;
    constexpr bool Q6 = C::Q6, MINS = C::MINS;
    constexpr int BM = C::BM, BN = C::BN, ROW = C::ROW, UPR = C::UPR;
    extern __shared__ __align__(16) uint8_t g_lds[];
    _Float16 * sA = (_Float16 *) g_lds;                     // [BM][ROW]: sc * q of the super-block (Q6_K: hi), slice-major
    _Float16 * sL = sA + BM * ROW;                          // Q6_K [BM][ROW]: lo
    _Float16 * sB = sL + (Q6 ? BM * ROW : 0);               // [BN][ROW]: q8, same order
    _Float16 * sM = sB + BN * ROW;                          // Q4_K / Q5_K [BM][16]: the min of 16-element group j (m[j / 2])
    _Float16 * sS = sM + (MINS ? BM * 16 : 0);              // Q4_K / Q5_K [BN][16]: bsums
    float * sdw = (float *) (sS + (MINS ? BN * 16 : 0));    // [BM] d
    float * sdm = sdw + BM;                                 // Q4_K / Q5_K [BM] dmin
    float * sdx = sdm + (MINS ? BM : 0);                    // [BN] activation d

    const int64_t M = G.n_rows, N = G.ncols, K = G.K, nsb = K / 256;
    const int tid = threadIdx.x, lane = tid % WAVE, wave = tid / WAVE;
    const int q = lane / 16, c = lane % 16;

    const int64_t n_ct = (N + BN - 1) / BN, tiles = ((M + BM - 1) / BM) * n_ct;
    int64_t t = blockIdx.x;
    if (tiles % 8 == 0) t = (int64_t) (blockIdx.x % 8) * (tiles / 8) + blockIdx.x / 8;
    const int64_t m0 = (t / n_ct) * BM, n0 = (t % n_ct) * BN;
    const int wr = (wave / 2) * 16 * WTM, wc = (wave % 2) * 16 * WTN;

    // staging units: weights u = (row u / UPR, sub-block pair u % 4 | Q6_K: 128-element half u % 2),
    // activations u = (column u / 4, sub-block pair u % 4); rows / columns past the end repeat the
    // last one
    uint4 rh[C::UA], rq[C::UA][Q6 ? 4 : 2], rqh[C::UA][2], rx[C::UB][4];
    uint2 rsc[C::UA], rs[C::UB];
    __half rdq[C::UA];
    float rd[C::UB];
    auto load = [&](int64_t sb) {
#pragma unroll
        for (int k = 0; k < C::UA; k++) {
            const int u = tid + 256 * k;
            if (u < BM * UPR) {
                const int64_t row = min(m0 + u / UPR, M - 1);
                const int64_t blk = row * nsb + sb;
                const int p = u % UPR;
                if constexpr (Q6) {
                    // planes: low bits [blocks][128], high bits [blocks][64], scales [blocks][16], d
                    const uint4 * ql = (const uint4 *) (G.w + blk * 128 + 64 * p);
                    const uint4 * qh = (const uint4 *) (G.wqh + blk * 64 + 32 * p);
#pragma unroll
                    for (int v = 0; v < 4; v++) rq[k][v] = ql[v];
                    rqh[k][0] = qh[0];
                    rqh[k][1] = qh[1];
                    rsc[k] = *(const uint2 *) (G.wsc + blk * 16 + 8 * p);
                    rdq[k] = G.wd[blk];
                } else {
                    const uint4 * b = (const uint4 *) (G.w + blk * C::BLK);
                    rh[k] = b[0];
                    if constexpr (TYPE == GGML_TYPE_Q5_K) {
                        // d, dmin, scales | qh[32] | qs[128]
                        rqh[k][0] = b[1];
                        rqh[k][1] = b[2];
                        rq[k][0] = b[3 + 2 * p];
                        rq[k][1] = b[4 + 2 * p];
                    } else {
                        rq[k][0] = b[1 + 2 * p];
                        rq[k][1] = b[2 + 2 * p];
                    }
                }
            }
        }
#pragma unroll
        for (int k = 0; k < C::UB; k++) {
            const int u = tid + 256 * k;
            if (u < BN * 4) {
                const int64_t col = min(n0 + u / 4, N - 1);
                const uint4 * p = (const uint4 *) (G.xq + col * K + sb * 256 + 64 * (u % 4));
#pragma unroll
                for (int v = 0; v < 4; v++) rx[k][v] = p[v];
                if constexpr (MINS) rs[k] = *(const uint2 *) (G.xbs + col * (K / 16) + sb * 16 + 4 * (u % 4));
                rd[k] = G.xd[col * nsb + sb];
            }
        }
    };
    auto store = [&]() {
#pragma unroll
        for (int k = 0; k < C::UA; k++) {
            const int u = tid + 256 * k;
            if (u < BM * UPR) {
                const int r = u / UPR, p = u % UPR;
                if constexpr (Q6) {
                    // half p: ql bytes 0-31 (a) and 32-63 (b), qh bytes 0-31; element 128 p + 32 m + j
                    // for byte j takes nibble m / 2 of a (m even) or b (m odd) and qh bits 2m, 2m + 1,
                    // and scale 8 p + 2 m + j / 16. Grouped by l, dword l holds bytes j = l + 8 t
                    // (t = 0..3): elements k = 16 p + 4 m + t of slice l, scales 2 m (t < 2), 2 m + 1.
                    uint32_t a[8] = { rq[k][0].x, rq[k][0].y, rq[k][0].z, rq[k][0].w, rq[k][1].x, rq[k][1].y, rq[k][1].z, rq[k][1].w };
                    uint32_t b[8] = { rq[k][2].x, rq[k][2].y, rq[k][2].z, rq[k][2].w, rq[k][3].x, rq[k][3].y, rq[k][3].z, rq[k][3].w };
                    uint32_t h[8] = { rqh[k][0].x, rqh[k][0].y, rqh[k][0].z, rqh[k][0].w, rqh[k][1].x, rqh[k][1].y, rqh[k][1].z, rqh[k][1].w };
                    q4k_group_by_l(a);
                    q4k_group_by_l(b);
                    q4k_group_by_l(h);
                    __half2 sc[8];
#pragma unroll
                    for (int g = 0; g < 8; g++) sc[g] = sbyte_h2(g < 4 ? rsc[k].x : rsc[k].y, g % 4);
#pragma unroll
                    for (int l = 0; l < 8; l++) {
                        const uint32_t v[4] = {
                            (a[l] & 0x0F0F0F0Fu) | ((h[l] & 0x03030303u) << 4),
                            (b[l] & 0x0F0F0F0Fu) | (((h[l] >> 2) & 0x03030303u) << 4),
                            ((a[l] >> 4) & 0x0F0F0F0Fu) | (((h[l] >> 4) & 0x03030303u) << 4),
                            ((b[l] >> 4) & 0x0F0F0F0Fu) | (((h[l] >> 6) & 0x03030303u) << 4),
                        };
                        uint32_t hi[8], lo[8];
#pragma unroll
                        for (int m = 0; m < 4; m++) q6x4_split(v[m], sc[2 * m], sc[2 * m + 1], hi[2 * m], hi[2 * m + 1], lo[2 * m], lo[2 * m + 1]);
                        uint4 * dh = (uint4 *) (sA + r * ROW + l * 32 + 16 * p);
                        uint4 * dl = (uint4 *) (sL + r * ROW + l * 32 + 16 * p);
                        dh[0] = make_uint4(hi[0], hi[1], hi[2], hi[3]);
                        dh[1] = make_uint4(hi[4], hi[5], hi[6], hi[7]);
                        dl[0] = make_uint4(lo[0], lo[1], lo[2], lo[3]);
                        dl[1] = make_uint4(lo[4], lo[5], lo[6], lo[7]);
                    }
                    if (p == 0) sdw[r] = __half2float(rdq[k]);
                } else {
                    int sca, ma, scb, mb;
                    q4k_sc_m(rh[k].y, rh[k].z, rh[k].w, 2 * p, sca, ma);
                    q4k_sc_m(rh[k].y, rh[k].z, rh[k].w, 2 * p + 1, scb, mb);
                    uint32_t w[8] = { rq[k][0].x, rq[k][0].y, rq[k][0].z, rq[k][0].w, rq[k][1].x, rq[k][1].y, rq[k][1].z, rq[k][1].w };
                    q4k_group_by_l(w);      // dword l: the pair's bytes l, l+8, l+16, l+24
                    uint32_t h[8];
                    if constexpr (TYPE == GGML_TYPE_Q5_K) {
                        // the fifth bit of byte j's low nibble is bit 2 p of qh[j], of its high nibble bit 2 p + 1
                        h[0] = rqh[k][0].x; h[1] = rqh[k][0].y; h[2] = rqh[k][0].z; h[3] = rqh[k][0].w;
                        h[4] = rqh[k][1].x; h[5] = rqh[k][1].y; h[6] = rqh[k][1].z; h[7] = rqh[k][1].w;
                        q4k_group_by_l(h);
                    }
                    const __half2 ha = __float2half2_rn((float) sca), hb = __float2half2_rn((float) scb);
#pragma unroll
                    for (int l = 0; l < 8; l++) {
                        // k = 8p + 0..3: sub-block 2p (low nibbles); k = 8p + 4..7: sub-block 2p + 1
                        uint32_t nl = w[l] & 0x0F0F0F0Fu, nh = (w[l] >> 4) & 0x0F0F0F0Fu;
                        if constexpr (TYPE == GGML_TYPE_Q5_K) {
                            nl |= ((h[l] >> (2 * p)) & 0x01010101u) << 4;
                            nh |= ((h[l] >> (2 * p + 1)) & 0x01010101u) << 4;
                        }
                        uint32_t l0, h0, l1, h1;
                        u4x4_scaled(nl, ha, l0, h0);
                        u4x4_scaled(nh, hb, l1, h1);
                        *(uint4 *) (sA + r * ROW + l * 32 + 8 * p) = make_uint4(l0, h0, l1, h1);
                    }
                    const __half2 mma = __float2half2_rn((float) ma), mmb = __float2half2_rn((float) mb);
                    *(uint2 *) (sM + r * 16 + 4 * p) = make_uint2(__builtin_bit_cast(uint32_t, mma), __builtin_bit_cast(uint32_t, mmb));
                    if (p == 0) {
                        sdw[r] = __half2float(__ushort_as_half((unsigned short) (rh[k].x & 0xffff)));
                        sdm[r] = __half2float(__ushort_as_half((unsigned short) (rh[k].x >> 16)));
                    }
                }
            }
        }
#pragma unroll
        for (int k = 0; k < C::UB; k++) {
            const int u = tid + 256 * k;
            if (u < BN * 4) {
                const int cc = u / 4, p = u % 4;
                const uint32_t v[16] = { rx[k][0].x, rx[k][0].y, rx[k][0].z, rx[k][0].w, rx[k][1].x, rx[k][1].y, rx[k][1].z, rx[k][1].w,
                                         rx[k][2].x, rx[k][2].y, rx[k][2].z, rx[k][2].w, rx[k][3].x, rx[k][3].y, rx[k][3].z, rx[k][3].w };
                // element l + 8 t of the pair's 64 sits in dword 2 t + l / 4, byte l % 4
                uint32_t ta[4], tb[4], tc[4], td[4];
                transpose4(v[0], v[2], v[4], v[6], ta);       // l = 0..3, t = 0..3
                transpose4(v[8], v[10], v[12], v[14], tb);    // l = 0..3, t = 4..7
                transpose4(v[1], v[3], v[5], v[7], tc);       // l = 4..7, t = 0..3
                transpose4(v[9], v[11], v[13], v[15], td);    // l = 4..7, t = 4..7
#pragma unroll
                for (int l = 0; l < 8; l++) {
                    uint32_t a0, a1, b0, b1;
                    i8x4_to_f16(l < 4 ? ta[l] : tc[l - 4], a0, a1);
                    i8x4_to_f16(l < 4 ? tb[l] : td[l - 4], b0, b1);
                    *(uint4 *) (sB + cc * ROW + l * 32 + 8 * p) = make_uint4(a0, a1, b0, b1);
                }
                if constexpr (MINS) {
                    const __half2 s01 = __halves2half2(__short2half_rn((short) (rs[k].x & 0xffff)), __short2half_rn((short) (rs[k].x >> 16)));
                    const __half2 s23 = __halves2half2(__short2half_rn((short) (rs[k].y & 0xffff)), __short2half_rn((short) (rs[k].y >> 16)));
                    *(uint2 *) (sS + cc * 16 + 4 * p) = make_uint2(__builtin_bit_cast(uint32_t, s01), __builtin_bit_cast(uint32_t, s23));
                }
                if (p == 0) sdx[cc] = rd[k];
            }
        }
    };

    float sums[WTM][WTN][8][4], mins[WTM][WTN][4];
#pragma unroll
    for (int i = 0; i < WTM; i++)
#pragma unroll
        for (int j = 0; j < WTN; j++)
#pragma unroll
            for (int r = 0; r < 4; r++) {
                mins[i][j][r] = 0.0f;
#pragma unroll
                for (int l = 0; l < 8; l++) sums[i][j][l][r] = 0.0f;
            }

    load(0);
    for (int64_t sb = 0; sb < nsb; sb++) {
        store();
        __syncthreads();
        if (sb + 1 < nsb) load(sb + 1);

        float dd[WTM][WTN][4];
        {
            f32x4 dw[WTM], dm[WTM];
            float dx[WTN];
#pragma unroll
            for (int i = 0; i < WTM; i++) {
                dw[i] = *(const f32x4 *) (sdw + wr + 16 * i + 4 * q);
                if constexpr (MINS) dm[i] = *(const f32x4 *) (sdm + wr + 16 * i + 4 * q);
            }
#pragma unroll
            for (int j = 0; j < WTN; j++) dx[j] = sdx[wc + 16 * j + c];
#pragma unroll
            for (int i = 0; i < WTM; i++)
#pragma unroll
                for (int j = 0; j < WTN; j++)
#pragma unroll
                    for (int r = 0; r < 4; r++) dd[i][j][r] = dw[i][r] * dx[j];
            if constexpr (MINS) {
                f16x4 am[WTM], bm[WTN];
#pragma unroll
                for (int i = 0; i < WTM; i++) am[i] = *(const f16x4 *) (sM + (wr + 16 * i + c) * 16 + 4 * q);
#pragma unroll
                for (int j = 0; j < WTN; j++) bm[j] = *(const f16x4 *) (sS + (wc + 16 * j + c) * 16 + 4 * q);
#pragma unroll
                for (int i = 0; i < WTM; i++)
#pragma unroll
                    for (int j = 0; j < WTN; j++) {
                        const f32x4 mv = __builtin_amdgcn_mfma_f32_16x16x16f16(am[i], bm[j], f32x4{ 0.0f, 0.0f, 0.0f, 0.0f }, 0, 0, 0);
#pragma unroll
                        for (int r = 0; r < 4; r++) {
                            const float dmin = dm[i][r] * dx[j];
                            mins[i][j][r] = mins[i][j][r] - dmin * mv[r];
                        }
                    }
            }
        }
#pragma unroll
        for (int l = 0; l < 8; l++) {
            f16x8 a[WTM], al[WTM], b[WTN];
#pragma unroll
            for (int i = 0; i < WTM; i++) {
                a[i] = *(const f16x8 *) (sA + (wr + 16 * i + c) * ROW + l * 32 + 8 * q);
                if constexpr (Q6) al[i] = *(const f16x8 *) (sL + (wr + 16 * i + c) * ROW + l * 32 + 8 * q);
            }
#pragma unroll
            for (int j = 0; j < WTN; j++) b[j] = *(const f16x8 *) (sB + (wc + 16 * j + c) * ROW + l * 32 + 8 * q);
#pragma unroll
            for (int i = 0; i < WTM; i++)
#pragma unroll
                for (int j = 0; j < WTN; j++) {
                    f32x4 sv = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[i], b[j], f32x4{ 0.0f, 0.0f, 0.0f, 0.0f }, 0, 0, 0);
                    if constexpr (Q6) {
                        const f32x4 sl = __builtin_amdgcn_mfma_f32_16x16x32_f16(al[i], b[j], f32x4{ 0.0f, 0.0f, 0.0f, 0.0f }, 0, 0, 0);
#pragma unroll
                        for (int r = 0; r < 4; r++) sv[r] = sv[r] + sl[r];
                    }
#pragma unroll
                    for (int r = 0; r < 4; r++) sums[i][j][l][r] = sums[i][j][l][r] + dd[i][j][r] * sv[r];
                }
        }
        __syncthreads();
    }

#pragma unroll
    for (int j = 0; j < WTN; j++) {
        const int64_t col = n0 + wc + 16 * j + c;
        if (col >= N) continue;
#pragma unroll
        for (int i = 0; i < WTM; i++) {
            const int64_t r0 = m0 + wr + 16 * i + 4 * q;
            if (r0 >= M) continue;
            float v[4];
#pragma unroll
            for (int r = 0; r < 4; r++) {
                float acc = mins[i][j][r];
#pragma unroll
                for (int l = 0; l < 8; l++) acc = acc + sums[i][j][l][r];
                v[r] = acc;
            }
            if (G.add) {
                const float * ap = G.add + col * G.add_stride + r0;
                for (int r = 0; r < 4; r++) if (r0 + r < M) v[r] = v[r] + ap[r];
            }
            float * yp = G.y + col * G.y_stride + r0;
            if (r0 + 3 < M) {
                *(float4 *) yp = make_float4(v[0], v[1], v[2], v[3]);
            } else {
                for (int r = 0; r < 4; r++) if (r0 + r < M) yp[r] = v[r];
            }
        }
    }
}

template <int TYPE, int WTM, int WTN>
void launch_gemm_k_t(const gemm_launch & G, hipStream_t st) {
    using C = gemm_k_cfg<TYPE, WTM, WTN>;
    static bool attr = false;
    if (!attr && C::LDS > 65536) {
        HIP_CHECK(hipFuncSetAttribute((const void *) gemm_k_kernel<TYPE, WTM, WTN>,
                                      hipFuncAttributeMaxDynamicSharedMemorySize, (int) C::LDS));
    }
    attr = true;
    const int64_t tiles = ((G.n_rows + C::BM - 1) / C::BM) * ((G.ncols + C::BN - 1) / C::BN);
    launch(gemm_k_kernel<TYPE, WTM, WTN>, dim3((unsigned) tiles), dim3(256), C::LDS, st, G);
}

template <int TYPE, int WTM, int WTN, int KB>
void launch_gemm_t(const gemm_launch & G, hipStream_t st) {
    using C = gemm_cfg<TYPE, WTM, WTN, KB>;
    static bool attr = false;
    if (!attr && C::LDS > 65536) {
        HIP_CHECK(hipFuncSetAttribute((const void *) gemm_q_kernel<TYPE, WTM, WTN, KB>,
                                      hipFuncAttributeMaxDynamicSharedMemorySize, (int) C::LDS));
    }
    attr = true;
    const int64_t tiles = ((G.n_rows + C::BM - 1) / C::BM) * ((G.ncols + C::BN - 1) / C::BN);
    launch(gemm_q_kernel<TYPE, WTM, WTN, KB>, dim3((unsigned) tiles), dim3(256), C::LDS, st, G);
}

int64_t n_tiles(const gemm_launch & G, int bm, int bn) { return ((G.n_rows + bm - 1) / bm) * ((G.ncols + bn - 1) / bn); }

// The workgroup tile of a launch. Q4_0 / Q8_0: the largest tile that still gives every CU two
// workgroups (Q4_0) or four (Q8_0, whose staging moves twice the weight bytes per block; measured:
// Phi-3 prefill 26.1 -> 24.9 ms, while Q4_0 is slower with the smaller tiles). K-quants: 64 x 64
// tiles where they give every CU a workgroup, else 32 x 64 (measured on Q4_K: the larger tile is
// faster down to one workgroup per CU).
enum gemm_tile { TILE_4x4x2, TILE_2x4x2, TILE_1x2x4, TILE_K_2x2, TILE_K_1x2 };

bool is_k_type(int type) { return type == GGML_TYPE_Q4_K || type == GGML_TYPE_Q5_K || type == GGML_TYPE_Q6_K; }

gemm_tile tile_of(const gemm_launch & G) {
    if (is_k_type(G.type)) return n_tiles(G, 64, 64) >= 256 ? TILE_K_2x2 : TILE_K_1x2;
    const int64_t target = G.type == GGML_TYPE_Q8_0 ? 1024 : 512;
    if (n_tiles(G, 128, 128) >= target) return TILE_4x4x2;
    if (n_tiles(G, 64, 128) >= target) return TILE_2x4x2;
    return TILE_1x2x4;
}

template <int TYPE>
void launch_gemm_type(const gemm_launch & G, hipStream_t st) {
    switch (tile_of(G)) {
        case TILE_4x4x2: launch_gemm_t<TYPE, 4, 4, 2>(G, st); break;
        case TILE_2x4x2: launch_gemm_t<TYPE, 2, 4, 2>(G, st); break;
        default: launch_gemm_t<TYPE, 1, 2, 4>(G, st); break;
    }
}

} // namespace

const char * gemm_tile_name(const gemm_launch & G) {
    switch (tile_of(G)) {
        case TILE_4x4x2: return "4x4x2";
        case TILE_2x4x2: return "2x4x2";
        case TILE_1x2x4: return "1x2x4";
        case TILE_K_2x2: return "2x2";
        default: return "1x2";
    }
}

bool gemm_supported(int type, int64_t K, int64_t n_rows) {
    if (is_k_type(type)) return K > 0 && K % 256 == 0 && n_rows > 0;
    return (type == GGML_TYPE_Q4_0 || type == GGML_TYPE_Q8_0) && K > 0 && K % 128 == 0 && n_rows > 0;
}

void launch_gemm(const gemm_launch & G, hipStream_t st) {
    if (!gemm_supported(G.type, G.K, G.n_rows) || G.ncols <= 0) {
        HIP_ABORT("gemm: unsupported geometry (type %d, K %lld, rows %lld, cols %lld)", G.type, (long long) G.K,
                  (long long) G.n_rows, (long long) G.ncols);
    }
    const uintptr_t align = (uintptr_t) G.y | (uintptr_t) G.add | (uintptr_t) G.w | (uintptr_t) G.xq;
    if (align % 16 || G.y_stride % 4 || (G.add && G.add_stride % 4)) {
        HIP_ABORT("gemm: operands must be 16-byte aligned with strides of whole float4s");
    }
    if (is_k_type(G.type)) {
        if (G.type != GGML_TYPE_Q6_K && (!G.xbs || ((uintptr_t) G.xbs % 8))) HIP_ABORT("gemm: Q4_K / Q5_K need Q8_K columns with 8-byte aligned bsums");
        if ((uintptr_t) G.xd % 4) HIP_ABORT("gemm: misaligned Q8_K scales");
        if (G.type == GGML_TYPE_Q6_K && (!G.wqh || !G.wsc || !G.wd || ((uintptr_t) G.wqh % 16) || ((uintptr_t) G.wsc % 8))) {
            HIP_ABORT("gemm: Q6_K needs its high-bit plane 16-byte and its scale plane 8-byte aligned");
        }
        const bool big = tile_of(G) == TILE_K_2x2;
        switch (G.type) {
            case GGML_TYPE_Q4_K: big ? launch_gemm_k_t<GGML_TYPE_Q4_K, 2, 2>(G, st) : launch_gemm_k_t<GGML_TYPE_Q4_K, 1, 2>(G, st); break;
            case GGML_TYPE_Q5_K: big ? launch_gemm_k_t<GGML_TYPE_Q5_K, 2, 2>(G, st) : launch_gemm_k_t<GGML_TYPE_Q5_K, 1, 2>(G, st); break;
            default: big ? launch_gemm_k_t<GGML_TYPE_Q6_K, 2, 2>(G, st) : launch_gemm_k_t<GGML_TYPE_Q6_K, 1, 2>(G, st); break;
        }
        return;
    }
    if (G.type == GGML_TYPE_Q4_0) launch_gemm_type<GGML_TYPE_Q4_0>(G, st);
    else launch_gemm_type<GGML_TYPE_Q8_0>(G, st);
}
