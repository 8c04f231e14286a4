// k_gemm.hip — the prefill GEMM: Q4_0 / Q8_0 weights times Q8_0-quantized activation columns on
// the int8 matrix cores.
//
// ggml-cpu computes every output of a quantized mul_mat as a float sum over the weight row's
// 32-element blocks, in block order, of an exact integer block dot scaled by the two fp16 block
// scales: Q8_0 sumf += sumi * (d_w * d_x), Q4_0 sumf += (sumi * d_w) * d_x. One
// v_mfma_i32_16x16x32_i8 yields the integer dots of one block for a tile of 16 weight rows x 16
// activation columns (exact in any order), so the kernel issues one MFMA per tile and block and
// adds the scaled terms to f32 accumulators in block order: every output is the same float as the
// GEMV's and the CPU reference's. The per-term float work (convert, two multiplies, one add) runs on
// the VALU and bounds the kernel, not the MFMA rate.
//
// Tiling: a workgroup is 2 x 2 waves; a wave owns WM x WN MFMA tiles. In a tile, lane l holds
// weight row l%16 and activation column l%16 with the k-slice 8(l/16)..8(l/16)+7 of the block (for
// Q4_0 the low nibbles of bytes 0-15 are elements 0-15 and the high nibbles 16-31, so the slice is 8
// bytes and one nibble half), and receives the results of rows 4(l/16)..4(l/16)+3 of column l%16.
// Each step loads KB blocks of every operand; the next step's loads are in flight while the current
// step is reduced. Workgroups are numbered so that the column tiles of one row tile run on one XCD
// and share its L2.
#include "kernels.h"

#include "ggml.h"

typedef int v4i __attribute__((ext_vector_type(4)));

namespace {

constexpr int KB = 4;   // blocks per pipeline step

// the lane's 8 int8 weights of one block from its 8 loaded bytes
template <int TYPE>
__device__ __forceinline__ long a_slice(uint64_t raw, int q) {
    if constexpr (TYPE == GGML_TYPE_Q8_0) {
        return (long) raw;
    } else {
        // nibble n -> int8 n - 8 in every byte: (n | 0x80) - 8 stays in [0x78, 0x87] (no borrow
        // between bytes), and flipping bit 7 turns it into n - 8 as a signed byte
        const int sh = (q >> 1) * 4;
        uint32_t lo = ((uint32_t) raw >> sh) & 0x0F0F0F0Fu;
        uint32_t hi = ((uint32_t) (raw >> 32) >> sh) & 0x0F0F0F0Fu;
        lo = ((lo | 0x80808080u) - 0x08080808u) ^ 0x80808080u;
        hi = ((hi | 0x80808080u) - 0x08080808u) ^ 0x80808080u;
        return (long) (((uint64_t) hi << 32) | lo);
    }
}

template <int WM, int WN>
struct gemm_stage {
    uint64_t a[WM][KB];    // weight bytes per tile row and block
    uint64_t b[WN][KB];    // activation int8 per tile column and block
    uint64_t wd[WM][4];    // fp16 d of KB blocks for each of the lane's 4 output rows
    float4   xd[WN];       // activation d of KB blocks for the lane's column
};

template <int TYPE, int WM, int WN>
__global__ __launch_bounds__(256) void gemm_q_kernel(const gemm_launch G) {
    constexpr int QB = TYPE == GGML_TYPE_Q4_0 ? Q4_0_QS : Q8_0_QS;
    constexpr int BM = 32 * WM, BN = 32 * WN;
    static_assert(KB == 4, "the scale loads move 4 blocks");
    const int64_t M = G.n_rows, N = G.ncols, K = G.K, nb = K / 32;
    const int lane = threadIdx.x % WAVE, wave = threadIdx.x / WAVE;
    const int q = lane / 16, c = lane % 16;

    const int64_t n_ct = (N + BN - 1) / BN, tiles = ((M + BM - 1) / BM) * n_ct;
    int64_t t = blockIdx.x;
    if (tiles % 8 == 0) t = (int64_t) (blockIdx.x % 8) * (tiles / 8) + blockIdx.x / 8;
    const int64_t row0 = (t / n_ct) * BM + (wave / 2) * 16 * WM;
    const int64_t col0 = (t % n_ct) * BN + (wave % 2) * 16 * WN;

    // operand rows / columns clamped into range (their results are not stored)
    const uint8_t * pa[WM];
    const __half * pd[WM];
    for (int i = 0; i < WM; i++) {
        const int64_t ra = min(row0 + 16 * i + c, M - 1);
        pa[i] = G.w + ra * nb * QB + (TYPE == GGML_TYPE_Q4_0 ? 8 * (q & 1) : 8 * q);
        pd[i] = G.wd + min(row0 + 16 * i + 4 * q, M - 4) * nb;
    }
    const int8_t * pb[WN];
    const float * px[WN];
    for (int j = 0; j < WN; j++) {
        const int64_t cb = min(col0 + 16 * j + c, N - 1);
        pb[j] = G.xq + cb * K + 8 * q;
        px[j] = G.xd + cb * nb;
    }

    auto load = [&](gemm_stage<WM, WN> & s, int64_t b) {
        for (int i = 0; i < WM; i++)
            for (int k = 0; k < KB; k++) s.a[i][k] = *(const uint64_t *) (pa[i] + (b + k) * QB);
        for (int j = 0; j < WN; j++)
            for (int k = 0; k < KB; k++) s.b[j][k] = *(const uint64_t *) (pb[j] + (b + k) * 32);
        for (int i = 0; i < WM; i++)
            for (int r = 0; r < 4; r++) s.wd[i][r] = *(const uint64_t *) (pd[i] + r * nb + b);
        for (int j = 0; j < WN; j++) s.xd[j] = *(const float4 *) (px[j] + b);
    };

    float acc[WM][WN][4];
    for (int i = 0; i < WM; i++)
        for (int j = 0; j < WN; j++)
            for (int r = 0; r < 4; r++) acc[i][j][r] = 0.0f;

    gemm_stage<WM, WN> cur, nxt;
    load(cur, 0);
    for (int64_t b = 0; b < nb; b += KB) {
        if (b + KB < nb) load(nxt, b + KB);
        for (int k = 0; k < KB; k++) {
            v4i s[WM][WN];
            for (int i = 0; i < WM; i++) {
                const long a = a_slice<TYPE>(cur.a[i][k], q);
                for (int j = 0; j < WN; j++) {
                    s[i][j] = __builtin_amdgcn_mfma_i32_16x16x32_i8(a, (long) cur.b[j][k], v4i{ 0, 0, 0, 0 }, 0, 0, 0);
                }
            }
            float dw[WM][4];
            for (int i = 0; i < WM; i++)
                for (int r = 0; r < 4; r++)
                    dw[i][r] = __half2float(__ushort_as_half((unsigned short) (cur.wd[i][r] >> (16 * k))));
            for (int j = 0; j < WN; j++) {
                const float dx = k == 0 ? cur.xd[j].x : k == 1 ? cur.xd[j].y : k == 2 ? cur.xd[j].z : cur.xd[j].w;
                for (int i = 0; i < WM; i++)
                    for (int r = 0; r < 4; r++) {
                        if constexpr (TYPE == GGML_TYPE_Q8_0) {
                            const float dd = dw[i][r] * dx;
                            acc[i][j][r] += (float) s[i][j][r] * dd;
                        } else {
                            acc[i][j][r] += ((float) s[i][j][r] * dw[i][r]) * dx;
                        }
                    }
            }
        }
        cur = nxt;
    }

    for (int j = 0; j < WN; j++) {
        const int64_t col = col0 + 16 * j + c;
        if (col >= N) continue;
        for (int i = 0; i < WM; i++) {
            const int64_t r0 = row0 + 16 * i + 4 * q;
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

template <int TYPE, int WM, int WN>
void launch_gemm_t(const gemm_launch & G, hipStream_t st) {
    const int64_t BM = 32 * WM, BN = 32 * WN;
    const int64_t tiles = ((G.n_rows + BM - 1) / BM) * ((G.ncols + BN - 1) / BN);
    launch(gemm_q_kernel<TYPE, WM, WN>, dim3((unsigned) tiles), dim3(256), 0, st, G);
}

template <int TYPE>
void launch_gemm_type(const gemm_launch & G, hipStream_t st) {
    // 64 x 128 tiles unless that leaves fewer than two workgroups per CU
    const int64_t big = ((G.n_rows + 63) / 64) * ((G.ncols + 127) / 128);
    if (big >= 512) launch_gemm_t<TYPE, 2, 4>(G, st);
    else launch_gemm_t<TYPE, 1, 4>(G, st);
}

} // namespace

bool gemm_supported(int type, int64_t K, int64_t n_rows) {
    return (type == GGML_TYPE_Q4_0 || type == GGML_TYPE_Q8_0) && K > 0 && K % (32 * KB) == 0 && n_rows > 0 &&
           n_rows % 4 == 0;
}

void launch_gemm(const gemm_launch & G, hipStream_t st) {
    if (!gemm_supported(G.type, G.K, G.n_rows) || G.ncols <= 0) {
        HIP_ABORT("gemm: unsupported geometry (type %d, K %lld, rows %lld, cols %lld)", G.type, (long long) G.K,
                  (long long) G.n_rows, (long long) G.ncols);
    }
    const uintptr_t align = (uintptr_t) G.y | (uintptr_t) G.add | (uintptr_t) G.w | (uintptr_t) G.wd |
                            (uintptr_t) G.xq | (uintptr_t) G.xd;
    if (align % 16 || G.y_stride % 4 || (G.add && G.add_stride % 4)) {
        HIP_ABORT("gemm: operands must be 16-byte aligned with strides of whole float4s");
    }
    if (G.type == GGML_TYPE_Q4_0) launch_gemm_type<GGML_TYPE_Q4_0>(G, st);
    else launch_gemm_type<GGML_TYPE_Q8_0>(G, st);
}
