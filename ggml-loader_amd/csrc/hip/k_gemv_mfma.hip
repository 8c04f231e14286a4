// k_gemv_mfma.hip — dense Q4_K products of a few columns (a multi-token decode step, a short
// prompt) on the matrix cores.
//
// y[c][r] = W[r] . x[c] (+ add[c][r]) for up to 16 columns per workgroup, in ggml-cpu's q4_K x q8_K
// arithmetic (the same floats as the GEMV and the prefill GEMM): per 256-element super-block i and
// output, eight integer sums aux[l] (l = element index mod 8) of sc * q4 * q8, sums[l] += (d_w d_x)
// aux[l]; the mins as sumf -= (dmin_w d_x) * sum(bsums * m); the output sumf + sums[0] + ... + sums[7].
//
// A workgroup takes 16 rows and 16 columns; wave w computes super-blocks w, w + 4, ... The integer
// sums come from the matrix cores with exact f16 operands (the prefill GEMM's staging): a lane of a
// wave holds row c's sub-block pair q of the super-block (the elements whose k = 8q .. 8q + 7 in
// every slice l, where slice l orders elements e = 8k + l by k), so it builds its MFMA A operands of
// sc * q4 in registers from its own 48 bytes of the block; one v_mfma_f32_16x16x32_f16 per slice
// gives aux[l] of the 16 x 16 tile (every product and partial sum an integer below 2^24), one
// v_mfma_f32_16x16x16f16 of the mins (m, as f16) against the bsums gives the mins sums. Each wave
// stages the activations of its own super-block (16 columns, as f16 in slice order) in LDS, so the
// staging needs no workgroup barrier. The nine float terms of each (row, column, super-block) go to
// LDS; after each chunk of four super-blocks one thread per (row, column) adds them to its nine
// running sums in super-block order, which is ggml's order.
//
// Every weight load is issued at entry (NCH chunks of three 16-byte loads per lane), and the next
// chunk's activations are loaded before the current chunk is computed.
#include "kernels.h"
#include "gemv_ops.h"

#include "ggml.h"

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

namespace {

constexpr int GM_THREADS = 256;
constexpr int GM_MAX_CHUNKS = 4;       // chunks of 4 super-blocks: K <= 4096
constexpr int GM_ROW = 256 + 8;        // f16 per staged (column, super-block): slice l at 32 l (+8 pad)
constexpr int GM_TS = 4 * 9 + 1;       // floats per (row, column) of a chunk's terms (+1: odd stride)

// per wave: the staged activations of its super-block [16 columns][GM_ROW] f16, their bsums
// [16][16] f16, their d [16], the block scales of its 16 rows d [16] and dmin [16]
constexpr int GM_WAVE_BYTES = 16 * GM_ROW * 2 + 16 * 16 * 2 + 16 * 4 * 3;
constexpr size_t GM_LDS = 4 * (size_t) GM_WAVE_BYTES + 256 * GM_TS * 4;

// 4 int8 (one dword) -> 4 f16 in two dwords (exact): bytes biased by 128 placed under the f16
// exponent of 1024 (0x64xx = 1024 + byte), then 1152 subtracted
__device__ __forceinline__ void i8x4_f16(uint32_t v, uint32_t & lo, uint32_t & hi) {
    const uint32_t u = v ^ 0x80808080u;
    lo = __builtin_amdgcn_perm(0x64646464u, u, 0x04010400u);
    hi = __builtin_amdgcn_perm(0x64646464u, u, 0x04030402u);
    const __half2 bias = __halves2half2(__ushort_as_half(0xE480), __ushort_as_half(0xE480));   // -1152
    lo = __builtin_bit_cast(uint32_t, __hadd2(__builtin_bit_cast(__half2, lo), bias));
    hi = __builtin_bit_cast(uint32_t, __hadd2(__builtin_bit_cast(__half2, hi), bias));
}

// 4 nibbles (0..15 in the byte lanes of n) -> 4 f16 of value nibble * sc (exact: at most 945)
__device__ __forceinline__ void u4x4_times(uint32_t n, __half2 sc, uint32_t & lo, uint32_t & hi) {
    lo = __builtin_amdgcn_perm(0x64646464u, n, 0x04010400u);
    hi = __builtin_amdgcn_perm(0x64646464u, n, 0x04030402u);
    const __half2 bias = __halves2half2(__ushort_as_half(0xE400), __ushort_as_half(0xE400));   // -1024
    lo = __builtin_bit_cast(uint32_t, __hmul2(__hadd2(__builtin_bit_cast(__half2, lo), bias), sc));
    hi = __builtin_bit_cast(uint32_t, __hmul2(__hadd2(__builtin_bit_cast(__half2, hi), bias), sc));
}

__device__ __forceinline__ void wave_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

template <int NCH>
__global__ __launch_bounds__(GM_THREADS, 2) void gemv_mfma_k_kernel(const gemv_kargs A_) {
    const gemv_kargs & a = kernargs_prefetched(A_);
    const gemv_launch & L = a.L;
    extern __shared__ __align__(16) uint8_t smem[];
    const int t = threadIdx.x, lane = t % WAVE, wave = t / WAVE;
    const int c = lane % 16, q = lane / 16;
    uint8_t * wb = smem + (size_t) wave * GM_WAVE_BYTES;
    _Float16 * sB = (_Float16 *) wb;                        // [16][GM_ROW]
    _Float16 * sS = sB + 16 * GM_ROW;                       // [16][16]
    float * sdx = (float *) (sS + 16 * 16);                 // [16]
    float * sdw = sdx + 16;                                 // [16]
    float * sdm = sdw + 16;                                 // [16]
    float * sT = (float *) (smem + 4 * (size_t) GM_WAVE_BYTES);   // [256 chains][GM_TS]

    const int K = L.K, nsb = K / 256;
    const int r0 = blockIdx.x * 16;
    const int mi = find_mat(a, r0);
    const gemv_mat & m = L.m[mi];
    const int lr0 = r0 - a.row_begin[mi];
    const int col0 = blockIdx.y * 16;

    // every weight load of this lane: row lr0 + c, pair q of super-block 4 ch + wave (clamped)
    uint4 wh[NCH], wq0[NCH], wq1[NCH];
    {
        const int64_t row = min(lr0 + c, m.n_rows - 1);
#pragma unroll
        for (int ch = 0; ch < NCH; ch++) {
            const int sb = min(4 * ch + wave, nsb - 1);
            const uint8_t * blk = m.w + (row * nsb + sb) * Q4_K_BYTES;
            wh[ch] = *(const uint4 *) blk;
            wq0[ch] = *(const uint4 *) (blk + 16 + 32 * q);
            wq1[ch] = *(const uint4 *) (blk + 32 + 32 * q);
        }
    }
    // the activation unit this thread stages for its wave's super-block: column (lane / 4), quarter
    // lane % 4 (64 int8, 4 bsums, the super-block's d); columns past the end repeat the last one
    const int xc = lane / 4, xp = lane % 4;
    const int64_t xcol = min(col0 + xc, L.ncols - 1);
    uint4 rx[4];
    uint2 rs;
    float rd;
    auto load_x = [&](int ch) {
        const int sb = min(4 * ch + wave, nsb - 1);
        const uint4 * src = (const uint4 *) (L.xq + xcol * K + sb * 256 + 64 * xp);
#pragma unroll
        for (int v = 0; v < 4; v++) rx[v] = src[v];
        rs = *(const uint2 *) (L.xbs + xcol * (K / 16) + sb * 16 + 4 * xp);
        rd = L.xd[xcol * nsb + sb];
    };
    auto store_x = [&]() {
        const uint32_t v[16] = { rx[0].x, rx[0].y, rx[0].z, rx[0].w, rx[1].x, rx[1].y, rx[1].z, rx[1].w,
                                 rx[2].x, rx[2].y, rx[2].z, rx[2].w, rx[3].x, rx[3].y, rx[3].z, rx[3].w };
        // element l + 8 u of the quarter's 64 sits in dword 2 u + l / 4, byte l % 4
        uint32_t ta[4], tb[4], tc[4], td[4];
        transpose4(v[0], v[2], v[4], v[6], ta);       // l = 0..3, u = 0..3
        transpose4(v[8], v[10], v[12], v[14], tb);    // l = 0..3, u = 4..7
        transpose4(v[1], v[3], v[5], v[7], tc);       // l = 4..7, u = 0..3
        transpose4(v[9], v[11], v[13], v[15], td);    // l = 4..7, u = 4..7
#pragma unroll
        for (int l = 0; l < 8; l++) {
            uint32_t a0, a1, b0, b1;
            i8x4_f16(l < 4 ? ta[l] : tc[l - 4], a0, a1);
            i8x4_f16(l < 4 ? tb[l] : td[l - 4], b0, b1);
            *(uint4 *) (sB + xc * GM_ROW + l * 32 + 8 * xp) = make_uint4(a0, a1, b0, b1);
        }
        const __half2 s01 = __halves2half2(__short2half_rn((short) (rs.x & 0xffff)), __short2half_rn((short) (rs.x >> 16)));
        const __half2 s23 = __halves2half2(__short2half_rn((short) (rs.y & 0xffff)), __short2half_rn((short) (rs.y >> 16)));
        *(uint2 *) (sS + xc * 16 + 4 * xp) = make_uint2(__builtin_bit_cast(uint32_t, s01), __builtin_bit_cast(uint32_t, s23));
        if (xp == 0) sdx[xc] = rd;
    };

    // running sums of chain t = (row t / 16, column t % 16): sumf (the mins) and sums[0..7]
    float sumf = 0.0f, sums[8];
#pragma unroll
    for (int l = 0; l < 8; l++) sums[l] = 0.0f;

    load_x(0);
#pragma unroll
    for (int ch = 0; ch < NCH; ch++) {
        const int sb = 4 * ch + wave;
        const int n_in = min(4, nsb - 4 * ch);            // super-blocks in this chunk (uniform)
        store_x();
        if (lane < 16) {
            sdw[lane] = __half2float(__ushort_as_half((unsigned short) (wh[ch].x & 0xffff)));
            sdm[lane] = __half2float(__ushort_as_half((unsigned short) (wh[ch].x >> 16)));
        }
        wave_sync();
        if (ch + 1 < NCH) load_x(ch + 1);
        if (sb < nsb) {
            int sca, ma, scb, mb;
            q4k_sc_m(wh[ch].y, wh[ch].z, wh[ch].w, 2 * q, sca, ma);
            q4k_sc_m(wh[ch].y, wh[ch].z, wh[ch].w, 2 * q + 1, scb, mb);
            uint32_t w8[8] = { wq0[ch].x, wq0[ch].y, wq0[ch].z, wq0[ch].w, wq1[ch].x, wq1[ch].y, wq1[ch].z, wq1[ch].w };
            q4k_group_by_l(w8);     // dword l: the pair's bytes l, l + 8, l + 16, l + 24
            const __half2 ha = __float2half2_rn((float) sca), hb = __float2half2_rn((float) scb);
            // D of the tiles: lane (c + 16 q) holds rows 4 q .. 4 q + 3 of column c
            const f32x4 dw = *(const f32x4 *) (sdw + 4 * q), dm = *(const f32x4 *) (sdm + 4 * q);
            const float dx = sdx[c];
            // the mins: m of the 16-element groups 4 q .. 4 q + 3 (sub-blocks 2 q, 2 q + 1) against the bsums
            const _Float16 fa = (_Float16) ma, fb = (_Float16) mb;
            const f16x4 am = { fa, fa, fb, fb };
            const f16x4 bm = *(const f16x4 *) (sS + c * 16 + 4 * q);
            const f32x4 mv = __builtin_amdgcn_mfma_f32_16x16x16f16(am, bm, f32x4{ 0.0f, 0.0f, 0.0f, 0.0f }, 0, 0, 0);
            float * tp = sT + (4 * q * 16 + c) * GM_TS + wave * 9;
#pragma unroll
            for (int l = 0; l < 8; l++) {
                uint32_t l0, h0, l1, h1;
                u4x4_times(w8[l] & 0x0F0F0F0Fu, ha, l0, h0);           // k = 8 q .. 8 q + 3: sub-block 2 q
                u4x4_times((w8[l] >> 4) & 0x0F0F0F0Fu, hb, l1, h1);    // k = 8 q + 4 .. 8 q + 7: sub-block 2 q + 1
                const f16x8 av = __builtin_bit_cast(f16x8, make_uint4(l0, h0, l1, h1));
                const f16x8 bv = *(const f16x8 *) (sB + c * GM_ROW + l * 32 + 8 * q);
                const f32x4 sv = __builtin_amdgcn_mfma_f32_16x16x32_f16(av, bv, f32x4{ 0.0f, 0.0f, 0.0f, 0.0f }, 0, 0, 0);
#pragma unroll
                for (int r = 0; r < 4; r++) tp[r * 16 * GM_TS + l] = (dw[r] * dx) * sv[r];
            }
#pragma unroll
            for (int r = 0; r < 4; r++) tp[r * 16 * GM_TS + 8] = (dm[r] * dx) * mv[r];
        }
        __syncthreads();
        // the chunk's terms, super-block by super-block in order
        {
            const float * tt = sT + t * GM_TS;
            for (int i = 0; i < n_in; i++) {
#pragma unroll
                for (int l = 0; l < 8; l++) sums[l] = sums[l] + tt[i * 9 + l];
                sumf = sumf - tt[i * 9 + 8];
            }
        }
        __syncthreads();
    }

    const int rr = t / 16, cc = t % 16;
    const int lrow = lr0 + rr, col = col0 + cc;
    if (lrow < m.n_rows && col < L.ncols) {
        float v = sumf;
#pragma unroll
        for (int l = 0; l < 8; l++) v = v + sums[l];
        if (m.add) v = v + m.add[(int64_t) col * m.add_stride + lrow];
        m.y[(int64_t) col * m.y_stride + lrow] = v;
    }
}

template <int NCH>
void launch_nch(const gemv_kargs & ka, hipStream_t st) {
    static bool attr = false;
    if (!attr) {
        HIP_CHECK(hipFuncSetAttribute((const void *) gemv_mfma_k_kernel<NCH>, hipFuncAttributeMaxDynamicSharedMemorySize, (int) GM_LDS));
        attr = true;
    }
    const dim3 grid((unsigned) (ka.total_rows / 16), (unsigned) ((ka.L.ncols + 15) / 16));
    launch(gemv_mfma_k_kernel<NCH>, grid, dim3(GM_THREADS), GM_LDS, st, ka);
}

}  // namespace

bool gemv_mfma_supported(const gemv_launch & L) {
    return L.type == GGML_TYPE_Q4_K && !L.swiglu && !L.ids && !L.norm.x && L.xq && L.xbs && L.xd && L.ncols >= 2 &&
           L.K % 256 == 0 && L.K <= 256 * 4 * GM_MAX_CHUNKS && L.n_mats >= 1 && L.n_mats <= GEMV_MAX_MATS;
}

void launch_gemv_mfma(const gemv_launch & L, hipStream_t st) {
    if (!gemv_mfma_supported(L)) HIP_ABORT("gemv_mfma: unsupported launch (type %d, K=%d, %d columns)", L.type, L.K, L.ncols);
    gemv_kargs ka{};
    ka.L = L;
    ka.rows_per_block = 16;
    // every matrix starts on a workgroup boundary
    int r = 0;
    for (int i = 0; i < L.n_mats; i++) {
        ka.row_begin[i] = r;
        r += (L.m[i].n_rows + 15) / 16 * 16;
    }
    for (int i = L.n_mats; i <= GEMV_MAX_MATS; i++) ka.row_begin[i] = r;
    ka.total_rows = r;
    const int nch = (L.K / 256 + 3) / 4;
    switch (nch) {
        case 1: launch_nch<1>(ka, st); break;
        case 2: launch_nch<2>(ka, st); break;
        case 3: launch_nch<3>(ka, st); break;
        default: launch_nch<4>(ka, st); break;
    }
}
