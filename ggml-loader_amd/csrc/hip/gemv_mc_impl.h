// gemv_mc_impl.h — the multi-column GEMV kernel template and its launch-shape choice, shared by
// one translation unit per weight type (k_gemv_mc_q4_0.hip, k_gemv_mc_q8_0.hip, k_gemv_mc_q4_k.hip),
// which compile in parallel; k_gemv_mc.hip holds the dispatch, the expert grouping and the entry
// points. See k_gemv_mc.hip for the arithmetic.
#pragma once

#include "kernels.h"
#include "gemv_ops.h"

#include "ggml.h"

namespace gemv_mc_detail {

struct gemv_mc_args {
    gemv_kargs a;
    int nc;                  // columns per workgroup (<= GEMV_MC_MAX_COLS)
    expert_groups g;         // g.cols set: workgroup column group blockIdx.y is item blockIdx.y
};

constexpr int MC_THREADS = 256;
constexpr size_t MC_MAX_LDS = 156 * 1024;   // dynamic LDS per workgroup (of 160 KB, the rest static)

// per-column bytes of the staged activation (16-byte multiple): Q8_0 [qs K][d nb f32][sums nb i32],
// Q8_K [qs K][d nsb f32][bsums K/16 i16]
template <int TYPE>
__host__ __device__ constexpr int mc_act_bytes(int K) {
    return TYPE == GGML_TYPE_Q4_K ? ((K + (K / 256) * 4 + (K / 16) * 2 + 15) & ~15) : K + (K / 32) * 8;
}
// floats per chain of terms: Q4_0/Q8_0 one per block (+4: consecutive chains start on other banks),
// Q4_K nine per super-block (+1)
template <int TYPE>
__host__ __device__ constexpr int mc_term_stride(int K) {
    return TYPE == GGML_TYPE_Q4_K ? (K / 256) * 9 + 1 : gemv_term_stride(K / 32);
}

// Copies n elements, i = 0 .. n - 1, from load(i) to store(i, v), element i on thread i % MC_THREADS:
// each thread loads up to MC_STAGE of its elements before it stores any, so they are in flight
// together. A block of N loads has N fixed at compile time and its loads and stores are
// unconditional: a load under a condition, even a uniform one, or a guarded store of a loaded
// value, gets a wait of its own. A thread past the end takes element i mod p2 instead (p2 the
// largest power of two <= n; it stores that element's value again), which spreads the repeated
// stores over the range: all of them on element n - 1 would serialize on one LDS address when a
// range is short (an expert's one or two columns). Up to MC_STAGE elements per thread run as straight-line code (a loop header waits for
// every load in flight, the weights included).
constexpr int MC_STAGE = 8;
template <int N, typename T, typename LD, typename STO>
__device__ __forceinline__ void stage_block(int n, int j0, LD & load, STO & store) {
    const int p2m = (1 << (31 - __clz(n))) - 1;
    T v[N];
    int idx[N];
#pragma unroll
    for (int j = 0; j < N; j++) {
        const int i = (int) threadIdx.x + (j0 + j) * MC_THREADS;
        idx[j] = i < n ? i : i & p2m;
        v[j] = load(idx[j]);
    }
#pragma unroll
    for (int j = 0; j < N; j++) store(idx[j], v[j]);
}
template <typename T, typename LD, typename STO>
__device__ __forceinline__ void stage_flat(int n, LD load, STO store) {
    const int per = (n + MC_THREADS - 1) / MC_THREADS;   // elements per thread (uniform)
    switch (per) {
        case 0: return;
        case 1: stage_block<1, T>(n, 0, load, store); return;
        case 2: stage_block<2, T>(n, 0, load, store); return;
        case 3: stage_block<3, T>(n, 0, load, store); return;
        case 4: stage_block<4, T>(n, 0, load, store); return;
        case 5: stage_block<5, T>(n, 0, load, store); return;
        case 6: stage_block<6, T>(n, 0, load, store); return;
        case 7: stage_block<7, T>(n, 0, load, store); return;
        case 8: stage_block<8, T>(n, 0, load, store); return;
        default:
            for (int j0 = 0; j0 < per; j0 += MC_STAGE) stage_block<MC_STAGE, T>(n, min(j0, per - MC_STAGE), load, store);
    }
}

// FLAT: consecutive columns of a multi-token step, staged as flat ranges (stage_flat); otherwise an
// expert's item, staged column by column
template <int TYPE, int LPR, bool SWIGLU, int ITS, bool FLAT>
__global__ __launch_bounds__(MC_THREADS) void gemv_mc_kernel(const gemv_mc_args A) {
    prefetch_kernargs<sizeof(gemv_mc_args)>();
    extern __shared__ __align__(16) uint8_t smem[];
    __shared__ int s_col[GEMV_MC_MAX_COLS];
    __shared__ int s_xcol[GEMV_MC_MAX_COLS];   // the activation column each reads
    constexpr int RPW = WAVE / LPR;
    constexpr int NCH = SWIGLU ? 2 : 1;
    const gemv_launch & L = A.a.L;
    const int K = L.K, nc = A.nc;
    const int t = threadIdx.x, lane = t % WAVE, wave = t / WAVE;
    const int g = lane / LPR, l = lane % LPR;
    const int rows_pb = A.a.rows_per_block;
    const int rib = wave * RPW + g;
    const int row = blockIdx.x * rows_pb + rib;
    const int mi = SWIGLU ? 0 : find_mat(A.a, blockIdx.x * rows_pb);   // uniform: the workgroup's matrix
    const int lrow = SWIGLU ? row : row - A.a.row_begin[mi];
    const bool valid = row < A.a.total_rows && lrow < L.m[mi].n_rows;

    // the workgroup's columns (an expert without columns here ends the workgroup before any load)
    int ncg, list_base = 0, first_col = 0;
    int64_t erow = 0;
    if (A.g.cols) {
        if ((int) blockIdx.y >= *A.g.n_items) return;
        const int32_t * item = A.g.items + 3 * blockIdx.y;
        erow = (int64_t) item[0] * L.expert_rows;
        list_base = item[1];
        ncg = item[2];
    } else {
        first_col = blockIdx.y * nc;
        ncg = min(nc, L.ncols - first_col);
    }

    // every weight load of this lane first (row and block clamped into the matrix)
    constexpr int QS = TYPE == GGML_TYPE_Q4_0 ? Q4_0_QS : Q8_0_QS;
    const int nb = K / 32, units = K / 64, nsb = K / 256;
    uint4 wa[NCH][ITS], wb[NCH][ITS], wh[NCH][ITS];
    uint32_t dwb[NCH][ITS];
#pragma unroll
    for (int ch = 0; ch < NCH; ch++) {
        const gemv_mat & wm = L.m[SWIGLU ? ch : mi];
        const int64_t wr = erow + min(lrow, wm.n_rows - 1);
#pragma unroll
        for (int it = 0; it < ITS; it++) {
            if constexpr (TYPE == GGML_TYPE_Q4_K) {
                const int u = min(l + it * LPR, units - 1);
                const uint8_t * blk = wm.w + wr * nsb * Q4_K_BYTES + (int64_t) (u >> 2) * Q4_K_BYTES;
                wh[ch][it] = *(const uint4 *) blk;
                wa[ch][it] = *(const uint4 *) (blk + 16 + 32 * (u & 3));
                wb[ch][it] = *(const uint4 *) (blk + 32 + 32 * (u & 3));
            } else {
                const int b = min(l + it * LPR, nb - 1);
                wa[ch][it] = *(const uint4 *) (wm.w + (wr * nb + b) * QS);
                if (TYPE == GGML_TYPE_Q8_0) wb[ch][it] = *(const uint4 *) (wm.w + (wr * nb + b) * QS + 16);
                dwb[ch][it] = ((const unsigned short *) wm.wd)[wr * nb + b];
            }
        }
    }

    // the columns' quantized activations into LDS
    const int ab = mc_act_bytes<TYPE>(K);
    if constexpr (!FLAT) {
        // an expert's item (a few columns): column by column, each column's index a scalar load.
        // Measured: kernels built with the flat staging below are slower for these items (C5
        // 16-token steps, expert gate/up 54.9 -> 61.9 us, down 45.2 -> 56.2 us per launch)
        if (t < ncg) s_col[t] = A.g.cols ? A.g.cols[list_base + t] : first_col + t;
        for (int k = 0; k < ncg; k++) {
            const int col = A.g.cols ? A.g.cols[list_base + k] : first_col + k;
            const int xcol = L.ids ? (col / L.n_slots) * L.x_cols + (col % L.n_slots) % L.x_cols : col;
            uint8_t * act = smem + (size_t) k * ab;
            for (int i = t; i < K / 16; i += MC_THREADS) ((int4 *) act)[i] = ((const int4 *) (L.xq + (int64_t) xcol * K))[i];
            if constexpr (TYPE == GGML_TYPE_Q4_K) {
                float * xd = (float *) (act + K);
                int16_t * xbs = (int16_t *) (act + K + nsb * 4);
                for (int i = t; i < nsb; i += MC_THREADS) xd[i] = L.xd[(int64_t) xcol * nsb + i];
                for (int i = t; i < K / 16; i += MC_THREADS) xbs[i] = L.xbs[(int64_t) xcol * (K / 16) + i];
            } else {
                float * xd = (float *) (act + K);
                int32_t * xs = (int32_t *) (act + K + nb * 4);
                for (int i = t; i < nb; i += MC_THREADS) {
                    xd[i] = L.xd[(int64_t) xcol * nb + i];
                    xs[i] = L.xs[(int64_t) xcol * nb + i];
                }
            }
        }
    } else {
        // consecutive columns of a multi-token step: each array of all the columns as one flat
        // range, MC_STAGE loads in flight per thread before their stores (one L2 round trip per
        // MC_STAGE * MC_THREADS pieces, not one per column; measured: C5 16-token QKV 46.1 -> 29.6
        // us, O 47.7 -> 33.3 us per launch)
        if (t < ncg) {
            s_col[t] = first_col + t;
            s_xcol[t] = L.ids ? ((first_col + t) / L.n_slots) * L.x_cols + ((first_col + t) % L.n_slots) % L.x_cols
                              : first_col + t;
        }
        __syncthreads();
        // qs: K / 16 pieces of 16 bytes per column
        stage_flat<int4>(ncg * (K / 16), [&](int i) {
            const int k = i / (K / 16);
            return ((const int4 *) (L.xq + (int64_t) s_xcol[k] * K))[i % (K / 16)];
        }, [&](int i, int4 v) { ((int4 *) (smem + (size_t) (i / (K / 16)) * ab))[i % (K / 16)] = v; });
        if constexpr (TYPE == GGML_TYPE_Q4_K) {
            stage_flat<float>(ncg * nsb, [&](int i) { return L.xd[(int64_t) s_xcol[i / nsb] * nsb + i % nsb]; },
                              [&](int i, float v) { ((float *) (smem + (size_t) (i / nsb) * ab + K))[i % nsb] = v; });
            // bsums: K / 16 int16 per column, as K / 32 dwords (the plane is 4-byte aligned only)
            stage_flat<int32_t>(ncg * (K / 32), [&](int i) {
                return ((const int32_t *) (L.xbs + (int64_t) s_xcol[i / (K / 32)] * (K / 16)))[i % (K / 32)];
            }, [&](int i, int32_t v) { ((int32_t *) (smem + (size_t) (i / (K / 32)) * ab + K + nsb * 4))[i % (K / 32)] = v; });
        } else {
            stage_flat<float>(ncg * nb, [&](int i) { return L.xd[(int64_t) s_xcol[i / nb] * nb + i % nb]; },
                              [&](int i, float v) { ((float *) (smem + (size_t) (i / nb) * ab + K))[i % nb] = v; });
            stage_flat<int32_t>(ncg * nb, [&](int i) { return L.xs[(int64_t) s_xcol[i / nb] * nb + i % nb]; },
                                [&](int i, int32_t v) { ((int32_t *) (smem + (size_t) (i / nb) * ab + K + nb * 4))[i % nb] = v; });
        }
    }
    __syncthreads();
    if constexpr (TYPE == GGML_TYPE_Q4_K && !FLAT) {
        for (int k = 0; k < ncg; k++) group_by_l_lds((int8_t *) (smem + (size_t) k * ab), K / 32);
        __syncthreads();
    } else if constexpr (TYPE == GGML_TYPE_Q4_K) {
        // each 32-byte group of every column regrouped by l, one group per thread
        for (int i = t; i < ncg * (K / 32); i += MC_THREADS) {
            uint4 * p = (uint4 *) (smem + (size_t) (i / (K / 32)) * ab + (i % (K / 32)) * 32);
            const uint4 lo4 = p[0], hi4 = p[1];
            uint32_t w8[8] = { lo4.x, lo4.y, lo4.z, lo4.w, hi4.x, hi4.y, hi4.z, hi4.w };
            q4k_group_by_l(w8);
            p[0] = make_uint4(w8[0], w8[1], w8[2], w8[3]);
            p[1] = make_uint4(w8[4], w8[5], w8[6], w8[7]);
        }
        __syncthreads();
    }

    // per-block terms of every (row, column, chain)
    const int stride = mc_term_stride<TYPE>(K);
    float * terms = (float *) (smem + (size_t) nc * ab);
    auto chain_of = [&](int r, int k, int ch) { return (r * nc + k) * NCH + ch; };
    if constexpr (TYPE == GGML_TYPE_Q4_0 || TYPE == GGML_TYPE_Q8_0) {
#pragma unroll
        for (int ch = 0; ch < NCH; ch++) {
#pragma unroll
            for (int it = 0; it < ITS; it++) {
                const int b = l + it * LPR;
                if (!valid || b >= nb) continue;
                const float dw = __half2float(__ushort_as_half((unsigned short) dwb[ch][it]));
                for (int k = 0; k < ncg; k++) {
                    const uint8_t * act = smem + (size_t) k * ab;
                    const int4 xa = *(const int4 *) (act + b * 32);
                    const int4 xb = *(const int4 *) (act + b * 32 + 16);
                    const float dx = ((const float *) (act + K))[b];
                    float tm;
                    if (TYPE == GGML_TYPE_Q4_0) {
                        const int sumi = dot_q4_0_block(wa[ch][it], xa, xb) - 8 * ((const int32_t *) (act + K + nb * 4))[b];
                        tm = ((float) sumi * dw) * dx;           // ggml: sumi*d_x*d_y
                    } else {
                        const int sumi = dot_q8_0_block(wa[ch][it], wb[ch][it], xa, xb);
                        tm = (float) sumi * (dw * dx);           // ggml: sumi*(d_x*d_y)
                    }
                    terms[chain_of(rib, k, ch) * stride + b] = tm;
                }
            }
        }
    } else {
#pragma unroll
        for (int ch = 0; ch < NCH; ch++) {
#pragma unroll
            for (int it = 0; it < ITS; it++) {
                if (it * LPR >= units) break;       // uniform across the workgroup
                const int u = l + it * LPR;
                const int sb = u >> 2, p = u & 3;
                const bool has = valid && u < units;
                const q4k_unit U = q4k_prepare(wh[ch][it], wa[ch][it], wb[ch][it], p);
                const uint32_t dd = wh[ch][it].x;
                for (int k = 0; k < ncg; k++) {
                    const uint8_t * act = smem + (size_t) k * ab;
                    int aux[8], mins = 0;
#pragma unroll
                    for (int q = 0; q < 8; q++) aux[q] = 0;
                    if (has) {
                        const int * xs = (const int *) (act + sb * 256 + 64 * p);
                        q4k_unit_dot(U, p, xs, xs + 8, (const int16_t *) (act + K + nsb * 4) + sb * 16, aux, mins);
                    }
                    // the 4 units of a super-block sit on 4 consecutive lanes: combine (exact integers)
#pragma unroll
                    for (int q = 0; q < 8; q++) {
                        aux[q] += dpp_i<0xB1>(aux[q]);   // quad lanes xor 1
                        aux[q] += dpp_i<0x4E>(aux[q]);   // quad lanes xor 2
                    }
                    mins += dpp_i<0xB1>(mins);
                    mins += dpp_i<0x4E>(mins);
                    if (has) {
                        const float yd = ((const float *) (act + K))[sb];
                        const float d = __half2float(__ushort_as_half((unsigned short) (dd & 0xffff))) * yd;
                        const float dmin = __half2float(__ushort_as_half((unsigned short) (dd >> 16))) * yd;
                        float t0 = 0.0f, t1 = 0.0f;
#pragma unroll
                        for (int q = 0; q < 8; q++) {
                            if (q == 2 * p) t0 = d * (float) aux[q];
                            if (q == 2 * p + 1) t1 = d * (float) aux[q];
                        }
                        float * tt = terms + chain_of(rib, k, ch) * stride + sb * 9;
                        tt[2 * p] = t0;
                        tt[2 * p + 1] = t1;
                        if (p == 0) tt[8] = dmin * (float) mins;
                    }
                }
            }
        }
    }
    __syncthreads();

    // ordered sums, one thread per chain (gate and up chains of a (row, column) on adjacent lanes)
    const int chain = t;
    const int r = chain / (nc * NCH), k = (chain / NCH) % nc, ch = chain % NCH;
    const int rrow = blockIdx.x * rows_pb + r;
    const bool has = r < rows_pb && k < ncg && rrow < A.a.total_rows &&
                     (SWIGLU || rrow - A.a.row_begin[mi] < L.m[mi].n_rows);
    float acc = 0.0f;
    if (has) {
        const float * tt = terms + chain * stride;
        if constexpr (TYPE == GGML_TYPE_Q4_K) {
            // sumf: the mins chain, then += sums[0..7] in order (each the super-blocks in order)
            float f = 0.0f;
            for (int i = 0; i < nsb; i++) f = f - tt[i * 9 + 8];
#pragma unroll
            for (int q = 0; q < 8; q++) {
                float v = 0.0f;
                for (int i = 0; i < nsb; i++) v = v + tt[i * 9 + q];
                f = f + v;
            }
            acc = f;
        } else {
            acc = ordered_sum(tt, nb);
        }
    }
    if constexpr (SWIGLU) {
        // act = silu(gate) * up (two roundings, as the silu and mul ops); up sits on the next lane
        const float uv = __shfl_down(acc, 1, WAVE);
        if (has && ch == 0) {
            const float sl = acc / (1.0f + exp_cr(-acc));
            L.m[0].y[(int64_t) s_col[k] * L.m[0].y_stride + rrow] = sl * uv;
        }
    } else if (has) {
        const int rl = rrow - A.a.row_begin[mi];
        const gemv_mat & m = L.m[mi];
        float v = acc;
        if (m.add) v = v + m.add[(int64_t) s_col[k] * m.add_stride + rl];
        m.y[(int64_t) s_col[k] * m.y_stride + rl] = v;
    }
}

template <int TYPE, int LPR, bool SWIGLU, int ITS, bool FLAT>
static void launch_mc_flat(gemv_mc_args & A, dim3 grid, size_t lds, hipStream_t st) {
    static size_t allowed = 64 * 1024;   // dynamic LDS this kernel may take
    if (lds > allowed) {
        HIP_CHECK(hipFuncSetAttribute((const void *) gemv_mc_kernel<TYPE, LPR, SWIGLU, ITS, FLAT>,
                                      hipFuncAttributeMaxDynamicSharedMemorySize, (int) lds));
        allowed = lds;
    }
    launch((gemv_mc_kernel<TYPE, LPR, SWIGLU, ITS, FLAT>), grid, dim3(MC_THREADS), lds, st, A);
}

template <int TYPE, int LPR, bool SWIGLU, int ITS>
static void launch_mc_its(gemv_mc_args & A, dim3 grid, size_t lds, hipStream_t st) {
    if (A.g.cols) launch_mc_flat<TYPE, LPR, SWIGLU, ITS, false>(A, grid, lds, st);
    else launch_mc_flat<TYPE, LPR, SWIGLU, ITS, true>(A, grid, lds, st);
}

// blocks (Q4_0/Q8_0) or 64-weight units (Q4_K) per lane held in registers
template <int TYPE, int LPR, bool SWIGLU>
static void launch_mc_t(gemv_mc_args & A, dim3 grid, size_t lds, hipStream_t st) {
    const int K = A.a.L.K;
    const int its = TYPE == GGML_TYPE_Q4_K ? (K / 64 + LPR - 1) / LPR : (K / 32 + LPR - 1) / LPR;
    if (its <= 1) launch_mc_its<TYPE, LPR, SWIGLU, 1>(A, grid, lds, st);
    else if (its <= 2) launch_mc_its<TYPE, LPR, SWIGLU, 2>(A, grid, lds, st);
    else if (its <= 4) launch_mc_its<TYPE, LPR, SWIGLU, 4>(A, grid, lds, st);
    else if (its <= 8) launch_mc_its<TYPE, LPR, SWIGLU, 8>(A, grid, lds, st);
    else if (its <= 12) launch_mc_its<TYPE, LPR, SWIGLU, 12>(A, grid, lds, st);
    else HIP_ABORT("gemv_mc: K=%d is too long", K);
}

template <int TYPE, bool SWIGLU>
static bool launch_mc_type(const gemv_launch & L, const expert_groups * G, int max_cols, hipStream_t st, bool dry) {
    constexpr int NCH = SWIGLU ? 2 : 1;
    const int K = L.K;
    const int n_units = TYPE == GGML_TYPE_Q4_K ? K / 64 : K / 32;
    const int want = G ? G->nc : std::min(GEMV_MC_MAX_COLS, L.ncols);
    const int rows_total = SWIGLU ? L.m[0].n_rows : [&] { int r = 0; for (int i = 0; i < L.n_mats; i++) r += L.m[i].n_rows; return r; }();
    for (int nc = want; nc >= 1; nc = (G || nc == 1) ? 0 : (nc + 1) / 2) {
        // the fewest lanes per row (most rows per workgroup) that still give the launch about two
        // workgroups per CU (grouped mul_mat_id: one row block per work item), else the most
        // workgroups that fit
        constexpr int TARGET_BLOCKS = 512;
        int pick = 0;
        for (int lpr : { 16, 32, 64 }) {
            const int rows_pb = (MC_THREADS / WAVE) * (WAVE / lpr);
            const int chains = rows_pb * NCH * nc;
            if (chains > MC_THREADS || (n_units + lpr - 1) / lpr > 12) continue;
            const size_t lds_c = (size_t) nc * mc_act_bytes<TYPE>(K) + (size_t) chains * mc_term_stride<TYPE>(K) * 4;
            if (lds_c > MC_MAX_LDS) continue;
            pick = lpr;
            const int64_t blocks = (int64_t) ((rows_total + rows_pb - 1) / rows_pb) * (G ? G->max_items : (L.ncols + nc - 1) / nc);
            if (blocks >= TARGET_BLOCKS) break;
        }
        if (pick) {
            const int lpr = pick;
            const int rows_pb = (MC_THREADS / WAVE) * (WAVE / lpr);
            const int chains = rows_pb * NCH * nc;
            const size_t lds = (size_t) nc * mc_act_bytes<TYPE>(K) + (size_t) chains * mc_term_stride<TYPE>(K) * 4;
            if (dry) return true;
            gemv_mc_args A{};
            A.a.L = L;
            A.a.rows_per_block = rows_pb;
            int r = 0;
            for (int i = 0; i < L.n_mats; i++) {
                A.a.row_begin[i] = r;
                r += SWIGLU ? 0 : (L.m[i].n_rows + rows_pb - 1) / rows_pb * rows_pb;
            }
            for (int i = L.n_mats; i <= GEMV_MAX_MATS; i++) A.a.row_begin[i] = r;
            A.a.total_rows = SWIGLU ? L.m[0].n_rows : r;
            if (SWIGLU) for (int i = 0; i <= GEMV_MAX_MATS; i++) A.a.row_begin[i] = 0;
            A.nc = nc;
            dim3 grid((unsigned) ((A.a.total_rows + rows_pb - 1) / rows_pb), 1);
            if (G) {
                A.g = *G;
                grid.y = (unsigned) G->max_items;
            } else {
                grid.y = (unsigned) ((L.ncols + nc - 1) / nc);
            }
            switch (lpr) {
                case 16: launch_mc_t<TYPE, 16, SWIGLU>(A, grid, lds, st); break;
                case 32: launch_mc_t<TYPE, 32, SWIGLU>(A, grid, lds, st); break;
                default: launch_mc_t<TYPE, 64, SWIGLU>(A, grid, lds, st); break;
            }
            return true;
        }
    }
    return false;
}

} // namespace gemv_mc_detail

// the launch (or, with dry, only the check that a workgroup shape fits) for one weight type
bool launch_mc_q4_0(bool swiglu, const gemv_launch & L, const expert_groups * G, int max_cols, hipStream_t st, bool dry);
bool launch_mc_q8_0(bool swiglu, const gemv_launch & L, const expert_groups * G, int max_cols, hipStream_t st, bool dry);
bool launch_mc_q4_k(bool swiglu, const gemv_launch & L, const expert_groups * G, int max_cols, hipStream_t st, bool dry);
