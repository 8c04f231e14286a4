// k_gemv_mc.hip — quantized GEMV over several activation columns per workgroup: each weight row
// block is read once for up to GEMV_MC_MAX_COLS columns (multi-token decode steps, prompts too
// short for the GEMM, Q4_K prompts) and, for ggml_mul_mat_id, once for all the tokens routed to
// its expert — the batched expert grouping of the reference's MoE engine (build_prefill_lists /
// matmul_batch, qwen_model.c:742-772, 862-939), here over the expert lists that moe_group_kernel
// builds on the device from the routing ids.
//
// Per (row, column) the arithmetic is k_gemv.hip's: the same integer block dots against the
// pre-quantized activation (Q8_0 / Q8_K), the same float terms, added in block order by one
// thread per (row, column[, gate/up]) chain, so the result is the CPU reference's float.
#include "kernels.h"
#include "gemv_ops.h"

#include "ggml.h"

namespace {

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

template <int TYPE, int LPR, bool SWIGLU, int ITS>
__global__ __launch_bounds__(MC_THREADS) void gemv_mc_kernel(const gemv_mc_args A) {
    extern __shared__ __align__(16) uint8_t smem[];
    __shared__ int s_col[GEMV_MC_MAX_COLS];
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
    __syncthreads();
    if constexpr (TYPE == GGML_TYPE_Q4_K) {
        for (int k = 0; k < ncg; k++) group_by_l_lds((int8_t *) (smem + (size_t) k * ab), K / 32);
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

template <int TYPE, int LPR, bool SWIGLU, int ITS>
static void launch_mc_its(gemv_mc_args & A, dim3 grid, size_t lds, hipStream_t st) {
    static size_t allowed = 64 * 1024;   // dynamic LDS this kernel may take
    if (lds > allowed) {
        HIP_CHECK(hipFuncSetAttribute((const void *) gemv_mc_kernel<TYPE, LPR, SWIGLU, ITS>,
                                      hipFuncAttributeMaxDynamicSharedMemorySize, (int) lds));
        allowed = lds;
    }
    launch((gemv_mc_kernel<TYPE, LPR, SWIGLU, ITS>), grid, dim3(MC_THREADS), lds, st, A);
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

template <bool SWIGLU>
static bool launch_mc_dispatch(const gemv_launch & L, const expert_groups * G, int max_cols, hipStream_t st, bool dry) {
    switch (L.type) {
        case GGML_TYPE_Q4_0: return launch_mc_type<GGML_TYPE_Q4_0, SWIGLU>(L, G, max_cols, st, dry);
        case GGML_TYPE_Q8_0: return launch_mc_type<GGML_TYPE_Q8_0, SWIGLU>(L, G, max_cols, st, dry);
        case GGML_TYPE_Q4_K: return launch_mc_type<GGML_TYPE_Q4_K, SWIGLU>(L, G, max_cols, st, dry);
        default: return false;
    }
}

// One workgroup: the columns (token, slot) of a mul_mat_id grouped by expert. Counts and cursors
// live in LDS (shared-memory atomics); the order inside an expert's list is arbitrary, which does
// not change any result (every column is computed on its own).
__global__ __launch_bounds__(256) void moe_group_kernel(const int32_t * ids, int64_t ids_stride, int n_slots, int n_tok,
                                                        int n_experts, const expert_groups g) {
    extern __shared__ int s_cnt[];
    int * s_cur = s_cnt + n_experts;
    const int t = threadIdx.x, ncol = n_slots * n_tok;
    for (int e = t; e < n_experts; e += 256) s_cnt[e] = 0;
    __syncthreads();
    for (int c = t; c < ncol; c += 256) {
        const int e = min(max(ids[(int64_t) (c / n_slots) * ids_stride + c % n_slots], 0), n_experts - 1);
        atomicAdd(&s_cnt[e], 1);
    }
    __syncthreads();
    if (t == 0) {
        int o = 0, n = 0;
        for (int e = 0; e < n_experts; e++) {
            s_cur[e] = o;
            g.offset[e] = o;
            g.count[e] = s_cnt[e];
            // the expert's columns in items of at most nc
            for (int j = 0; j < s_cnt[e]; j += g.nc, n++) {
                g.items[3 * n] = e;
                g.items[3 * n + 1] = o + j;
                g.items[3 * n + 2] = min(g.nc, s_cnt[e] - j);
            }
            o += s_cnt[e];
        }
        *g.n_items = n;
    }
    __syncthreads();
    for (int c = t; c < ncol; c += 256) {
        const int e = min(max(ids[(int64_t) (c / n_slots) * ids_stride + c % n_slots], 0), n_experts - 1);
        g.cols[atomicAdd(&s_cur[e], 1)] = c;
    }
}

} // namespace

bool gemv_mc_supported(const gemv_launch & L, int max_cols) {
    if (L.norm.x || !L.xq || L.ncols < 1 || max_cols < 1) return false;
    if (L.type == GGML_TYPE_Q4_K ? L.K % 256 != 0 : L.K % 32 != 0) return false;
    return L.swiglu ? launch_mc_dispatch<true>(L, nullptr, max_cols, nullptr, true)
                    : launch_mc_dispatch<false>(L, nullptr, max_cols, nullptr, true);
}

bool gemv_mc_fits(int type, int K, bool swiglu, int nc) {
    gemv_launch L{};
    L.type = type;
    L.K = K;
    L.ncols = GEMV_MC_MAX_COLS;
    L.n_mats = swiglu ? 2 : 1;
    L.swiglu = swiglu;
    L.xq = (const int8_t *) &L;   // any non-null pointer: nothing is launched
    if (type == GGML_TYPE_Q4_K ? K % 256 != 0 : K % 32 != 0) return false;
    expert_groups g{};
    g.nc = nc;
    const expert_groups * G = nc > 0 ? &g : nullptr;
    return swiglu ? launch_mc_dispatch<true>(L, G, GEMV_MC_MAX_COLS, nullptr, true)
                  : launch_mc_dispatch<false>(L, G, GEMV_MC_MAX_COLS, nullptr, true);
}

void launch_gemv_mc(const gemv_launch & L, const expert_groups * G, int max_cols, hipStream_t st) {
    if (L.swiglu && (L.n_mats != 2 || L.m[0].n_rows != L.m[1].n_rows)) HIP_ABORT("gemv_mc: swiglu needs two equal matrices");
    if (G && (!L.ids || L.n_slots < 1 || L.x_cols < 1 || L.n_experts < 1)) HIP_ABORT("gemv_mc: bad mul_mat_id geometry");
    if (!gemv_mc_supported(L, G ? max_cols : L.ncols) || (G && !gemv_mc_fits(L.type, L.K, L.swiglu, G->nc))) {
        HIP_ABORT("gemv_mc: unsupported launch (type %d, K=%d)", L.type, L.K);
    }
    const bool ok = L.swiglu ? launch_mc_dispatch<true>(L, G, max_cols, st, false) : launch_mc_dispatch<false>(L, G, max_cols, st, false);
    if (!ok) HIP_ABORT("gemv_mc: no workgroup shape fits (type %d, K=%d)", L.type, L.K);
}

void launch_moe_group(const int32_t * ids, int64_t ids_stride, int n_slots, int n_tok, int n_experts, const expert_groups & g,
                      hipStream_t st) {
    if (n_experts < 1 || n_experts > 4096 || n_slots < 1 || n_tok < 1) HIP_ABORT("moe_group: %d experts", n_experts);
    const int ncol = n_slots * n_tok;
    if (g.nc < 1 || g.nc > GEMV_MC_MAX_COLS || g.max_items < std::min(n_experts, ncol) + (ncol + g.nc - 1) / g.nc) {
        HIP_ABORT("moe_group: %d items of %d columns cannot hold %d columns", g.max_items, g.nc, ncol);
    }
    launch(moe_group_kernel, dim3(1), dim3(256), (size_t) n_experts * 2 * sizeof(int), st, ids, ids_stride, n_slots, n_tok,
           n_experts, g);
}
