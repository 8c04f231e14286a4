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
#include "gemv_mc_impl.h"

#include "ggml.h"

namespace {

using namespace gemv_mc_detail;

template <bool SWIGLU>
static bool launch_mc_dispatch(const gemv_launch & L, const expert_groups * G, int max_cols, hipStream_t st, bool dry) {
    switch (L.type) {
        case GGML_TYPE_Q4_0: return launch_mc_q4_0(SWIGLU, L, G, max_cols, st, dry);
        case GGML_TYPE_Q8_0: return launch_mc_q8_0(SWIGLU, L, G, max_cols, st, dry);
        case GGML_TYPE_Q4_K: return launch_mc_q4_k(SWIGLU, L, G, max_cols, st, dry);
        default: return false;
    }
}

// One workgroup: the columns (token, slot) of a mul_mat_id grouped by expert. Counts and cursors
// live in LDS (shared-memory atomics); the order inside an expert's list is arbitrary, which does
// not change any result (every column is computed on its own).
// inclusive sum over the workgroup's 256 threads (wave shuffles, then the waves' totals in order)
__device__ __forceinline__ int block_scan_256(int v, int * s_w) {
    const int lane = threadIdx.x % WAVE, wave = threadIdx.x / WAVE;
#pragma unroll
    for (int o = 1; o < WAVE; o <<= 1) {
        const int u = __shfl_up(v, o, WAVE);
        if (lane >= o) v += u;
    }
    if (lane == WAVE - 1) s_w[wave] = v;
    __syncthreads();
    for (int w = 0; w < wave; w++) v += s_w[w];
    return v;
}

// The expert lists of a mul_mat_id's columns: count per expert, each expert's start in cols, the
// work items (expert, start, up to nc columns) in expert order, and the columns by expert. Each
// thread takes a contiguous run of experts; its run's first column and first item come from a
// scan over the threads' run totals, so no thread walks all experts.
__global__ __launch_bounds__(256) void moe_group_kernel(const int32_t * ids, int64_t ids_stride, int n_slots, int n_tok,
                                                        int n_experts, const expert_groups g) {
    extern __shared__ int s_cnt[];
    int * s_cur = s_cnt + n_experts;
    __shared__ int s_w[256 / WAVE];
    const int t = threadIdx.x, ncol = n_slots * n_tok;
    for (int e = t; e < n_experts; e += 256) s_cnt[e] = 0;
    __syncthreads();
    // the column's expert (read once, kept for the scatter below when one column per thread covers
    // the launch's columns)
    int ec[4];
#pragma unroll
    for (int k = 0; k < 4; k++) {
        const int c = t + k * 256;
        ec[k] = -1;
        if (c < ncol) {
            const int tk = c / n_slots;
            ec[k] = min(max(ids[(int64_t) tk * ids_stride + (c - tk * n_slots)], 0), n_experts - 1);
            atomicAdd(&s_cnt[ec[k]], 1);
        }
    }
    for (int c = t + 4 * 256; c < ncol; c += 256) {
        const int tk = c / n_slots;
        atomicAdd(&s_cnt[min(max(ids[(int64_t) tk * ids_stride + (c - tk * n_slots)], 0), n_experts - 1)], 1);
    }
    __syncthreads();
    // this thread's run of experts [e0, e1): its columns and items, then the scans
    const int per = (n_experts + 255) / 256;
    const int e0 = min(t * per, n_experts), e1 = min(e0 + per, n_experts);
    int cols = 0, its = 0;
    for (int e = e0; e < e1; e++) {
        cols += s_cnt[e];
        its += (s_cnt[e] + g.nc - 1) / g.nc;
    }
    const int cend = block_scan_256(cols, s_w);
    __syncthreads();                                   // s_w reused by the second scan
    const int iend = block_scan_256(its, s_w);
    int o = cend - cols, n = iend - its;
    for (int e = e0; e < e1; e++) {
        const int cnt = s_cnt[e];
        s_cur[e] = o;
        g.offset[e] = o;
        g.count[e] = cnt;
        // the expert's columns in items of at most nc
        for (int j = 0; j < cnt; j += g.nc, n++) {
            g.items[3 * n] = e;
            g.items[3 * n + 1] = o + j;
            g.items[3 * n + 2] = min(g.nc, cnt - j);
        }
        o += cnt;
    }
    if (t == 255) *g.n_items = iend;
    __syncthreads();
#pragma unroll
    for (int k = 0; k < 4; k++) {
        if (ec[k] >= 0) g.cols[atomicAdd(&s_cur[ec[k]], 1)] = t + k * 256;
    }
    for (int c = t + 4 * 256; c < ncol; c += 256) {
        const int tk = c / n_slots;
        const int e = min(max(ids[(int64_t) tk * ids_stride + (c - tk * n_slots)], 0), n_experts - 1);
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
