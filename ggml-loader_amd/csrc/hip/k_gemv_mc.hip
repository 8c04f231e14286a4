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
