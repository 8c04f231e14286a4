// k_gemv_mc_q4_k.hip — the multi-column GEMV kernels for Q4_K weights (gemv_mc_impl.h).
#include "gemv_mc_impl.h"

bool launch_mc_q4_k(bool swiglu, const gemv_launch & L, const expert_groups * G, int max_cols, hipStream_t st, bool dry) {
    return swiglu ? gemv_mc_detail::launch_mc_type<GGML_TYPE_Q4_K, true>(L, G, max_cols, st, dry)
                  : gemv_mc_detail::launch_mc_type<GGML_TYPE_Q4_K, false>(L, G, max_cols, st, dry);
}
