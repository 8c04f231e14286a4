// k_gemv_mc_q4_0.hip — the multi-column GEMV kernels for Q4_0 weights (gemv_mc_impl.h).
#include "gemv_mc_impl.h"

bool launch_mc_q4_0(bool swiglu, const gemv_launch & L, const expert_groups * G, int max_cols, hipStream_t st, bool dry) {
    return swiglu ? gemv_mc_detail::launch_mc_type<GGML_TYPE_Q4_0, true>(L, G, max_cols, st, dry)
                  : gemv_mc_detail::launch_mc_type<GGML_TYPE_Q4_0, false>(L, G, max_cols, st, dry);
}
