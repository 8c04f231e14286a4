// Test infrastructure only: calls the reference's own sampler (GGML-Loader src/model.cpp:1668-1728,
// init_sampler + sample), compiled from its source by Makefile.ref, so that the tests can pin the
// oracle's restatement (oracle_sample) on it. Each call samples the same logits and window again
// with the sampler's generator running on, as a decode loop calls it.
#include "model.h"

#include <vector>

extern "C" int ref_sample_run(const float * logits, int64_t n, const int32_t * recent, int64_t n_recent, float temp,
                              int32_t top_k, float top_p, float repeat_penalty, int32_t repeat_last_n, uint32_t seed,
                              int n_calls, int32_t * out) {
    sampler_params sp;
    sp.temp = temp;
    sp.top_k = top_k;
    sp.top_p = top_p;
    sp.repeat_penalty = repeat_penalty;
    sp.repeat_last_n = repeat_last_n;
    sp.seed = seed;
    sampler smp = init_sampler(sp);
    const std::vector<int32_t> rec(recent, recent + n_recent);
    for (int c = 0; c < n_calls; c++) {
        std::vector<float> l(logits, logits + n);
        out[c] = sample(smp, l, rec);
    }
    return 0;
}
