// ggml-hip.h — the MI355X (gfx950) backend, selected as `--backend hip`.
//
// The first three entry points mirror the Vulkan trio init_backend() calls (model.cpp:800-813:
// ggml_backend_vk_get_device_count / _get_device_description / _init); init_backend("hip") calls
// these instead. Device memory, weights, the F16 KV cache and activations live in HIP buffers
// owned by the backend; ggml_backend_graph_compute runs the graph with hand-written gfx950
// kernels and returns when the results are complete.
#pragma once

#include "ggml-backend.h"

#ifdef __cplusplus
extern "C" {
#endif

// replaces ggml_backend_vk_get_device_count (model.cpp:801)
GGML_API int  ggml_backend_hip_get_device_count(void);
// replaces ggml_backend_vk_get_device_description (model.cpp:806)
GGML_API void ggml_backend_hip_get_device_description(int device, char * description, size_t description_size);
// replaces ggml_backend_vk_init (model.cpp:808); NULL if the device cannot be opened
GGML_API ggml_backend_t ggml_backend_hip_init(int device);
GGML_API bool ggml_backend_is_hip(ggml_backend_t backend);
GGML_API ggml_backend_buffer_type_t ggml_backend_hip_buffer_type(int device);

// ---- extensions of this backend (no counterpart in the reference) ----

// Bytes of device scratch ggml_backend_hip_graph_compute_static can give a graph's kernels.
#define GGML_HIP_STATIC_SCRATCH_BYTES (64 << 20)

// ggml_backend_graph_compute without any device allocation: no counterpart in the reference; for
// callers that cannot allocate (serving loops, harnesses that forbid hipMalloc). The kernels'
// scratch (attention scores and partials, quantized activations, expert groups, argmax parts)
// comes from a file-scope device array of GGML_HIP_STATIC_SCRATCH_BYTES that every GPU the
// library runs on holds until the process ends; the graph's tensors are the caller's as with
// ggml_backend_graph_compute, and the result is the same. Like ggml_backend_graph_compute it
// launches on the backend's own stream and returns after the device finished, so it cannot be
// recorded by a caller's HIP graph capture. A graph needing more scratch is rejected with
// GGML_STATUS_ALLOC_FAILED and a message, but only at the node where the array ran out: the
// kernels queued before that node have run, including any KV-cache append folded into an earlier
// attention, so cache rows of the step may already be written; the outputs are undefined. Calls
// share their GPU's array and keep its last contents (no kernel relies on it starting at zero):
// calls that overlap on one GPU (several threads or backends) race. Fails with profiling on (it
// creates events).
GGML_API enum ggml_status ggml_backend_hip_graph_compute_static(ggml_backend_t backend, struct ggml_cgraph * cgraph);

// Token sampling on the device: replaces `int32_t sample(sampler &, std::vector<float> & logits,
// const std::vector<int32_t> & recent_tokens)` (model.h:432-435, model.cpp:1675-1728) for logits
// that stay in device memory. Same parameters (model.h:418-425, minus the seed) and the same result:
// the repetition penalty over the last repeat_last_n entries of recent (a negative repeat_last_n
// takes all of them; ids outside the row are skipped), then argmax for temp <= 0 (first index of
// the maximum), else temperature, top-k (top_k <= 0 or >= the row length: no cut), top-p (>= 1:
// no cut) and the weighted draw of std::discrete_distribution on the uniform variate u in [0, 1)
// that the caller's generator supplies (libstdc++ draws it as std::generate_canonical<double, 53>
// of its std::mt19937). *used_draw reports whether the draw consumed u: it does not for temp <= 0
// or when fewer than two tokens survive the cuts, and the reference's generator is then not
// advanced either, so a caller keeps u for its next call. Logits with equal values are ordered by
// ascending token id before the cuts (std::partial_sort leaves their order unspecified). logits:
// an F32 tensor in this backend's buffer, row `row` (ggml row index over ne[1..3]) contiguous.
// Synchronous: returns when the token id is on the host. Fails (GGML_STATUS_FAILED, with a message
// on stderr) for another backend or buffer, a bad row, or a maximum that is not finite.
struct ggml_hip_sampler_params {
    float   temp;
    int32_t top_k;
    float   top_p;
    float   repeat_penalty;
    int32_t repeat_last_n;
};
GGML_API enum ggml_status ggml_backend_hip_sample(ggml_backend_t backend, const struct ggml_tensor * logits, int64_t row,
                                                  const struct ggml_hip_sampler_params * params,
                                                  const int32_t * recent, size_t n_recent, double u,
                                                  int32_t * token, bool * used_draw);

// Graph-level fusion (fused norm+quantize, QKV/gate-up multi-GEMV, rope+KV append, split-KV
// decode attention). On by default; off runs one kernel per ggml node. Used by the parity tests
// to check both paths against the oracle.
GGML_API void ggml_backend_hip_set_fusion(ggml_backend_t backend, bool enable);

// Per-kernel timing with HIP events recorded on the backend's own stream. While enabled, every
// launch of graph_compute is bracketed by events; stats accumulate per kernel name until reset.
// The entry "host_enqueue" holds the host time each graph_compute spends walking the graph and
// submitting its kernels (one count per compute).
GGML_API void ggml_backend_hip_set_profiling(ggml_backend_t backend, bool enable);
// Restricts the events to kernels whose name starts with prefix (NULL or "" = every kernel), so a
// timed run can measure one kernel without bracketing every launch.
GGML_API void ggml_backend_hip_set_profile_filter(ggml_backend_t backend, const char * prefix);
// Times one graph compute in every `every` (1 = all) while profiling is on: reading back the
// events costs host time after each timed compute, which sampling keeps out of most steps.
GGML_API void ggml_backend_hip_set_profile_sampling(ggml_backend_t backend, int every);
GGML_API void ggml_backend_hip_reset_profile(ggml_backend_t backend);
// Number of distinct kernel names recorded.
GGML_API int  ggml_backend_hip_profile_count(ggml_backend_t backend);
// Entry i: name, number of launches, total milliseconds, total algorithmic bytes (weights,
// activations and KV bytes the launches must touch once). Returns false if i is out of range.
GGML_API bool ggml_backend_hip_profile_entry(ggml_backend_t backend, int i, char * name, size_t name_size,
                                             int64_t * launches, double * total_ms, double * total_bytes);

#ifdef __cplusplus
}
#endif
