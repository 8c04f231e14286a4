// ggml-alloc.h — graph activation allocator.
//
// Reference call sites: init_decode_session (model.cpp:1486, ggml_gallocr_new with the backend's
// default buffer type), forward_step (model.cpp:1563, ggml_gallocr_alloc_graph every step: the
// graph shape changes as n_kv grows, so the plan is redone and the buffer grows when needed),
// free_decode_session (model.cpp:1492).
#pragma once

#include "ggml.h"

#ifdef __cplusplus
extern "C" {
#endif

// the buffer-type handle of ggml-backend.h (declared here as well, so that ggml-backend.h can
// include this header the way the reference's model.h expects: model.h:380 names ggml_gallocr_t
// with only ggml-backend.h included)
typedef struct ggml_backend_buffer_type * ggml_backend_buffer_type_t;
typedef struct ggml_gallocr * ggml_gallocr_t;

GGML_API ggml_gallocr_t ggml_gallocr_new(ggml_backend_buffer_type_t buft);
GGML_API void           ggml_gallocr_free(ggml_gallocr_t galloc);

// Assigns device memory to every tensor of the graph that has no data yet (nodes and leafs);
// views get their storage from their view_src. Returns false if allocation failed.
GGML_API bool   ggml_gallocr_alloc_graph(ggml_gallocr_t galloc, struct ggml_cgraph * graph);
GGML_API bool   ggml_gallocr_reserve(ggml_gallocr_t galloc, struct ggml_cgraph * graph);
GGML_API size_t ggml_gallocr_get_buffer_size(ggml_gallocr_t galloc, int buffer_id);

#ifdef __cplusplus
}
#endif
