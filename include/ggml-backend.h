// ggml-backend.h — backend / buffer API (the plugin surface the forward pass runs through).
//
// Every function keeps ggml's name and semantics. Call sites in the reference:
//   ggml_backend_alloc_ctx_tensors  model.cpp:736, 834, 859
//   ggml_backend_tensor_set / _get  model.cpp:763, 777, 1568-1592
//   ggml_backend_graph_compute      model.cpp:1588 (synchronous: complete on return)
//   ggml_backend_buffer_free        cmd_bench.cpp:158-160
//   ggml_backend_buffer_get_size    cmd_bench.cpp:119
//   ggml_backend_buffer_clear       cmd_chat.cpp:759
//   ggml_backend_get_default_buffer_type  model.cpp:1486
//   ggml_backend_free               cmd_bench.cpp:162
#pragma once

#include "ggml.h"
#include "ggml-alloc.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef struct ggml_backend_buffer_type * ggml_backend_buffer_type_t;
typedef struct ggml_backend_buffer      * ggml_backend_buffer_t;
typedef struct ggml_backend             * ggml_backend_t;

enum ggml_status {
    GGML_STATUS_ALLOC_FAILED = -2,
    GGML_STATUS_FAILED       = -1,
    GGML_STATUS_SUCCESS      = 0,
    GGML_STATUS_ABORTED      = 1,
};

// ---- buffer types ----
GGML_API const char *          ggml_backend_buft_name(ggml_backend_buffer_type_t buft);
GGML_API ggml_backend_buffer_t ggml_backend_buft_alloc_buffer(ggml_backend_buffer_type_t buft, size_t size);
GGML_API size_t                ggml_backend_buft_get_alignment(ggml_backend_buffer_type_t buft);
GGML_API size_t                ggml_backend_buft_get_alloc_size(ggml_backend_buffer_type_t buft, const struct ggml_tensor * tensor);
GGML_API bool                  ggml_backend_buft_is_host(ggml_backend_buffer_type_t buft);

// ---- buffers ----
GGML_API const char * ggml_backend_buffer_name(ggml_backend_buffer_t buffer);
GGML_API void   ggml_backend_buffer_free(ggml_backend_buffer_t buffer);
GGML_API void * ggml_backend_buffer_get_base(ggml_backend_buffer_t buffer);
GGML_API size_t ggml_backend_buffer_get_size(ggml_backend_buffer_t buffer);
GGML_API void   ggml_backend_buffer_clear(ggml_backend_buffer_t buffer, uint8_t value);
GGML_API bool   ggml_backend_buffer_is_host(ggml_backend_buffer_t buffer);
GGML_API ggml_backend_buffer_type_t ggml_backend_buffer_get_type(ggml_backend_buffer_t buffer);
// sets tensor->buffer/data for a tensor placed at `addr` inside `buffer` (used by allocators)
GGML_API enum ggml_status ggml_backend_tensor_alloc(ggml_backend_buffer_t buffer, struct ggml_tensor * tensor, void * addr);
GGML_API enum ggml_status ggml_backend_view_init(struct ggml_tensor * tensor);

// ---- backends ----
GGML_API const char * ggml_backend_name(ggml_backend_t backend);
GGML_API void         ggml_backend_free(ggml_backend_t backend);
GGML_API ggml_backend_buffer_type_t ggml_backend_get_default_buffer_type(ggml_backend_t backend);
GGML_API ggml_backend_buffer_t      ggml_backend_alloc_buffer(ggml_backend_t backend, size_t size);
GGML_API size_t ggml_backend_get_alignment(ggml_backend_t backend);
GGML_API void   ggml_backend_synchronize(ggml_backend_t backend);
GGML_API enum ggml_status ggml_backend_graph_compute(ggml_backend_t backend, struct ggml_cgraph * cgraph);
// ggml's asynchronous variant: the graph's work is queued on the backend and may still run after
// the call returns (ggml_backend_synchronize waits for it). Tensor uploads and later graphs on the
// same backend are ordered after it. Backends without queued execution compute synchronously.
GGML_API enum ggml_status ggml_backend_graph_compute_async(ggml_backend_t backend, struct ggml_cgraph * cgraph);

// Called after a backend has computed a node (its data is complete and readable with
// ggml_backend_tensor_get). `ask` is always false here; return false to stop reporting. Used by
// debugging and parity tools to compare intermediate tensors across backends.
typedef bool (*ggml_backend_eval_callback)(struct ggml_tensor * t, bool ask, void * user_data);
GGML_API void ggml_backend_set_eval_callback(ggml_backend_t backend, ggml_backend_eval_callback cb, void * user_data);

// synchronous host<->tensor copies (offset/size in bytes of the tensor's GGML layout)
GGML_API void ggml_backend_tensor_set(struct ggml_tensor * tensor, const void * data, size_t offset, size_t size);
GGML_API void ggml_backend_tensor_get(const struct ggml_tensor * tensor, void * data, size_t offset, size_t size);
GGML_API void ggml_backend_tensor_memset(struct ggml_tensor * tensor, uint8_t value, size_t offset, size_t size);

// allocates one buffer holding every tensor of ctx that has no data yet (model.cpp:736)
GGML_API ggml_backend_buffer_t ggml_backend_alloc_ctx_tensors(struct ggml_context * ctx, ggml_backend_t backend);
GGML_API ggml_backend_buffer_t ggml_backend_alloc_ctx_tensors_from_buft(struct ggml_context * ctx, ggml_backend_buffer_type_t buft);

// ---- backend registry ----
// Backends register a factory under a name ("CPU", "HIP"); callers create one by name.
// `params` is backend specific (device index for HIP, NULL for CPU).
typedef ggml_backend_t (*ggml_backend_init_fn)(const char * params);
GGML_API void           ggml_backend_register(const char * name, ggml_backend_init_fn init);
GGML_API ggml_backend_t ggml_backend_init_by_name(const char * name, const char * params);
GGML_API size_t         ggml_backend_reg_count(void);
// dlopen()s a backend library (which registers itself when loaded); false on failure
GGML_API bool           ggml_backend_load(const char * path);
GGML_API const char *   ggml_backend_reg_name(size_t i);

#ifdef __cplusplus
}
#endif
