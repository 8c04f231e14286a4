// ggml-backend-impl.h — interface a backend implements to plug into ggml-backend.h.
//
// This is the plugin contract between the core library and the device backends (the HIP backend
// in this package and the CPU reference backend used as the test oracle). It mirrors the role of
// ggml's own ggml-backend-impl.h: a buffer-type vtable, a buffer vtable and a backend vtable.
#pragma once

#include "ggml-backend.h"

#ifdef __cplusplus
extern "C" {
#endif

struct ggml_backend_buffer_type_i {
    const char *          (*get_name)      (ggml_backend_buffer_type_t buft);
    ggml_backend_buffer_t (*alloc_buffer)  (ggml_backend_buffer_type_t buft, size_t size);
    size_t                (*get_alignment) (ggml_backend_buffer_type_t buft);
    size_t                (*get_alloc_size)(ggml_backend_buffer_type_t buft, const struct ggml_tensor * tensor); // NULL => ggml_nbytes
    bool                  (*is_host)       (ggml_backend_buffer_type_t buft);
    // true: the graph allocator gives every tensor of a graph its own memory instead of recycling
    // the memory of tensors whose consumers have run (lets a backend reorder/fuse nodes freely)
    bool                  (*no_reuse)      (ggml_backend_buffer_type_t buft);
};

struct ggml_backend_buffer_type {
    struct ggml_backend_buffer_type_i iface;
    void * context;
};

struct ggml_backend_buffer_i {
    void   (*free_buffer)(ggml_backend_buffer_t buffer);
    void * (*get_base)   (ggml_backend_buffer_t buffer);
    // called once per tensor when it is placed in the buffer (may be NULL)
    enum ggml_status (*init_tensor)(ggml_backend_buffer_t buffer, struct ggml_tensor * tensor);
    void   (*set_tensor) (ggml_backend_buffer_t buffer, struct ggml_tensor * tensor, const void * data, size_t offset, size_t size);
    void   (*get_tensor) (ggml_backend_buffer_t buffer, const struct ggml_tensor * tensor, void * data, size_t offset, size_t size);
    void   (*memset_tensor)(ggml_backend_buffer_t buffer, struct ggml_tensor * tensor, uint8_t value, size_t offset, size_t size);
    void   (*clear)      (ggml_backend_buffer_t buffer, uint8_t value);
};

struct ggml_backend_buffer {
    struct ggml_backend_buffer_i iface;
    ggml_backend_buffer_type_t   buft;
    void * context;
    size_t size;
};

GGML_API ggml_backend_buffer_t ggml_backend_buffer_init(ggml_backend_buffer_type_t buft,
        struct ggml_backend_buffer_i iface, void * context, size_t size);

struct ggml_backend_i {
    const char * (*get_name)(ggml_backend_t backend);
    void         (*free)(ggml_backend_t backend);
    ggml_backend_buffer_type_t (*get_default_buffer_type)(ggml_backend_t backend);
    enum ggml_status (*graph_compute)(ggml_backend_t backend, struct ggml_cgraph * cgraph);
    void         (*synchronize)(ggml_backend_t backend); // may be NULL
    void         (*set_eval_callback)(ggml_backend_t backend, ggml_backend_eval_callback cb, void * user_data); // may be NULL
    enum ggml_status (*graph_compute_async)(ggml_backend_t backend, struct ggml_cgraph * cgraph); // may be NULL
};

struct ggml_backend {
    struct ggml_backend_i iface;
    void * context;
};

// graph internals needed by backends and allocators
struct ggml_cgraph {
    int size;
    int n_nodes;
    int n_leafs;
    struct ggml_tensor ** nodes;
    struct ggml_tensor ** leafs;
    // open-addressing set of visited tensors (capacity hash_size)
    size_t hash_size;
    struct ggml_tensor ** hash_keys;
};

#ifdef __cplusplus
}
#endif
