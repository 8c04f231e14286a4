// ggml-backend.cpp — backend-independent half of the backend API: buffer/tensor plumbing,
// context allocation (ggml_backend_alloc_ctx_tensors) and the backend registry.
#include "ggml-backend-impl.h"
#include "ggml-vulkan.h"

#include <cstdio>
#include <dlfcn.h>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <string>
#include <vector>

#define BK_ABORT(...) do { fprintf(stderr, "ggml-backend error: " __VA_ARGS__); fputc('\n', stderr); abort(); } while (0)

extern "C" {

// ---- buffer types ----
const char * ggml_backend_buft_name(ggml_backend_buffer_type_t buft) { return buft->iface.get_name(buft); }
ggml_backend_buffer_t ggml_backend_buft_alloc_buffer(ggml_backend_buffer_type_t buft, size_t size) {
    return buft->iface.alloc_buffer(buft, size);
}
size_t ggml_backend_buft_get_alignment(ggml_backend_buffer_type_t buft) { return buft->iface.get_alignment(buft); }
size_t ggml_backend_buft_get_alloc_size(ggml_backend_buffer_type_t buft, const struct ggml_tensor * tensor) {
    return buft->iface.get_alloc_size ? buft->iface.get_alloc_size(buft, tensor) : ggml_nbytes(tensor);
}
bool ggml_backend_buft_is_host(ggml_backend_buffer_type_t buft) { return buft->iface.is_host && buft->iface.is_host(buft); }

// ---- buffers ----
ggml_backend_buffer_t ggml_backend_buffer_init(ggml_backend_buffer_type_t buft, struct ggml_backend_buffer_i iface,
                                               void * context, size_t size) {
    ggml_backend_buffer * b = new ggml_backend_buffer();
    b->iface = iface;
    b->buft = buft;
    b->context = context;
    b->size = size;
    return b;
}

const char * ggml_backend_buffer_name(ggml_backend_buffer_t buffer) { return ggml_backend_buft_name(buffer->buft); }

void ggml_backend_buffer_free(ggml_backend_buffer_t buffer) {
    if (!buffer) return;
    if (buffer->iface.free_buffer) buffer->iface.free_buffer(buffer);
    delete buffer;
}

void * ggml_backend_buffer_get_base(ggml_backend_buffer_t buffer) { return buffer->iface.get_base(buffer); }
size_t ggml_backend_buffer_get_size(ggml_backend_buffer_t buffer) { return buffer->size; }
void ggml_backend_buffer_clear(ggml_backend_buffer_t buffer, uint8_t value) { buffer->iface.clear(buffer, value); }
bool ggml_backend_buffer_is_host(ggml_backend_buffer_t buffer) { return ggml_backend_buft_is_host(buffer->buft); }
ggml_backend_buffer_type_t ggml_backend_buffer_get_type(ggml_backend_buffer_t buffer) { return buffer->buft; }

enum ggml_status ggml_backend_tensor_alloc(ggml_backend_buffer_t buffer, struct ggml_tensor * tensor, void * addr) {
    if (tensor->buffer != nullptr || tensor->data != nullptr || tensor->view_src != nullptr) {
        BK_ABORT("tensor '%s' is already allocated", tensor->name);
    }
    char * base = (char *) ggml_backend_buffer_get_base(buffer);
    if ((char *) addr < base || (char *) addr + ggml_backend_buft_get_alloc_size(buffer->buft, tensor) > base + buffer->size) {
        BK_ABORT("tensor '%s' does not fit in its buffer", tensor->name);
    }
    tensor->buffer = buffer;
    tensor->data = addr;
    if (buffer->iface.init_tensor) return buffer->iface.init_tensor(buffer, tensor);
    return GGML_STATUS_SUCCESS;
}

enum ggml_status ggml_backend_view_init(struct ggml_tensor * tensor) {
    ggml_tensor * src = tensor->view_src;
    if (!src || !src->buffer || !src->data) BK_ABORT("view '%s' has no allocated source", tensor->name);
    tensor->buffer = src->buffer;
    tensor->data = (char *) src->data + tensor->view_offs;
    if (src->buffer->iface.init_tensor) return src->buffer->iface.init_tensor(src->buffer, tensor);
    return GGML_STATUS_SUCCESS;
}

// ---- tensor data access ----
static ggml_backend_buffer_t tensor_buffer(const ggml_tensor * t) {
    return t->view_src ? t->view_src->buffer : t->buffer;
}

void ggml_backend_tensor_set(struct ggml_tensor * tensor, const void * data, size_t offset, size_t size) {
    ggml_backend_buffer_t buf = tensor_buffer(tensor);
    if (size == 0) return;
    if (!buf || !tensor->data) BK_ABORT("tensor_set: tensor '%s' is not allocated", tensor->name);
    if (offset + size > ggml_nbytes(tensor)) BK_ABORT("tensor_set: write out of bounds for '%s'", tensor->name);
    buf->iface.set_tensor(buf, tensor, data, offset, size);
}

void ggml_backend_tensor_get(const struct ggml_tensor * tensor, void * data, size_t offset, size_t size) {
    ggml_backend_buffer_t buf = tensor_buffer(tensor);
    if (size == 0) return;
    if (!buf || !tensor->data) BK_ABORT("tensor_get: tensor '%s' is not allocated", tensor->name);
    if (offset + size > ggml_nbytes(tensor)) BK_ABORT("tensor_get: read out of bounds for '%s'", tensor->name);
    buf->iface.get_tensor(buf, tensor, data, offset, size);
}

void ggml_backend_tensor_memset(struct ggml_tensor * tensor, uint8_t value, size_t offset, size_t size) {
    ggml_backend_buffer_t buf = tensor_buffer(tensor);
    if (size == 0) return;
    if (!buf || !tensor->data) BK_ABORT("tensor_memset: tensor '%s' is not allocated", tensor->name);
    if (offset + size > ggml_nbytes(tensor)) BK_ABORT("tensor_memset: out of bounds for '%s'", tensor->name);
    if (!buf->iface.memset_tensor) BK_ABORT("tensor_memset: not supported by buffer type %s", ggml_backend_buffer_name(buf));
    buf->iface.memset_tensor(buf, tensor, value, offset, size);
}

// ---- backends ----
const char * ggml_backend_name(ggml_backend_t backend) { return backend ? backend->iface.get_name(backend) : "NULL"; }
void ggml_backend_free(ggml_backend_t backend) { if (backend) backend->iface.free(backend); }
ggml_backend_buffer_type_t ggml_backend_get_default_buffer_type(ggml_backend_t backend) {
    return backend->iface.get_default_buffer_type(backend);
}
ggml_backend_buffer_t ggml_backend_alloc_buffer(ggml_backend_t backend, size_t size) {
    return ggml_backend_buft_alloc_buffer(ggml_backend_get_default_buffer_type(backend), size);
}
size_t ggml_backend_get_alignment(ggml_backend_t backend) {
    return ggml_backend_buft_get_alignment(ggml_backend_get_default_buffer_type(backend));
}
void ggml_backend_set_eval_callback(ggml_backend_t backend, ggml_backend_eval_callback cb, void * user_data) {
    if (!backend->iface.set_eval_callback) BK_ABORT("backend %s does not report node evaluations", ggml_backend_name(backend));
    backend->iface.set_eval_callback(backend, cb, user_data);
}
void ggml_backend_synchronize(ggml_backend_t backend) { if (backend->iface.synchronize) backend->iface.synchronize(backend); }
enum ggml_status ggml_backend_graph_compute(ggml_backend_t backend, struct ggml_cgraph * cgraph) {
    enum ggml_status st = backend->iface.graph_compute(backend, cgraph);
    ggml_backend_synchronize(backend);
    return st;
}
enum ggml_status ggml_backend_graph_compute_async(ggml_backend_t backend, struct ggml_cgraph * cgraph) {
    if (backend->iface.graph_compute_async) return backend->iface.graph_compute_async(backend, cgraph);
    return backend->iface.graph_compute(backend, cgraph);
}

// ---- allocate every data-less tensor of a context in one buffer ----
ggml_backend_buffer_t ggml_backend_alloc_ctx_tensors_from_buft(struct ggml_context * ctx, ggml_backend_buffer_type_t buft) {
    const size_t align = ggml_backend_buft_get_alignment(buft);
    size_t total = 0;
    for (ggml_tensor * t = ggml_get_first_tensor(ctx); t; t = ggml_get_next_tensor(ctx, t)) {
        if (t->data || t->view_src) continue;
        total = GGML_PAD(total, align) + ggml_backend_buft_get_alloc_size(buft, t);
    }
    if (total == 0) return nullptr;
    ggml_backend_buffer_t buf = ggml_backend_buft_alloc_buffer(buft, GGML_PAD(total, align));
    if (!buf) return nullptr;
    char * base = (char *) ggml_backend_buffer_get_base(buf);
    size_t off = 0;
    for (ggml_tensor * t = ggml_get_first_tensor(ctx); t; t = ggml_get_next_tensor(ctx, t)) {
        if (t->data || t->view_src) continue;
        off = GGML_PAD(off, align);
        ggml_backend_tensor_alloc(buf, t, base + off);
        off += ggml_backend_buft_get_alloc_size(buft, t);
    }
    for (ggml_tensor * t = ggml_get_first_tensor(ctx); t; t = ggml_get_next_tensor(ctx, t)) {
        if (t->view_src && !t->data) ggml_backend_view_init(t);
    }
    return buf;
}

ggml_backend_buffer_t ggml_backend_alloc_ctx_tensors(struct ggml_context * ctx, ggml_backend_t backend) {
    return ggml_backend_alloc_ctx_tensors_from_buft(ctx, ggml_backend_get_default_buffer_type(backend));
}

// ---- registry ----
namespace {
struct reg_entry { std::string name; ggml_backend_init_fn init; };
std::mutex & reg_mutex() { static std::mutex m; return m; }
std::vector<reg_entry> & reg_list() { static std::vector<reg_entry> v; return v; }

bool name_eq(const std::string & a, const char * b) {
    if (a.size() != strlen(b)) return false;
    for (size_t i = 0; i < a.size(); i++) if (tolower((unsigned char) a[i]) != tolower((unsigned char) b[i])) return false;
    return true;
}
}

void ggml_backend_register(const char * name, ggml_backend_init_fn init) {
    std::lock_guard<std::mutex> lk(reg_mutex());
    for (reg_entry & e : reg_list()) if (name_eq(e.name, name)) { e.init = init; return; }
    reg_list().push_back({ name, init });
}

ggml_backend_t ggml_backend_init_by_name(const char * name, const char * params) {
    ggml_backend_init_fn fn = nullptr;
    {
        std::lock_guard<std::mutex> lk(reg_mutex());
        for (const reg_entry & e : reg_list()) if (name_eq(e.name, name)) fn = e.init;
    }
    return fn ? fn(params) : nullptr;
}

bool ggml_backend_load(const char * path) {
    void * h = dlopen(path, RTLD_NOW | RTLD_GLOBAL);
    if (!h) {
        fprintf(stderr, "ggml_backend_load: %s\n", dlerror());
        return false;
    }
    return true;
}

size_t ggml_backend_reg_count(void) { std::lock_guard<std::mutex> lk(reg_mutex()); return reg_list().size(); }

// ggml-vulkan.h: this build has no Vulkan backend (model.cpp:800-813 then reports that no Vulkan
// device is available)
int ggml_backend_vk_get_device_count(void) { return 0; }
void ggml_backend_vk_get_device_description(int device, char * description, size_t description_size) {
    (void) device;
    if (description && description_size) description[0] = '\0';
}
ggml_backend_t ggml_backend_vk_init(size_t dev_num) {
    (void) dev_num;
    return nullptr;
}
const char * ggml_backend_reg_name(size_t i) {
    std::lock_guard<std::mutex> lk(reg_mutex());
    return i < reg_list().size() ? reg_list()[i].name.c_str() : nullptr;
}

} // extern "C"
