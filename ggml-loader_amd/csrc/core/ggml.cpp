// ggml.cpp — tensor metadata, contexts, op constructors and graph building.
//
// Host-only bookkeeping: no arithmetic on tensor data happens here. The semantics of every op
// constructor (result shape/type, which srcs it records, which op_params it stores) follow
// ggml's public API as GGML-Loader's build_graph uses it (reference src/model.cpp:1296-1474).
#include "ggml.h"
#include "ggml-backend-impl.h"

#include <cassert>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>

#define GGML_ABORT(...) do { fprintf(stderr, "ggml error: " __VA_ARGS__); fputc('\n', stderr); abort(); } while (0)
#define GGML_CHECK(c) do { if (!(c)) GGML_ABORT("%s:%d: check failed: %s", __FILE__, __LINE__, #c); } while (0)

// ---------------------------------------------------------------------------------------------
// type traits

namespace {
struct type_traits { const char * name; int64_t blck; size_t size; bool quantized; };

// indexed by ggml_type id; ids not listed are unknown (size 0)
type_traits g_traits[GGML_TYPE_COUNT];

struct traits_init {
    traits_init() {
        auto set = [](int id, const char * n, int64_t b, size_t s, bool q) { g_traits[id] = { n, b, s, q }; };
        set(GGML_TYPE_F32,  "f32",  1, 4, false);
        set(GGML_TYPE_F16,  "f16",  1, 2, false);
        set(GGML_TYPE_Q4_0, "q4_0", 32, 18, true);
        set(GGML_TYPE_Q4_1, "q4_1", 32, 20, true);
        set(GGML_TYPE_Q5_0, "q5_0", 32, 22, true);
        set(GGML_TYPE_Q5_1, "q5_1", 32, 24, true);
        set(GGML_TYPE_Q8_0, "q8_0", 32, 34, true);
        set(GGML_TYPE_Q8_1, "q8_1", 32, 36, true);
        set(GGML_TYPE_Q2_K, "q2_K", 256, 84, true);
        set(GGML_TYPE_Q3_K, "q3_K", 256, 110, true);
        set(GGML_TYPE_Q4_K, "q4_K", 256, 144, true);
        set(GGML_TYPE_Q5_K, "q5_K", 256, 176, true);
        set(GGML_TYPE_Q6_K, "q6_K", 256, 210, true);
        set(GGML_TYPE_Q8_K, "q8_K", 256, 292, true);
        set(16, "iq2_xxs", 256, 66, true);
        set(17, "iq2_xs", 256, 74, true);
        set(18, "iq3_xxs", 256, 98, true);
        set(19, "iq1_s", 256, 50, true);
        set(20, "iq4_nl", 32, 18, true);
        set(21, "iq3_s", 256, 110, true);
        set(22, "iq2_s", 256, 82, true);
        set(23, "iq4_xs", 256, 136, true);
        set(GGML_TYPE_I8,   "i8",   1, 1, false);
        set(GGML_TYPE_I16,  "i16",  1, 2, false);
        set(GGML_TYPE_I32,  "i32",  1, 4, false);
        set(GGML_TYPE_I64,  "i64",  1, 8, false);
        set(GGML_TYPE_F64,  "f64",  1, 8, false);
        set(29, "iq1_m", 256, 56, true);
        set(GGML_TYPE_BF16, "bf16", 1, 2, false);
        set(34, "tq1_0", 256, 54, true);
        set(35, "tq2_0", 256, 66, true);
        set(39, "mxfp4", 32, 17, true);
    }
} g_traits_init;

const type_traits & traits(enum ggml_type t) {
    static const type_traits unknown = { "unknown", 0, 0, false };
    if ((int) t < 0 || (int) t >= GGML_TYPE_COUNT || g_traits[t].size == 0) return unknown;
    return g_traits[t];
}
} // namespace

extern "C" {

const char * ggml_type_name(enum ggml_type type) { return traits(type).name; }
size_t  ggml_type_size(enum ggml_type type) { return traits(type).size; }
int64_t ggml_blck_size(enum ggml_type type) { return traits(type).blck; }
bool    ggml_is_quantized(enum ggml_type type) { return traits(type).quantized; }

size_t ggml_row_size(enum ggml_type type, int64_t ne) {
    const type_traits & t = traits(type);
    GGML_CHECK(t.blck > 0 && ne % t.blck == 0);
    return (size_t) (ne / t.blck) * t.size;
}

const char * ggml_op_name(enum ggml_op op) {
    static const char * names[GGML_OP_COUNT] = {
        "NONE", "DUP", "ADD", "MUL", "SCALE", "SQR", "RMS_NORM", "MUL_MAT", "MUL_MAT_ID", "CPY", "CONT",
        "RESHAPE", "VIEW", "PERMUTE", "TRANSPOSE", "GET_ROWS", "SOFT_MAX", "ROPE", "FLASH_ATTN_EXT",
        "ARGMAX", "UNARY", "DIV", "SUM_ROWS", "ARGSORT", "SUB", "CONCAT", "L2_NORM", "GLU", "SSM_CONV",
        "SSM_SCAN", "GATED_DELTA_NET",
    };
    return ((int) op >= 0 && op < GGML_OP_COUNT) ? names[op] : "?";
}

// ---------------------------------------------------------------------------------------------
// half / bfloat16 conversions (IEEE binary16, round-to-nearest-even)

static inline uint32_t f32_bits(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline float bits_f32(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

float ggml_fp16_to_fp32(ggml_fp16_t h) {
    const uint32_t sign = (uint32_t) (h & 0x8000u) << 16;
    const uint32_t e = (h >> 10) & 0x1f;
    const uint32_t m = h & 0x3ff;
    if (e == 0) {
        // zero or subnormal: m * 2^-24, exact in fp32
        const float v = (float) m * 5.9604644775390625e-08f;
        return sign ? -v : v;
    }
    if (e == 31) return bits_f32(sign | 0x7f800000u | (m << 13));
    return bits_f32(sign | ((e + 112) << 23) | (m << 13));
}

ggml_fp16_t ggml_fp32_to_fp16(float f) {
    const uint32_t x = f32_bits(f);
    const uint32_t sign = (x >> 16) & 0x8000u;
    const uint32_t mag = x & 0x7fffffffu;
    if (mag >= 0x7f800000u) { // inf / nan
        return (ggml_fp16_t) (sign | 0x7c00u | (mag > 0x7f800000u ? (0x200u | ((mag >> 13) & 0x3ffu)) : 0u));
    }
    if (mag >= 0x477ff000u) return (ggml_fp16_t) (sign | 0x7c00u); // rounds to +-inf
    if (mag < 0x38800000u) { // result is subnormal (or zero) in binary16
        const uint32_t e = mag >> 23;
        if (e < 102) return (ggml_fp16_t) sign;
        const uint32_t M = (mag & 0x7fffffu) | 0x800000u;
        const uint32_t shift = 126 - e;
        uint32_t q = M >> shift;
        const uint32_t rem = M & ((1u << shift) - 1);
        const uint32_t half = 1u << (shift - 1);
        if (rem > half || (rem == half && (q & 1u))) q++;
        return (ggml_fp16_t) (sign | q);
    }
    uint32_t h = (mag >> 13) - (112u << 10);
    const uint32_t rem = mag & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h++;
    return (ggml_fp16_t) (sign | h);
}

float ggml_bf16_to_fp32(ggml_bf16_t h) { return bits_f32((uint32_t) h.bits << 16); }

ggml_bf16_t ggml_fp32_to_bf16(float f) {
    uint32_t u = f32_bits(f);
    ggml_bf16_t r;
    if ((u & 0x7fffffffu) > 0x7f800000u) { r.bits = (uint16_t) ((u >> 16) | 64); return r; }
    r.bits = (uint16_t) ((u + (0x7fffu + ((u >> 16) & 1u))) >> 16);
    return r;
}

void ggml_fp16_to_fp32_row(const ggml_fp16_t * x, float * y, int64_t n) { for (int64_t i = 0; i < n; i++) y[i] = ggml_fp16_to_fp32(x[i]); }
void ggml_fp32_to_fp16_row(const float * x, ggml_fp16_t * y, int64_t n) { for (int64_t i = 0; i < n; i++) y[i] = ggml_fp32_to_fp16(x[i]); }

} // extern "C"

// ---------------------------------------------------------------------------------------------
// contexts: one linear arena holding object headers, tensor structs, graphs and (optionally) data

namespace {
enum obj_kind { OBJ_TENSOR = 0, OBJ_GRAPH = 1 };
struct ggml_object {
    size_t offs;           // payload offset from the arena base
    size_t size;           // payload size
    ggml_object * next;
    int kind;
    char pad[4];
};
constexpr size_t OBJ_SIZE = sizeof(ggml_object);
} // namespace

struct ggml_context {
    size_t mem_size;
    void * mem_buffer;
    bool   mem_owned;
    bool   no_alloc;
    int    n_objects;
    ggml_object * first;
    ggml_object * last;
};

static ggml_object * ctx_new_object(ggml_context * ctx, int kind, size_t size) {
    const size_t cur_end = ctx->last ? ctx->last->offs + ctx->last->size : 0;
    const size_t size_needed = GGML_PAD(size, GGML_MEM_ALIGN);
    char * base = (char *) ctx->mem_buffer;
    ggml_object * obj = (ggml_object *) (base + cur_end);
    if (cur_end + OBJ_SIZE + size_needed > ctx->mem_size) {
        GGML_ABORT("not enough space in the context's memory pool (needed %zu, available %zu)",
                   cur_end + OBJ_SIZE + size_needed, ctx->mem_size);
    }
    obj->offs = cur_end + OBJ_SIZE;
    obj->size = size_needed;
    obj->next = nullptr;
    obj->kind = kind;
    if (ctx->last) ctx->last->next = obj; else ctx->first = obj;
    ctx->last = obj;
    ctx->n_objects++;
    return obj;
}

extern "C" {

size_t ggml_tensor_overhead(void) { return OBJ_SIZE + GGML_PAD(sizeof(ggml_tensor), GGML_MEM_ALIGN); }

static size_t graph_hash_size(size_t size) {
    size_t n = 64;
    while (n < 2 * size) n <<= 1;
    return n;
}

static size_t graph_nbytes(size_t size) {
    return sizeof(ggml_cgraph) + 2 * size * sizeof(ggml_tensor *) + graph_hash_size(size) * sizeof(ggml_tensor *);
}

size_t ggml_graph_overhead_custom(size_t size, bool grads) {
    (void) grads;
    return OBJ_SIZE + GGML_PAD(graph_nbytes(size), GGML_MEM_ALIGN);
}
size_t ggml_graph_overhead(void) { return ggml_graph_overhead_custom(GGML_DEFAULT_GRAPH_SIZE, false); }

struct ggml_context * ggml_init(struct ggml_init_params params) {
    ggml_context * ctx = (ggml_context *) calloc(1, sizeof(ggml_context));
    if (!ctx) return nullptr;
    size_t mem_size = params.mem_size ? params.mem_size : GGML_MEM_ALIGN;
    ctx->mem_size = mem_size;
    if (params.mem_buffer) {
        ctx->mem_buffer = params.mem_buffer;
        ctx->mem_owned = false;
    } else {
        ctx->mem_buffer = aligned_alloc(64, GGML_PAD(mem_size, 64));
        if (!ctx->mem_buffer) { free(ctx); return nullptr; }
        ctx->mem_owned = true;
    }
    ctx->no_alloc = params.no_alloc;
    return ctx;
}

void ggml_free(struct ggml_context * ctx) {
    if (!ctx) return;
    if (ctx->mem_owned) free(ctx->mem_buffer);
    free(ctx);
}

size_t ggml_used_mem(const struct ggml_context * ctx) { return ctx->last ? ctx->last->offs + ctx->last->size : 0; }
bool ggml_get_no_alloc(struct ggml_context * ctx) { return ctx->no_alloc; }
void ggml_set_no_alloc(struct ggml_context * ctx, bool no_alloc) { ctx->no_alloc = no_alloc; }

static ggml_tensor * obj_tensor(const ggml_context * ctx, ggml_object * obj) {
    return (ggml_tensor *) ((char *) ctx->mem_buffer + obj->offs);
}

struct ggml_tensor * ggml_get_first_tensor(const struct ggml_context * ctx) {
    for (ggml_object * o = ctx->first; o; o = o->next) if (o->kind == OBJ_TENSOR) return obj_tensor(ctx, o);
    return nullptr;
}

struct ggml_tensor * ggml_get_next_tensor(const struct ggml_context * ctx, struct ggml_tensor * tensor) {
    ggml_object * o = (ggml_object *) ((char *) tensor - OBJ_SIZE);
    for (o = o->next; o; o = o->next) if (o->kind == OBJ_TENSOR) return obj_tensor(ctx, o);
    return nullptr;
}

struct ggml_tensor * ggml_get_tensor(struct ggml_context * ctx, const char * name) {
    for (ggml_object * o = ctx->first; o; o = o->next) {
        if (o->kind != OBJ_TENSOR) continue;
        ggml_tensor * t = obj_tensor(ctx, o);
        if (strcmp(t->name, name) == 0) return t;
    }
    return nullptr;
}

// ---------------------------------------------------------------------------------------------
// tensors

static ggml_tensor * new_tensor_impl(ggml_context * ctx, enum ggml_type type, int n_dims, const int64_t * ne,
                                     ggml_tensor * view_src, size_t view_offs) {
    GGML_CHECK(n_dims >= 1 && n_dims <= GGML_MAX_DIMS);
    GGML_CHECK(traits(type).size > 0);
    if (view_src && view_src->view_src) {
        view_offs += view_src->view_offs;
        view_src = view_src->view_src;
    }
    int64_t nes[GGML_MAX_DIMS] = { 1, 1, 1, 1 };
    for (int i = 0; i < n_dims; i++) nes[i] = ne[i];
    size_t data_size = ggml_row_size(type, nes[0]);
    for (int i = 1; i < GGML_MAX_DIMS; i++) data_size *= (size_t) nes[i];
    if (view_src) GGML_CHECK(data_size == 0 || view_offs + data_size <= ggml_nbytes(view_src));

    const size_t alloc_data = (view_src == nullptr && !ctx->no_alloc) ? data_size : 0;
    ggml_object * obj = ctx_new_object(ctx, OBJ_TENSOR, sizeof(ggml_tensor) + alloc_data);
    ggml_tensor * t = obj_tensor(ctx, obj);
    memset(t, 0, sizeof(ggml_tensor));
    t->type = type;
    for (int i = 0; i < GGML_MAX_DIMS; i++) t->ne[i] = nes[i];
    t->nb[0] = traits(type).size;
    t->nb[1] = t->nb[0] * (size_t) (t->ne[0] / traits(type).blck);
    for (int i = 2; i < GGML_MAX_DIMS; i++) t->nb[i] = t->nb[i - 1] * (size_t) t->ne[i - 1];
    t->op = GGML_OP_NONE;
    t->view_src = view_src;
    t->view_offs = view_offs;
    if (view_src) {
        t->buffer = view_src->buffer;
        t->data = view_src->data ? (char *) view_src->data + view_offs : nullptr;
    } else if (alloc_data) {
        t->data = (char *) t + sizeof(ggml_tensor);
    }
    return t;
}

struct ggml_tensor * ggml_new_tensor(struct ggml_context * ctx, enum ggml_type type, int n_dims, const int64_t * ne) {
    return new_tensor_impl(ctx, type, n_dims, ne, nullptr, 0);
}
struct ggml_tensor * ggml_new_tensor_1d(struct ggml_context * ctx, enum ggml_type type, int64_t ne0) {
    return ggml_new_tensor(ctx, type, 1, &ne0);
}
struct ggml_tensor * ggml_new_tensor_2d(struct ggml_context * ctx, enum ggml_type type, int64_t ne0, int64_t ne1) {
    const int64_t ne[2] = { ne0, ne1 };
    return ggml_new_tensor(ctx, type, 2, ne);
}
struct ggml_tensor * ggml_new_tensor_3d(struct ggml_context * ctx, enum ggml_type type, int64_t ne0, int64_t ne1, int64_t ne2) {
    const int64_t ne[3] = { ne0, ne1, ne2 };
    return ggml_new_tensor(ctx, type, 3, ne);
}
struct ggml_tensor * ggml_new_tensor_4d(struct ggml_context * ctx, enum ggml_type type, int64_t ne0, int64_t ne1, int64_t ne2, int64_t ne3) {
    const int64_t ne[4] = { ne0, ne1, ne2, ne3 };
    return ggml_new_tensor(ctx, type, 4, ne);
}
struct ggml_tensor * ggml_dup_tensor(struct ggml_context * ctx, const struct ggml_tensor * src) {
    return ggml_new_tensor(ctx, src->type, GGML_MAX_DIMS, src->ne);
}

struct ggml_tensor * ggml_set_name(struct ggml_tensor * tensor, const char * name) {
    size_t i;
    for (i = 0; i < GGML_MAX_NAME - 1 && name[i]; i++) tensor->name[i] = name[i];
    tensor->name[i] = '\0';
    return tensor;
}
const char * ggml_get_name(const struct ggml_tensor * tensor) { return tensor->name; }

static void format_name(ggml_tensor * t, const char * fmt, const char * a, const char * b = nullptr) {
    snprintf(t->name, GGML_MAX_NAME, fmt, a, b);
}

struct ggml_tensor * ggml_view_tensor(struct ggml_context * ctx, struct ggml_tensor * src) {
    ggml_tensor * r = new_tensor_impl(ctx, src->type, GGML_MAX_DIMS, src->ne, src, 0);
    format_name(r, "%s (view)", src->name);
    for (int i = 0; i < GGML_MAX_DIMS; i++) r->nb[i] = src->nb[i];
    return r;
}

void ggml_set_input(struct ggml_tensor * tensor) { tensor->flags |= GGML_TENSOR_FLAG_INPUT; }
void ggml_set_output(struct ggml_tensor * tensor) { tensor->flags |= GGML_TENSOR_FLAG_OUTPUT; }

int64_t ggml_nelements(const struct ggml_tensor * t) { return t->ne[0] * t->ne[1] * t->ne[2] * t->ne[3]; }
int64_t ggml_nrows(const struct ggml_tensor * t) { return t->ne[1] * t->ne[2] * t->ne[3]; }

size_t ggml_nbytes(const struct ggml_tensor * t) {
    for (int i = 0; i < GGML_MAX_DIMS; i++) if (t->ne[i] <= 0) return 0;
    const int64_t blck = ggml_blck_size(t->type);
    size_t nbytes;
    if (blck == 1) {
        nbytes = ggml_type_size(t->type);
        for (int i = 0; i < GGML_MAX_DIMS; i++) nbytes += (size_t) (t->ne[i] - 1) * t->nb[i];
    } else {
        nbytes = (size_t) (t->ne[0] / blck) * t->nb[0];
        for (int i = 1; i < GGML_MAX_DIMS; i++) nbytes += (size_t) (t->ne[i] - 1) * t->nb[i];
    }
    return nbytes;
}

int ggml_n_dims(const struct ggml_tensor * t) {
    for (int i = GGML_MAX_DIMS - 1; i >= 1; --i) if (t->ne[i] > 1) return i + 1;
    return 1;
}

bool ggml_is_contiguous(const struct ggml_tensor * t) {
    size_t expect = ggml_type_size(t->type);
    if (t->ne[0] != ggml_blck_size(t->type) && t->nb[0] != expect) return false;
    expect = ggml_row_size(t->type, t->ne[0]);
    for (int i = 1; i < GGML_MAX_DIMS; i++) {
        if (t->ne[i] != 1 && t->nb[i] != expect) return false;
        expect *= (size_t) t->ne[i];
    }
    return true;
}

bool ggml_is_transposed(const struct ggml_tensor * t) { return t->nb[0] > t->nb[1]; }
bool ggml_is_permuted(const struct ggml_tensor * t) { return t->nb[0] > t->nb[1] || t->nb[1] > t->nb[2] || t->nb[2] > t->nb[3]; }

bool ggml_are_same_shape(const struct ggml_tensor * a, const struct ggml_tensor * b) {
    return a->ne[0] == b->ne[0] && a->ne[1] == b->ne[1] && a->ne[2] == b->ne[2] && a->ne[3] == b->ne[3];
}

bool ggml_can_repeat(const struct ggml_tensor * t0, const struct ggml_tensor * t1) {
    for (int i = 0; i < GGML_MAX_DIMS; i++) if (t0->ne[i] <= 0 || t1->ne[i] % t0->ne[i] != 0) return false;
    return true;
}

// ---------------------------------------------------------------------------------------------
// op constructors

static void set_op_params(ggml_tensor * t, const void * params, size_t size) {
    GGML_CHECK(size <= GGML_MAX_OP_PARAMS);
    memcpy(t->op_params, params, size);
}
static void set_op_param_f32(ggml_tensor * t, int i, float v) { memcpy(&t->op_params[i], &v, 4); }
static void set_op_param_i32(ggml_tensor * t, int i, int32_t v) { t->op_params[i] = v; }

struct ggml_tensor * ggml_get_rows(struct ggml_context * ctx, struct ggml_tensor * a, struct ggml_tensor * b) {
    GGML_CHECK(a->ne[2] == b->ne[1]);
    GGML_CHECK(b->ne[3] == 1);
    GGML_CHECK(b->type == GGML_TYPE_I32);
    const enum ggml_type type = a->type == GGML_TYPE_I32 ? GGML_TYPE_I32 : GGML_TYPE_F32;
    ggml_tensor * r = ggml_new_tensor_4d(ctx, type, a->ne[0], b->ne[0], b->ne[1], b->ne[2]);
    r->op = GGML_OP_GET_ROWS;
    r->src[0] = a;
    r->src[1] = b;
    return r;
}

struct ggml_tensor * ggml_rms_norm(struct ggml_context * ctx, struct ggml_tensor * a, float eps) {
    ggml_tensor * r = ggml_dup_tensor(ctx, a);
    set_op_param_f32(r, 0, eps);
    r->op = GGML_OP_RMS_NORM;
    r->src[0] = a;
    return r;
}

static ggml_tensor * binary_op(ggml_context * ctx, ggml_tensor * a, ggml_tensor * b, enum ggml_op op) {
    GGML_CHECK(ggml_can_repeat(b, a));
    ggml_tensor * r = ggml_dup_tensor(ctx, a);
    r->op = op;
    r->src[0] = a;
    r->src[1] = b;
    return r;
}
struct ggml_tensor * ggml_mul(struct ggml_context * ctx, struct ggml_tensor * a, struct ggml_tensor * b) { return binary_op(ctx, a, b, GGML_OP_MUL); }
struct ggml_tensor * ggml_add(struct ggml_context * ctx, struct ggml_tensor * a, struct ggml_tensor * b) { return binary_op(ctx, a, b, GGML_OP_ADD); }
struct ggml_tensor * ggml_div(struct ggml_context * ctx, struct ggml_tensor * a, struct ggml_tensor * b) { return binary_op(ctx, a, b, GGML_OP_DIV); }
struct ggml_tensor * ggml_sub(struct ggml_context * ctx, struct ggml_tensor * a, struct ggml_tensor * b) { return binary_op(ctx, a, b, GGML_OP_SUB); }

struct ggml_tensor * ggml_l2_norm(struct ggml_context * ctx, struct ggml_tensor * a, float eps) {
    ggml_tensor * r = ggml_dup_tensor(ctx, a);
    set_op_param_f32(r, 0, eps);
    r->op = GGML_OP_L2_NORM;
    r->src[0] = a;
    return r;
}

struct ggml_tensor * ggml_concat(struct ggml_context * ctx, struct ggml_tensor * a, struct ggml_tensor * b, int dim) {
    GGML_CHECK(dim >= 0 && dim < GGML_MAX_DIMS && a->type == b->type);
    int64_t ne[GGML_MAX_DIMS];
    for (int d = 0; d < GGML_MAX_DIMS; d++) {
        if (d == dim) {
            ne[d] = a->ne[d] + b->ne[d];
        } else {
            GGML_CHECK(a->ne[d] == b->ne[d]);
            ne[d] = a->ne[d];
        }
    }
    ggml_tensor * r = ggml_new_tensor(ctx, a->type, GGML_MAX_DIMS, ne);
    set_op_param_i32(r, 0, dim);
    r->op = GGML_OP_CONCAT;
    r->src[0] = a;
    r->src[1] = b;
    return r;
}

struct ggml_tensor * ggml_swiglu_split(struct ggml_context * ctx, struct ggml_tensor * a, struct ggml_tensor * b) {
    GGML_CHECK(ggml_are_same_shape(a, b));
    ggml_tensor * r = ggml_dup_tensor(ctx, a);
    set_op_param_i32(r, 0, GGML_GLU_OP_SWIGLU);
    r->op = GGML_OP_GLU;
    r->src[0] = a;
    r->src[1] = b;
    return r;
}

struct ggml_tensor * ggml_ssm_conv(struct ggml_context * ctx, struct ggml_tensor * sx, struct ggml_tensor * c) {
    GGML_CHECK(sx->ne[1] == c->ne[1] && sx->ne[0] >= c->ne[0] - 1);
    const int64_t n_t = sx->ne[0] - c->ne[0] + 1;
    ggml_tensor * r = ggml_new_tensor_3d(ctx, GGML_TYPE_F32, c->ne[1], n_t, sx->ne[2]);
    r->op = GGML_OP_SSM_CONV;
    r->src[0] = sx;
    r->src[1] = c;
    return r;
}

struct ggml_tensor * ggml_ssm_scan(struct ggml_context * ctx, struct ggml_tensor * s, struct ggml_tensor * x,
        struct ggml_tensor * dt, struct ggml_tensor * A, struct ggml_tensor * B, struct ggml_tensor * C,
        struct ggml_tensor * ids, int version) {
    ggml_tensor * r = ggml_new_tensor_1d(ctx, GGML_TYPE_F32, ggml_nelements(x) + ggml_nelements(s));
    set_op_param_i32(r, 0, version);
    r->op = GGML_OP_SSM_SCAN;
    r->src[0] = s; r->src[1] = x; r->src[2] = dt; r->src[3] = A; r->src[4] = B; r->src[5] = C; r->src[6] = ids;
    return r;
}

struct ggml_tensor * ggml_gated_delta_net(struct ggml_context * ctx, struct ggml_tensor * q, struct ggml_tensor * k,
        struct ggml_tensor * v, struct ggml_tensor * g, struct ggml_tensor * beta, struct ggml_tensor * state, int version) {
    ggml_tensor * r = ggml_new_tensor_1d(ctx, GGML_TYPE_F32, ggml_nelements(v) + ggml_nelements(state));
    set_op_param_i32(r, 0, version);
    r->op = GGML_OP_GATED_DELTA_NET;
    r->src[0] = q; r->src[1] = k; r->src[2] = v; r->src[3] = g; r->src[4] = beta; r->src[5] = state;
    return r;
}

struct ggml_tensor * ggml_scale(struct ggml_context * ctx, struct ggml_tensor * a, float s) {
    ggml_tensor * r = ggml_dup_tensor(ctx, a);
    set_op_param_f32(r, 0, s);
    r->op = GGML_OP_SCALE;
    r->src[0] = a;
    return r;
}

struct ggml_tensor * ggml_sqr(struct ggml_context * ctx, struct ggml_tensor * a) {
    ggml_tensor * r = ggml_dup_tensor(ctx, a);
    r->op = GGML_OP_SQR;
    r->src[0] = a;
    return r;
}

struct ggml_tensor * ggml_mul_mat(struct ggml_context * ctx, struct ggml_tensor * a, struct ggml_tensor * b) {
    GGML_CHECK(a->ne[0] == b->ne[0]);
    GGML_CHECK(b->ne[2] % a->ne[2] == 0 && b->ne[3] % a->ne[3] == 0);
    GGML_CHECK(!ggml_is_transposed(a));
    ggml_tensor * r = ggml_new_tensor_4d(ctx, GGML_TYPE_F32, a->ne[1], b->ne[1], b->ne[2], b->ne[3]);
    r->op = GGML_OP_MUL_MAT;
    r->src[0] = a;
    r->src[1] = b;
    return r;
}

struct ggml_tensor * ggml_mul_mat_id(struct ggml_context * ctx, struct ggml_tensor * as, struct ggml_tensor * b, struct ggml_tensor * ids) {
    GGML_CHECK(!ggml_is_transposed(as));
    GGML_CHECK(ids->type == GGML_TYPE_I32);
    GGML_CHECK(as->ne[3] == 1 && b->ne[3] == 1);
    GGML_CHECK(ids->ne[2] == 1 && ids->ne[3] == 1);
    GGML_CHECK(ids->ne[1] == b->ne[2]);
    GGML_CHECK(as->ne[0] == b->ne[0]);
    GGML_CHECK(ids->ne[0] % b->ne[1] == 0);
    ggml_tensor * r = ggml_new_tensor_4d(ctx, GGML_TYPE_F32, as->ne[1], ids->ne[0], b->ne[2], 1);
    r->op = GGML_OP_MUL_MAT_ID;
    r->src[0] = as;
    r->src[1] = b;
    r->src[2] = ids;
    return r;
}

static ggml_tensor * reshape_impl(ggml_context * ctx, ggml_tensor * a, int n, const int64_t * ne) {
    GGML_CHECK(ggml_is_contiguous(a));
    int64_t prod = 1;
    for (int i = 0; i < n; i++) prod *= ne[i];
    GGML_CHECK(prod == ggml_nelements(a));
    ggml_tensor * r = new_tensor_impl(ctx, a->type, n, ne, a, 0);
    format_name(r, "%s (reshaped)", a->name);
    r->op = GGML_OP_RESHAPE;
    r->src[0] = a;
    return r;
}
struct ggml_tensor * ggml_reshape_1d(struct ggml_context * ctx, struct ggml_tensor * a, int64_t ne0) {
    const int64_t ne[1] = { ne0 }; return reshape_impl(ctx, a, 1, ne);
}
struct ggml_tensor * ggml_reshape_2d(struct ggml_context * ctx, struct ggml_tensor * a, int64_t ne0, int64_t ne1) {
    const int64_t ne[2] = { ne0, ne1 }; return reshape_impl(ctx, a, 2, ne);
}
struct ggml_tensor * ggml_reshape_3d(struct ggml_context * ctx, struct ggml_tensor * a, int64_t ne0, int64_t ne1, int64_t ne2) {
    const int64_t ne[3] = { ne0, ne1, ne2 }; return reshape_impl(ctx, a, 3, ne);
}
struct ggml_tensor * ggml_reshape_4d(struct ggml_context * ctx, struct ggml_tensor * a, int64_t ne0, int64_t ne1, int64_t ne2, int64_t ne3) {
    const int64_t ne[4] = { ne0, ne1, ne2, ne3 }; return reshape_impl(ctx, a, 4, ne);
}

static ggml_tensor * view_impl(ggml_context * ctx, ggml_tensor * a, int n, const int64_t * ne, size_t offset) {
    ggml_tensor * r = new_tensor_impl(ctx, a->type, n, ne, a, offset);
    format_name(r, "%s (view)", a->name);
    set_op_params(r, &offset, sizeof(offset));
    r->op = GGML_OP_VIEW;
    r->src[0] = a;
    return r;
}
struct ggml_tensor * ggml_view_1d(struct ggml_context * ctx, struct ggml_tensor * a, int64_t ne0, size_t offset) {
    const int64_t ne[1] = { ne0 };
    return view_impl(ctx, a, 1, ne, offset);
}
struct ggml_tensor * ggml_view_2d(struct ggml_context * ctx, struct ggml_tensor * a, int64_t ne0, int64_t ne1, size_t nb1, size_t offset) {
    const int64_t ne[2] = { ne0, ne1 };
    ggml_tensor * r = view_impl(ctx, a, 2, ne, offset);
    r->nb[1] = nb1;
    r->nb[2] = nb1 * ne1;
    r->nb[3] = r->nb[2];
    return r;
}
struct ggml_tensor * ggml_view_3d(struct ggml_context * ctx, struct ggml_tensor * a, int64_t ne0, int64_t ne1, int64_t ne2, size_t nb1, size_t nb2, size_t offset) {
    const int64_t ne[3] = { ne0, ne1, ne2 };
    ggml_tensor * r = view_impl(ctx, a, 3, ne, offset);
    r->nb[1] = nb1;
    r->nb[2] = nb2;
    r->nb[3] = nb2 * ne2;
    return r;
}
struct ggml_tensor * ggml_view_4d(struct ggml_context * ctx, struct ggml_tensor * a, int64_t ne0, int64_t ne1, int64_t ne2, int64_t ne3, size_t nb1, size_t nb2, size_t nb3, size_t offset) {
    const int64_t ne[4] = { ne0, ne1, ne2, ne3 };
    ggml_tensor * r = view_impl(ctx, a, 4, ne, offset);
    r->nb[1] = nb1;
    r->nb[2] = nb2;
    r->nb[3] = nb3;
    return r;
}

struct ggml_tensor * ggml_permute(struct ggml_context * ctx, struct ggml_tensor * a, int axis0, int axis1, int axis2, int axis3) {
    const int ax[4] = { axis0, axis1, axis2, axis3 };
    for (int i = 0; i < 4; i++) {
        GGML_CHECK(ax[i] >= 0 && ax[i] < GGML_MAX_DIMS);
        for (int j = 0; j < i; j++) GGML_CHECK(ax[i] != ax[j]);
    }
    ggml_tensor * r = ggml_view_tensor(ctx, a);
    format_name(r, "%s (permuted)", a->name);
    int64_t ne[4];
    size_t nb[4];
    for (int i = 0; i < 4; i++) { ne[ax[i]] = a->ne[i]; nb[ax[i]] = a->nb[i]; }
    for (int i = 0; i < 4; i++) { r->ne[i] = ne[i]; r->nb[i] = nb[i]; }
    r->op = GGML_OP_PERMUTE;
    r->src[0] = a;
    for (int i = 0; i < 4; i++) set_op_param_i32(r, i, ax[i]);
    return r;
}

struct ggml_tensor * ggml_transpose(struct ggml_context * ctx, struct ggml_tensor * a) {
    ggml_tensor * r = ggml_view_tensor(ctx, a);
    format_name(r, "%s (transposed)", a->name);
    r->ne[0] = a->ne[1]; r->ne[1] = a->ne[0];
    r->nb[0] = a->nb[1]; r->nb[1] = a->nb[0];
    r->op = GGML_OP_TRANSPOSE;
    r->src[0] = a;
    return r;
}

struct ggml_tensor * ggml_cont_4d(struct ggml_context * ctx, struct ggml_tensor * a, int64_t ne0, int64_t ne1, int64_t ne2, int64_t ne3) {
    GGML_CHECK(ggml_nelements(a) == ne0 * ne1 * ne2 * ne3);
    ggml_tensor * r = ggml_new_tensor_4d(ctx, a->type, ne0, ne1, ne2, ne3);
    format_name(r, "%s (cont)", a->name);
    r->op = GGML_OP_CONT;
    r->src[0] = a;
    return r;
}
struct ggml_tensor * ggml_cont(struct ggml_context * ctx, struct ggml_tensor * a) {
    return ggml_cont_4d(ctx, a, a->ne[0], a->ne[1], a->ne[2], a->ne[3]);
}
struct ggml_tensor * ggml_cont_2d(struct ggml_context * ctx, struct ggml_tensor * a, int64_t ne0, int64_t ne1) {
    return ggml_cont_4d(ctx, a, ne0, ne1, 1, 1);
}
struct ggml_tensor * ggml_cont_3d(struct ggml_context * ctx, struct ggml_tensor * a, int64_t ne0, int64_t ne1, int64_t ne2) {
    return ggml_cont_4d(ctx, a, ne0, ne1, ne2, 1);
}

struct ggml_tensor * ggml_cpy(struct ggml_context * ctx, struct ggml_tensor * a, struct ggml_tensor * b) {
    GGML_CHECK(ggml_nelements(a) == ggml_nelements(b));
    ggml_tensor * r = ggml_view_tensor(ctx, b);
    if (b->name[0]) format_name(r, "%s (copy of %s)", b->name, a->name);
    else format_name(r, "%s (copy)", a->name);
    r->op = GGML_OP_CPY;
    r->src[0] = a;
    r->src[1] = b;
    return r;
}

struct ggml_tensor * ggml_cast(struct ggml_context * ctx, struct ggml_tensor * a, enum ggml_type type) {
    ggml_tensor * r = ggml_new_tensor(ctx, type, GGML_MAX_DIMS, a->ne);
    format_name(r, "%s (copy)", a->name);
    r->op = GGML_OP_CPY;
    r->src[0] = a;
    r->src[1] = r;
    return r;
}

struct ggml_tensor * ggml_rope_ext(struct ggml_context * ctx, struct ggml_tensor * a, struct ggml_tensor * b,
        struct ggml_tensor * c, int n_dims, int mode, int n_ctx_orig, float freq_base, float freq_scale,
        float ext_factor, float attn_factor, float beta_fast, float beta_slow) {
    GGML_CHECK(b->type == GGML_TYPE_I32 && b->ne[0] == a->ne[2]);
    GGML_CHECK(n_dims <= a->ne[0] && n_dims % 2 == 0);
    if (c) GGML_CHECK(c->type == GGML_TYPE_F32 && c->ne[0] >= n_dims / 2);
    ggml_tensor * r = ggml_dup_tensor(ctx, a);
    int32_t params[15] = { 0, n_dims, mode, 0, n_ctx_orig };
    memcpy(params + 5,  &freq_base,   4);
    memcpy(params + 6,  &freq_scale,  4);
    memcpy(params + 7,  &ext_factor,  4);
    memcpy(params + 8,  &attn_factor, 4);
    memcpy(params + 9,  &beta_fast,   4);
    memcpy(params + 10, &beta_slow,   4);
    set_op_params(r, params, sizeof(params));
    r->op = GGML_OP_ROPE;
    r->src[0] = a;
    r->src[1] = b;
    r->src[2] = c;
    return r;
}

static float rope_corr_dim(int n_dims, int n_ctx_orig, float n_rot, float base) {
    return n_dims * logf(n_ctx_orig / (n_rot * 2 * (float) M_PI)) / (2 * logf(base));
}

void ggml_rope_yarn_corr_dims(int n_dims, int n_ctx_orig, float freq_base, float beta_fast, float beta_slow, float dims[2]) {
    const float start = floorf(rope_corr_dim(n_dims, n_ctx_orig, beta_fast, freq_base));
    const float end   = ceilf(rope_corr_dim(n_dims, n_ctx_orig, beta_slow, freq_base));
    dims[0] = start > 0 ? start : 0;
    dims[1] = end < (float) (n_dims - 1) ? end : (float) (n_dims - 1);
}

struct ggml_tensor * ggml_soft_max_ext(struct ggml_context * ctx, struct ggml_tensor * a, struct ggml_tensor * mask, float scale, float max_bias) {
    GGML_CHECK(ggml_is_contiguous(a));
    if (mask) {
        GGML_CHECK(mask->type == GGML_TYPE_F16 || mask->type == GGML_TYPE_F32);
        GGML_CHECK(ggml_is_contiguous(mask));
        GGML_CHECK(mask->ne[0] == a->ne[0] && mask->ne[1] >= a->ne[1]);
    }
    ggml_tensor * r = ggml_dup_tensor(ctx, a);
    set_op_param_f32(r, 0, scale);
    set_op_param_f32(r, 1, max_bias);
    r->op = GGML_OP_SOFT_MAX;
    r->src[0] = a;
    r->src[1] = mask;
    return r;
}
struct ggml_tensor * ggml_soft_max(struct ggml_context * ctx, struct ggml_tensor * a) { return ggml_soft_max_ext(ctx, a, nullptr, 1.0f, 0.0f); }

struct ggml_tensor * ggml_unary(struct ggml_context * ctx, struct ggml_tensor * a, enum ggml_unary_op op) {
    ggml_tensor * r = ggml_dup_tensor(ctx, a);
    set_op_param_i32(r, 0, (int32_t) op);
    r->op = GGML_OP_UNARY;
    r->src[0] = a;
    return r;
}
struct ggml_tensor * ggml_silu(struct ggml_context * ctx, struct ggml_tensor * a) { return ggml_unary(ctx, a, GGML_UNARY_OP_SILU); }
struct ggml_tensor * ggml_relu(struct ggml_context * ctx, struct ggml_tensor * a) { return ggml_unary(ctx, a, GGML_UNARY_OP_RELU); }
struct ggml_tensor * ggml_sigmoid(struct ggml_context * ctx, struct ggml_tensor * a) { return ggml_unary(ctx, a, GGML_UNARY_OP_SIGMOID); }
struct ggml_tensor * ggml_abs(struct ggml_context * ctx, struct ggml_tensor * a) { return ggml_unary(ctx, a, GGML_UNARY_OP_ABS); }
struct ggml_tensor * ggml_softplus(struct ggml_context * ctx, struct ggml_tensor * a) { return ggml_unary(ctx, a, GGML_UNARY_OP_SOFTPLUS); }
enum ggml_unary_op ggml_get_unary_op(const struct ggml_tensor * t) { return (enum ggml_unary_op) t->op_params[0]; }

struct ggml_tensor * ggml_flash_attn_ext(struct ggml_context * ctx, struct ggml_tensor * q, struct ggml_tensor * k,
        struct ggml_tensor * v, struct ggml_tensor * mask, float scale, float max_bias, float logit_softcap) {
    GGML_CHECK(q->ne[0] == k->ne[0]);
    GGML_CHECK(k->ne[1] == v->ne[1]);
    GGML_CHECK(q->ne[2] % k->ne[2] == 0);
    if (mask) {
        GGML_CHECK(ggml_is_contiguous(mask));
        GGML_CHECK(mask->ne[0] == k->ne[1] && mask->ne[1] >= q->ne[1]);
    }
    ggml_tensor * r = ggml_new_tensor_4d(ctx, GGML_TYPE_F32, v->ne[0], q->ne[2], q->ne[1], q->ne[3]);
    set_op_param_f32(r, 0, scale);
    set_op_param_f32(r, 1, max_bias);
    set_op_param_f32(r, 2, logit_softcap);
    r->op = GGML_OP_FLASH_ATTN_EXT;
    r->src[0] = q;
    r->src[1] = k;
    r->src[2] = v;
    r->src[3] = mask;
    return r;
}

struct ggml_tensor * ggml_sum_rows(struct ggml_context * ctx, struct ggml_tensor * a) {
    GGML_CHECK(a->type == GGML_TYPE_F32);
    ggml_tensor * r = ggml_new_tensor_4d(ctx, GGML_TYPE_F32, 1, a->ne[1], a->ne[2], a->ne[3]);
    r->op = GGML_OP_SUM_ROWS;
    r->src[0] = a;
    return r;
}

struct ggml_tensor * ggml_argsort(struct ggml_context * ctx, struct ggml_tensor * a, enum ggml_sort_order order) {
    GGML_CHECK(a->type == GGML_TYPE_F32);
    ggml_tensor * r = ggml_new_tensor_4d(ctx, GGML_TYPE_I32, a->ne[0], a->ne[1], a->ne[2], a->ne[3]);
    r->op_params[0] = (int32_t) order;
    r->op = GGML_OP_ARGSORT;
    r->src[0] = a;
    return r;
}

struct ggml_tensor * ggml_top_k(struct ggml_context * ctx, struct ggml_tensor * a, int k) {
    GGML_CHECK(k > 0 && k <= a->ne[0]);
    ggml_tensor * s = ggml_argsort(ctx, a, GGML_SORT_ORDER_DESC);
    return ggml_view_4d(ctx, s, k, s->ne[1], s->ne[2], s->ne[3], s->nb[1], s->nb[2], s->nb[3], 0);
}

struct ggml_tensor * ggml_argmax(struct ggml_context * ctx, struct ggml_tensor * a) {
    GGML_CHECK(a->type == GGML_TYPE_F32 && a->ne[2] == 1 && a->ne[3] == 1);
    ggml_tensor * r = ggml_new_tensor_1d(ctx, GGML_TYPE_I32, a->ne[1]);
    r->op = GGML_OP_ARGMAX;
    r->src[0] = a;
    return r;
}

// ---------------------------------------------------------------------------------------------
// graphs

struct ggml_cgraph * ggml_new_graph_custom(struct ggml_context * ctx, size_t size, bool grads) {
    (void) grads;
    ggml_object * obj = ctx_new_object(ctx, OBJ_GRAPH, graph_nbytes(size));
    ggml_cgraph * g = (ggml_cgraph *) ((char *) ctx->mem_buffer + obj->offs);
    ggml_tensor ** p = (ggml_tensor **) (g + 1);
    g->size = (int) size;
    g->n_nodes = 0;
    g->n_leafs = 0;
    g->nodes = p;
    g->leafs = p + size;
    g->hash_size = graph_hash_size(size);
    g->hash_keys = p + 2 * size;
    memset(g->hash_keys, 0, g->hash_size * sizeof(ggml_tensor *));
    return g;
}
struct ggml_cgraph * ggml_new_graph(struct ggml_context * ctx) { return ggml_new_graph_custom(ctx, GGML_DEFAULT_GRAPH_SIZE, false); }

// returns true if t was newly inserted
static bool graph_visit_insert(ggml_cgraph * g, ggml_tensor * t) {
    const size_t mask = g->hash_size - 1;
    size_t h = (((uintptr_t) t) >> 4) * 0x9E3779B97F4A7C15ull;
    h = (h >> 17) & mask;
    while (g->hash_keys[h]) {
        if (g->hash_keys[h] == t) return false;
        h = (h + 1) & mask;
    }
    g->hash_keys[h] = t;
    return true;
}

static void graph_visit(ggml_cgraph * g, ggml_tensor * t) {
    if (!graph_visit_insert(g, t)) return;
    for (int i = 0; i < GGML_MAX_SRC; i++) {
        if (t->src[i]) graph_visit(g, t->src[i]);
    }
    if (t->op == GGML_OP_NONE) {
        if (g->n_leafs >= g->size) GGML_ABORT("graph leaf capacity %d exceeded", g->size);
        g->leafs[g->n_leafs++] = t;
    } else {
        if (g->n_nodes >= g->size) GGML_ABORT("graph node capacity %d exceeded", g->size);
        g->nodes[g->n_nodes++] = t;
    }
}

void ggml_build_forward_expand(struct ggml_cgraph * cgraph, struct ggml_tensor * tensor) { graph_visit(cgraph, tensor); }

int ggml_graph_n_nodes(struct ggml_cgraph * g) { return g->n_nodes; }
struct ggml_tensor * ggml_graph_node(struct ggml_cgraph * g, int i) {
    if (i < 0) i += g->n_nodes;
    GGML_CHECK(i >= 0 && i < g->n_nodes);
    return g->nodes[i];
}
int ggml_graph_n_leafs(struct ggml_cgraph * g) { return g->n_leafs; }
struct ggml_tensor * ggml_graph_leaf(struct ggml_cgraph * g, int i) {
    GGML_CHECK(i >= 0 && i < g->n_leafs);
    return g->leafs[i];
}

} // extern "C"
