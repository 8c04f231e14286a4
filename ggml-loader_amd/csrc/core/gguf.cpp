// gguf.cpp — GGUF v2/v3 container: reader (metadata + tensor directory + optional data load)
// and writer (header/metadata, tensor infos, aligned tensor data).
//
// On-disk layout (little endian): "GGUF", u32 version, u64 n_tensors, u64 n_kv, n_kv x
// {string key, u32 type, value}, n_tensors x {string name, u32 n_dims, u64 ne[n_dims], u32 type,
// u64 offset}, zero padding to general.alignment (default 32), tensor data (each tensor at its
// offset, aligned). Strings are u64 length + bytes. This is the format the reference reads in
// load_weights_filtered (model.cpp:667-784) and src/moe_stream/gguf_index.c:189-346.
#include "gguf.h"
#include "ggml-backend.h"

#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <string>
#include <vector>

namespace {

struct gguf_kv {
    std::string key;
    gguf_type type = GGUF_TYPE_UINT8;
    gguf_type arr_type = GGUF_TYPE_UINT8; // arrays only
    std::vector<uint8_t> data;            // scalar value bytes, or packed array elements
    std::vector<std::string> strs;        // string value (1 entry) or string array
    size_t n = 0;                         // array length
};

struct gguf_tinfo {
    std::string name;
    int n_dims = 0;
    int64_t ne[GGML_MAX_DIMS] = { 1, 1, 1, 1 };
    ggml_type type = GGML_TYPE_F32;
    size_t offset = 0;
    size_t size = 0;
    const void * data = nullptr; // writer: source of the bytes
};

size_t scalar_size(gguf_type t) {
    switch (t) {
        case GGUF_TYPE_UINT8: case GGUF_TYPE_INT8: case GGUF_TYPE_BOOL: return 1;
        case GGUF_TYPE_UINT16: case GGUF_TYPE_INT16: return 2;
        case GGUF_TYPE_UINT32: case GGUF_TYPE_INT32: case GGUF_TYPE_FLOAT32: return 4;
        case GGUF_TYPE_UINT64: case GGUF_TYPE_INT64: case GGUF_TYPE_FLOAT64: return 8;
        default: return 0;
    }
}

[[noreturn]] void fail(const char * msg, const char * key) {
    fprintf(stderr, "gguf error: %s (key '%s')\n", msg, key ? key : "");
    abort();
}

struct reader {
    FILE * f;
    bool ok = true;
    bool read(void * dst, size_t n) {
        if (!ok) return false;
        if (n && fread(dst, 1, n, f) != n) ok = false;
        return ok;
    }
    template <typename T> bool get(T & v) { return read(&v, sizeof(T)); }
    bool str(std::string & s) {
        uint64_t n = 0;
        if (!get(n)) return false;
        if (n > (1ull << 32)) { ok = false; return false; }
        s.resize(n);
        return read(&s[0], n);
    }
};

} // namespace

struct gguf_context {
    uint32_t version = GGUF_VERSION;
    std::vector<gguf_kv> kv;
    std::vector<gguf_tinfo> tensors;
    size_t alignment = GGUF_DEFAULT_ALIGNMENT;
    size_t data_offset = 0; // reader: file offset of the data section
    size_t data_size = 0;   // total bytes of the data section (padded)
};

static size_t pad_to(size_t x, size_t a) { return (x + a - 1) / a * a; }

static int64_t find_key_impl(const gguf_context * ctx, const char * key) {
    for (size_t i = 0; i < ctx->kv.size(); i++) if (ctx->kv[i].key == key) return (int64_t) i;
    return -1;
}

static const gguf_kv & kv_at(const gguf_context * ctx, int64_t id) {
    if (id < 0 || (size_t) id >= ctx->kv.size()) fail("key id out of range", nullptr);
    return ctx->kv[id];
}

template <typename T>
static T get_scalar(const gguf_context * ctx, int64_t id, gguf_type want) {
    const gguf_kv & e = kv_at(ctx, id);
    if (e.type != want) fail("value type mismatch", e.key.c_str());
    T v;
    memcpy(&v, e.data.data(), sizeof(T));
    return v;
}

static const gguf_tinfo & tinfo(const gguf_context * ctx, int64_t id) {
    if (id < 0 || (size_t) id >= ctx->tensors.size()) fail("tensor id out of range", nullptr);
    return ctx->tensors[id];
}

static gguf_kv & kv_slot(gguf_context * ctx, const char * key) {
    int64_t id = find_key_impl(ctx, key);
    if (id >= 0) {
        ctx->kv[id] = gguf_kv();
        ctx->kv[id].key = key;
        return ctx->kv[id];
    }
    ctx->kv.emplace_back();
    ctx->kv.back().key = key;
    return ctx->kv.back();
}

template <typename T>
static void set_scalar(gguf_context * ctx, const char * key, gguf_type type, T v) {
    gguf_kv & e = kv_slot(ctx, key);
    e.type = type;
    e.data.resize(sizeof(T));
    memcpy(e.data.data(), &v, sizeof(T));
    if (strcmp(key, GGUF_KEY_GENERAL_ALIGNMENT) == 0 && type == GGUF_TYPE_UINT32) ctx->alignment = (size_t) (uint32_t) v;
}

static void put(std::vector<uint8_t> & b, const void * p, size_t n) {
    const uint8_t * q = (const uint8_t *) p;
    b.insert(b.end(), q, q + n);
}
template <typename T> static void put_v(std::vector<uint8_t> & b, T v) { put(b, &v, sizeof(T)); }
static void put_s(std::vector<uint8_t> & b, const std::string & s) { put_v<uint64_t>(b, s.size()); put(b, s.data(), s.size()); }

extern "C" {

struct gguf_context * gguf_init_empty(void) { return new gguf_context(); }

void gguf_free(struct gguf_context * ctx) { delete ctx; }

const char * gguf_type_name(enum gguf_type type) {
    static const char * names[] = { "u8", "i8", "u16", "i16", "u32", "i32", "f32", "bool", "str", "arr", "u64", "i64", "f64" };
    return (type >= 0 && type < GGUF_TYPE_COUNT) ? names[type] : "?";
}

struct gguf_context * gguf_init_from_file(const char * fname, struct gguf_init_params params) {
    FILE * f = fopen(fname, "rb");
    if (!f) {
        fprintf(stderr, "gguf: failed to open '%s'\n", fname);
        return nullptr;
    }
    reader r{ f };
    char magic[4];
    gguf_context * ctx = new gguf_context();
    auto bad = [&](const char * what) -> gguf_context * {
        fprintf(stderr, "gguf: '%s': %s\n", fname, what);
        fclose(f);
        delete ctx;
        return nullptr;
    };
    if (!r.read(magic, 4) || memcmp(magic, GGUF_MAGIC, 4) != 0) return bad("bad magic");
    if (!r.get(ctx->version) || ctx->version < 2 || ctx->version > 3) return bad("unsupported version");
    uint64_t n_tensors = 0, n_kv = 0;
    if (!r.get(n_tensors) || !r.get(n_kv)) return bad("truncated header");
    ctx->kv.resize(n_kv);
    for (uint64_t i = 0; i < n_kv; i++) {
        gguf_kv & e = ctx->kv[i];
        uint32_t t = 0;
        if (!r.str(e.key) || !r.get(t) || t >= GGUF_TYPE_COUNT) return bad("bad kv header");
        e.type = (gguf_type) t;
        if (e.type == GGUF_TYPE_STRING) {
            e.strs.resize(1);
            if (!r.str(e.strs[0])) return bad("bad string value");
        } else if (e.type == GGUF_TYPE_ARRAY) {
            uint32_t at = 0;
            uint64_t n = 0;
            if (!r.get(at) || !r.get(n) || at >= GGUF_TYPE_COUNT || at == GGUF_TYPE_ARRAY) return bad("bad array header");
            e.arr_type = (gguf_type) at;
            e.n = n;
            if (e.arr_type == GGUF_TYPE_STRING) {
                e.strs.resize(n);
                for (uint64_t j = 0; j < n; j++) if (!r.str(e.strs[j])) return bad("bad string array");
            } else {
                e.data.resize(n * scalar_size(e.arr_type));
                if (!r.read(e.data.data(), e.data.size())) return bad("bad array data");
            }
        } else {
            e.data.resize(scalar_size(e.type));
            if (!r.read(e.data.data(), e.data.size())) return bad("bad scalar value");
        }
    }
    const int64_t ai = gguf_find_key(ctx, GGUF_KEY_GENERAL_ALIGNMENT);
    if (ai >= 0) {
        if (ctx->kv[ai].type != GGUF_TYPE_UINT32) return bad("general.alignment must be u32");
        uint32_t a;
        memcpy(&a, ctx->kv[ai].data.data(), 4);
        if (a == 0 || (a & (a - 1))) return bad("alignment is not a power of two");
        ctx->alignment = a;
    }
    ctx->tensors.resize(n_tensors);
    for (uint64_t i = 0; i < n_tensors; i++) {
        gguf_tinfo & ti = ctx->tensors[i];
        uint32_t nd = 0, type = 0;
        if (!r.str(ti.name) || !r.get(nd) || nd < 1 || nd > GGML_MAX_DIMS) return bad("bad tensor info");
        ti.n_dims = (int) nd;
        for (uint32_t d = 0; d < nd; d++) {
            uint64_t v;
            if (!r.get(v)) return bad("bad tensor dims");
            ti.ne[d] = (int64_t) v;
        }
        uint64_t off = 0;
        if (!r.get(type) || !r.get(off)) return bad("bad tensor type/offset");
        ti.type = (ggml_type) type;
        ti.offset = off;
        if (ggml_type_size(ti.type) == 0) return bad("unknown tensor type");
        const int64_t blck = ggml_blck_size(ti.type);
        if (ti.ne[0] % blck != 0) return bad("row size not a multiple of the block size");
        ti.size = ggml_row_size(ti.type, ti.ne[0]) * (size_t) (ti.ne[1] * ti.ne[2] * ti.ne[3]);
        if (off % ctx->alignment != 0) return bad("tensor offset not aligned");
    }
    long pos = ftell(f);
    ctx->data_offset = pad_to((size_t) pos, ctx->alignment);
    for (const gguf_tinfo & ti : ctx->tensors) {
        const size_t end = ti.offset + ti.size;
        if (end > ctx->data_size) ctx->data_size = end;
    }

    if (params.ctx) {
        const size_t n = ctx->tensors.size();
        size_t mem = (n + 1) * ggml_tensor_overhead();
        if (!params.no_alloc) mem += ctx->data_size + n * GGML_MEM_ALIGN;
        ggml_init_params ip = { mem, nullptr, params.no_alloc };
        ggml_context * gctx = ggml_init(ip);
        if (!gctx) return bad("out of memory for the tensor context");
        for (const gguf_tinfo & ti : ctx->tensors) {
            ggml_tensor * t = ggml_new_tensor(gctx, ti.type, GGML_MAX_DIMS, ti.ne);
            ggml_set_name(t, ti.name.c_str());
            if (!params.no_alloc) {
                if (fseek(f, (long) (ctx->data_offset + ti.offset), SEEK_SET) != 0 ||
                    fread(t->data, 1, ti.size, f) != ti.size) {
                    ggml_free(gctx);
                    return bad("failed to read tensor data");
                }
            }
        }
        *params.ctx = gctx;
    }
    fclose(f);
    return ctx;
}

uint32_t gguf_get_version(const struct gguf_context * ctx) { return ctx->version; }
size_t gguf_get_alignment(const struct gguf_context * ctx) { return ctx->alignment; }
size_t gguf_get_data_offset(const struct gguf_context * ctx) { return ctx->data_offset; }

int64_t gguf_get_n_kv(const struct gguf_context * ctx) { return (int64_t) ctx->kv.size(); }

int64_t gguf_find_key(const struct gguf_context * ctx, const char * key) {
    for (size_t i = 0; i < ctx->kv.size(); i++) if (ctx->kv[i].key == key) return (int64_t) i;
    return -1;
}


const char * gguf_get_key(const struct gguf_context * ctx, int64_t key_id) { return kv_at(ctx, key_id).key.c_str(); }
enum gguf_type gguf_get_kv_type(const struct gguf_context * ctx, int64_t key_id) { return kv_at(ctx, key_id).type; }
enum gguf_type gguf_get_arr_type(const struct gguf_context * ctx, int64_t key_id) {
    const gguf_kv & e = kv_at(ctx, key_id);
    if (e.type != GGUF_TYPE_ARRAY) fail("not an array", e.key.c_str());
    return e.arr_type;
}


uint8_t  gguf_get_val_u8 (const struct gguf_context * c, int64_t k) { return get_scalar<uint8_t >(c, k, GGUF_TYPE_UINT8); }
int8_t   gguf_get_val_i8 (const struct gguf_context * c, int64_t k) { return get_scalar<int8_t  >(c, k, GGUF_TYPE_INT8); }
uint16_t gguf_get_val_u16(const struct gguf_context * c, int64_t k) { return get_scalar<uint16_t>(c, k, GGUF_TYPE_UINT16); }
int16_t  gguf_get_val_i16(const struct gguf_context * c, int64_t k) { return get_scalar<int16_t >(c, k, GGUF_TYPE_INT16); }
uint32_t gguf_get_val_u32(const struct gguf_context * c, int64_t k) { return get_scalar<uint32_t>(c, k, GGUF_TYPE_UINT32); }
int32_t  gguf_get_val_i32(const struct gguf_context * c, int64_t k) { return get_scalar<int32_t >(c, k, GGUF_TYPE_INT32); }
float    gguf_get_val_f32(const struct gguf_context * c, int64_t k) { return get_scalar<float   >(c, k, GGUF_TYPE_FLOAT32); }
uint64_t gguf_get_val_u64(const struct gguf_context * c, int64_t k) { return get_scalar<uint64_t>(c, k, GGUF_TYPE_UINT64); }
int64_t  gguf_get_val_i64(const struct gguf_context * c, int64_t k) { return get_scalar<int64_t >(c, k, GGUF_TYPE_INT64); }
double   gguf_get_val_f64(const struct gguf_context * c, int64_t k) { return get_scalar<double  >(c, k, GGUF_TYPE_FLOAT64); }
bool     gguf_get_val_bool(const struct gguf_context * c, int64_t k) { return get_scalar<uint8_t>(c, k, GGUF_TYPE_BOOL) != 0; }

const char * gguf_get_val_str(const struct gguf_context * ctx, int64_t key_id) {
    const gguf_kv & e = kv_at(ctx, key_id);
    if (e.type != GGUF_TYPE_STRING) fail("not a string", e.key.c_str());
    return e.strs[0].c_str();
}

size_t gguf_get_arr_n(const struct gguf_context * ctx, int64_t key_id) {
    const gguf_kv & e = kv_at(ctx, key_id);
    if (e.type != GGUF_TYPE_ARRAY) fail("not an array", e.key.c_str());
    return e.n;
}

const void * gguf_get_arr_data(const struct gguf_context * ctx, int64_t key_id) {
    const gguf_kv & e = kv_at(ctx, key_id);
    if (e.type != GGUF_TYPE_ARRAY || e.arr_type == GGUF_TYPE_STRING) fail("not a numeric array", e.key.c_str());
    return e.data.data();
}

const char * gguf_get_arr_str(const struct gguf_context * ctx, int64_t key_id, size_t i) {
    const gguf_kv & e = kv_at(ctx, key_id);
    if (e.type != GGUF_TYPE_ARRAY || e.arr_type != GGUF_TYPE_STRING) fail("not a string array", e.key.c_str());
    if (i >= e.strs.size()) fail("string array index out of range", e.key.c_str());
    return e.strs[i].c_str();
}

int64_t gguf_get_n_tensors(const struct gguf_context * ctx) { return (int64_t) ctx->tensors.size(); }
int64_t gguf_find_tensor(const struct gguf_context * ctx, const char * name) {
    for (size_t i = 0; i < ctx->tensors.size(); i++) if (ctx->tensors[i].name == name) return (int64_t) i;
    return -1;
}

size_t gguf_get_tensor_offset(const struct gguf_context * c, int64_t id) { return tinfo(c, id).offset; }
const char * gguf_get_tensor_name(const struct gguf_context * c, int64_t id) { return tinfo(c, id).name.c_str(); }
enum ggml_type gguf_get_tensor_type(const struct gguf_context * c, int64_t id) { return tinfo(c, id).type; }
size_t gguf_get_tensor_size(const struct gguf_context * c, int64_t id) { return tinfo(c, id).size; }
int gguf_get_tensor_n_dims(const struct gguf_context * c, int64_t id) { return tinfo(c, id).n_dims; }
const int64_t * gguf_get_tensor_ne(const struct gguf_context * c, int64_t id) { return tinfo(c, id).ne; }

// ---- writer ----



void gguf_set_val_u8  (struct gguf_context * c, const char * k, uint8_t  v) { set_scalar(c, k, GGUF_TYPE_UINT8, v); }
void gguf_set_val_i8  (struct gguf_context * c, const char * k, int8_t   v) { set_scalar(c, k, GGUF_TYPE_INT8, v); }
void gguf_set_val_u16 (struct gguf_context * c, const char * k, uint16_t v) { set_scalar(c, k, GGUF_TYPE_UINT16, v); }
void gguf_set_val_i16 (struct gguf_context * c, const char * k, int16_t  v) { set_scalar(c, k, GGUF_TYPE_INT16, v); }
void gguf_set_val_u32 (struct gguf_context * c, const char * k, uint32_t v) { set_scalar(c, k, GGUF_TYPE_UINT32, v); }
void gguf_set_val_i32 (struct gguf_context * c, const char * k, int32_t  v) { set_scalar(c, k, GGUF_TYPE_INT32, v); }
void gguf_set_val_f32 (struct gguf_context * c, const char * k, float    v) { set_scalar(c, k, GGUF_TYPE_FLOAT32, v); }
void gguf_set_val_u64 (struct gguf_context * c, const char * k, uint64_t v) { set_scalar(c, k, GGUF_TYPE_UINT64, v); }
void gguf_set_val_i64 (struct gguf_context * c, const char * k, int64_t  v) { set_scalar(c, k, GGUF_TYPE_INT64, v); }
void gguf_set_val_f64 (struct gguf_context * c, const char * k, double   v) { set_scalar(c, k, GGUF_TYPE_FLOAT64, v); }
void gguf_set_val_bool(struct gguf_context * c, const char * k, bool     v) { set_scalar(c, k, GGUF_TYPE_BOOL, (uint8_t) (v ? 1 : 0)); }

void gguf_set_val_str(struct gguf_context * ctx, const char * key, const char * val) {
    gguf_kv & e = kv_slot(ctx, key);
    e.type = GGUF_TYPE_STRING;
    e.strs.assign(1, std::string(val));
}

void gguf_set_arr_data(struct gguf_context * ctx, const char * key, enum gguf_type type, const void * data, size_t n) {
    if (type == GGUF_TYPE_STRING || type == GGUF_TYPE_ARRAY || scalar_size(type) == 0) fail("bad array element type", key);
    gguf_kv & e = kv_slot(ctx, key);
    e.type = GGUF_TYPE_ARRAY;
    e.arr_type = type;
    e.n = n;
    e.data.resize(n * scalar_size(type));
    if (n) memcpy(e.data.data(), data, e.data.size());
}

void gguf_set_arr_str(struct gguf_context * ctx, const char * key, const char ** data, size_t n) {
    gguf_kv & e = kv_slot(ctx, key);
    e.type = GGUF_TYPE_ARRAY;
    e.arr_type = GGUF_TYPE_STRING;
    e.n = n;
    e.strs.clear();
    for (size_t i = 0; i < n; i++) e.strs.emplace_back(data[i]);
}

static void add_tinfo(gguf_context * ctx, const char * name, ggml_type type, int n_dims, const int64_t * ne, const void * data) {
    if (gguf_find_tensor(ctx, name) >= 0) fail("duplicate tensor name", name);
    gguf_tinfo ti;
    ti.name = name;
    ti.n_dims = n_dims;
    for (int i = 0; i < n_dims; i++) ti.ne[i] = ne[i];
    ti.type = type;
    ti.size = ggml_row_size(type, ti.ne[0]) * (size_t) (ti.ne[1] * ti.ne[2] * ti.ne[3]);
    size_t off = 0;
    if (!ctx->tensors.empty()) {
        const gguf_tinfo & last = ctx->tensors.back();
        off = pad_to(last.offset + last.size, ctx->alignment);
    }
    ti.offset = off;
    ti.data = data;
    ctx->tensors.push_back(ti);
}

void gguf_add_tensor(struct gguf_context * ctx, const struct ggml_tensor * tensor) {
    add_tinfo(ctx, tensor->name, tensor->type, ggml_n_dims(tensor), tensor->ne, tensor->data);
}

void gguf_add_tensor_info(struct gguf_context * ctx, const char * name, enum ggml_type type, int n_dims, const int64_t * ne) {
    add_tinfo(ctx, name, type, n_dims, ne, nullptr);
}

static std::vector<uint8_t> build_meta(const gguf_context * ctx) {
    std::vector<uint8_t> b;
    put(b, GGUF_MAGIC, 4);
    put_v<uint32_t>(b, GGUF_VERSION);
    put_v<uint64_t>(b, ctx->tensors.size());
    put_v<uint64_t>(b, ctx->kv.size());
    for (const gguf_kv & e : ctx->kv) {
        put_s(b, e.key);
        put_v<uint32_t>(b, (uint32_t) e.type);
        if (e.type == GGUF_TYPE_STRING) {
            put_s(b, e.strs[0]);
        } else if (e.type == GGUF_TYPE_ARRAY) {
            put_v<uint32_t>(b, (uint32_t) e.arr_type);
            put_v<uint64_t>(b, e.n);
            if (e.arr_type == GGUF_TYPE_STRING) for (const std::string & s : e.strs) put_s(b, s);
            else put(b, e.data.data(), e.data.size());
        } else {
            put(b, e.data.data(), e.data.size());
        }
    }
    for (const gguf_tinfo & ti : ctx->tensors) {
        put_s(b, ti.name);
        put_v<uint32_t>(b, (uint32_t) ti.n_dims);
        for (int d = 0; d < ti.n_dims; d++) put_v<uint64_t>(b, (uint64_t) ti.ne[d]);
        put_v<uint32_t>(b, (uint32_t) ti.type);
        put_v<uint64_t>(b, (uint64_t) ti.offset);
    }
    b.resize(pad_to(b.size(), ctx->alignment), 0);
    return b;
}

size_t gguf_get_meta_size(const struct gguf_context * ctx) { return build_meta(ctx).size(); }

bool gguf_write_to_file(const struct gguf_context * ctx, const char * fname, bool only_meta) {
    FILE * f = fopen(fname, "wb");
    if (!f) return false;
    std::vector<uint8_t> meta = build_meta(ctx);
    bool ok = fwrite(meta.data(), 1, meta.size(), f) == meta.size();
    if (ok && !only_meta) {
        size_t pos = 0;
        std::vector<uint8_t> zeros(ctx->alignment, 0);
        for (const gguf_tinfo & ti : ctx->tensors) {
            if (!ti.data) { ok = false; break; }
            if (ti.offset > pos) ok = ok && fwrite(zeros.data(), 1, ti.offset - pos, f) == ti.offset - pos;
            ok = ok && fwrite(ti.data, 1, ti.size, f) == ti.size;
            pos = ti.offset + ti.size;
            if (!ok) break;
        }
        size_t end = pad_to(pos, ctx->alignment);
        if (ok && end > pos) ok = fwrite(zeros.data(), 1, end - pos, f) == end - pos;
    }
    ok = (fclose(f) == 0) && ok;
    return ok;
}

} // extern "C"
