// model.cpp — forward-pass runtime: hparams, weight binding/loading, KV cache, graph building and
// the per-token step. Mirrors the reference's src/model.cpp path function by function (citations
// inline). Failures throw gl_error; the exit-on-error entry points of the reference are kept by
// the CLI, which reports the message and exits 1 exactly where the reference does.
#include "model.h"
#include "runtime_error.h"

#include "ggml-hip.h"

#include <algorithm>
#include <random>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <emmintrin.h>

// ---- gguf metadata helpers (model.cpp:15-59) ----

static int64_t kv_find(const gguf_context * ctx, const char * key) {
    int64_t id = gguf_find_key(ctx, key);
    if (id < 0) throw gl_error(std::string("missing gguf key '") + key + "'");
    return id;
}

static long long kv_int(const gguf_context * ctx, const char * key) {
    int64_t id = kv_find(ctx, key);
    switch (gguf_get_kv_type(ctx, id)) {
        case GGUF_TYPE_UINT8:  return gguf_get_val_u8(ctx, id);
        case GGUF_TYPE_INT8:   return gguf_get_val_i8(ctx, id);
        case GGUF_TYPE_UINT16: return gguf_get_val_u16(ctx, id);
        case GGUF_TYPE_INT16:  return gguf_get_val_i16(ctx, id);
        case GGUF_TYPE_UINT32: return gguf_get_val_u32(ctx, id);
        case GGUF_TYPE_INT32:  return gguf_get_val_i32(ctx, id);
        case GGUF_TYPE_UINT64: return (long long) gguf_get_val_u64(ctx, id);
        case GGUF_TYPE_INT64:  return gguf_get_val_i64(ctx, id);
        default: throw gl_error(std::string("key '") + key + "' is not an integer type");
    }
}

static double kv_float(const gguf_context * ctx, const char * key) {
    int64_t id = kv_find(ctx, key);
    switch (gguf_get_kv_type(ctx, id)) {
        case GGUF_TYPE_FLOAT32: return gguf_get_val_f32(ctx, id);
        case GGUF_TYPE_FLOAT64: return gguf_get_val_f64(ctx, id);
        default: throw gl_error(std::string("key '") + key + "' is not a float type");
    }
}

static std::string kv_string(const gguf_context * ctx, const char * key) {
    int64_t id = kv_find(ctx, key);
    if (gguf_get_kv_type(ctx, id) != GGUF_TYPE_STRING) throw gl_error(std::string("key '") + key + "' is not a string type");
    return gguf_get_val_str(ctx, id);
}

// model.cpp:74-206 (transformer archs only)
hparams load_hparams(const gguf_context * ctx) {
    hparams h{};
    h.arch_name = kv_string(ctx, "general.architecture");
    if      (h.arch_name == "phi3")     h.arch = arch_t::PHI3;
    else if (h.arch_name == "qwen2")    h.arch = arch_t::QWEN2;
    else if (h.arch_name == "qwen3")    h.arch = arch_t::QWEN3;
    else if (h.arch_name == "llama")    h.arch = arch_t::LLAMA;
    else if (h.arch_name == "qwen3moe") h.arch = arch_t::QWEN3MOE;
    else throw gl_error("unsupported architecture '" + h.arch_name + "' (supported: phi3, qwen2, qwen3, llama, qwen3moe)");

    auto pfx = [&](const char * suffix) { return h.arch_name + "." + suffix; };

    h.n_embd  = kv_int(ctx, pfx("embedding_length").c_str());
    h.n_head  = kv_int(ctx, pfx("attention.head_count").c_str());
    h.n_layer = kv_int(ctx, pfx("block_count").c_str());
    h.n_ctx_train = kv_int(ctx, pfx("context_length").c_str());
    h.rms_eps = gguf_find_key(ctx, pfx("attention.layer_norm_rms_epsilon").c_str()) >= 0
                    ? (float) kv_float(ctx, pfx("attention.layer_norm_rms_epsilon").c_str()) : 0.0f;
    h.n_head_kv = kv_int(ctx, pfx("attention.head_count_kv").c_str());
    h.n_ff      = kv_int(ctx, pfx("feed_forward_length").c_str());
    h.rope_freq_base = (float) kv_float(ctx, pfx("rope.freq_base").c_str());

    std::string key_len_key = pfx("attention.key_length");
    h.n_embd_head = gguf_find_key(ctx, key_len_key.c_str()) >= 0 ? kv_int(ctx, key_len_key.c_str()) : h.n_embd / h.n_head;
    std::string rot_key = pfx("rope.dimension_count");
    h.n_rot = gguf_find_key(ctx, rot_key.c_str()) >= 0 ? kv_int(ctx, rot_key.c_str()) : h.n_embd_head;

    std::string ctx_orig_key = pfx("rope.scaling.original_context_length");
    h.has_rope_scaling = gguf_find_key(ctx, ctx_orig_key.c_str()) >= 0;
    if (h.has_rope_scaling) {
        h.n_ctx_orig       = kv_int(ctx, ctx_orig_key.c_str());
        h.rope_attn_factor = (float) kv_float(ctx, pfx("rope.scaling.attn_factor").c_str());
    } else {
        h.n_ctx_orig       = kv_int(ctx, pfx("context_length").c_str());
        h.rope_attn_factor = 1.0f;
    }

    // per-arch flags (model.cpp:155-159); qwen3moe shares qwen3's attention (QK-Norm, NEOX)
    h.qkv_fused    = (h.arch == arch_t::PHI3);
    h.has_qkv_bias = (h.arch == arch_t::QWEN2);
    h.has_qk_norm  = (h.arch == arch_t::QWEN3 || h.arch == arch_t::QWEN3MOE);
    h.ffn_fused    = (h.arch == arch_t::PHI3);
    h.rope_neox    = (h.arch != arch_t::LLAMA);

    if (h.arch == arch_t::QWEN3MOE) {
        h.n_expert      = kv_int(ctx, pfx("expert_count").c_str());
        h.n_expert_used = kv_int(ctx, pfx("expert_used_count").c_str());
        h.n_ff_exp      = kv_int(ctx, pfx("expert_feed_forward_length").c_str());
    }

    h.bos_id = gguf_find_key(ctx, "tokenizer.ggml.bos_token_id") >= 0 ? kv_int(ctx, "tokenizer.ggml.bos_token_id") : -1;
    h.eos_id = gguf_find_key(ctx, "tokenizer.ggml.eos_token_id") >= 0 ? kv_int(ctx, "tokenizer.ggml.eos_token_id") : -1;
    return h;
}

// ---- weights (model.cpp:525-665) ----

static struct ggml_tensor * must_get(struct ggml_context * ctx, const std::string & name) {
    struct ggml_tensor * t = ggml_get_tensor(ctx, name.c_str());
    if (!t) throw gl_error("missing tensor '" + name + "'");
    return t;
}

model load_model(struct ggml_context * wctx, const hparams & hp) {
    model m;
    m.token_embd  = must_get(wctx, "token_embd.weight");
    m.output_norm = must_get(wctx, "output_norm.weight");
    struct ggml_tensor * output_w = ggml_get_tensor(wctx, "output.weight");
    m.output = output_w ? output_w : m.token_embd;
    if (hp.has_rope_scaling) m.rope_factors = must_get(wctx, "rope_factors_short.weight");

    m.layers.resize(hp.n_layer);
    for (int64_t il = 0; il < hp.n_layer; il++) {
        std::string p = "blk." + std::to_string(il) + ".";
        layer_weights & l = m.layers[il];
        l.attn_norm   = must_get(wctx, p + "attn_norm.weight");
        l.attn_output = must_get(wctx, p + "attn_output.weight");
        l.ffn_norm    = must_get(wctx, p + "ffn_norm.weight");

        if (hp.qkv_fused) {
            l.attn_qkv = must_get(wctx, p + "attn_qkv.weight");
        } else {
            l.attn_q = must_get(wctx, p + "attn_q.weight");
            l.attn_k = must_get(wctx, p + "attn_k.weight");
            l.attn_v = must_get(wctx, p + "attn_v.weight");
            if (hp.has_qkv_bias) {
                l.attn_q_bias = must_get(wctx, p + "attn_q.bias");
                l.attn_k_bias = must_get(wctx, p + "attn_k.bias");
                l.attn_v_bias = must_get(wctx, p + "attn_v.bias");
            }
            if (hp.has_qk_norm) {
                l.attn_q_norm = must_get(wctx, p + "attn_q_norm.weight");
                l.attn_k_norm = must_get(wctx, p + "attn_k_norm.weight");
            }
        }

        if (hp.arch == arch_t::QWEN3MOE) {
            l.ffn_gate_inp  = must_get(wctx, p + "ffn_gate_inp.weight");
            l.ffn_gate_exps = must_get(wctx, p + "ffn_gate_exps.weight");
            l.ffn_up_exps   = must_get(wctx, p + "ffn_up_exps.weight");
            l.ffn_down_exps = must_get(wctx, p + "ffn_down_exps.weight");
        } else {
            l.ffn_down = must_get(wctx, p + "ffn_down.weight");
            if (hp.ffn_fused) {
                l.ffn_up_gate = must_get(wctx, p + "ffn_up.weight");
            } else {
                l.ffn_gate = must_get(wctx, p + "ffn_gate.weight");
                l.ffn_up   = must_get(wctx, p + "ffn_up.weight");
            }
        }
    }
    return m;
}

// model.cpp:667-788 (no prefix filter, no BF16 conversion: the in-scope archs ship none)
weights_store load_weights(const char * path, ggml_backend_t backend, struct gguf_context ** out_gguf) {
    struct ggml_context * meta_ctx = nullptr;
    struct gguf_init_params gp = { /*.no_alloc =*/ true, /*.ctx =*/ &meta_ctx };
    struct gguf_context * gctx = gguf_init_from_file(path, gp);
    if (!gctx || !meta_ctx) throw gl_error(std::string("failed to load '") + path + "'");

    const int64_t n_tensors = gguf_get_n_tensors(gctx);
    struct ggml_init_params ip = {
        /*.mem_size   =*/ (size_t) n_tensors * ggml_tensor_overhead() + ggml_graph_overhead(),
        /*.mem_buffer =*/ nullptr,
        /*.no_alloc   =*/ true,
    };
    struct ggml_context * wctx = ggml_init(ip);
    for (int64_t i = 0; i < n_tensors; i++) {
        const char * name = gguf_get_tensor_name(gctx, i);
        struct ggml_tensor * t = ggml_dup_tensor(wctx, ggml_get_tensor(meta_ctx, name));
        ggml_set_name(t, name);
    }

    weights_store ws;
    ws.ctx = wctx;
    ws.buffer = ggml_backend_alloc_ctx_tensors(wctx, backend);
    if (!ws.buffer) throw gl_error(std::string("failed to allocate backend memory for weights from '") + path + "'");

    FILE * f = fopen(path, "rb");
    if (!f) throw gl_error(std::string("failed to reopen '") + path + "' to read tensor data");
    const size_t data_base = gguf_get_data_offset(gctx);
    std::vector<uint8_t> buf;
    for (int64_t i = 0; i < n_tensors; i++) {
        const char * name = gguf_get_tensor_name(gctx, i);
        struct ggml_tensor * t = ggml_get_tensor(wctx, name);
        const size_t file_size = ggml_nbytes(t);
        const size_t offset = data_base + gguf_get_tensor_offset(gctx, i);
        buf.resize(file_size);
        if (fseek(f, (long) offset, SEEK_SET) != 0 || fread(buf.data(), 1, file_size, f) != file_size) {
            fclose(f);
            throw gl_error(std::string("failed to read tensor '") + name + "' from '" + path + "'");
        }
        ggml_backend_tensor_set(t, buf.data(), 0, file_size);
    }
    fclose(f);
    *out_gguf = gctx;
    ggml_free(meta_ctx);
    return ws;
}

// model.cpp:790-817 with a `hip` branch shaped like the vulkan one
ggml_backend_t init_backend(const std::string & name, int n_threads) {
    if (name == "cpu") {
        // the CPU backend is the reference restatement (oracle/), registered as "CPU" when loaded
        const std::string params = std::to_string(n_threads);
        ggml_backend_t backend = ggml_backend_init_by_name("CPU", params.c_str());
        if (!backend) throw gl_error("failed to initialize the cpu backend (the CPU reference library is not loaded)");
        return backend;
    }
    if (name == "hip") {
        if (ggml_backend_hip_get_device_count() == 0) throw gl_error("backend 'hip' requested but no HIP device is available");
        char desc[256];
        ggml_backend_hip_get_device_description(0, desc, sizeof(desc));
        fprintf(stderr, "hip device 0: %s\n", desc);
        ggml_backend_t backend = ggml_backend_hip_init(0);
        if (!backend) throw gl_error("failed to initialize the hip backend (device 0)");
        return backend;
    }
    throw gl_error("unknown backend '" + name + "' (expected cpu or hip)");
}

// ---- persistent KV cache (model.cpp:821-885) ----

kv_cache init_kv_cache(const model & m, const hparams & hp, ggml_backend_t backend, int64_t n_ctx) {
    kv_cache kv;
    const int64_t head_dim = hp.n_embd_head;
    size_t buf_size = ggml_tensor_overhead() * (size_t) (hp.n_layer * 2 + 8);
    struct ggml_init_params ip = { buf_size, nullptr, /*.no_alloc =*/ true };
    kv.ctx = ggml_init(ip);
    kv.k.resize(hp.n_layer);
    kv.v.resize(hp.n_layer);
    for (int64_t il = 0; il < hp.n_layer; il++) {
        kv.k[il] = ggml_new_tensor_3d(kv.ctx, GGML_TYPE_F16, head_dim, hp.n_head_kv, n_ctx);
        kv.v[il] = ggml_new_tensor_3d(kv.ctx, GGML_TYPE_F16, head_dim, hp.n_head_kv, n_ctx);
    }
    kv.buffer = ggml_backend_alloc_ctx_tensors(kv.ctx, backend);
    if (!kv.buffer) {
        char msg[256];
        snprintf(msg, sizeof(msg), "failed to allocate KV cache (%lld positions x %lld layers, %.0f MiB requested)",
                 (long long) n_ctx, (long long) hp.n_layer, (double) kv_cache_bytes(m, hp, n_ctx) / (1024.0 * 1024.0));
        throw gl_error(msg);
    }
    return kv;
}

size_t kv_cache_bytes(const model & m, const hparams & hp, int64_t n_ctx) {
    (void) m;
    const size_t es = ggml_type_size(GGML_TYPE_F16);
    return (size_t) (hp.n_embd_head * hp.n_head_kv) * es * 2 * (size_t) hp.n_layer * (size_t) n_ctx;
}

// ---- graph construction (model.cpp:1061-1474) ----

struct built_graph {
    struct ggml_cgraph * gf;
    struct ggml_tensor * tokens;
    struct ggml_tensor * positions;
    struct ggml_tensor * mask;
    struct ggml_tensor * logits;
};

static struct ggml_tensor * rms_norm_mul(struct ggml_context * ctx, struct ggml_tensor * x, struct ggml_tensor * w, float eps) {
    return ggml_mul(ctx, ggml_rms_norm(ctx, x, eps), w);
}

// model.cpp:1082-1108
static void build_qkv(struct ggml_context * ctx, const hparams & hp, const layer_weights & l, struct ggml_tensor * x,
                      int64_t n_new, int64_t head_dim, int64_t n_head_kv,
                      struct ggml_tensor ** out_Q, struct ggml_tensor ** out_K, struct ggml_tensor ** out_V) {
    const size_t es = sizeof(float);
    if (hp.qkv_fused) {
        struct ggml_tensor * qkv = ggml_mul_mat(ctx, l.attn_qkv, x);
        *out_Q = ggml_view_3d(ctx, qkv, head_dim, hp.n_head, n_new, head_dim * es, qkv->nb[1], 0);
        *out_K = ggml_view_3d(ctx, qkv, head_dim, n_head_kv, n_new, head_dim * es, qkv->nb[1], hp.n_head * head_dim * es);
        *out_V = ggml_view_3d(ctx, qkv, head_dim, n_head_kv, n_new, head_dim * es, qkv->nb[1], (hp.n_head + n_head_kv) * head_dim * es);
    } else {
        struct ggml_tensor * q = ggml_mul_mat(ctx, l.attn_q, x);
        struct ggml_tensor * k = ggml_mul_mat(ctx, l.attn_k, x);
        struct ggml_tensor * v = ggml_mul_mat(ctx, l.attn_v, x);
        if (hp.has_qkv_bias) {
            q = ggml_add(ctx, q, l.attn_q_bias);
            k = ggml_add(ctx, k, l.attn_k_bias);
            v = ggml_add(ctx, v, l.attn_v_bias);
        }
        *out_Q = ggml_reshape_3d(ctx, q, head_dim, hp.n_head, n_new);
        *out_K = ggml_reshape_3d(ctx, k, head_dim, n_head_kv, n_new);
        *out_V = ggml_reshape_3d(ctx, v, head_dim, n_head_kv, n_new);
    }
}

// model.cpp:1113-1127
static struct ggml_tensor * build_ffn_act(struct ggml_context * ctx, const hparams & hp, const layer_weights & l,
                                          struct ggml_tensor * y, int64_t n_new) {
    struct ggml_tensor * gate;
    struct ggml_tensor * up;
    if (hp.ffn_fused) {
        struct ggml_tensor * gate_up = ggml_mul_mat(ctx, l.ffn_up_gate, y);
        gate = ggml_view_2d(ctx, gate_up, hp.n_ff, n_new, gate_up->nb[1], 0);
        up   = ggml_view_2d(ctx, gate_up, hp.n_ff, n_new, gate_up->nb[1], hp.n_ff * sizeof(float));
    } else {
        gate = ggml_mul_mat(ctx, l.ffn_gate, y);
        up   = ggml_mul_mat(ctx, l.ffn_up, y);
    }
    return ggml_mul(ctx, ggml_silu(ctx, gate), up);
}

// Routed expert FFN for qwen3moe. The routing restates the reference MoE engine's moe_route
// (src/moe_stream/qwen_model.c:551-606: softmax over all experts, top-k with ties to the lower
// id, renormalize the k weights) and the expert sum of moe_block (:608-734: out = sum_k w_k *
// down_k(silu(gate_k(x)) * up_k(x))). The expert GEMVs are ggml_mul_mat_id.
static struct ggml_tensor * build_moe_ffn(struct ggml_context * ctx, const hparams & hp, const layer_weights & l,
                                          struct ggml_tensor * y, int64_t n_new, built_graph & bg);

// Graph capacity: the reference's GGML_DEFAULT_GRAPH_SIZE (model.cpp:1486) for the dense archs. A
// qwen3moe layer adds the router, top-k, renormalization, three mul_mat_id and the per-slot expert
// sum (about 60 tensors more), which overflows it at 48 layers.
static size_t graph_size_of(const hparams & hp) {
    return hp.n_expert > 0 ? std::max<size_t>(GGML_DEFAULT_GRAPH_SIZE, (size_t) hp.n_layer * 160 + 256)
                           : (size_t) GGML_DEFAULT_GRAPH_SIZE;
}

// model.cpp:1296-1474 (transformer archs)
static built_graph build_graph(struct ggml_context * ctx, const model & m, const hparams & hp, kv_cache & kv,
                               int64_t n_past, int64_t n_new, bool use_flash_attn,
                               struct ggml_tensor * tokens_in = nullptr) {
    built_graph bg{};
    bg.gf = ggml_new_graph_custom(ctx, graph_size_of(hp), false);

    const int64_t head_dim = hp.n_embd_head;
    const int64_t n_kv     = n_past + n_new;
    const float   kq_scale = 1.0f / sqrtf((float) head_dim);

    bg.tokens    = tokens_in ? tokens_in : ggml_new_tensor_1d(ctx, GGML_TYPE_I32, n_new);
    bg.positions = ggml_new_tensor_1d(ctx, GGML_TYPE_I32, n_new);
    bg.mask      = ggml_new_tensor_2d(ctx, GGML_TYPE_F32, n_kv, n_new);

    struct ggml_tensor * cur = ggml_get_rows(ctx, m.token_embd, bg.tokens);

    const float rope_ext_factor = hp.has_rope_scaling ? 1.0f : 0.0f;
    const float rope_beta_fast  = hp.has_rope_scaling ? 32.0f : 0.0f;
    const float rope_beta_slow  = hp.has_rope_scaling ? 1.0f : 0.0f;

    for (int64_t il = 0; il < hp.n_layer; il++) {
        const layer_weights & l = m.layers[il];
        struct ggml_tensor * residual = cur;
        struct ggml_tensor * x = rms_norm_mul(ctx, cur, l.attn_norm, hp.rms_eps);
        const int64_t n_head_kv = kv.k[il]->ne[1];

        struct ggml_tensor * Qcur;
        struct ggml_tensor * Kcur;
        struct ggml_tensor * Vcur;
        build_qkv(ctx, hp, l, x, n_new, head_dim, n_head_kv, &Qcur, &Kcur, &Vcur);

        if (hp.has_qk_norm) {
            Qcur = rms_norm_mul(ctx, Qcur, l.attn_q_norm, hp.rms_eps);
            Kcur = rms_norm_mul(ctx, Kcur, l.attn_k_norm, hp.rms_eps);
        }

        const int rope_mode = hp.rope_neox ? GGML_ROPE_TYPE_NEOX : GGML_ROPE_TYPE_NORMAL;
        Qcur = ggml_rope_ext(ctx, Qcur, bg.positions, m.rope_factors, (int) hp.n_rot, rope_mode, (int) hp.n_ctx_orig,
                             hp.rope_freq_base, 1.0f, rope_ext_factor, hp.rope_attn_factor, rope_beta_fast, rope_beta_slow);
        Kcur = ggml_rope_ext(ctx, Kcur, bg.positions, m.rope_factors, (int) hp.n_rot, rope_mode, (int) hp.n_ctx_orig,
                             hp.rope_freq_base, 1.0f, rope_ext_factor, hp.rope_attn_factor, rope_beta_fast, rope_beta_slow);

        struct ggml_tensor * k_dst = ggml_view_3d(ctx, kv.k[il], head_dim, n_head_kv, n_new,
                                                  kv.k[il]->nb[1], kv.k[il]->nb[2], n_past * kv.k[il]->nb[2]);
        struct ggml_tensor * v_dst = ggml_view_3d(ctx, kv.v[il], head_dim, n_head_kv, n_new,
                                                  kv.v[il]->nb[1], kv.v[il]->nb[2], n_past * kv.v[il]->nb[2]);
        ggml_build_forward_expand(bg.gf, ggml_cpy(ctx, Kcur, k_dst));
        ggml_build_forward_expand(bg.gf, ggml_cpy(ctx, Vcur, v_dst));

        struct ggml_tensor * K_full = ggml_view_3d(ctx, kv.k[il], head_dim, n_head_kv, n_kv, kv.k[il]->nb[1], kv.k[il]->nb[2], 0);
        struct ggml_tensor * V_full = ggml_view_3d(ctx, kv.v[il], head_dim, n_head_kv, n_kv, kv.v[il]->nb[1], kv.v[il]->nb[2], 0);

        struct ggml_tensor * Q = ggml_permute(ctx, Qcur, 0, 2, 1, 3);
        struct ggml_tensor * K = ggml_permute(ctx, K_full, 0, 2, 1, 3);

        if (use_flash_attn) {
            struct ggml_tensor * V_flash = ggml_permute(ctx, V_full, 0, 2, 1, 3);
            struct ggml_tensor * mask_f16 = ggml_cast(ctx, bg.mask, GGML_TYPE_F16);
            struct ggml_tensor * attn_out = ggml_flash_attn_ext(ctx, Q, K, V_flash, mask_f16, kq_scale, 0.0f, 0.0f);
            cur = ggml_cont_2d(ctx, attn_out, hp.n_head * head_dim, n_new);
        } else {
            struct ggml_tensor * KQ = ggml_mul_mat(ctx, K, Q);
            KQ = ggml_soft_max_ext(ctx, KQ, bg.mask, kq_scale, 0.0f);
            struct ggml_tensor * V_trans = ggml_cont_3d(ctx, ggml_permute(ctx, V_full, 1, 2, 0, 3), n_kv, head_dim, n_head_kv);
            struct ggml_tensor * KQV = ggml_mul_mat(ctx, V_trans, KQ);
            struct ggml_tensor * merged = ggml_permute(ctx, KQV, 0, 2, 1, 3);
            cur = ggml_cont_2d(ctx, merged, hp.n_head * head_dim, n_new);
        }

        cur = ggml_mul_mat(ctx, l.attn_output, cur);
        cur = ggml_add(ctx, cur, residual);

        residual = cur;
        struct ggml_tensor * y = rms_norm_mul(ctx, cur, l.ffn_norm, hp.rms_eps);
        if (hp.arch == arch_t::QWEN3MOE) {
            cur = build_moe_ffn(ctx, hp, l, y, n_new, bg);
        } else {
            struct ggml_tensor * ffn_act = build_ffn_act(ctx, hp, l, y, n_new);
            cur = ggml_mul_mat(ctx, l.ffn_down, ffn_act);
        }
        cur = ggml_add(ctx, cur, residual);
    }

    cur = rms_norm_mul(ctx, cur, m.output_norm, hp.rms_eps);
    bg.logits = ggml_mul_mat(ctx, m.output, cur);
    ggml_build_forward_expand(bg.gf, bg.logits);
    return bg;
}

static struct ggml_tensor * build_moe_ffn(struct ggml_context * ctx, const hparams & hp, const layer_weights & l,
                                          struct ggml_tensor * y, int64_t n_new, built_graph & bg) {
    (void) bg;
    const int64_t n_embd = hp.n_embd, n_expert = hp.n_expert, k = hp.n_expert_used;
    // router: logits [n_expert, n_new] from the f32 router, softmax over all experts
    struct ggml_tensor * probs = ggml_soft_max_ext(ctx, ggml_mul_mat(ctx, l.ffn_gate_inp, y), nullptr, 1.0f, 0.0f);
    // top-k by probability (stable: an earlier expert wins a tie), then their probabilities,
    // renormalized to sum to one
    struct ggml_tensor * selected = ggml_top_k(ctx, probs, (int) k);                          // I32 [k, n_new]
    struct ggml_tensor * w = ggml_get_rows(ctx, ggml_reshape_3d(ctx, probs, 1, n_expert, n_new), selected);  // [1, k, n_new]
    w = ggml_reshape_2d(ctx, w, k, n_new);
    w = ggml_div(ctx, w, ggml_sum_rows(ctx, w));
    w = ggml_reshape_3d(ctx, w, 1, k, n_new);
    // experts: gate/up on the token's activation, SwiGLU, down on each slot's activation
    struct ggml_tensor * x = ggml_reshape_3d(ctx, y, n_embd, 1, n_new);
    struct ggml_tensor * gate = ggml_mul_mat_id(ctx, l.ffn_gate_exps, x, selected);           // [n_ff_exp, k, n_new]
    struct ggml_tensor * up = ggml_mul_mat_id(ctx, l.ffn_up_exps, x, selected);
    struct ggml_tensor * act = ggml_mul(ctx, ggml_silu(ctx, gate), up);
    struct ggml_tensor * experts = ggml_mul_mat_id(ctx, l.ffn_down_exps, act, selected);     // [n_embd, k, n_new]
    experts = ggml_mul(ctx, experts, w);
    // out = w_0 down_0 + w_1 down_1 + ... in slot order
    struct ggml_tensor * out = ggml_view_2d(ctx, experts, n_embd, n_new, experts->nb[2], 0);
    for (int64_t i = 1; i < k; i++) {
        out = ggml_add(ctx, out, ggml_view_2d(ctx, experts, n_embd, n_new, experts->nb[2], (size_t) i * experts->nb[1]));
    }
    return out;
}

// model.cpp:1476-1494
decode_session init_decode_session(ggml_backend_t backend, const hparams & hp, bool use_flash_attn) {
    decode_session ds;
    const size_t n = graph_size_of(hp);
    size_t buf_size = ggml_tensor_overhead() * n + ggml_graph_overhead_custom(n, false);
    ds.graph_buf.resize(buf_size);
    ds.galloc = ggml_gallocr_new(ggml_backend_get_default_buffer_type(backend));
    ds.use_flash_attn = use_flash_attn;
    return ds;
}

void free_decode_session(decode_session & ds) {
    ggml_gallocr_free(ds.galloc);
    ds.galloc = nullptr;
}

// model.cpp:1496-1597. logits_out (n_vocab floats, may be null) receives the last column's logits; with greedy_out
// set instead, the graph ends in the argmax of that column (ggml_argmax: the first index of the
// maximum, the pick of argmax() below) and only the index is read back.
struct sample_job {
    sampler * smp;
    const std::vector<int32_t> * recent;
    int32_t token;
};

// a step of a device-fed greedy chain: its token is chain->tok, its argmax goes back there and to
// chain->hist[index]
struct chain_job {
    decode_chain * chain;
    int64_t index;
};

static void run_step(const model & m, const hparams & hp, kv_cache & kv, decode_session & ds, ggml_backend_t backend,
                     int64_t n_past, const std::vector<int32_t> & new_tokens, int64_t n_vocab, float * logits_out,
                     int32_t * greedy_out, sample_job * sj = nullptr, chain_job * cj = nullptr) {
    const int64_t n_new = (int64_t) new_tokens.size();
    const int64_t n_kv  = n_past + n_new;
    if (n_new <= 0) throw gl_error("forward_step: no tokens");
    if (n_kv > kv.k[0]->ne[2]) throw gl_error("forward_step: n_past + n_new exceeds the KV cache size");

    struct ggml_init_params gip = { ds.graph_buf.size(), ds.graph_buf.data(), /*.no_alloc =*/ true };
    struct ggml_context * gctx_build = ggml_init(gip);

    built_graph bg = build_graph(gctx_build, m, hp, kv, n_past, n_new, ds.use_flash_attn, cj ? cj->chain->tok : nullptr);
    struct ggml_tensor * pick = nullptr;
    if (cj) {
        struct ggml_tensor * last = ggml_view_1d(gctx_build, bg.logits, n_vocab, (size_t) (n_new - 1) * bg.logits->nb[1]);
        pick = ggml_argmax(gctx_build, last);
        struct ggml_tensor * next = ggml_cpy(gctx_build, pick, cj->chain->tok);
        struct ggml_tensor * rec = ggml_cpy(gctx_build, pick, ggml_view_1d(gctx_build, cj->chain->hist, 1, (size_t) cj->index * sizeof(int32_t)));
        ggml_build_forward_expand(bg.gf, next);
        ggml_build_forward_expand(bg.gf, rec);
    } else if (greedy_out) {
        struct ggml_tensor * last = ggml_view_1d(gctx_build, bg.logits, n_vocab, (size_t) (n_new - 1) * bg.logits->nb[1]);
        pick = ggml_argmax(gctx_build, last);
        ggml_set_output(pick);
        ggml_build_forward_expand(bg.gf, pick);
    }
    if (sj) {
        if (!ggml_backend_is_hip(backend)) {
            ggml_free(gctx_build);
            throw gl_error("forward_step_sample: device sampling needs the hip backend");
        }
        ggml_set_output(bg.logits);
    }

    if (!ggml_gallocr_alloc_graph(ds.galloc, bg.gf)) {
        ggml_free(gctx_build);
        throw gl_error("graph allocation failed");
    }

    if (!cj) ggml_backend_tensor_set(bg.tokens, new_tokens.data(), 0, n_new * sizeof(int32_t));

    std::vector<int32_t> positions(n_new);
    for (int64_t i = 0; i < n_new; i++) positions[i] = (int32_t) (n_past + i);
    ggml_backend_tensor_set(bg.positions, positions.data(), 0, n_new * sizeof(int32_t));

    std::vector<float> mask((size_t) (n_kv * n_new));
    for (int64_t q = 0; q < n_new; q++) {
        const int64_t abs_q = n_past + q;
        for (int64_t k = 0; k < n_kv; k++) mask[q * n_kv + k] = (k <= abs_q) ? 0.0f : -INFINITY;
    }
    ggml_backend_tensor_set(bg.mask, mask.data(), 0, mask.size() * sizeof(float));

    if (cj) {
        // queued: the next step's graph is built while this one runs
        ggml_backend_graph_compute_async(backend, bg.gf);
        ggml_free(gctx_build);
        return;
    }
    ggml_backend_graph_compute(backend, bg.gf);

    if (sj) {
        // model.cpp:1675-1728 on the last column, with the generator's next variate
        sampler & smp = *sj->smp;
        if (!smp.has_u) {
            smp.u = std::generate_canonical<double, 53>(smp.rng);
            smp.has_u = true;
        }
        const ggml_hip_sampler_params sp = { smp.params.temp, smp.params.top_k, smp.params.top_p,
                                             smp.params.repeat_penalty, smp.params.repeat_last_n };
        bool used = false;
        const enum ggml_status st = ggml_backend_hip_sample(backend, bg.logits, n_new - 1, &sp, sj->recent->data(),
                                                            sj->recent->size(), smp.u, &sj->token, &used);
        if (st != GGML_STATUS_SUCCESS) {
            ggml_free(gctx_build);
            throw gl_error("forward_step_sample: device sampling failed");
        }
        if (used) smp.has_u = false;
    } else if (greedy_out) {
        ggml_backend_tensor_get(pick, greedy_out, 0, sizeof(int32_t));
    } else if (logits_out) {
        const size_t last_col_offset = (size_t) (n_new - 1) * n_vocab * sizeof(float);
        ggml_backend_tensor_get(bg.logits, logits_out, last_col_offset, n_vocab * sizeof(float));
    }
    ggml_free(gctx_build);
}

std::vector<float> forward_step(const model & m, const hparams & hp, kv_cache & kv, decode_session & ds,
                                ggml_backend_t backend, int64_t n_past, const std::vector<int32_t> & new_tokens,
                                int64_t n_vocab) {
    std::vector<float> last_logits(n_vocab);
    run_step(m, hp, kv, ds, backend, n_past, new_tokens, n_vocab, last_logits.data(), nullptr);
    return last_logits;
}

void forward_step_into(const model & m, const hparams & hp, kv_cache & kv, decode_session & ds, ggml_backend_t backend,
                       int64_t n_past, const std::vector<int32_t> & new_tokens, int64_t n_vocab, float * logits) {
    run_step(m, hp, kv, ds, backend, n_past, new_tokens, n_vocab, logits, nullptr);
}

int32_t forward_step_greedy(const model & m, const hparams & hp, kv_cache & kv, decode_session & ds,
                            ggml_backend_t backend, int64_t n_past, const std::vector<int32_t> & new_tokens,
                            int64_t n_vocab) {
    int32_t tok = 0;
    run_step(m, hp, kv, ds, backend, n_past, new_tokens, n_vocab, nullptr, &tok);
    return tok;
}

decode_chain init_decode_chain(ggml_backend_t backend, int32_t first_token, int64_t n_steps) {
    decode_chain dc;
    struct ggml_init_params ip = { 2 * ggml_tensor_overhead(), nullptr, /*.no_alloc =*/ true };
    dc.ctx = ggml_init(ip);
    dc.tok = ggml_new_tensor_1d(dc.ctx, GGML_TYPE_I32, 1);
    dc.hist = ggml_new_tensor_1d(dc.ctx, GGML_TYPE_I32, std::max<int64_t>(n_steps, 1));
    dc.buf = ggml_backend_alloc_ctx_tensors(dc.ctx, backend);
    if (!dc.buf) {
        ggml_free(dc.ctx);
        throw gl_error("decode chain: allocation failed");
    }
    ggml_backend_tensor_set(dc.tok, &first_token, 0, sizeof(int32_t));
    dc.n_steps = n_steps;
    return dc;
}

void free_decode_chain(decode_chain & dc) {
    if (dc.buf) ggml_backend_buffer_free(dc.buf);
    if (dc.ctx) ggml_free(dc.ctx);
    dc = decode_chain{};
}

void forward_step_chained(const model & m, const hparams & hp, kv_cache & kv, decode_session & ds, ggml_backend_t backend,
                          int64_t n_past, int64_t n_vocab, decode_chain & chain, int64_t index) {
    if (index < 0 || index >= chain.n_steps) throw gl_error("forward_step_chained: step index out of range");
    chain_job cj = { &chain, index };
    run_step(m, hp, kv, ds, backend, n_past, { 0 }, n_vocab, nullptr, nullptr, nullptr, &cj);
}

// model.cpp:1668-1673
sampler init_sampler(const sampler_params & params) {
    sampler smp;
    smp.params = params;
    smp.rng.seed(params.seed != 0 ? params.seed : std::random_device{}());
    return smp;
}

int32_t forward_step_sample(const model & m, const hparams & hp, kv_cache & kv, decode_session & ds,
                            ggml_backend_t backend, int64_t n_past, const std::vector<int32_t> & new_tokens,
                            int64_t n_vocab, sampler & smp, const std::vector<int32_t> & recent_tokens) {
    sample_job sj = { &smp, &recent_tokens, 0 };
    run_step(m, hp, kv, ds, backend, n_past, new_tokens, n_vocab, nullptr, nullptr, &sj);
    return sj.token;
}

// model.cpp:1624-1657 (the Vulkan-only chunking policy is kept for callers that ask for it)
std::vector<float> prefill(const model & m, const hparams & hp, kv_cache & kv, decode_session & ds,
                           ggml_backend_t backend, int64_t n_past, const std::vector<int32_t> & tokens,
                           int64_t n_vocab, bool use_chunking) {
    constexpr size_t kFastChunk = 8;
    constexpr size_t kBadZoneMax = 32;
    if (!use_chunking || tokens.size() <= kFastChunk || tokens.size() > kBadZoneMax) {
        return forward_step(m, hp, kv, ds, backend, n_past, tokens, n_vocab);
    }
    std::vector<float> last_logits;
    for (size_t off = 0; off < tokens.size(); off += kFastChunk) {
        const size_t n = std::min(kFastChunk, tokens.size() - off);
        std::vector<int32_t> chunk(tokens.begin() + off, tokens.begin() + off + n);
        last_logits = forward_step(m, hp, kv, ds, backend, n_past + (int64_t) off, chunk, n_vocab);
    }
    return last_logits;
}

// model.cpp:1659-1666: greedy, first index of the maximum wins
int32_t argmax(const std::vector<float> & logits) {
    // the first index of the largest value: the maximum from eight running maxima in two SSE
    // registers (no loop-carried branch), then its first occurrence; a leading NaN keeps index 0,
    // as the single-pass compare does
    const float * v = logits.data();
    const size_t n = logits.size();
    // maxps(a, b) returns a > b ? a : b, so a NaN value never replaces a running maximum
    __m128 m0 = _mm_set1_ps(v[0]), m1 = m0;
    size_t i = 0;
    for (; i + 8 <= n; i += 8) {
        m0 = _mm_max_ps(_mm_loadu_ps(v + i), m0);
        m1 = _mm_max_ps(_mm_loadu_ps(v + i + 4), m1);
    }
    float m[8];
    _mm_storeu_ps(m, m0);
    _mm_storeu_ps(m + 4, m1);
    float best = v[0];
    for (int k = 0; k < 8; k++) best = m[k] > best ? m[k] : best;
    for (; i < n; i++) best = v[i] > best ? v[i] : best;
    for (size_t j = 0; j < n; j++) {
        if (v[j] == best) return (int32_t) j;
    }
    return 0;
}
