// model.h — per-token forward-pass runtime over the ggml API (host side of the boundary).
//
// Mirrors GGML-Loader's model runtime for the path this build accelerates (reference
// src/model.h:63-408, src/model.cpp:15-206, 523-885, 1061-1728): the same structs, function names,
// argument meanings and exit-on-error behaviour, restricted to the transformer architectures in
// scope (llama, qwen2, qwen3, phi3) plus qwen3moe, whose expert FFN runs through
// ggml_mul_mat_id. Tokenizer/chat templates, the hybrid SSM archs, dory and phone-RAM context
// sizing are out of scope.
#pragma once

#include "ggml.h"
#include "ggml-alloc.h"
#include "ggml-backend.h"
#include "gguf.h"

#include <cstdint>
#include <random>
#include <string>
#include <vector>

enum class arch_t { PHI3, QWEN2, QWEN3, LLAMA, QWEN3MOE };

// model.h:63-161
struct hparams {
    arch_t      arch;
    std::string arch_name;

    int64_t n_embd;
    int64_t n_head;
    int64_t n_head_kv;
    int64_t n_embd_head;
    int64_t n_layer;
    int64_t n_ctx_train;
    int64_t n_ff;
    int64_t n_rot;
    bool    rope_neox;
    float   rms_eps;
    float   rope_freq_base;

    bool    has_rope_scaling;
    int64_t n_ctx_orig;
    float   rope_attn_factor;

    bool qkv_fused;
    bool has_qkv_bias;
    bool has_qk_norm;
    bool ffn_fused;

    // qwen3moe (expert FFN in every layer)
    int64_t n_expert      = 0;
    int64_t n_expert_used = 0;
    int64_t n_ff_exp      = 0;

    int64_t bos_id;
    int64_t eos_id;
};

hparams load_hparams(const gguf_context * ctx);

// model.h:94-129
struct layer_weights {
    struct ggml_tensor * attn_norm = nullptr;
    struct ggml_tensor * attn_qkv = nullptr;
    struct ggml_tensor * attn_q = nullptr;
    struct ggml_tensor * attn_k = nullptr;
    struct ggml_tensor * attn_v = nullptr;
    struct ggml_tensor * attn_q_bias = nullptr;
    struct ggml_tensor * attn_k_bias = nullptr;
    struct ggml_tensor * attn_v_bias = nullptr;
    struct ggml_tensor * attn_q_norm = nullptr;
    struct ggml_tensor * attn_k_norm = nullptr;
    struct ggml_tensor * attn_output = nullptr;
    struct ggml_tensor * ffn_norm = nullptr;
    struct ggml_tensor * ffn_up_gate = nullptr;
    struct ggml_tensor * ffn_gate = nullptr;
    struct ggml_tensor * ffn_up = nullptr;
    struct ggml_tensor * ffn_down = nullptr;
    // qwen3moe
    struct ggml_tensor * ffn_gate_inp = nullptr;  // router [n_embd, n_expert] f32
    struct ggml_tensor * ffn_gate_exps = nullptr; // [n_embd, n_ff_exp, n_expert]
    struct ggml_tensor * ffn_up_exps = nullptr;   // [n_embd, n_ff_exp, n_expert]
    struct ggml_tensor * ffn_down_exps = nullptr; // [n_ff_exp, n_embd, n_expert]
};

struct model {
    struct ggml_tensor * token_embd = nullptr;
    struct ggml_tensor * output = nullptr;
    struct ggml_tensor * output_norm = nullptr;
    struct ggml_tensor * rope_factors = nullptr;
    std::vector<layer_weights> layers;
};

model load_model(struct ggml_context * wctx, const hparams & hp);

struct weights_store {
    struct ggml_context * ctx = nullptr;
    ggml_backend_buffer_t buffer = nullptr;
};
weights_store load_weights(const char * path, ggml_backend_t backend, struct gguf_context ** out_gguf);

// model.cpp:790-817, with the `hip` branch this build adds
ggml_backend_t init_backend(const std::string & name, int n_threads);

struct kv_cache {
    struct ggml_context * ctx = nullptr;
    ggml_backend_buffer_t buffer = nullptr;
    std::vector<struct ggml_tensor *> k;
    std::vector<struct ggml_tensor *> v;
};
kv_cache init_kv_cache(const model & m, const hparams & hp, ggml_backend_t backend, int64_t n_ctx);
size_t kv_cache_bytes(const model & m, const hparams & hp, int64_t n_ctx);

struct decode_session {
    std::vector<uint8_t> graph_buf;
    ggml_gallocr_t galloc = nullptr;
    bool use_flash_attn = false;
};
decode_session init_decode_session(ggml_backend_t backend, const hparams & hp, bool use_flash_attn = false);
void free_decode_session(decode_session & ds);

std::vector<float> forward_step(const model & m, const hparams & hp, kv_cache & kv, decode_session & ds,
                                ggml_backend_t backend, int64_t n_past, const std::vector<int32_t> & new_tokens,
                                int64_t n_vocab);
// forward_step writing the last column's logits (n_vocab floats) to logits, or nothing when it is null
void forward_step_into(const model & m, const hparams & hp, kv_cache & kv, decode_session & ds, ggml_backend_t backend,
                       int64_t n_past, const std::vector<int32_t> & new_tokens, int64_t n_vocab, float * logits);
// forward_step + the greedy pick of the last column computed on the backend (only the index is
// read back; the same token as argmax(forward_step(...)))
int32_t forward_step_greedy(const model & m, const hparams & hp, kv_cache & kv, decode_session & ds,
                            ggml_backend_t backend, int64_t n_past, const std::vector<int32_t> & new_tokens,
                            int64_t n_vocab);

std::vector<float> prefill(const model & m, const hparams & hp, kv_cache & kv, decode_session & ds,
                           ggml_backend_t backend, int64_t n_past, const std::vector<int32_t> & tokens,
                           int64_t n_vocab, bool use_chunking);

int32_t argmax(const std::vector<float> & logits);

// A greedy decode fed on the device: the token of a step lives in a one-element device tensor
// (tok) that the step's graph reads (get_rows) and overwrites with the argmax of its last logits
// column (ggml_cpy), which is also copied into hist[index]. Each step is queued with
// ggml_backend_graph_compute_async, so the host builds the next step while the device runs this
// one and never waits in between; ggml_backend_synchronize then hist give the tokens, the ones
// argmax(forward_step(...)) would have picked step by step.
struct decode_chain {
    struct ggml_context * ctx = nullptr;
    ggml_backend_buffer_t buf = nullptr;
    struct ggml_tensor * tok = nullptr;    // I32 [1]
    struct ggml_tensor * hist = nullptr;   // I32 [n_steps]
    int64_t n_steps = 0;
};
decode_chain init_decode_chain(ggml_backend_t backend, int32_t first_token, int64_t n_steps);
void free_decode_chain(decode_chain & dc);
void forward_step_chained(const model & m, const hparams & hp, kv_cache & kv, decode_session & ds, ggml_backend_t backend,
                          int64_t n_past, int64_t n_vocab, decode_chain & chain, int64_t index);

// model.h:410-430: sampling parameters (temp <= 0 is greedy) and state. The generator is the
// reference's std::mt19937; a uniform variate it has produced for a draw stays pending until a
// draw consumes it (the reference's generator is not advanced when no draw happens).
struct sampler_params {
    float    temp           = 0.0f;
    int      top_k          = 40;
    float    top_p          = 0.95f;
    float    repeat_penalty = 1.0f;
    int      repeat_last_n  = 64;
    uint32_t seed           = 0;   // 0 = seed from std::random_device
};
struct sampler {
    sampler_params params;
    std::mt19937 rng;
    bool has_u = false;
    double u = 0.0;
};
// model.cpp:1668-1673
sampler init_sampler(const sampler_params & params);
// forward_step + sample(smp, logits, recent_tokens) (model.cpp:1675-1728) of the last column, on
// the device (HIP backend): only the token id is read back
int32_t forward_step_sample(const model & m, const hparams & hp, kv_cache & kv, decode_session & ds,
                            ggml_backend_t backend, int64_t n_past, const std::vector<int32_t> & new_tokens,
                            int64_t n_vocab, sampler & smp, const std::vector<int32_t> & recent_tokens);
