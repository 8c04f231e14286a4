// capi.cpp — C-ABI sessions over the forward-pass runtime (include/ggml-loader.h).
#include "ggml-loader.h"
#include "model.h"
#include "runtime_error.h"

#include <omp.h>

#include <chrono>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <vector>

struct gl_session {
    ggml_backend_t backend = nullptr;
    gguf_context * gguf = nullptr;
    weights_store ws;
    hparams hp;
    model m;
    kv_cache kv;
    decode_session ds;
    int64_t n_vocab = 0;
    int64_t n_ctx = 0;
    bool ds_ready = false;
};

static void set_err(char * err, size_t n, const char * msg) {
    if (err && n) snprintf(err, n, "%s", msg);
}

static void session_release(gl_session * s) {
    if (!s) return;
    if (s->ds_ready) free_decode_session(s->ds);
    if (s->kv.buffer) ggml_backend_buffer_free(s->kv.buffer);
    if (s->kv.ctx) ggml_free(s->kv.ctx);
    if (s->ws.buffer) ggml_backend_buffer_free(s->ws.buffer);
    if (s->ws.ctx) ggml_free(s->ws.ctx);
    if (s->gguf) gguf_free(s->gguf);
    if (s->backend) ggml_backend_free(s->backend);
    delete s;
}

extern "C" {

gl_session * gl_session_open(const char * model_path, const char * backend, int n_threads, int64_t n_ctx,
                             int flash_attn, char * err, size_t err_size) {
    gl_session * s = new gl_session();
    try {
        // same order as cmd_bench.cpp:106-129
        s->backend = init_backend(backend ? backend : "hip", n_threads);
        s->ws = load_weights(model_path, s->backend, &s->gguf);
        s->hp = load_hparams(s->gguf);
        s->m = load_model(s->ws.ctx, s->hp);
        s->n_vocab = s->m.token_embd->ne[1];
        if (n_ctx < 1) throw gl_error("n_ctx must be >= 1");
        s->n_ctx = n_ctx;
        s->kv = init_kv_cache(s->m, s->hp, s->backend, n_ctx);
        s->ds = init_decode_session(s->backend, s->hp, flash_attn != 0);
        s->ds_ready = true;
    } catch (const std::exception & e) {
        set_err(err, err_size, e.what());
        session_release(s);
        return nullptr;
    }
    return s;
}

void gl_session_free(gl_session * s) { session_release(s); }

ggml_backend_t gl_session_backend(gl_session * s) { return s ? s->backend : nullptr; }

int64_t gl_session_get(const gl_session * s, const char * name) {
    const std::string n = name;
    const hparams & h = s->hp;
    if (n == "n_vocab") return s->n_vocab;
    if (n == "n_embd") return h.n_embd;
    if (n == "n_layer") return h.n_layer;
    if (n == "n_head") return h.n_head;
    if (n == "n_head_kv") return h.n_head_kv;
    if (n == "head_dim") return h.n_embd_head;
    if (n == "n_ff") return h.n_ff;
    if (n == "n_ctx") return s->n_ctx;
    if (n == "n_expert") return h.n_expert;
    if (n == "n_expert_used") return h.n_expert_used;
    if (n == "weights_bytes") return (int64_t) ggml_backend_buffer_get_size(s->ws.buffer);
    return -1;
}

int gl_forward_step(gl_session * s, int64_t n_past, const int32_t * tokens, int64_t n_new, float * logits,
                    char * err, size_t err_size) {
    try {
        for (int64_t i = 0; i < n_new; i++) {
            if (tokens[i] < 0 || tokens[i] >= s->n_vocab) throw gl_error("token id out of range");
        }
        std::vector<int32_t> toks(tokens, tokens + n_new);
        forward_step_into(s->m, s->hp, s->kv, s->ds, s->backend, n_past, toks, s->n_vocab, logits);
    } catch (const std::exception & e) {
        set_err(err, err_size, e.what());
        return 1;
    }
    return 0;
}

int gl_generate(gl_session * s, int64_t n_past, const int32_t * prompt, int64_t n_prompt, int n_steps,
                const gl_sampler_params * params, int32_t * tokens_out, double * seconds, char * err, size_t err_size) {
    try {
        if (!params || !prompt || n_prompt < 1 || n_steps < 1) throw gl_error("gl_generate: bad arguments");
        for (int64_t i = 0; i < n_prompt; i++) {
            if (prompt[i] < 0 || prompt[i] >= s->n_vocab) throw gl_error("token id out of range");
        }
        sampler_params sp;
        sp.temp = params->temp;
        sp.top_k = params->top_k;
        sp.top_p = params->top_p;
        sp.repeat_penalty = params->repeat_penalty;
        sp.repeat_last_n = params->repeat_last_n;
        sp.seed = params->seed;
        sampler smp = init_sampler(sp);
        auto t0 = std::chrono::steady_clock::now();
        // cmd_run.cpp:503-510: the prompt in one step, then the first sample over all_tokens
        std::vector<int32_t> all_tokens(prompt, prompt + n_prompt);
        int64_t pos = n_past + n_prompt;
        int32_t next = forward_step_sample(s->m, s->hp, s->kv, s->ds, s->backend, n_past, all_tokens, s->n_vocab, smp,
                                           all_tokens);
        tokens_out[0] = next;
        // cmd_run.cpp:582-619: feed the token, extend all_tokens, sample again
        for (int i = 1; i < n_steps; i++) {
            all_tokens.push_back(next);
            next = forward_step_sample(s->m, s->hp, s->kv, s->ds, s->backend, pos, { next }, s->n_vocab, smp, all_tokens);
            pos++;
            tokens_out[i] = next;
        }
        auto t1 = std::chrono::steady_clock::now();
        if (seconds) *seconds = std::chrono::duration<double>(t1 - t0).count();
    } catch (const std::exception & e) {
        set_err(err, err_size, e.what());
        return 1;
    }
    return 0;
}

int gl_decode_loop(gl_session * s, int64_t n_past, int32_t first_token, int n_steps, int fixed_pos,
                   int32_t * tokens_out, double * seconds, char * err, size_t err_size) {
    try {
        if (first_token < 0 || first_token >= s->n_vocab) throw gl_error("token id out of range");
        if (n_steps < 1) throw gl_error("n_steps must be >= 1");
        // cmd_bench.cpp:52-61: the n_tg loop of forward_step + argmax. The argmax of the last logits
        // column runs on the backend and feeds the next step there (decode_chain), so the host
        // queues step after step without waiting; the timed region ends when the last step is done.
        decode_chain dc = init_decode_chain(s->backend, first_token, n_steps);
        try {
            ggml_backend_synchronize(s->backend);
            auto t0 = std::chrono::steady_clock::now();
            for (int i = 0; i < n_steps; i++) {
                const int64_t pos = fixed_pos ? n_past : n_past + i;
                forward_step_chained(s->m, s->hp, s->kv, s->ds, s->backend, pos, s->n_vocab, dc, i);
            }
            ggml_backend_synchronize(s->backend);
            auto t1 = std::chrono::steady_clock::now();
            if (seconds) *seconds = std::chrono::duration<double>(t1 - t0).count();
            if (tokens_out) ggml_backend_tensor_get(dc.hist, tokens_out, 0, (size_t) n_steps * sizeof(int32_t));
        } catch (...) {
            ggml_backend_synchronize(s->backend);
            free_decode_chain(dc);
            throw;
        }
        free_decode_chain(dc);
    } catch (const std::exception & e) {
        set_err(err, err_size, e.what());
        return 1;
    }
    return 0;
}

int gl_kv_fill_random(gl_session * s, int64_t n_pos, uint64_t seed, char * err, size_t err_size) {
    try {
        if (n_pos < 0 || n_pos > s->n_ctx) throw gl_error("kv fill: n_pos out of range");
        if (n_pos == 0) return 0;
        const int64_t per_pos = s->hp.n_embd_head * s->hp.n_head_kv;
        const int64_t n = per_pos * n_pos;
        std::vector<float> f((size_t) n);
        std::vector<ggml_fp16_t> h((size_t) n);
        for (int64_t il = 0; il < s->hp.n_layer; il++) {
            for (int is_v = 0; is_v < 2; is_v++) {
                const uint64_t key = seed * 0x9E3779B97F4A7C15ull + (uint64_t) (il * 2 + is_v) * 0xD1B54A32D192ED03ull;
                gl_fill_normal(f.data(), n, key, 0, 0.0f, 1.0f);
                #pragma omp parallel for schedule(static)
                for (int64_t i = 0; i < n; i++) h[i] = ggml_fp32_to_fp16(f[i]);
                ggml_tensor * t = is_v ? s->kv.v[il] : s->kv.k[il];
                ggml_backend_tensor_set(t, h.data(), 0, (size_t) n * sizeof(ggml_fp16_t));
            }
        }
    } catch (const std::exception & e) {
        set_err(err, err_size, e.what());
        return 1;
    }
    return 0;
}

int gl_kv_read(gl_session * s, int layer, int is_v, void * dst, size_t offset, size_t size) {
    if (layer < 0 || layer >= (int) s->kv.k.size()) return 1;
    ggml_tensor * t = is_v ? s->kv.v[layer] : s->kv.k[layer];
    if (offset + size > ggml_nbytes(t)) return 1;
    ggml_backend_tensor_get(t, dst, offset, size);
    return 0;
}

} // extern "C"
