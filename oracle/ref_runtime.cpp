// Test infrastructure only: the reference's own model runtime (GGML-Loader src/model.cpp and
// src/dory.c, compiled unchanged from their sources by Makefile.ref against include/) driven on a
// backend the caller hands in, in the order cmd_bench.cpp:106-129 and :161-168 use it:
// load_weights, load_hparams, load_model, init_kv_cache, init_ssm_state, init_decode_session, then
// forward_step / prefill, then the same teardown. The backend is the only thing that differs from
// the reference's own program: the tests pass the hip backend (ggml_backend_hip_init) or the
// oracle's CPU backend, so the reference's unchanged caller runs on this library.
#include "model.h"

#include <cstdio>
#include <cstring>
#include <vector>

namespace {

struct ref_rt {
    ggml_backend_t backend = nullptr;
    gguf_context * gguf = nullptr;
    weights_store ws;
    hparams hp;
    model m;
    kv_cache kv;
    ssm_state ss;
    decode_session ds;
    int64_t n_vocab = 0;
};

int give(const std::vector<float> & logits, float * out, int64_t n_vocab) {
    if ((int64_t) logits.size() != n_vocab) return -1;
    std::memcpy(out, logits.data(), (size_t) n_vocab * sizeof(float));
    return 0;
}

}  // namespace

extern "C" void * ref_rt_open(const char * path, ggml_backend_t backend, int64_t n_ctx, int flash_attn) {
    ref_rt * r = new ref_rt;
    r->backend = backend;
    r->ws = load_weights(path, backend, &r->gguf);
    r->hp = load_hparams(r->gguf);
    r->m = load_model(r->ws.ctx, r->hp);
    r->n_vocab = r->m.token_embd->ne[1];
    r->kv = init_kv_cache(r->m, r->hp, backend, n_ctx);
    r->ss = init_ssm_state(r->hp, backend);
    r->ds = init_decode_session(backend, r->hp, flash_attn != 0);
    return r;
}

extern "C" int64_t ref_rt_n_vocab(void * h) { return ((ref_rt *) h)->n_vocab; }

// the bytes of the K/V storage set to `value` (init_kv_cache leaves them as allocated)
extern "C" void ref_rt_kv_fill(void * h, uint8_t value) {
    ref_rt * r = (ref_rt *) h;
    ggml_backend_buffer_clear(r->kv.buffer, value);
}

// forward_step (model.cpp:1496-1597): logits of the last of the n tokens
extern "C" int ref_rt_forward(void * h, int64_t n_past, const int32_t * tokens, int64_t n, float * logits) {
    ref_rt * r = (ref_rt *) h;
    const std::vector<int32_t> toks(tokens, tokens + n);
    return give(forward_step(r->m, r->hp, r->kv, r->ds, r->backend, n_past, toks, r->n_vocab, &r->ss), logits,
                r->n_vocab);
}

// prefill (model.cpp:1623-1657): chunked as the reference chunks (dory always; use_chunking as given)
extern "C" int ref_rt_prefill(void * h, int64_t n_past, const int32_t * tokens, int64_t n, int use_chunking,
                              float * logits) {
    ref_rt * r = (ref_rt *) h;
    const std::vector<int32_t> toks(tokens, tokens + n);
    return give(prefill(r->m, r->hp, r->kv, r->ds, r->backend, n_past, toks, r->n_vocab, use_chunking != 0, &r->ss),
                logits, r->n_vocab);
}

// cmd_bench.cpp:161-168 minus the backend, which stays the caller's
extern "C" void ref_rt_close(void * h) {
    ref_rt * r = (ref_rt *) h;
    free_decode_session(r->ds);
    free_ssm_state(r->ss);
    ggml_backend_buffer_free(r->kv.buffer);
    ggml_free(r->kv.ctx);
    ggml_backend_buffer_free(r->ws.buffer);
    ggml_free(r->ws.ctx);
    gguf_free(r->gguf);
    delete r;
}
