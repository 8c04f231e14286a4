// ggml-loader.h — C-ABI over the forward-pass runtime (for FFI callers: Python ctypes in this
// repository's tests and bench, or any cgo/JNI binding).
//
// Each entry point wraps one reference runtime function so a caller can drive the same sequence
// cmd_bench/cmd_run do (cmd_bench.cpp:41-64, 106-129; cmd_run.cpp:397-620):
//   gl_session_open   init_backend + load_weights + load_hparams + load_model + init_kv_cache +
//                     init_decode_session (model.cpp:667-885, 1476-1494)
//   gl_forward_step   forward_step (model.cpp:1496-1597): logits of the last new token
//   gl_decode_loop    run_cycle's tg loop (cmd_bench.cpp:52-59): n steps of forward_step + argmax
//                     (the argmax runs on the backend; one index is read back per step)
//   gl_generate       cmd_run's sampled generation (temperature / top-k / top-p / repeat penalty
//                     sampled on the device; one index is read back per step)
//   gl_synth_model    writes the seeded synthetic GGUF models the benchmark configs describe
// Errors return non-zero (or NULL) and write a message into err; nothing here calls exit().
#pragma once

#include "ggml-backend.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef struct gl_session gl_session;

GGML_API gl_session * gl_session_open(const char * model_path, const char * backend, int n_threads, int64_t n_ctx,
                                      int flash_attn, char * err, size_t err_size);
GGML_API void         gl_session_free(gl_session * s);
GGML_API ggml_backend_t gl_session_backend(gl_session * s);
// "n_vocab", "n_embd", "n_layer", "n_head", "n_head_kv", "head_dim", "n_ff", "n_ctx", "n_expert",
// "n_expert_used", "weights_bytes"; -1 for an unknown name
GGML_API int64_t      gl_session_get(const gl_session * s, const char * name);

// logits: n_vocab floats for the last of the n_new tokens (NULL: computed, not read back)
GGML_API int gl_forward_step(gl_session * s, int64_t n_past, const int32_t * tokens, int64_t n_new, float * logits,
                             char * err, size_t err_size);
// Greedy decode: n_steps x {forward_step(n_past_i, {tok}); tok = argmax} (the first index of the
// maximum of the last logits column, picked by the graph's argmax op on the backend). With fixed_pos != 0 every
// step runs at n_past (the same position), otherwise n_past advances by one per step. tokens_out
// (n_steps entries, may be NULL) receives each step's argmax; *seconds receives the wall time.
GGML_API int gl_decode_loop(gl_session * s, int64_t n_past, int32_t first_token, int n_steps, int fixed_pos,
                            int32_t * tokens_out, double * seconds, char * err, size_t err_size);

// Sampled generation as cmd_run drives it (cmd_run.cpp:503-510, 576-620), on the HIP backend:
// forward_step of the prompt at n_past, then n_steps - 1 single-token steps, each followed by
// sample(smp, logits, all_tokens) (model.cpp:1675-1728) of the last logits column on the device,
// where all_tokens is the prompt plus every token fed so far and smp is init_sampler(params)
// (model.cpp:1668-1673; seed 0 = std::random_device). tokens_out (n_steps entries) receives the
// sampled tokens: the first from the prompt's logits, then one per step. No stop tokens.
typedef struct gl_sampler_params {
    float    temp;
    int32_t  top_k;
    float    top_p;
    float    repeat_penalty;
    int32_t  repeat_last_n;
    uint32_t seed;
} gl_sampler_params;
GGML_API int gl_generate(gl_session * s, int64_t n_past, const int32_t * prompt, int64_t n_prompt, int n_steps,
                         const gl_sampler_params * params, int32_t * tokens_out, double * seconds, char * err,
                         size_t err_size);

// Fills positions [0, n_pos) of every layer's K and V cache with N(0,1) values stored as F16
// (seeded, deterministic).
GGML_API int gl_kv_fill_random(gl_session * s, int64_t n_pos, uint64_t seed, char * err, size_t err_size);
// Raw F16 bytes of one layer's K (is_v = 0) or V cache.
GGML_API int gl_kv_read(gl_session * s, int layer, int is_v, void * dst, size_t offset, size_t size);

typedef struct {
    const char * arch;       // "llama", "qwen2", "qwen3", "phi3", "qwen3moe"
    int64_t n_embd, n_layer, n_head, n_head_kv, head_dim, n_ff, n_vocab, n_ctx_train;
    int64_t n_expert, n_expert_used, n_ff_exp;
    float   rope_theta, rms_eps;
    int32_t wtype;           // ggml type of the linear weights
    int32_t embd_type;       // token_embd.weight type
    int32_t output_type;     // output.weight type
    int32_t tied_output;     // non-zero: no output.weight (the head reuses token_embd)
    float   w_std;           // linear weights ~ N(0, w_std)
    float   norm_std;        // norm weights ~ 1 + N(0, norm_std)
    uint64_t seed;
    int32_t n_threads;
    int32_t share_experts;   // non-zero: every layer's expert tensors hold layer 0's values
    int32_t rope_scaling_orig_ctx; // non-zero: phi3 LongRoPE keys ({arch}.rope.scaling.original_context_length
                                   // = this, .rope.scaling.attn_factor) and rope_factors_short.weight
    float   rope_attn_factor;      // the LongRoPE attention factor written with those keys
    int32_t kquant_mix;            // 1 (with wtype Q4_K): a Q4_K_M-style mix of K-quant types, see below
} gl_synth_params;

// Weights are N(0, w_std) floats from a counter-based generator (splitmix64 -> Box-Muller in
// double), quantized with the ggml reference quantizer of the requested type. share_experts
// (qwen3moe) writes layer 0's quantized expert tensors into every layer: the expert weights of a
// 48-layer, 128-expert model are 29e9 values, minutes of quantization; routers, attention and norm
// weights stay distinct per layer, so routing still differs from layer to layer.
// rope_scaling_orig_ctx (phi3 LongRoPE, reference model.cpp:145-153, 555-557): the frequency
// factors rope_factors_short.weight F32[head_dim / 2] are 2 + N(0, 0.25) values (seeded).
// kquant_mix 1 mixes types the way llama.cpp's Q4_K_M files do (the reference's published
// workloads: README.md:162, moe_stream/VULKAN.md:646-651): output.weight Q6_K; attn_v and
// ffn_down (ffn_down_exps) Q6_K in even layers; attn_q, ffn_gate and ffn_up (and their _exps) Q5_K
// in odd layers; every other matrix wtype.
GGML_API int gl_synth_model(const char * path, const gl_synth_params * p, char * err, size_t err_size);

// The seeded normal generator the synthetic models use: out[i] = mean + std * z(seed, first + i).
GGML_API void gl_fill_normal(float * out, int64_t n, uint64_t seed, int64_t first, float mean, float std);

#ifdef __cplusplus
}
#endif
