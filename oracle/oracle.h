/*
 * oracle.h — CPU reference (test oracle) for GGML-Loader's per-token forward pass.
 *
 * TEST INFRASTRUCTURE ONLY. Nothing in the product (ggml-loader_amd/) includes, links or loads
 * this; only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg use it, and only as
 * the checker / baseline, never as the thing measured or shipped.
 *
 * It restates the arithmetic of ggml's CPU backend (upstream ggml is an un-vendored, absent
 * submodule in the reference: .gitmodules:1-3), the way GGML-Loader's `--backend cpu` computes
 * forward_step (model.cpp:790-799, 1496-1597), in plain C with a fixed float operation order
 * (-ffp-contract=off). It is also registered as the "CPU" ggml backend so the same graph that the
 * HIP backend runs can be computed here (ggml_backend_cpu_init, include/ggml-cpu.h).
 *
 * What pins each primitive (tests/test_oracle.py, tests/test_host.py; golden vectors made by
 * tests/golden/make_golden.py from the reference's src/moe_stream sources via Makefile.ref):
 *   fp16 <-> fp32              IEEE binary16 (numpy): all 65536 codes; 3M f32 patterns incl. ties
 *   Q4_0 decode                closed form over every nibble at every position, 8 scales
 *   Q8_0, Q4_K decode          reference dequant_row golden vectors, bit-exact (dequant.c:94-251)
 *   Q4_0 quantizer             tests/test_oracle_pins.py: d = binary16(max / -8), codes x/d rounded
 *                              half up (constructed ties at power-of-two scales), clipped to 15
 *                              exactly where x/d >= 7.5; a planted truncation fails
 *   Q8_0/Q8_K quantizers       error bounds (round to nearest within d/2), zero and constant
 *                              blocks, Q8_K block sums; the product's quantizers byte-identical
 *   Q5_K/Q6_K decode           reference dequant_row golden vectors (dequant.c:135-197), bit-exact
 *   Q5_K/Q6_K quantizers, dots tests/test_kquants.py: codes within half a step under the decoded
 *                              scales, largest scale codes, make_qx_quants against a float64
 *                              statement of its search; dots against fp64 brute force
 *   Q4_K quantizer             tests/test_oracle_pins.py: make_qkx2_quants against a float64
 *                              statement of ggml's search (same pick where float32 rounding cannot
 *                              decide it), scale/min codes of the float64 optimum under weights
 *                              av_x + |x|, d/dmin = binary16(max / 63), nibbles re-rounded; planted
 *                              mistakes (no search, unit weights) fail
 *   vec dots / gemv            fp64 brute force over the same quantized operands; one-hot columns;
 *                              reference sc_matmul golden (Q4_K) within the activation-quantization
 *                              bound. ggml-cpu's block-sum order itself: parity unpinned
 *   rms_norm, softmax, silu    reference sc_rmsnorm / sc_softmax / sc_swiglu golden vectors
 *                              (tolerance: float vs double sums); softmax masks and row sums
 *   rope                       reference sc_rope golden (NEOX); position 0 identity; pair norms;
 *                              theta_0 = pos; NORMAL == NEOX on interleaved pairs; partial dims;
 *                              frequency factors, attn_factor, freq_scale and the YaRN ramp by
 *                              identities and float64 rotations (tests/test_oracle_pins.py)
 *   attention chain            n_kv = 1 -> V; equal keys -> mean of V (exact); fp64 GQA brute force
 *                              that also rejects the h % n_head_kv mapping; the reference MoE
 *                              engine's own qwen3moe forward (qwen_model.c attention_block: q/k
 *                              norms, NEOX rope, f32 KV, GQA) built by Makefile.ref: logits of 32
 *                              decode steps at 32/4 heads x 128 within 1e-3 (F32 matrices) or
 *                              2.5e-2 median / 1e-1 (Q4_K), fixtures made by
 *                              tests/golden/make_qwen_ref.py; a planted head mapping, rope pairing
 *                              or dropped softmax scale (oracle_set_planted) fails that check
 *   moe_route                  brute-force top-k (ties -> lower id) and renormalized softmax
 *   sample                     the reference's own sample() built from model.cpp (Makefile.ref):
 *                              identical ids over seeded draw sequences on tie-free logits, and the
 *                              same weight slot with ties; closed forms (top-k 1, two tokens, the
 *                              draw as a step function of u with steps of the probabilities)
 *   forward_step               float64 numpy transformer on synthetic GGUFs of 4 archs, rejecting
 *                              the other RoPE pair layout
 */
#ifndef GGML_LOADER_ORACLE_H
#define GGML_LOADER_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* IEEE binary16 conversions (round to nearest even) */
float    oracle_fp16_to_fp32(uint16_t h);
uint16_t oracle_fp32_to_fp16(float f);

/* reference quantizers (restating ggml quantize_row_*_ref) over k elements */
void oracle_quantize_q4_0(const float * x, void * y, int64_t k);
void oracle_quantize_q8_0(const float * x, void * y, int64_t k);
void oracle_quantize_q4_K(const float * x, void * y, int64_t k);
void oracle_quantize_q8_K(const float * x, void * y, int64_t k);
void oracle_quantize_q5_K(const float * x, void * y, int64_t k);
void oracle_quantize_q6_K(const float * x, void * y, int64_t k);

/* ggml's make_qkx2_quants (the per-sub-block weighted grid search inside the Q4_K quantizer):
   n <= 256 values with weights, codes 0..nmax into L, returns the scale and writes -min */
float oracle_make_qkx2_quants(int n, int nmax, const float * x, const float * weights, uint8_t * L, float * the_min,
                              float rmin, float rdelta, int nstep);

/* ggml's make_qx_quants with rmse_type 1 (the Q6_K sub-block search): n <= 256 values, codes
   -nmax..nmax-1 stored + nmax in L; returns the scale */
float oracle_make_qx_quants(int n, int nmax, const float * x, int8_t * L);

/* row decoders (type = ggml type id: 0 f32, 1 f16, 2 q4_0, 8 q8_0, 12 q4_K, 13 q5_K, 14 q6_K,
   30 bf16); 0 on unknown type */
int oracle_dequantize(int type, const void * x, float * y, int64_t k);

/* block dot products with the activation already in the weight's dot type */
float oracle_vec_dot_q4_0_q8_0(int64_t n, const void * x, const void * y);
float oracle_vec_dot_q8_0_q8_0(int64_t n, const void * x, const void * y);
float oracle_vec_dot_q4_K_q8_K(int64_t n, const void * x, const void * y);
float oracle_vec_dot_q5_K_q8_K(int64_t n, const void * x, const void * y);
float oracle_vec_dot_q6_K_q8_K(int64_t n, const void * x, const void * y);

/* y[r] = W[r] . x for nrows rows of a weight of type `type`, with ggml-cpu's activation
   quantization (Q4_0/Q8_0 -> Q8_0, Q4_K -> Q8_K, F16 -> F16, F32 exact) */
void oracle_gemv(int type, const void * w, int64_t nrows, int64_t k, const float * x, float * y, int n_threads);

/* RoPE of one vector of ne0 floats at position pos (ggml_rope_ext semantics, ext_factor 0
   unless given) */
void oracle_rope(float * dst, const float * src, int64_t ne0, int n_dims, int mode, int32_t pos,
                 float freq_base, float freq_scale, float ext_factor, float attn_factor,
                 float beta_fast, float beta_slow, int n_ctx_orig, const float * freq_factors);

/* MoE router as in the reference's moe_route (qwen_model.c:551-606): softmax over n_expert
   logits, top-k by insertion (ties keep the lower id), renormalize the k weights */
void oracle_moe_route(const float * logits, int n_expert, int top_k, int32_t * ids, float * w);

/* experiment hook: the order of the Q4_0 / Q8_0 dots' block-term sums (0 = ggml-cpu's block
   order, the default; 1 = a 32-lane wave reduction), tests/exactness_experiment.py only */
void oracle_set_block_sum_order(int mode);

/* test hook: plants a known mistake (0 = none, the default), to show that a check fails on it:
   bit 1 = query head h reads KV head h % n_head_kv; bit 2 = rope's NEOX and NORMAL pairings
   exchanged; bit 4 = soft_max and flash_attn_ext without their scale (tests/test_ref_qwen.py);
   bit 8 = Q4_0 codes truncated (x/d + 8) instead of rounded (+ 8.5); bit 16 = make_qkx2_quants
   without its scale search; bit 32 = Q4_K sub-block weights 1 instead of av_x + |x|; bit 64 = the
   YaRN ramp's extrapolated and interpolated angles exchanged; bit 128 = rope freq_factors
   multiplying the angle instead of dividing it; bit 256 = make_qx_quants without its rescaling
   search (tests/test_oracle_pins.py, tests/test_kquants.py) */
void oracle_set_planted(int bits);

/* sample() (model.cpp:1675-1728) on n logits with the window recent[0..n_recent) and the
   uniform variate u of the weighted draw; *used_draw = 1 when the draw consumed u. Equal logits
   order by ascending id. Returns the token id, or -1 when temp > 0 and the largest logit is not
   finite. */
int32_t oracle_sample(const float * logits, int64_t n, const int32_t * recent, int64_t n_recent, float temp,
                      int32_t top_k, float top_p, float repeat_penalty, int32_t repeat_last_n, double u,
                      int32_t * used_draw);

#ifdef __cplusplus
}
#endif

#endif
