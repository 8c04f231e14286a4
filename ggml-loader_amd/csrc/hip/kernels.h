// kernels.h — host-side launchers of the gfx950 kernels. Every launcher takes plain device
// pointers, sizes and the stream it enqueues on; shape checks happen in the caller (the graph
// executor) before launch.
#pragma once

#include "hip_common.h"

#include <hip/hip_ext.h>

#include <chrono>

// Timing of one executor op. While stop is set, the op's kernels are launched through
// hipExtLaunchKernel, which stamps start (first launch) and stop (each launch; the last one wins)
// from the kernel dispatches themselves, so timing puts no event markers between kernels.
struct launch_timing {
    hipEvent_t start = nullptr;
    hipEvent_t stop = nullptr;
    int launches = 0;
    // host time spent inside the launch calls (accumulated while api_on; profiled computes only)
    bool api_on = false;
    double api_ms = 0.0;
};
extern thread_local launch_timing g_launch_timing;

template <typename... KArgs, typename... Args>
inline void launch(void (*kernel)(KArgs...), dim3 grid, dim3 block, size_t shmem, hipStream_t st, Args... args) {
    launch_timing & t = g_launch_timing;
    const auto t0 = t.api_on ? std::chrono::steady_clock::now() : std::chrono::steady_clock::time_point{};
    if (t.stop) {
        hipExtLaunchKernelGGL(kernel, grid, block, (std::uint32_t) shmem, st, t.launches == 0 ? t.start : nullptr, t.stop, 0,
                              args...);
        t.launches++;
    } else {
        hipLaunchKernelGGL(kernel, grid, block, shmem, st, args...);
    }
    HIP_CHECK(hipGetLastError());
    if (t.api_on) t.api_ms += std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - t0).count();
}

// A strided view of a tensor (ggml ne/nb convention, nb in bytes).
struct tview {
    char *  data;
    int     type;    // ggml_type
    int64_t ne[4];
    int64_t nb[4];
};

// the K-quant weight types (Q4_K, Q5_K, Q6_K): 256-weight super-blocks, dotted against Q8_K
// activations
__host__ __device__ constexpr bool is_kquant(int type) { return type == 12 || type == 13 || type == 14; }

// ---------------------------------------------------------------------------------------------
// weight layout conversion (GGUF bytes <-> device planes), on the stream
void launch_repack_q(int type, const uint8_t * raw, uint8_t * qs_plane, __half * d_plane,
                     int64_t nblocks, int64_t first_block, hipStream_t st);
void launch_unpack_q(int type, uint8_t * raw, const uint8_t * qs_plane, const __half * d_plane,
                     int64_t nblocks, int64_t first_block, hipStream_t st);
// Q6_K blocks (210 bytes, so only 2-byte aligned in GGUF order: {ql[128], qh[64], i8 scales[16],
// f16 d}) as four planes inside the tensor's
// own allocation, same size: [ql: nb x 128][qh: nb x 64][scales: nb x 16][d: nb x f16], block b's
// fields at ql + 128 b, qh + 64 b, sc + 16 b, d + b; every 16-byte piece a kernel loads is aligned
struct q6k_planes {
    uint8_t * ql;
    uint8_t * qh;
    int8_t *  sc;
    __half *  d;
};
void launch_repack_q6k(const uint8_t * raw, q6k_planes p, int64_t nblocks, int64_t first_block, hipStream_t st);
void launch_unpack_q6k(uint8_t * raw, q6k_planes p, int64_t nblocks, int64_t first_block, hipStream_t st);

// ---------------------------------------------------------------------------------------------
// activation quantization of ncols columns of K floats (column c at x + c*x_col_stride floats)
struct q8_act { int8_t * qs; float * d; int32_t * s; };     // Q8_0 semantics, per-column K / K/32 / K/32
struct q8k_act { int8_t * qs; float * d; int16_t * bsums; }; // Q8_K semantics, per-column K / K/256 / K/16

void launch_quantize_q8(const float * x, int64_t x_col_stride, int64_t K, int64_t ncols, q8_act out, hipStream_t st);
void launch_quantize_q8k(const float * x, int64_t x_col_stride, int64_t K, int64_t ncols, q8k_act out, hipStream_t st);

// ---------------------------------------------------------------------------------------------
// quantized GEMV / small-batch GEMM: y[c][r] = W[r] . x[c] (+ add[c][r]) for up to 4 weight
// matrices of one type and row length K sharing the same activation (one launch).
constexpr int GEMV_MAX_MATS = 4;
constexpr int GEMV_MAX_K = 16384;          // Q4_0 / Q8_0 rows
// longest rows of a gate/up pair in one SwiGLU launch (both chains' weight blocks stay in registers)
constexpr int gemv_swiglu_max_k(int type) {
    return type == 8 /* GGML_TYPE_Q8_0 */ ? 4096 : type == 12 /* GGML_TYPE_Q4_K */ ? 16384
         : type == 13 /* GGML_TYPE_Q5_K */ ? 12288 : type == 14 /* GGML_TYPE_Q6_K */ ? 8192 : 6144;
}

struct gemv_mat {
    const uint8_t * w;     // Q4_0/Q8_0: qs plane of the first row; Q4_K/Q5_K: first block; Q6_K: ql plane
    const __half *  wd;    // Q4_0/Q8_0/Q6_K: d plane of the first row
    const uint8_t * wqh;   // Q6_K: qh plane of the first row
    const int8_t *  wsc;   // Q6_K: scales plane of the first row
    float *         y;     // output column 0
    const float *   add;   // optional residual added to the output (nullptr: none)
    int64_t         y_stride;   // floats between output columns
    int64_t         add_stride;
    int32_t         n_rows;
};

// ---------------------------------------------------------------------------------------------
// prefill GEMM on the matrix cores: y[c][r] = W[r] . x[c] (+ add[c][r]) for Q4_0 / Q8_0 weights
// in the plane layout with Q8_0-quantized activation columns, or Q4_K weights (ggml blocks) with
// Q8_K-quantized columns; the same floats as the GEMV.
constexpr int GEMM_MIN_COLS = 64;   // narrower products stay on the GEMV, except:
// an output projection this tall (an LM head) takes the GEMM from GEMM_WIDE_MIN_COLS columns: its
// weights stream once at the GEMM's rate, where the multi-column GEMV would stage every column's
// activation once per 16-row workgroup
constexpr int GEMM_WIDE_MIN_COLS = 16;
constexpr int64_t GEMM_WIDE_MIN_ROWS = 65536;

struct gemm_launch {
    int             type;      // GGML_TYPE_Q4_0 / Q8_0 / Q4_K / Q5_K / Q6_K
    int64_t         K;         // row length (a multiple of 128; of 256 for the K-quants)
    int64_t         n_rows;
    int64_t         ncols;
    const uint8_t * w;         // Q4_0 / Q8_0: qs plane of row 0; Q4_K / Q5_K: row 0's first block; Q6_K: its low-bit plane
    const __half *  wd;        // Q4_0 / Q8_0 / Q6_K: d plane of row 0
    const uint8_t * wqh;       // Q6_K: high-bit plane of row 0 (64 bytes per block)
    const int8_t *  wsc;       // Q6_K: scale plane of row 0 (16 per block)
    const int8_t *  xq;        // activation column c at xq + c * K
    const float *   xd;        // and its scales at xd + c * K / 32 (Q8_0) or xd + c * K / 256 (Q8_K)
    const int16_t * xbs;       // Q8_K: the column's 16-element sums at xbs + c * K / 16
    float *         y;         // output column c at y + c * y_stride
    int64_t         y_stride;
    const float *   add;       // optional residual, column c at add + c * add_stride
    int64_t         add_stride;
};

bool gemm_supported(int type, int64_t K, int64_t n_rows);
void launch_gemm(const gemm_launch & G, hipStream_t st);
// the workgroup tile launch_gemm picks (kernel template arguments: "4x4x2", "2x4x2", "1x2x4" for
// Q4_0 / Q8_0 warp tiles x k-blocks; "2x2", "1x2" for the K-quants), for profile names
const char * gemm_tile_name(const gemm_launch & G);

// Activation prologue of a GEMV: every workgroup quantizes its column of x itself, either as
// rms_norm(x) * w (rms set: ggml's rms_norm -> mul -> quantize_row_q8_0 / q8_K chain, same
// roundings) or as x (the activation quantization ggml-cpu applies inside mul_mat).
struct gemv_norm {
    const float * x;       // column c at x + c * x_stride (nullptr: no prologue)
    int64_t       x_stride;
    const float * w;       // norm weight [K] (rms only; nullptr: rms_norm without the multiply)
    float         eps;
    int           rms;
    // x holds doubles (x_stride counted in doubles), each rounded to float and then quantized as
    // is (rms 0): the decode attention's accumulated output (attn_launch::acc)
    int           f64;
};

// largest K the act_quant kernel (and the Q4_K GEMV's prologue) handles: with rms, one 32-element
// Q8_0 block or one 16-element Q8_K group per thread of a 256-thread workgroup; without, up to 8 of
// them per thread
constexpr int act_quant_max_k(int type, bool rms) {
    return (is_kquant(type) ? 16 : 32) * 256 * (rms ? 1 : 8);
}
// largest K a GEMV's activation prologue handles: the Q4_0 / Q8_0 kernel holds up to 2 (rms) or 4
// float4 chunks per thread of a 512-thread workgroup
constexpr int gemv_prologue_max_k(int type, bool rms) {
    return is_kquant(type) ? act_quant_max_k(type, rms) : (rms ? 4096 : 8192);
}
// SwiGLU launches that quantize act for the down projection (out_q): 32 rows per workgroup of 1024
// threads, K up to 4096
constexpr int GEMV_SWIGLU_QOUT_MAX_K = 4096;
// longest row of the register-resident rms_norm kernel (32 elements per thread); longer rows go
// through the strided kernel
constexpr int RMS_NORM_MAX_ROW = 256 * 32;

struct gemv_launch {
    int        type;       // GGML_TYPE_Q4_0 / Q8_0 / Q4_K
    int        K;
    int        ncols;
    int        n_mats;
    gemv_mat   m[GEMV_MAX_MATS];
    // activation (already quantized; column c at +c*K int8 and +c*K/32 (q8) or K/256 (q8K) scales),
    // unused when norm.x is set
    const int8_t *  xq;
    const float *   xd;
    const int32_t * xs;    // q8: block sums
    const int16_t * xbs;   // q8K: 16-wise sums
    gemv_norm  norm;
    // ggml_mul_mat_id: grid column c is (token c / n_slots, slot c % n_slots); it reads the rows of
    // expert ids[token * ids_stride + slot] (expert e's rows begin e * expert_rows rows into every
    // matrix; ids are clamped to [0, n_experts)) and activation column token * x_cols + slot % x_cols
    const int32_t * ids;   // nullptr: a plain GEMV
    int64_t    ids_stride;
    int        n_slots;
    int        x_cols;
    int        n_experts;
    int64_t    expert_rows;
    // mul_mat_id of one token whose routing has not run (route_logits set; single-column Q4_K
    // SwiGLU kernel only): every workgroup routes the token itself from the router logits
    // (n_experts of them, times route_scale; moe_route_256) and reads the expert of its slot, and
    // the launch writes the n_slots expert ids to ids and their renormalized weights to route_w,
    // which later launches read
    const float * route_logits;
    float *    route_w;
    // SwiGLU epilogue: m[0] = gate, m[1] = up (same n_rows); writes act = silu(g) * u to m[0].y
    bool       swiglu;
    float      route_scale;
    // with swiglu (Q4_0 / Q8_0 weights, n_rows % 32 == 0, K <= GEMV_SWIGLU_QOUT_MAX_K): act also
    // quantized to Q8_0 here (quantize_row_q8_0 semantics; column c's blocks at +c * n_rows), for a
    // down projection that reads it pre-quantized
    q8_act     out_q;
};

void launch_gemv(const gemv_launch & L, hipStream_t st);
// whether launch_gemv takes a double-valued column (gemv_norm::f64) for this launch: one column,
// no SwiGLU, no experts; Q4_0 / Q8_0 on the single-column kernel, K-quants on the multi-unit one
bool gemv_f64_input_supported(const gemv_launch & L);
// the single-column Q4_0 / Q8_0 kernel (k_gemv_q.hip), which launch_gemv uses when this holds
bool gemv_q_supported(const gemv_launch & L);
void launch_gemv_q(const gemv_launch & L, hipStream_t st);
// the single-column Q4_K kernel (k_gemv_q4k.hip), likewise (GGML_HIP_NO_Q4K_GEMV=1 turns it off)
bool gemv_q4k_enabled();
bool gemv_q4k_supported(const gemv_launch & L);
void launch_gemv_q4k(const gemv_launch & L, hipStream_t st);
// Dense Q4_K products of 2 or more pre-quantized columns with K <= 4096 on the matrix cores
// (k_gemv_mfma.hip): 16 rows x 16 columns per workgroup, the same floats as the GEMV
bool gemv_mfma_supported(const gemv_launch & L);
void launch_gemv_mfma(const gemv_launch & L, hipStream_t st);
// Several activation columns per workgroup (k_gemv_mc.hip): each weight row block is read once for
// up to GEMV_MC_MAX_COLS columns; the activation must be quantized already (L.xq, no L.norm). With
// groups (mul_mat_id): the workgroups of expert e take the columns the ids route to e, listed by
// launch_moe_group; max_cols is then the most columns one expert can get (the token count).
constexpr int GEMV_MC_MAX_COLS = 16;
struct expert_groups {
    int32_t * count;           // [n_experts] columns routed to each expert
    int32_t * offset;          // [n_experts] start of each expert's list in cols
    int32_t * cols;            // [n_slots * n_tok] grid columns (token * n_slots + slot), by expert
    int32_t * items;           // [max_items][3] workgroup columns: expert, start in cols, count (<= nc)
    int32_t * n_items;         // items in use
    int nc;                    // columns per item
    int max_items;             // n_experts (or the column count, if smaller) + columns / nc
};
bool gemv_mc_supported(const gemv_launch & L, int max_cols);
// a workgroup shape exists for this row length (nc > 0: with exactly nc columns per workgroup)
bool gemv_mc_fits(int type, int K, bool swiglu, int nc = 0);
void launch_gemv_mc(const gemv_launch & L, const expert_groups * G, int max_cols, hipStream_t st);
void launch_moe_group(const int32_t * ids, int64_t ids_stride, int n_slots, int n_tok, int n_experts, const expert_groups & g,
                      hipStream_t st);
// L.norm's prologue for L.ncols columns of L.K, written once to q8 (Q4_0/Q8_0 consumers) or q8k (Q4_K)
void launch_act_quant(const gemv_launch & L, const q8_act & q8, const q8k_act & q8k, hipStream_t st);
// consumers with more rows than this get the activation quantized once instead of per workgroup
constexpr int GEMV_PROLOGUE_MAX_ROWS = 32768;

// ---------------------------------------------------------------------------------------------
// element-wise / normalization / positional kernels

// y[c] = rmsnorm(x[c]) (* w), for ncols rows of n floats; optional fused activation quantization
void launch_rms_norm(const float * x, int64_t x_stride, const float * w, float * y, int64_t y_stride,
                     int64_t n, int64_t ncols, float eps, const q8_act * q8, const q8k_act * q8k, hipStream_t st);
// generic strided rms_norm over ne0 of every row
void launch_rms_norm_strided(const tview & x, const tview & y, float eps, hipStream_t st);

// dst = a (op) broadcast(b); op: 0 add, 1 mul, 2 div, 3 sub
void launch_binary(int op, const tview & a, const tview & b, const tview & dst, hipStream_t st);
// unary: 0 silu, 1 relu, 2 sigmoid, 3 sqr, 4 scale(s), 5 abs, 6 softplus
void launch_unary(int op, float s, const tview & a, const tview & dst, hipStream_t st);
// each row over ne0 divided by max(|row|_2, eps) (ggml_l2_norm)
void launch_l2_norm(const tview & a, const tview & dst, float eps, hipStream_t st);
// a and b joined along dim (ggml_concat; F32 / F16 / I32)
void launch_concat(const tview & a, const tview & b, const tview & dst, int dim, hipStream_t st);
// silu(a) * b (ggml_swiglu_split)
void launch_glu(const tview & a, const tview & b, const tview & dst, hipStream_t st);
// element-wise copy with type conversion in row-major element order (shapes may differ)
void launch_cpy(const tview & src, const tview & dst, hipStream_t st);
// dst rows = dequantized rows of a selected by I32 ids (Q4_0 / Q8_0: qs_plane, d_plane; Q6_K: q6;
// with first_block the block of a's first element in them)
void launch_get_rows(const tview & a, const tview & ids, const tview & dst, const uint8_t * qs_plane,
                     const __half * d_plane, const q6k_planes & q6, int64_t first_block, hipStream_t st);

struct rope_params {
    int   n_dims;
    int   mode;
    float freq_scale;
    float ext_factor;
    float attn_factor;
    float corr_dims[2];
    float theta_scale;     // powf(freq_base, -2/n_dims), evaluated on the host
};
void launch_rope(const tview & src, const int32_t * pos, const float * freq_factors, const tview & dst,
                 const rope_params & p, hipStream_t st);

// Up to ROPE_MAX_JOBS independent jobs in one launch: RoPE of src into dst (pos set; dst F32, or
// F16 when the rotation is stored straight into the KV cache) or a converting copy (pos null).
constexpr int ROPE_MAX_JOBS = 4;
struct rope_job {
    tview src, dst;
    const int32_t * pos;
    const float * ff;          // optional frequency factors
    rope_params p;
    int64_t n;                 // work items: rotation pairs, or elements for a copy (rows with norm_x)
    const float2 * cs;         // optional (cos, sin) table [token][n_dims / 2] (launch_rope_table)
    // optional QK-Norm of the rows before the rotation (rms_norm(x) * w, the ops' roundings): the
    // rotated rows are (head, token) rows of src's shape read from norm_x + head * norm_nb1 +
    // token * norm_nb2 (floats, src.ne[0] <= 256 contiguous), one wave per row; src's data unused
    const float * norm_x;
    int64_t norm_nb1, norm_nb2;
    const float * norm_w;
    float norm_eps;
};
struct rope_batch {
    rope_job job[ROPE_MAX_JOBS];
    int64_t first_block[ROPE_MAX_JOBS];
    int n_jobs;
};
void launch_rope_batch(rope_batch & B, hipStream_t st);
constexpr int64_t ROPE_TABLE_MIN_TOKENS = 16;   // RoPE jobs over at least this many tokens read a table
// (cos, sin) of every rotation pair of n_pos tokens at positions pos, [n_pos][p.n_dims / 2]: what
// every rotation of those tokens with these parameters uses (prefill: all heads of Q and K of every
// layer), formed once
void launch_rope_table(const int32_t * pos, int64_t n_pos, const rope_params & p, const float * ff, float2 * out, hipStream_t st);

void launch_soft_max(const tview & a, const tview * mask, const tview & dst, float scale, float max_bias, hipStream_t st);
// dst = silu(gate) * up (2-D f32 views), with its Q8_0 (q) or Q8_K (qk) quantization when set
void launch_swiglu(const tview & gate, const tview & up, const tview & dst, const q8_act * q, const q8k_act * qk, hipStream_t st);

// ---------------------------------------------------------------------------------------------
// MoE routing and expert combination
void launch_sum_rows(const tview & a, const tview & dst, hipStream_t st);
constexpr int ARGSORT_MAX_ROW = 16384;
void launch_argsort(const tview & a, const tview & dst, bool desc, hipStream_t st);
// out[:, t] = sum over slots s in order of e[:, s, t] * w[s, t] (+ res[:, t]); strides in floats
struct moe_wsum {
    const float * e;   int64_t e_nb1, e_nb2;
    const float * w;   int64_t w_nb1, w_nb2;
    const float * res; int64_t res_nb1;
    float *       out; int64_t out_nb1;
    int64_t n_embd, n_tok;
    int k;
};
void launch_moe_wsum(const moe_wsum & M, hipStream_t st);
// the weighted sum, then the next rms_norm * nw of each token's row quantized to Q8_K (one launch;
// n_embd a multiple of 256, at most 4096; rows 16-byte aligned)
bool wsum_norm_q8k_supported(const moe_wsum & M, const float * nw);
void launch_wsum_norm_q8k(const moe_wsum & M, const float * nw, float eps, q8k_act q8k, hipStream_t st);
void launch_argmax(const tview & a, int32_t * out, hipStream_t st);
// one wide row in two launches over ARGMAX_PARTS partial results (part_v / part_i: that many
// entries of device scratch); the same index as launch_argmax
constexpr int ARGMAX_PARTS = 128;
constexpr int64_t ARGMAX_ROW_MIN = 16384;   // narrower rows take the one-workgroup kernel
// out2 / out3 (optional): further destinations of the index (the decode loop's copies of the pick)
void launch_argmax_row(const tview & a, int32_t * out, float * part_v, int * part_i, hipStream_t st,
                       int32_t * out2 = nullptr, int32_t * out3 = nullptr);

// generic F32/F16/BF16 mul_mat (src0 rows contiguous): one wave per output element
void launch_mul_mat_generic(const tview & src0, const tview & src1, const tview & dst, hipStream_t st);
// dst[:, c] = W^T (rms_norm(x[:, c]) * nw) for an F32 W [K, rows] (the MoE router), also writing
// the normalized columns to y_out (the rms_norm -> mul output, for the norm's other consumers)
// and, with q8k.qs set (K % 256 == 0), their Q8_K quantization
constexpr int64_t MUL_MAT_ROWS_NORM_MAX_K = 8192;
bool mul_mat_rows_norm_supported(const tview & w, int64_t K);
void launch_mul_mat_rows_norm(const tview & w, const float * x, int64_t x_stride, const float * nw, float eps, float * y_out,
                              int64_t y_stride, const tview & dst, int64_t ncols, q8k_act q8k, hipStream_t st);

// MoE routing of one token per workgroup: softmax over the router logits (the soft_max op's
// arithmetic), the k most probable experts in the stable descending order of argsort (ties: the
// lower expert id first), and their probabilities divided by their float sum (sum_rows in double).
constexpr int MOE_ROUTE_MAX_EXPERTS = 1024;
constexpr int MOE_ROUTE_MAX_K = 32;
struct moe_route {
    const float * logits;      // [n_expert] floats per token, token stride logits_nb1
    int64_t       logits_nb1;
    int n_expert, k, n_tok;
    float scale;
    int32_t *     ids;         // k expert ids per token (stride ids_nb1)
    int64_t       ids_nb1;
    float *       w;           // k renormalized weights per token (stride w_nb1)
    int64_t       w_nb1;
};
void launch_moe_route(const moe_route & R, hipStream_t st);

// ---------------------------------------------------------------------------------------------
// decode attention over the F16 KV cache: out[h*hd + i, q] for q < n_q, h < n_head
// A per-head RMSNorm * w (QK-Norm) folded into the rotation of a RoPE source: element e of row
// (head, token) is (x[e] * scale) * w[e], scale = 1 / sqrt(mean(x^2) + eps) over the row's hd
// elements (the rms_norm -> mul ops' roundings). x == nullptr: none.
struct qk_norm {
    const float * x;           // row (head, token) at x + head * nb1 + token * nb2 (floats), contiguous
    int64_t       nb1, nb2;
    const float * w;           // [hd]
    float         eps;
};

struct attn_launch {
    const float *  q;          // Q (post-RoPE) element (i, head, token) at q + i + head*q_nb1 + token*q_nb2 (floats)
    int64_t        q_nb1, q_nb2;
    const __half * k;          // K cache: element (i, kv_head, pos) at k + i + kv_head*k_nb1 + pos*k_nb2 (halves)
    int64_t        k_nb1, k_nb2;
    const __half * v;
    int64_t        v_nb1, v_nb2;
    const void *   mask;       // [n_kv, >= n_q] rows of mask_nb1 bytes; F32 or F16; nullptr = none
    int            mask_f16;
    int64_t        mask_nb1;
    float *        out;        // out + i + head*hd + token*out_nb1 (floats)
    int64_t        out_nb1;
    int n_kv, n_q, n_head, n_head_kv, hd;
    float scale;
    // split-KV scratch (attn_scratch_bytes): scores, row statistics, per-chunk partials
    float *        scratch;
    int64_t        scratch_bytes;
    // quantized copy of out for the o-projection (Q8_0 semantics), optional
    q8_act         out_q;
    // or its Q8_K copy (quantize_row_q8_K semantics; n_head * hd a multiple of 256 and 256 a
    // multiple of hd: one combination workgroup per 256-dim super-block), optional
    q8k_act        out_q8k;
    // one query (n_q == 1): instead of per-chunk partials and a combination launch, the PV
    // workgroups add their chunk partials into acc[head * hd + i] (doubles; exact sums, so their
    // order does not matter; zeroed by the scores launch), and out / out_q are not written: the
    // o-projection's prologue reads acc (gemv_norm::f64). nullptr: the partials and combination.
    double *       acc;
    // RoPE of the new tokens folded in (rope set; decode only): Q is read from rq.src and rotated
    // in the scores kernel (the rotated Q is not stored); the workgroup whose position chunk holds
    // new position n_kv - n_q + t rotates K row t of rk.src into rk.dst (the K cache) and copies V
    // row t of rv.src into rv.dst (the V cache)
    int            rope;
    rope_job       rq, rk, rv;
    // with rope: Q and K rows normalized before the rotation (Qwen3's QK-Norm), read from qn.x /
    // kn.x instead of rq.src / rk.src
    qk_norm        qn, kn;
    // with rope: the (cos, sin) table of the new tokens' rotation pairs, [n_q][n_dims / 2]; every
    // layer rotates with the same positions, so the first attention of a graph computes it and
    // stores it here (cs_mode 1, workgroup 0), the later ones read it (cs_mode 2); 0: compute only
    float2 *       cs_tab;
    int            cs_mode;
    // flash_attn_ext's contract: a position whose mask is -inf takes no part in that query's row,
    // whatever its K and V hold (ggml-cpu skips it; the never-written cells of a ring cache may hold
    // any bits). Every path gives such a position the score -inf without reading its dot; with
    // skip_masked the V rows of positions masked for every query of a workgroup are also read as
    // zero, so that 0 * (non-finite V) cannot reach the sums. The manual chain, which never attends
    // an unwritten position, leaves it 0.
    int            skip_masked;
    // flash_attn_ext's probabilities: ggml's flash op never materializes KQ, so p = exp(s - M) / S
    // stays a float into the PV sums (1); the manual chain's V mul_mat converts p to F16 first (0)
    int            p_f32;
    // Set by launch_attn_decode from the fields above (callers leave them zero): the rows the
    // decode kernels read, with 32-bit element strides, so that their per-lane offsets are 32-bit.
    // Q source rows (before QK-Norm and RoPE) at sq + head * sq1 + token * sq2; with RoPE the new
    // tokens' K and V source rows at sk / sv + kv_head * s?1 + token * s?2, otherwise q (valid,
    // unused), as are the QK-Norm weights sqw / skw without the norm and the positions spos
    // without RoPE.
    const float *  sq, * sk, * sv, * sqw, * skw;
    const int32_t * spos;
    int32_t        sq1, sq2, sk1, sk2, sv1, sv2;
    int32_t        s_half;         // rotation pairs per row (1 without RoPE)
    int32_t        s_mask_stride;  // elements per mask row
    int32_t        k_s2, v_s2;     // k_nb2, v_nb2
    int32_t        s_gqa;          // n_head / n_head_kv
    float          s_inv_gqa;      // 1 / s_gqa
};
int64_t attn_scratch_bytes(int n_kv, int n_q, int n_head, int hd);
// split-KV decode attention for 1 <= n_q <= ATT_DECODE_MAX_Q queries (groups of 4 per workgroup;
// RoPE folded in only for n_q <= 4)
constexpr int ATT_DECODE_MAX_Q = 64;
void launch_attn_decode(const attn_launch & A, hipStream_t st);
// n_q > 4 (prefill): one workgroup per (16-query tile, head), a row's scores in LDS (no scratch, no
// quantized output); n_kv up to attn_prefill_max_kv(hd), 0 for an unsupported head dim
int attn_prefill_max_kv(int hd);
void launch_attn_prefill(const attn_launch & A, hipStream_t st);

// ---- token sampling (k_sample.hip) ----
// One row of F32 logits, the window's penalized ids (distinct, ascending) with their occurrence
// counts, the sampler's parameters and the uniform variate u of the draw. out (device, 3 ints):
// the token id, whether u was used (the weighted draw ran over two or more weights), a status.
constexpr int SMP_BOUND_K = 1024;    // largest top-k of the one-launch path
constexpr int SMP_MAX_CAND = 4096;   // candidates the one-launch path holds (and rows it sorts whole)
constexpr int SMP_MAX_PEN = 1024;    // penalized ids the one-launch path holds
constexpr int SMP_CHUNK = 4096;      // probabilities staged per pass of the sequential sums
enum { SMP_OK = 0, SMP_OVERFLOW = 1, SMP_NONFINITE = 2 };
struct sample_request {
    const float * logits;
    int           n;
    const int *   pen_ids;
    const int *   pen_cnt;
    int           n_pen;
    float         temp;
    int           top_k;
    float         top_p;
    float         penalty;
    double        u;
    int *         out;
};
// the one-launch path takes the request (it may still report SMP_OVERFLOW: then take the sorted path)
bool sample_fast_path(const sample_request & r);
void launch_sample(const sample_request & r, hipStream_t st);
// the sorted path: ws of sample_sorted_ws_bytes(n) bytes
size_t sample_sorted_ws_bytes(int n);
void launch_sample_sorted(const sample_request & r, void * ws, size_t ws_bytes, hipStream_t st);
