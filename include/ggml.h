// ggml.h — tensor/graph core of the MI355X-native GGML-Loader build.
//
// This is the subset of the ggml C API that GGML-Loader's per-token forward pass is written
// against (reference: src/model.cpp, src/model.h, src/cmd_bench.cpp, src/cmd_run.cpp). Every
// declaration keeps ggml's name, argument meaning and shape conventions, so code written for ggml
// compiles unchanged against it. Each group cites the reference call sites it serves.
//
// Conventions (identical to ggml):
//   * ne[i] = number of elements along dim i, ne[0] is the contiguous dim.
//   * nb[i] = stride in BYTES along dim i; for block-quantized types nb[0] is the block size in
//     bytes and nb[1] = ne[0]/blck_size * nb[0].
//   * Ops build a DAG lazily; nothing is computed until a backend runs the graph.
#pragma once

#include <stdbool.h>
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#ifndef GGML_API
#define GGML_API __attribute__((visibility("default")))
#endif

// The reference builds every translation unit with GGML_MAX_NAME=128 (CMakeLists.txt:23); the
// tensor struct layout below depends on it, so it is fixed here rather than left to the caller.
#ifndef GGML_MAX_NAME
#define GGML_MAX_NAME 128
#endif
#define GGML_MAX_DIMS           4
#define GGML_MAX_SRC            10
#define GGML_MAX_OP_PARAMS      64
#define GGML_DEFAULT_GRAPH_SIZE 2048
#define GGML_MEM_ALIGN          16
#define GGML_PAD(x, n) (((x) + (n) - 1) & ~((n) - 1))

// RoPE modes used by build_graph (model.cpp:1395)
#define GGML_ROPE_TYPE_NORMAL 0
#define GGML_ROPE_TYPE_NEOX   2

typedef uint16_t ggml_fp16_t;
typedef struct { uint16_t bits; } ggml_bf16_t;

// Type ids are the on-disk GGUF tensor type ids, so they cannot be renumbered.
enum ggml_type {
    GGML_TYPE_F32  = 0,
    GGML_TYPE_F16  = 1,
    GGML_TYPE_Q4_0 = 2,
    GGML_TYPE_Q4_1 = 3,
    GGML_TYPE_Q5_0 = 6,
    GGML_TYPE_Q5_1 = 7,
    GGML_TYPE_Q8_0 = 8,
    GGML_TYPE_Q8_1 = 9,
    GGML_TYPE_Q2_K = 10,
    GGML_TYPE_Q3_K = 11,
    GGML_TYPE_Q4_K = 12,
    GGML_TYPE_Q5_K = 13,
    GGML_TYPE_Q6_K = 14,
    GGML_TYPE_Q8_K = 15,
    GGML_TYPE_I8   = 24,
    GGML_TYPE_I16  = 25,
    GGML_TYPE_I32  = 26,
    GGML_TYPE_I64  = 27,
    GGML_TYPE_F64  = 28,
    GGML_TYPE_BF16 = 30,
    GGML_TYPE_COUNT = 40,
};

#define QK4_0 32
#define QK8_0 32
#define QK_K  256

enum ggml_op {
    GGML_OP_NONE = 0,
    GGML_OP_DUP,
    GGML_OP_ADD,
    GGML_OP_MUL,
    GGML_OP_SCALE,
    GGML_OP_SQR,
    GGML_OP_RMS_NORM,
    GGML_OP_MUL_MAT,
    GGML_OP_MUL_MAT_ID,
    GGML_OP_CPY,
    GGML_OP_CONT,
    GGML_OP_RESHAPE,
    GGML_OP_VIEW,
    GGML_OP_PERMUTE,
    GGML_OP_TRANSPOSE,
    GGML_OP_GET_ROWS,
    GGML_OP_SOFT_MAX,
    GGML_OP_ROPE,
    GGML_OP_FLASH_ATTN_EXT,
    GGML_OP_ARGMAX,
    GGML_OP_UNARY,
    GGML_OP_DIV,
    GGML_OP_SUM_ROWS,
    GGML_OP_ARGSORT,
    // ops of the reference's other graphs (model.cpp:1156-1295 Mamba2 / gated-delta mixers,
    // dory.c:722-724): built by the constructors below
    GGML_OP_SUB,
    GGML_OP_CONCAT,
    GGML_OP_L2_NORM,
    GGML_OP_GLU,
    GGML_OP_SSM_CONV,
    GGML_OP_SSM_SCAN,
    GGML_OP_GATED_DELTA_NET,
    GGML_OP_COUNT,
};

enum ggml_unary_op {
    GGML_UNARY_OP_RELU = 0,
    GGML_UNARY_OP_SILU,
    GGML_UNARY_OP_SIGMOID,
    GGML_UNARY_OP_ABS,
    GGML_UNARY_OP_SOFTPLUS,
    GGML_UNARY_OP_COUNT,
};

enum ggml_glu_op {
    GGML_GLU_OP_SWIGLU = 0,
};

enum ggml_tensor_flag {
    GGML_TENSOR_FLAG_INPUT  = 1,
    GGML_TENSOR_FLAG_OUTPUT = 2,
};

struct ggml_backend_buffer;

// Same field set and meaning as ggml's tensor; model.cpp reads ne/nb/type/name directly
// (e.g. model.cpp:721-729, 1351, 1407-1412).
struct ggml_tensor {
    enum ggml_type type;
    struct ggml_backend_buffer * buffer;

    int64_t ne[GGML_MAX_DIMS];
    size_t  nb[GGML_MAX_DIMS];

    enum ggml_op op;
    int32_t op_params[GGML_MAX_OP_PARAMS / sizeof(int32_t)];
    int32_t flags;

    struct ggml_tensor * src[GGML_MAX_SRC];

    struct ggml_tensor * view_src;
    size_t               view_offs;

    void * data;
    char   name[GGML_MAX_NAME];
    void * extra;
    char   padding[8];
};

struct ggml_context;
struct ggml_cgraph;

struct ggml_init_params {
    size_t mem_size;   // bytes
    void * mem_buffer; // if NULL, memory is allocated internally
    bool   no_alloc;   // don't allocate memory for tensor data
};

// ---- type traits / conversions (model.cpp:726, 755, 771-775) ----
GGML_API const char * ggml_type_name(enum ggml_type type);
GGML_API size_t  ggml_type_size(enum ggml_type type);   // bytes per block
GGML_API int64_t ggml_blck_size(enum ggml_type type);   // elements per block
GGML_API size_t  ggml_row_size(enum ggml_type type, int64_t ne);
GGML_API bool    ggml_is_quantized(enum ggml_type type);
GGML_API const char * ggml_op_name(enum ggml_op op);

GGML_API float       ggml_fp16_to_fp32(ggml_fp16_t h);
GGML_API ggml_fp16_t ggml_fp32_to_fp16(float f);
GGML_API float       ggml_bf16_to_fp32(ggml_bf16_t h);
GGML_API ggml_bf16_t ggml_fp32_to_bf16(float f);
GGML_API void ggml_fp16_to_fp32_row(const ggml_fp16_t * x, float * y, int64_t n);
GGML_API void ggml_fp32_to_fp16_row(const float * x, ggml_fp16_t * y, int64_t n);

// ---- context (model.cpp:708-713, 843-845, 1552-1557) ----
GGML_API struct ggml_context * ggml_init(struct ggml_init_params params);
GGML_API void   ggml_free(struct ggml_context * ctx);
GGML_API size_t ggml_used_mem(const struct ggml_context * ctx);
GGML_API bool   ggml_get_no_alloc(struct ggml_context * ctx);
GGML_API void   ggml_set_no_alloc(struct ggml_context * ctx, bool no_alloc);
GGML_API size_t ggml_tensor_overhead(void);
GGML_API size_t ggml_graph_overhead(void);
GGML_API size_t ggml_graph_overhead_custom(size_t size, bool grads);

GGML_API struct ggml_tensor * ggml_get_first_tensor(const struct ggml_context * ctx);
GGML_API struct ggml_tensor * ggml_get_next_tensor(const struct ggml_context * ctx, struct ggml_tensor * tensor);
GGML_API struct ggml_tensor * ggml_get_tensor(struct ggml_context * ctx, const char * name);

// ---- tensors (model.cpp:719, 855-856, 1306-1308) ----
GGML_API struct ggml_tensor * ggml_new_tensor(struct ggml_context * ctx, enum ggml_type type, int n_dims, const int64_t * ne);
GGML_API struct ggml_tensor * ggml_new_tensor_1d(struct ggml_context * ctx, enum ggml_type type, int64_t ne0);
GGML_API struct ggml_tensor * ggml_new_tensor_2d(struct ggml_context * ctx, enum ggml_type type, int64_t ne0, int64_t ne1);
GGML_API struct ggml_tensor * ggml_new_tensor_3d(struct ggml_context * ctx, enum ggml_type type, int64_t ne0, int64_t ne1, int64_t ne2);
GGML_API struct ggml_tensor * ggml_new_tensor_4d(struct ggml_context * ctx, enum ggml_type type, int64_t ne0, int64_t ne1, int64_t ne2, int64_t ne3);
GGML_API struct ggml_tensor * ggml_dup_tensor(struct ggml_context * ctx, const struct ggml_tensor * src);
GGML_API struct ggml_tensor * ggml_view_tensor(struct ggml_context * ctx, struct ggml_tensor * src);
GGML_API struct ggml_tensor * ggml_set_name(struct ggml_tensor * tensor, const char * name);
GGML_API const char *         ggml_get_name(const struct ggml_tensor * tensor);
GGML_API void ggml_set_input(struct ggml_tensor * tensor);
GGML_API void ggml_set_output(struct ggml_tensor * tensor);

GGML_API int64_t ggml_nelements(const struct ggml_tensor * tensor);
GGML_API int64_t ggml_nrows(const struct ggml_tensor * tensor);
GGML_API size_t  ggml_nbytes(const struct ggml_tensor * tensor);
GGML_API int     ggml_n_dims(const struct ggml_tensor * tensor);
GGML_API bool    ggml_is_contiguous(const struct ggml_tensor * tensor);
GGML_API bool    ggml_is_permuted(const struct ggml_tensor * tensor);
GGML_API bool    ggml_is_transposed(const struct ggml_tensor * tensor);
GGML_API bool    ggml_are_same_shape(const struct ggml_tensor * a, const struct ggml_tensor * b);
GGML_API bool    ggml_can_repeat(const struct ggml_tensor * t0, const struct ggml_tensor * t1); // t0 tiles t1 exactly

// ---- ops on the forward_step path (model.cpp:1071-1474) ----
GGML_API struct ggml_tensor * ggml_get_rows(struct ggml_context * ctx, struct ggml_tensor * a, struct ggml_tensor * b);
GGML_API struct ggml_tensor * ggml_rms_norm(struct ggml_context * ctx, struct ggml_tensor * a, float eps);
GGML_API struct ggml_tensor * ggml_mul(struct ggml_context * ctx, struct ggml_tensor * a, struct ggml_tensor * b);
GGML_API struct ggml_tensor * ggml_add(struct ggml_context * ctx, struct ggml_tensor * a, struct ggml_tensor * b);
GGML_API struct ggml_tensor * ggml_scale(struct ggml_context * ctx, struct ggml_tensor * a, float s);
GGML_API struct ggml_tensor * ggml_sqr(struct ggml_context * ctx, struct ggml_tensor * a);
GGML_API struct ggml_tensor * ggml_mul_mat(struct ggml_context * ctx, struct ggml_tensor * a, struct ggml_tensor * b);
// as: [K, N, n_expert], b: [K, n_b, n_tokens], ids: I32 [n_expert_used, n_tokens]
// -> F32 [N, n_expert_used, n_tokens]; column (e, t) = as[:, :, ids[e, t]] . b[:, e % n_b, t]
GGML_API struct ggml_tensor * ggml_mul_mat_id(struct ggml_context * ctx, struct ggml_tensor * as, struct ggml_tensor * b, struct ggml_tensor * ids);

GGML_API struct ggml_tensor * ggml_reshape_1d(struct ggml_context * ctx, struct ggml_tensor * a, int64_t ne0);
GGML_API struct ggml_tensor * ggml_reshape_2d(struct ggml_context * ctx, struct ggml_tensor * a, int64_t ne0, int64_t ne1);
GGML_API struct ggml_tensor * ggml_reshape_3d(struct ggml_context * ctx, struct ggml_tensor * a, int64_t ne0, int64_t ne1, int64_t ne2);
GGML_API struct ggml_tensor * ggml_reshape_4d(struct ggml_context * ctx, struct ggml_tensor * a, int64_t ne0, int64_t ne1, int64_t ne2, int64_t ne3);
GGML_API struct ggml_tensor * ggml_view_1d(struct ggml_context * ctx, struct ggml_tensor * a, int64_t ne0, size_t offset);
GGML_API struct ggml_tensor * ggml_view_2d(struct ggml_context * ctx, struct ggml_tensor * a, int64_t ne0, int64_t ne1, size_t nb1, size_t offset);
GGML_API struct ggml_tensor * ggml_view_3d(struct ggml_context * ctx, struct ggml_tensor * a, int64_t ne0, int64_t ne1, int64_t ne2, size_t nb1, size_t nb2, size_t offset);
GGML_API struct ggml_tensor * ggml_view_4d(struct ggml_context * ctx, struct ggml_tensor * a, int64_t ne0, int64_t ne1, int64_t ne2, int64_t ne3, size_t nb1, size_t nb2, size_t nb3, size_t offset);
GGML_API struct ggml_tensor * ggml_permute(struct ggml_context * ctx, struct ggml_tensor * a, int axis0, int axis1, int axis2, int axis3);
GGML_API struct ggml_tensor * ggml_transpose(struct ggml_context * ctx, struct ggml_tensor * a);
GGML_API struct ggml_tensor * ggml_cont(struct ggml_context * ctx, struct ggml_tensor * a);
GGML_API struct ggml_tensor * ggml_cont_2d(struct ggml_context * ctx, struct ggml_tensor * a, int64_t ne0, int64_t ne1);
GGML_API struct ggml_tensor * ggml_cont_3d(struct ggml_context * ctx, struct ggml_tensor * a, int64_t ne0, int64_t ne1, int64_t ne2);
GGML_API struct ggml_tensor * ggml_cont_4d(struct ggml_context * ctx, struct ggml_tensor * a, int64_t ne0, int64_t ne1, int64_t ne2, int64_t ne3);
// copies a into b (converting type); returns a view of b
GGML_API struct ggml_tensor * ggml_cpy(struct ggml_context * ctx, struct ggml_tensor * a, struct ggml_tensor * b);
GGML_API struct ggml_tensor * ggml_cast(struct ggml_context * ctx, struct ggml_tensor * a, enum ggml_type type);

// b: I32 positions [a->ne[2]]; c: optional F32 frequency factors [n_dims/2]
GGML_API struct ggml_tensor * ggml_rope_ext(struct ggml_context * ctx, struct ggml_tensor * a, struct ggml_tensor * b,
        struct ggml_tensor * c, int n_dims, int mode, int n_ctx_orig, float freq_base, float freq_scale,
        float ext_factor, float attn_factor, float beta_fast, float beta_slow);
GGML_API void ggml_rope_yarn_corr_dims(int n_dims, int n_ctx_orig, float freq_base, float beta_fast, float beta_slow, float dims[2]);

// softmax(a*scale + mask) over ne0; mask F32/F16 [ne0, >=ne1], broadcast over dims 2,3
GGML_API struct ggml_tensor * ggml_soft_max(struct ggml_context * ctx, struct ggml_tensor * a);
GGML_API struct ggml_tensor * ggml_soft_max_ext(struct ggml_context * ctx, struct ggml_tensor * a, struct ggml_tensor * mask, float scale, float max_bias);

GGML_API struct ggml_tensor * ggml_unary(struct ggml_context * ctx, struct ggml_tensor * a, enum ggml_unary_op op);
GGML_API struct ggml_tensor * ggml_silu(struct ggml_context * ctx, struct ggml_tensor * a);
GGML_API struct ggml_tensor * ggml_relu(struct ggml_context * ctx, struct ggml_tensor * a);
GGML_API struct ggml_tensor * ggml_sigmoid(struct ggml_context * ctx, struct ggml_tensor * a);
GGML_API enum ggml_unary_op   ggml_get_unary_op(const struct ggml_tensor * tensor);

// q: [D, n_q, n_head, ne3], k: [D, n_kv, n_head_kv, ne3], v: [Dv, n_kv, n_head_kv, ne3] (not transposed),
// mask: F16 [n_kv, >=n_q]; result F32 [Dv, n_head, n_q, ne3] (model.cpp:1426-1434)
GGML_API struct ggml_tensor * ggml_flash_attn_ext(struct ggml_context * ctx, struct ggml_tensor * q, struct ggml_tensor * k,
        struct ggml_tensor * v, struct ggml_tensor * mask, float scale, float max_bias, float logit_softcap);

// index of the max of each row (first max wins) -> I32 [a->ne[1]]
GGML_API struct ggml_tensor * ggml_argmax(struct ggml_context * ctx, struct ggml_tensor * a);

// ---- ops of the reference's other architectures (model.cpp:1156-1295, dory.c:722-724) ----
// a - b, b repeated over a (like ggml_add)
GGML_API struct ggml_tensor * ggml_sub(struct ggml_context * ctx, struct ggml_tensor * a, struct ggml_tensor * b);
GGML_API struct ggml_tensor * ggml_abs(struct ggml_context * ctx, struct ggml_tensor * a);
// log(1 + exp(x)) (x itself above 20)
GGML_API struct ggml_tensor * ggml_softplus(struct ggml_context * ctx, struct ggml_tensor * a);
// each row over ne0 divided by max(|row|_2, eps)
GGML_API struct ggml_tensor * ggml_l2_norm(struct ggml_context * ctx, struct ggml_tensor * a, float eps);
// a and b joined along dim (the other extents equal)
GGML_API struct ggml_tensor * ggml_concat(struct ggml_context * ctx, struct ggml_tensor * a, struct ggml_tensor * b, int dim);
// silu(a) * b (same shapes)
GGML_API struct ggml_tensor * ggml_swiglu_split(struct ggml_context * ctx, struct ggml_tensor * a, struct ggml_tensor * b);
// sx: [d_conv - 1 + n_t, d_inner, n_s], c: [d_conv, d_inner] -> F32 [d_inner, n_t, n_s]
GGML_API struct ggml_tensor * ggml_ssm_conv(struct ggml_context * ctx, struct ggml_tensor * sx, struct ggml_tensor * c);
// selective scan: F32 1-D [nelements(x) + nelements(s)], y followed by the new state (model.cpp:1187-1196)
GGML_API struct ggml_tensor * ggml_ssm_scan(struct ggml_context * ctx, struct ggml_tensor * s, struct ggml_tensor * x,
        struct ggml_tensor * dt, struct ggml_tensor * A, struct ggml_tensor * B, struct ggml_tensor * C,
        struct ggml_tensor * ids, int version);
// gated delta rule: F32 1-D [nelements(v) + nelements(state)], y followed by the new state
// (model.cpp:1273-1281)
GGML_API struct ggml_tensor * ggml_gated_delta_net(struct ggml_context * ctx, struct ggml_tensor * q, struct ggml_tensor * k,
        struct ggml_tensor * v, struct ggml_tensor * g, struct ggml_tensor * beta, struct ggml_tensor * state, int version);

// ---- MoE routing (the router of qwen_model.c:551-606 as graph ops) ----
enum ggml_sort_order {
    GGML_SORT_ORDER_ASC,
    GGML_SORT_ORDER_DESC,
};
// a / b, b repeated over a (like ggml_mul)
GGML_API struct ggml_tensor * ggml_div(struct ggml_context * ctx, struct ggml_tensor * a, struct ggml_tensor * b);
// F32 [1, ne1, ne2, ne3]: the sum of each row
GGML_API struct ggml_tensor * ggml_sum_rows(struct ggml_context * ctx, struct ggml_tensor * a);
// I32, same shape: the indices that sort each row; equal values keep ascending index order (the
// router's rule: an earlier expert wins a tie)
GGML_API struct ggml_tensor * ggml_argsort(struct ggml_context * ctx, struct ggml_tensor * a, enum ggml_sort_order order);
// I32 [k, ne1, ne2, ne3]: a view of the first k columns of ggml_argsort(a, DESC)
GGML_API struct ggml_tensor * ggml_top_k(struct ggml_context * ctx, struct ggml_tensor * a, int k);

// ---- graph (model.cpp:1300, 1413-1414, 1472) ----
GGML_API struct ggml_cgraph * ggml_new_graph(struct ggml_context * ctx);
GGML_API struct ggml_cgraph * ggml_new_graph_custom(struct ggml_context * ctx, size_t size, bool grads);
GGML_API void ggml_build_forward_expand(struct ggml_cgraph * cgraph, struct ggml_tensor * tensor);
GGML_API int  ggml_graph_n_nodes(struct ggml_cgraph * cgraph);
GGML_API struct ggml_tensor * ggml_graph_node(struct ggml_cgraph * cgraph, int i); // i < 0: from the end
GGML_API int  ggml_graph_n_leafs(struct ggml_cgraph * cgraph);
GGML_API struct ggml_tensor * ggml_graph_leaf(struct ggml_cgraph * cgraph, int i);

// ---- quantization (ggml's public quantizer entry points; used to write synthetic GGUF models) ----
// Quantizes nrows rows of n_per_row floats starting at row `start`; returns bytes written.
GGML_API size_t ggml_quantize_chunk(enum ggml_type type, const float * src, void * dst, int64_t start,
                                    int64_t nrows, int64_t n_per_row, const float * imatrix);
GGML_API void quantize_row_q4_0_ref(const float * x, void * y, int64_t k);
GGML_API void quantize_row_q8_0_ref(const float * x, void * y, int64_t k);
GGML_API void quantize_row_q4_K_ref(const float * x, void * y, int64_t k);
GGML_API void quantize_row_q8_K_ref(const float * x, void * y, int64_t k);
GGML_API void dequantize_row_q4_0(const void * x, float * y, int64_t k);
GGML_API void dequantize_row_q8_0(const void * x, float * y, int64_t k);
GGML_API void dequantize_row_q4_K(const void * x, float * y, int64_t k);
// generic row decode for F32/F16/BF16/Q4_0/Q8_0/Q4_K (used by tensor inspection tools)
GGML_API bool ggml_dequantize_row(enum ggml_type type, const void * x, float * y, int64_t k);

#ifdef __cplusplus
}
#endif
