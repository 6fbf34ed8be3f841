// ggml.h (compat subset) -- STANDALONE-BUILD STAND-IN for ggml's public header.
//
// ggml itself is not vendored (CrispEmbed pins it as a git submodule,
// .gitmodules:1-4).  This file transcribes the parts of ggml's C API that the
// MI355X backend and its test driver use, so they build without ggml.  A real
// integration compiles ggml_backend_mi355.cpp against ggml's own headers instead
// (include path switch only; the backend source does not change).
// The struct layouts and the ggml_type / ggml_status / ggml_unary_op values follow
// upstream ggml as published in 2025 (NOT verified against CrispEmbed's fork pin
// 890278a8).  The ggml_op enum is a local subset with its own numbering: code names
// ops, never their values, so the backend compiles unchanged against ggml's header.
#pragma once
#include <stdbool.h>
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define GGML_API __attribute__((visibility("default")))
#define GGML_MAX_DIMS 4
#define GGML_MAX_OP_PARAMS 64
#define GGML_MAX_SRC 10
#define GGML_MAX_NAME 64

enum ggml_status {
    GGML_STATUS_ALLOC_FAILED = -2,
    GGML_STATUS_FAILED = -1,
    GGML_STATUS_SUCCESS = 0,
    GGML_STATUS_ABORTED = 1,
};

enum ggml_type {
    GGML_TYPE_F32 = 0,
    GGML_TYPE_F16 = 1,
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
    GGML_TYPE_I8 = 24,
    GGML_TYPE_I16 = 25,
    GGML_TYPE_I32 = 26,
    GGML_TYPE_COUNT = 40,
};

// Only the ops the backend and its tests name are listed; the numeric values are
// the compat build's own (code refers to them by name).
enum ggml_op {
    GGML_OP_NONE = 0,
    GGML_OP_DUP,
    GGML_OP_ADD,
    GGML_OP_SUB,
    GGML_OP_MUL,
    GGML_OP_DIV,
    GGML_OP_NORM,
    GGML_OP_RMS_NORM,
    GGML_OP_MUL_MAT,
    GGML_OP_MUL_MAT_ID,
    GGML_OP_SCALE,
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
    GGML_OP_UNARY,
    GGML_OP_ARGSORT,
    GGML_OP_REPEAT,
    GGML_OP_COUNT,
};

enum ggml_sort_order {
    GGML_SORT_ORDER_ASC,
    GGML_SORT_ORDER_DESC,
};

enum ggml_unary_op {
    GGML_UNARY_OP_ABS,
    GGML_UNARY_OP_SGN,
    GGML_UNARY_OP_NEG,
    GGML_UNARY_OP_STEP,
    GGML_UNARY_OP_TANH,
    GGML_UNARY_OP_ELU,
    GGML_UNARY_OP_RELU,
    GGML_UNARY_OP_SIGMOID,
    GGML_UNARY_OP_GELU,
    GGML_UNARY_OP_GELU_QUICK,
    GGML_UNARY_OP_SILU,
    GGML_UNARY_OP_HARDSWISH,
    GGML_UNARY_OP_HARDSIGMOID,
    GGML_UNARY_OP_EXP,
    GGML_UNARY_OP_GELU_ERF,
    GGML_UNARY_OP_COUNT,
};

enum ggml_tensor_flag {
    GGML_TENSOR_FLAG_INPUT = 1,
    GGML_TENSOR_FLAG_OUTPUT = 2,
    GGML_TENSOR_FLAG_PARAM = 4,
    GGML_TENSOR_FLAG_LOSS = 8,
};

struct ggml_backend_buffer;

struct ggml_tensor {
    enum ggml_type type;
    struct ggml_backend_buffer *buffer;
    int64_t ne[GGML_MAX_DIMS];  // number of elements
    size_t nb[GGML_MAX_DIMS];   // stride in bytes
    enum ggml_op op;
    int32_t op_params[GGML_MAX_OP_PARAMS / sizeof(int32_t)];
    int32_t flags;
    struct ggml_tensor *src[GGML_MAX_SRC];
    struct ggml_tensor *view_src;
    size_t view_offs;
    void *data;
    char name[GGML_MAX_NAME];
    void *extra;
    char padding[8];
};

struct ggml_context;
struct ggml_cgraph;

struct ggml_init_params {
    size_t mem_size;
    void *mem_buffer;
    bool no_alloc;
};

GGML_API int64_t ggml_blck_size(enum ggml_type type);
GGML_API size_t ggml_type_size(enum ggml_type type);
GGML_API size_t ggml_row_size(enum ggml_type type, int64_t ne);
GGML_API const char *ggml_type_name(enum ggml_type type);
GGML_API const char *ggml_op_name(enum ggml_op op);
GGML_API int64_t ggml_nelements(const struct ggml_tensor *tensor);
GGML_API int64_t ggml_nrows(const struct ggml_tensor *tensor);
GGML_API size_t ggml_nbytes(const struct ggml_tensor *tensor);
GGML_API bool ggml_is_contiguous(const struct ggml_tensor *tensor);
GGML_API bool ggml_is_empty(const struct ggml_tensor *tensor);
GGML_API const char *ggml_get_name(const struct ggml_tensor *tensor);
GGML_API struct ggml_tensor *ggml_set_name(struct ggml_tensor *tensor, const char *name);
GGML_API void ggml_set_input(struct ggml_tensor *tensor);
GGML_API void ggml_set_output(struct ggml_tensor *tensor);

GGML_API size_t ggml_tensor_overhead(void);
GGML_API size_t ggml_graph_overhead(void);
GGML_API size_t ggml_graph_overhead_custom(size_t size, bool grads);
GGML_API struct ggml_context *ggml_init(struct ggml_init_params params);
GGML_API void ggml_free(struct ggml_context *ctx);
GGML_API struct ggml_tensor *ggml_new_tensor_1d(struct ggml_context *ctx, enum ggml_type type, int64_t ne0);
GGML_API struct ggml_tensor *ggml_new_tensor_2d(struct ggml_context *ctx, enum ggml_type type, int64_t ne0,
                                               int64_t ne1);
GGML_API struct ggml_tensor *ggml_new_tensor_3d(struct ggml_context *ctx, enum ggml_type type, int64_t ne0,
                                               int64_t ne1, int64_t ne2);
GGML_API struct ggml_tensor *ggml_new_tensor_4d(struct ggml_context *ctx, enum ggml_type type, int64_t ne0,
                                               int64_t ne1, int64_t ne2, int64_t ne3);
GGML_API struct ggml_tensor *ggml_get_first_tensor(const struct ggml_context *ctx);
GGML_API struct ggml_tensor *ggml_get_next_tensor(const struct ggml_context *ctx, struct ggml_tensor *tensor);
GGML_API struct ggml_tensor *ggml_mul_mat(struct ggml_context *ctx, struct ggml_tensor *a, struct ggml_tensor *b);
// as [k, n, n_exp], b [k, 1|n_used, T], ids I32 [n_used, T] -> [n, n_used, T]
GGML_API struct ggml_tensor *ggml_mul_mat_id(struct ggml_context *ctx, struct ggml_tensor *as, struct ggml_tensor *b,
                                            struct ggml_tensor *ids);
GGML_API struct ggml_tensor *ggml_add(struct ggml_context *ctx, struct ggml_tensor *a, struct ggml_tensor *b);
GGML_API struct ggml_tensor *ggml_reshape_2d(struct ggml_context *ctx, struct ggml_tensor *a, int64_t ne0,
                                            int64_t ne1);
GGML_API struct ggml_tensor *ggml_reshape_3d(struct ggml_context *ctx, struct ggml_tensor *a, int64_t ne0,
                                            int64_t ne1, int64_t ne2);
GGML_API struct ggml_tensor *ggml_reshape_4d(struct ggml_context *ctx, struct ggml_tensor *a, int64_t ne0,
                                            int64_t ne1, int64_t ne2, int64_t ne3);
GGML_API struct ggml_tensor *ggml_view_1d(struct ggml_context *ctx, struct ggml_tensor *a, int64_t ne0, size_t offset);
GGML_API struct ggml_tensor *ggml_view_2d(struct ggml_context *ctx, struct ggml_tensor *a, int64_t ne0, int64_t ne1,
                                         size_t nb1, size_t offset);
GGML_API struct ggml_tensor *ggml_permute(struct ggml_context *ctx, struct ggml_tensor *a, int axis0, int axis1,
                                         int axis2, int axis3);
GGML_API struct ggml_tensor *ggml_cont(struct ggml_context *ctx, struct ggml_tensor *a);
GGML_API struct ggml_tensor *ggml_cpy(struct ggml_context *ctx, struct ggml_tensor *a, struct ggml_tensor *b);
GGML_API struct ggml_tensor *ggml_sub(struct ggml_context *ctx, struct ggml_tensor *a, struct ggml_tensor *b);
GGML_API struct ggml_tensor *ggml_mul(struct ggml_context *ctx, struct ggml_tensor *a, struct ggml_tensor *b);
GGML_API struct ggml_tensor *ggml_div(struct ggml_context *ctx, struct ggml_tensor *a, struct ggml_tensor *b);
GGML_API struct ggml_tensor *ggml_get_rows(struct ggml_context *ctx, struct ggml_tensor *a, struct ggml_tensor *b);
GGML_API struct ggml_tensor *ggml_norm(struct ggml_context *ctx, struct ggml_tensor *a, float eps);
GGML_API struct ggml_tensor *ggml_rms_norm(struct ggml_context *ctx, struct ggml_tensor *a, float eps);
GGML_API struct ggml_tensor *ggml_unary(struct ggml_context *ctx, struct ggml_tensor *a, enum ggml_unary_op op);
GGML_API struct ggml_tensor *ggml_gelu_erf(struct ggml_context *ctx, struct ggml_tensor *a);
GGML_API struct ggml_tensor *ggml_gelu(struct ggml_context *ctx, struct ggml_tensor *a);
GGML_API struct ggml_tensor *ggml_silu(struct ggml_context *ctx, struct ggml_tensor *a);
GGML_API struct ggml_tensor *ggml_relu(struct ggml_context *ctx, struct ggml_tensor *a);
GGML_API enum ggml_unary_op ggml_get_unary_op(const struct ggml_tensor *tensor);
// q [hd, Tq, nh, B], k / v [hd, Tk, nkv, B], mask F16 or NULL -> [hd, nh, Tq, B] F32;
// op_params: scale, max_bias, logit_softcap
GGML_API struct ggml_tensor *ggml_flash_attn_ext(struct ggml_context *ctx, struct ggml_tensor *q, struct ggml_tensor *k,
                                                struct ggml_tensor *v, struct ggml_tensor *mask, float scale,
                                                float max_bias, float logit_softcap);
GGML_API struct ggml_tensor *ggml_graph_get_tensor(const struct ggml_cgraph *cgraph, const char *name);
// softmax over ne0 of a * scale + mask (mask NULL or F16/F32); op_params: scale, max_bias
GGML_API struct ggml_tensor *ggml_soft_max(struct ggml_context *ctx, struct ggml_tensor *a);
GGML_API struct ggml_tensor *ggml_soft_max_ext(struct ggml_context *ctx, struct ggml_tensor *a,
                                              struct ggml_tensor *mask, float scale, float max_bias);
// I32 indices sorting each row; op_params[0] = order.  top_k: the first k columns, descending
GGML_API struct ggml_tensor *ggml_argsort(struct ggml_context *ctx, struct ggml_tensor *a, enum ggml_sort_order order);
GGML_API struct ggml_tensor *ggml_top_k(struct ggml_context *ctx, struct ggml_tensor *a, int k);
// a tiled to b's shape
GGML_API struct ggml_tensor *ggml_repeat(struct ggml_context *ctx, struct ggml_tensor *a, struct ggml_tensor *b);
#define GGML_ROPE_TYPE_NEOX 2
// a [n_dims.., n_head, T, B], b I32 positions [T], c freq factors or NULL; op_params:
// 0, n_dims, mode, 0, n_ctx_orig, then floats freq_base, freq_scale, ext_factor, attn_factor,
// beta_fast, beta_slow
GGML_API struct ggml_tensor *ggml_rope_ext(struct ggml_context *ctx, struct ggml_tensor *a, struct ggml_tensor *b,
                                          struct ggml_tensor *c, int n_dims, int mode, int n_ctx_orig, float freq_base,
                                          float freq_scale, float ext_factor, float attn_factor, float beta_fast,
                                          float beta_slow);
GGML_API struct ggml_cgraph *ggml_new_graph(struct ggml_context *ctx);
GGML_API struct ggml_cgraph *ggml_new_graph_custom(struct ggml_context *ctx, size_t size, bool grads);
GGML_API void ggml_build_forward_expand(struct ggml_cgraph *cgraph, struct ggml_tensor *tensor);
GGML_API int ggml_graph_n_nodes(struct ggml_cgraph *cgraph);
GGML_API struct ggml_tensor *ggml_graph_node(struct ggml_cgraph *cgraph, int i);
// Stand-in only (not ggml API): ggml's internal ggml_graph_view(cgraph, i0, i1), which the
// scheduler uses to compute a graph in pieces, as an allocated object; nodes [i0, i1), use
// counts of the whole graph.  Free with ggml_compat_graph_view_free.
GGML_API struct ggml_cgraph *ggml_compat_graph_view(struct ggml_cgraph *cgraph, int i0, int i1);
GGML_API void ggml_compat_graph_view_free(struct ggml_cgraph *view);

#ifdef __cplusplus
}
#endif
