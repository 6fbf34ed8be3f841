// ggml.h (compat subset) -- STANDALONE-BUILD STAND-IN for ggml's public header.
//
// ggml itself is not vendored (CrispEmbed pins it as a git submodule,
// .gitmodules:1-4).  This file transcribes the parts of ggml's C API that the
// MI355X backend and its test driver use, so they build without ggml.  A real
// integration compiles ggml_backend_mi355.cpp against ggml's own headers instead
// (include path switch only; the backend source does not change).
// The struct layouts and enum values follow upstream ggml as published in 2025
// and are NOT verified against CrispEmbed's fork pin 890278a8.
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
    GGML_TYPE_COUNT = 40,
};

// Only the ops the backend names are listed; the numeric values are the compat
// build's own (code refers to them by name).
enum ggml_op {
    GGML_OP_NONE = 0,
    GGML_OP_DUP,
    GGML_OP_ADD,
    GGML_OP_MUL,
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
    GGML_OP_COUNT,
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
GGML_API struct ggml_context *ggml_init(struct ggml_init_params params);
GGML_API void ggml_free(struct ggml_context *ctx);
GGML_API struct ggml_tensor *ggml_new_tensor_1d(struct ggml_context *ctx, enum ggml_type type, int64_t ne0);
GGML_API struct ggml_tensor *ggml_new_tensor_2d(struct ggml_context *ctx, enum ggml_type type, int64_t ne0,
                                               int64_t ne1);
GGML_API struct ggml_tensor *ggml_new_tensor_3d(struct ggml_context *ctx, enum ggml_type type, int64_t ne0,
                                               int64_t ne1, int64_t ne2);
GGML_API struct ggml_tensor *ggml_get_first_tensor(const struct ggml_context *ctx);
GGML_API struct ggml_tensor *ggml_get_next_tensor(const struct ggml_context *ctx, struct ggml_tensor *tensor);
GGML_API struct ggml_tensor *ggml_mul_mat(struct ggml_context *ctx, struct ggml_tensor *a, struct ggml_tensor *b);
GGML_API struct ggml_tensor *ggml_add(struct ggml_context *ctx, struct ggml_tensor *a, struct ggml_tensor *b);
GGML_API struct ggml_tensor *ggml_reshape_2d(struct ggml_context *ctx, struct ggml_tensor *a, int64_t ne0,
                                            int64_t ne1);
GGML_API struct ggml_cgraph *ggml_new_graph(struct ggml_context *ctx);
GGML_API void ggml_build_forward_expand(struct ggml_cgraph *cgraph, struct ggml_tensor *tensor);
GGML_API int ggml_graph_n_nodes(struct ggml_cgraph *cgraph);
GGML_API struct ggml_tensor *ggml_graph_node(struct ggml_cgraph *cgraph, int i);

#ifdef __cplusplus
}
#endif
