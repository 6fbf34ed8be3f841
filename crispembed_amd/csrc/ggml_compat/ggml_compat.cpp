// ggml_compat.cpp -- STANDALONE-BUILD STAND-IN for the parts of ggml-base that
// the MI355X backend and its test driver call (tensor metadata helpers, the
// backend registry, buffer/backend dispatch through the interface tables, and a
// context allocator).  It is built into libggml-compat.so, which a real
// integration replaces with ggml itself; libggml-mi355.so only needs these
// symbols from whichever library provides them.  Behaviour follows ggml's
// published API; it is not a copy of ggml's implementation.
#include <algorithm>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <vector>

#include "ggml-backend-impl.h"
#include "ggml-impl.h"
#include "ggml.h"

// ---------------------------------------------------------------------------
// type traits (only the types this project uses)
// ---------------------------------------------------------------------------
extern "C" int64_t ggml_blck_size(enum ggml_type type) {
    switch (type) {
        case GGML_TYPE_F32:
        case GGML_TYPE_F16:
        case GGML_TYPE_I32: return 1;
        case GGML_TYPE_Q8_0: return 32;
        case GGML_TYPE_Q4_K:
        case GGML_TYPE_Q6_K:
        case GGML_TYPE_Q8_K: return 256;
        default: return 0;
    }
}

extern "C" size_t ggml_type_size(enum ggml_type type) {
    switch (type) {
        case GGML_TYPE_F32:
        case GGML_TYPE_I32: return 4;
        case GGML_TYPE_F16: return 2;
        case GGML_TYPE_Q8_0: return 34;
        case GGML_TYPE_Q4_K: return 144;
        case GGML_TYPE_Q6_K: return 210;
        case GGML_TYPE_Q8_K: return 292;
        default: return 0;
    }
}

extern "C" const char *ggml_type_name(enum ggml_type type) {
    switch (type) {
        case GGML_TYPE_F32: return "f32";
        case GGML_TYPE_F16: return "f16";
        case GGML_TYPE_Q8_0: return "q8_0";
        case GGML_TYPE_Q4_K: return "q4_K";
        case GGML_TYPE_Q6_K: return "q6_K";
        case GGML_TYPE_Q8_K: return "q8_K";
        case GGML_TYPE_I32: return "i32";
        default: return "?";
    }
}

extern "C" const char *ggml_op_name(enum ggml_op op) {
    switch (op) {
        case GGML_OP_NONE: return "NONE";
        case GGML_OP_DUP: return "DUP";
        case GGML_OP_ADD: return "ADD";
        case GGML_OP_SUB: return "SUB";
        case GGML_OP_MUL: return "MUL";
        case GGML_OP_DIV: return "DIV";
        case GGML_OP_NORM: return "NORM";
        case GGML_OP_RMS_NORM: return "RMS_NORM";
        case GGML_OP_MUL_MAT: return "MUL_MAT";
        case GGML_OP_MUL_MAT_ID: return "MUL_MAT_ID";
        case GGML_OP_SCALE: return "SCALE";
        case GGML_OP_CPY: return "CPY";
        case GGML_OP_CONT: return "CONT";
        case GGML_OP_RESHAPE: return "RESHAPE";
        case GGML_OP_VIEW: return "VIEW";
        case GGML_OP_PERMUTE: return "PERMUTE";
        case GGML_OP_TRANSPOSE: return "TRANSPOSE";
        case GGML_OP_GET_ROWS: return "GET_ROWS";
        case GGML_OP_SOFT_MAX: return "SOFT_MAX";
        case GGML_OP_ROPE: return "ROPE";
        case GGML_OP_FLASH_ATTN_EXT: return "FLASH_ATTN_EXT";
        case GGML_OP_UNARY: return "UNARY";
        case GGML_OP_ARGSORT: return "ARGSORT";
        case GGML_OP_REPEAT: return "REPEAT";
        default: return "OP";
    }
}

extern "C" size_t ggml_row_size(enum ggml_type type, int64_t ne) {
    const int64_t b = ggml_blck_size(type);
    return b ? ggml_type_size(type) * (size_t)(ne / b) : 0;
}

extern "C" int64_t ggml_nelements(const struct ggml_tensor *t) { return t->ne[0] * t->ne[1] * t->ne[2] * t->ne[3]; }
extern "C" int64_t ggml_nrows(const struct ggml_tensor *t) { return t->ne[1] * t->ne[2] * t->ne[3]; }

extern "C" size_t ggml_nbytes(const struct ggml_tensor *t) {
    for (int i = 0; i < GGML_MAX_DIMS; i++)
        if (t->ne[i] <= 0) return 0;
    const int64_t b = ggml_blck_size(t->type);
    size_t n;
    if (b == 1) {
        n = ggml_type_size(t->type);
        for (int i = 0; i < GGML_MAX_DIMS; i++) n += (size_t)(t->ne[i] - 1) * t->nb[i];
    } else {
        n = (size_t)(t->ne[0] * t->nb[0] / b);
        for (int i = 1; i < GGML_MAX_DIMS; i++) n += (size_t)(t->ne[i] - 1) * t->nb[i];
    }
    return n;
}

extern "C" bool ggml_is_contiguous(const struct ggml_tensor *t) {
    size_t next = ggml_type_size(t->type);
    if (t->ne[0] != ggml_blck_size(t->type) && t->nb[0] != next) return false;
    next *= (size_t)(t->ne[0] / ggml_blck_size(t->type));
    for (int i = 1; i < GGML_MAX_DIMS; i++) {
        if (t->ne[i] != 1) {
            if (t->nb[i] != next) return false;
            next *= (size_t)t->ne[i];
        }
    }
    return true;
}

extern "C" bool ggml_is_empty(const struct ggml_tensor *t) {
    for (int i = 0; i < GGML_MAX_DIMS; i++)
        if (t->ne[i] == 0) return true;
    return false;
}

extern "C" const char *ggml_get_name(const struct ggml_tensor *t) { return t->name; }
extern "C" struct ggml_tensor *ggml_set_name(struct ggml_tensor *t, const char *name) {
    std::snprintf(t->name, sizeof(t->name), "%s", name);
    return t;
}
extern "C" void ggml_set_input(struct ggml_tensor *t) { t->flags |= 1; }
extern "C" void ggml_set_output(struct ggml_tensor *t) { t->flags |= 2; }

// ---------------------------------------------------------------------------
// contexts, tensors, graphs
// ---------------------------------------------------------------------------
struct ggml_context {
    bool no_alloc = true;
    std::vector<ggml_tensor *> tensors;
    std::vector<ggml_cgraph *> graphs;
};

struct ggml_cgraph {
    std::vector<ggml_tensor *> nodes;
    std::vector<ggml_tensor *> leafs;
    // a view of nodes [i0, i1) of another graph (ggml_graph_view): use counts are the whole
    // graph's, as in ggml, where a view shares its parent's use-count table
    const ggml_cgraph *parent = nullptr;
};

extern "C" size_t ggml_tensor_overhead(void) { return sizeof(ggml_tensor) + 16; }
extern "C" size_t ggml_graph_overhead(void) { return 4096; }
// the node list grows as needed: no size limit to reserve
extern "C" size_t ggml_graph_overhead_custom(size_t, bool) { return 4096; }

extern "C" struct ggml_context *ggml_init(struct ggml_init_params params) {
    ggml_context *ctx = new ggml_context;
    ctx->no_alloc = params.no_alloc;
    return ctx;
}

extern "C" void ggml_free(struct ggml_context *ctx) {
    if (!ctx) return;
    for (ggml_tensor *t : ctx->tensors) {
        if (!ctx->no_alloc && !t->view_src && !t->buffer) std::free(t->data);
        delete t;
    }
    for (ggml_cgraph *g : ctx->graphs) delete g;
    delete ctx;
}

static ggml_tensor *new_tensor(ggml_context *ctx, ggml_type type, int n_dims, const int64_t *ne) {
    ggml_tensor *t = new ggml_tensor;
    std::memset(t, 0, sizeof(*t));
    t->type = type;
    for (int i = 0; i < GGML_MAX_DIMS; i++) t->ne[i] = i < n_dims ? ne[i] : 1;
    t->nb[0] = ggml_type_size(type);
    t->nb[1] = t->nb[0] * (size_t)(t->ne[0] / ggml_blck_size(type));
    for (int i = 2; i < GGML_MAX_DIMS; i++) t->nb[i] = t->nb[i - 1] * (size_t)t->ne[i - 1];
    t->op = GGML_OP_NONE;
    if (!ctx->no_alloc) t->data = std::calloc(1, ggml_nbytes(t) ? ggml_nbytes(t) : 1);
    ctx->tensors.push_back(t);
    return t;
}

extern "C" struct ggml_tensor *ggml_new_tensor_1d(struct ggml_context *ctx, enum ggml_type type, int64_t ne0) {
    const int64_t ne[1] = {ne0};
    return new_tensor(ctx, type, 1, ne);
}
extern "C" struct ggml_tensor *ggml_new_tensor_2d(struct ggml_context *ctx, enum ggml_type type, int64_t ne0,
                                                  int64_t ne1) {
    const int64_t ne[2] = {ne0, ne1};
    return new_tensor(ctx, type, 2, ne);
}
extern "C" struct ggml_tensor *ggml_new_tensor_3d(struct ggml_context *ctx, enum ggml_type type, int64_t ne0,
                                                  int64_t ne1, int64_t ne2) {
    const int64_t ne[3] = {ne0, ne1, ne2};
    return new_tensor(ctx, type, 3, ne);
}

extern "C" struct ggml_tensor *ggml_new_tensor_4d(struct ggml_context *ctx, enum ggml_type type, int64_t ne0,
                                                  int64_t ne1, int64_t ne2, int64_t ne3) {
    const int64_t ne[4] = {ne0, ne1, ne2, ne3};
    return new_tensor(ctx, type, 4, ne);
}

extern "C" struct ggml_tensor *ggml_get_first_tensor(const struct ggml_context *ctx) {
    return ctx->tensors.empty() ? nullptr : ctx->tensors.front();
}
extern "C" struct ggml_tensor *ggml_get_next_tensor(const struct ggml_context *ctx, struct ggml_tensor *t) {
    auto it = std::find(ctx->tensors.begin(), ctx->tensors.end(), t);
    if (it == ctx->tensors.end() || ++it == ctx->tensors.end()) return nullptr;
    return *it;
}

// result = a * b^T in ggml's convention: a [K, N], b [K, M, ...] -> [N, M, ...]
extern "C" struct ggml_tensor *ggml_mul_mat(struct ggml_context *ctx, struct ggml_tensor *a, struct ggml_tensor *b) {
    const int64_t ne[4] = {a->ne[1], b->ne[1], b->ne[2], b->ne[3]};
    ggml_tensor *r = new_tensor(ctx, GGML_TYPE_F32, 4, ne);
    r->op = GGML_OP_MUL_MAT;
    r->src[0] = a;
    r->src[1] = b;
    return r;
}

extern "C" struct ggml_tensor *ggml_mul_mat_id(struct ggml_context *ctx, struct ggml_tensor *as,
                                               struct ggml_tensor *b, struct ggml_tensor *ids) {
    const int64_t ne[4] = {as->ne[1], ids->ne[0], b->ne[2], 1};
    ggml_tensor *r = new_tensor(ctx, GGML_TYPE_F32, 4, ne);
    r->op = GGML_OP_MUL_MAT_ID;
    r->src[0] = as;
    r->src[1] = b;
    r->src[2] = ids;
    return r;
}

static ggml_tensor *binary(ggml_context *ctx, ggml_tensor *a, ggml_tensor *b, ggml_op op) {
    ggml_tensor *r = new_tensor(ctx, a->type, 4, a->ne);
    r->op = op;
    r->src[0] = a;
    r->src[1] = b;
    return r;
}

extern "C" struct ggml_tensor *ggml_add(struct ggml_context *ctx, struct ggml_tensor *a, struct ggml_tensor *b) {
    return binary(ctx, a, b, GGML_OP_ADD);
}
extern "C" struct ggml_tensor *ggml_sub(struct ggml_context *ctx, struct ggml_tensor *a, struct ggml_tensor *b) {
    return binary(ctx, a, b, GGML_OP_SUB);
}
extern "C" struct ggml_tensor *ggml_mul(struct ggml_context *ctx, struct ggml_tensor *a, struct ggml_tensor *b) {
    return binary(ctx, a, b, GGML_OP_MUL);
}
extern "C" struct ggml_tensor *ggml_div(struct ggml_context *ctx, struct ggml_tensor *a, struct ggml_tensor *b) {
    return binary(ctx, a, b, GGML_OP_DIV);
}

// A tensor sharing `a`'s memory: shape ne, strides nb, `offset` bytes into a's data.
static ggml_tensor *view_of(ggml_context *ctx, ggml_tensor *a, const int64_t *ne, const size_t *nb, size_t offset,
                            ggml_op op) {
    const bool na = ctx->no_alloc;
    ctx->no_alloc = true;
    ggml_tensor *r = new_tensor(ctx, a->type, 4, ne);
    ctx->no_alloc = na;
    for (int i = 0; i < GGML_MAX_DIMS; i++) r->nb[i] = nb[i];
    r->op = op;
    r->src[0] = a;
    r->view_src = a->view_src ? a->view_src : a;
    r->view_offs = a->view_offs + offset;
    r->data = a->data ? (char *)a->data + offset : nullptr;
    r->buffer = a->buffer;
    return r;
}

static ggml_tensor *reshape(ggml_context *ctx, ggml_tensor *a, int n, const int64_t *ne_in) {
    if (!ggml_is_contiguous(a)) {
        std::fprintf(stderr, "ggml_reshape: tensor '%s' is not contiguous\n", a->name);
        std::abort();
    }
    int64_t ne[4] = {1, 1, 1, 1};
    for (int i = 0; i < n; i++) ne[i] = ne_in[i];
    if (ne[0] * ne[1] * ne[2] * ne[3] != ggml_nelements(a)) {
        std::fprintf(stderr, "ggml_reshape: element count of '%s' changes\n", a->name);
        std::abort();
    }
    size_t nb[4];
    nb[0] = ggml_type_size(a->type);
    nb[1] = nb[0] * (size_t)(ne[0] / ggml_blck_size(a->type));
    for (int i = 2; i < 4; i++) nb[i] = nb[i - 1] * (size_t)ne[i - 1];
    return view_of(ctx, a, ne, nb, 0, GGML_OP_RESHAPE);
}

extern "C" struct ggml_tensor *ggml_reshape_2d(struct ggml_context *ctx, struct ggml_tensor *a, int64_t ne0,
                                               int64_t ne1) {
    const int64_t ne[2] = {ne0, ne1};
    return reshape(ctx, a, 2, ne);
}
extern "C" struct ggml_tensor *ggml_reshape_3d(struct ggml_context *ctx, struct ggml_tensor *a, int64_t ne0,
                                               int64_t ne1, int64_t ne2) {
    const int64_t ne[3] = {ne0, ne1, ne2};
    return reshape(ctx, a, 3, ne);
}
extern "C" struct ggml_tensor *ggml_reshape_4d(struct ggml_context *ctx, struct ggml_tensor *a, int64_t ne0,
                                               int64_t ne1, int64_t ne2, int64_t ne3) {
    const int64_t ne[4] = {ne0, ne1, ne2, ne3};
    return reshape(ctx, a, 4, ne);
}

extern "C" struct ggml_tensor *ggml_view_1d(struct ggml_context *ctx, struct ggml_tensor *a, int64_t ne0,
                                            size_t offset) {
    const int64_t ne[4] = {ne0, 1, 1, 1};
    const size_t es = ggml_type_size(a->type);
    const size_t nb[4] = {es, es * (size_t)ne0, es * (size_t)ne0, es * (size_t)ne0};
    return view_of(ctx, a, ne, nb, offset, GGML_OP_VIEW);
}

extern "C" struct ggml_tensor *ggml_view_2d(struct ggml_context *ctx, struct ggml_tensor *a, int64_t ne0,
                                            int64_t ne1, size_t nb1, size_t offset) {
    const int64_t ne[4] = {ne0, ne1, 1, 1};
    const size_t nb[4] = {ggml_type_size(a->type), nb1, nb1 * (size_t)ne1, nb1 * (size_t)ne1};
    return view_of(ctx, a, ne, nb, offset, GGML_OP_VIEW);
}

// result dim axis_i is a's dim i
extern "C" struct ggml_tensor *ggml_permute(struct ggml_context *ctx, struct ggml_tensor *a, int axis0, int axis1,
                                            int axis2, int axis3) {
    const int ax[4] = {axis0, axis1, axis2, axis3};
    int64_t ne[4];
    size_t nb[4];
    for (int i = 0; i < 4; i++) {
        ne[ax[i]] = a->ne[i];
        nb[ax[i]] = a->nb[i];
    }
    ggml_tensor *r = view_of(ctx, a, ne, nb, 0, GGML_OP_PERMUTE);
    std::memcpy(r->op_params, ax, sizeof(ax));  // the axes, as ggml records them
    return r;
}

extern "C" struct ggml_tensor *ggml_cont(struct ggml_context *ctx, struct ggml_tensor *a) {
    ggml_tensor *r = new_tensor(ctx, a->type, 4, a->ne);
    r->op = GGML_OP_CONT;
    r->src[0] = a;
    return r;
}

// copies a into b; the result is a view of b
extern "C" struct ggml_tensor *ggml_cpy(struct ggml_context *ctx, struct ggml_tensor *a, struct ggml_tensor *b) {
    ggml_tensor *r = view_of(ctx, b, b->ne, b->nb, 0, GGML_OP_CPY);
    r->src[0] = a;
    r->src[1] = b;
    return r;
}

extern "C" struct ggml_tensor *ggml_get_rows(struct ggml_context *ctx, struct ggml_tensor *a, struct ggml_tensor *b) {
    const int64_t ne[4] = {a->ne[0], b->ne[0], b->ne[1], b->ne[2]};
    ggml_tensor *r = new_tensor(ctx, GGML_TYPE_F32, 4, ne);
    r->op = GGML_OP_GET_ROWS;
    r->src[0] = a;
    r->src[1] = b;
    return r;
}

static ggml_tensor *norm_op(ggml_context *ctx, ggml_tensor *a, float eps, ggml_op op) {
    ggml_tensor *r = new_tensor(ctx, a->type, 4, a->ne);
    r->op = op;
    std::memcpy(r->op_params, &eps, sizeof(float));
    r->src[0] = a;
    return r;
}
extern "C" struct ggml_tensor *ggml_norm(struct ggml_context *ctx, struct ggml_tensor *a, float eps) {
    return norm_op(ctx, a, eps, GGML_OP_NORM);
}
extern "C" struct ggml_tensor *ggml_rms_norm(struct ggml_context *ctx, struct ggml_tensor *a, float eps) {
    return norm_op(ctx, a, eps, GGML_OP_RMS_NORM);
}

extern "C" struct ggml_tensor *ggml_unary(struct ggml_context *ctx, struct ggml_tensor *a, enum ggml_unary_op op) {
    ggml_tensor *r = new_tensor(ctx, a->type, 4, a->ne);
    r->op = GGML_OP_UNARY;
    r->op_params[0] = (int32_t)op;
    r->src[0] = a;
    return r;
}
extern "C" struct ggml_tensor *ggml_gelu_erf(struct ggml_context *ctx, struct ggml_tensor *a) {
    return ggml_unary(ctx, a, GGML_UNARY_OP_GELU_ERF);
}
extern "C" struct ggml_tensor *ggml_gelu(struct ggml_context *ctx, struct ggml_tensor *a) {
    return ggml_unary(ctx, a, GGML_UNARY_OP_GELU);
}
extern "C" struct ggml_tensor *ggml_silu(struct ggml_context *ctx, struct ggml_tensor *a) {
    return ggml_unary(ctx, a, GGML_UNARY_OP_SILU);
}
extern "C" struct ggml_tensor *ggml_relu(struct ggml_context *ctx, struct ggml_tensor *a) {
    return ggml_unary(ctx, a, GGML_UNARY_OP_RELU);
}
extern "C" enum ggml_unary_op ggml_get_unary_op(const struct ggml_tensor *t) {
    return (enum ggml_unary_op)t->op_params[0];
}

extern "C" struct ggml_tensor *ggml_soft_max_ext(struct ggml_context *ctx, struct ggml_tensor *a,
                                                 struct ggml_tensor *mask, float scale, float max_bias) {
    ggml_tensor *r = new_tensor(ctx, a->type, 4, a->ne);
    r->op = GGML_OP_SOFT_MAX;
    const float p[2] = {scale, max_bias};
    std::memcpy(r->op_params, p, sizeof(p));
    r->src[0] = a;
    r->src[1] = mask;
    return r;
}
extern "C" struct ggml_tensor *ggml_soft_max(struct ggml_context *ctx, struct ggml_tensor *a) {
    return ggml_soft_max_ext(ctx, a, nullptr, 1.0f, 0.0f);
}

extern "C" struct ggml_tensor *ggml_argsort(struct ggml_context *ctx, struct ggml_tensor *a,
                                            enum ggml_sort_order order) {
    ggml_tensor *r = new_tensor(ctx, GGML_TYPE_I32, 4, a->ne);
    r->op = GGML_OP_ARGSORT;
    r->op_params[0] = (int32_t)order;
    r->src[0] = a;
    return r;
}

extern "C" struct ggml_tensor *ggml_top_k(struct ggml_context *ctx, struct ggml_tensor *a, int k) {
    ggml_tensor *s = ggml_argsort(ctx, a, GGML_SORT_ORDER_DESC);
    const int64_t ne[4] = {k, s->ne[1], s->ne[2], s->ne[3]};
    return view_of(ctx, s, ne, s->nb, 0, GGML_OP_VIEW);
}

extern "C" struct ggml_tensor *ggml_repeat(struct ggml_context *ctx, struct ggml_tensor *a, struct ggml_tensor *b) {
    ggml_tensor *r = new_tensor(ctx, a->type, 4, b->ne);
    r->op = GGML_OP_REPEAT;
    r->src[0] = a;
    return r;
}

extern "C" struct ggml_tensor *ggml_rope_ext(struct ggml_context *ctx, struct ggml_tensor *a, struct ggml_tensor *b,
                                             struct ggml_tensor *c, int n_dims, int mode, int n_ctx_orig,
                                             float freq_base, float freq_scale, float ext_factor, float attn_factor,
                                             float beta_fast, float beta_slow) {
    ggml_tensor *r = new_tensor(ctx, a->type, 4, a->ne);
    r->op = GGML_OP_ROPE;
    const int32_t ip[5] = {0, n_dims, mode, 0, n_ctx_orig};
    std::memcpy(r->op_params, ip, sizeof(ip));
    const float fp[6] = {freq_base, freq_scale, ext_factor, attn_factor, beta_fast, beta_slow};
    std::memcpy(r->op_params + 5, fp, sizeof(fp));
    r->src[0] = a;
    r->src[1] = b;
    r->src[2] = c;
    return r;
}

extern "C" struct ggml_tensor *ggml_flash_attn_ext(struct ggml_context *ctx, struct ggml_tensor *q,
                                                   struct ggml_tensor *k, struct ggml_tensor *v,
                                                   struct ggml_tensor *mask, float scale, float max_bias,
                                                   float logit_softcap) {
    const int64_t ne[4] = {v->ne[0], q->ne[2], q->ne[1], q->ne[3]};
    ggml_tensor *r = new_tensor(ctx, GGML_TYPE_F32, 4, ne);
    r->op = GGML_OP_FLASH_ATTN_EXT;
    const float p[3] = {scale, max_bias, logit_softcap};
    std::memcpy(r->op_params, p, sizeof(p));
    r->src[0] = q;
    r->src[1] = k;
    r->src[2] = v;
    r->src[3] = mask;
    return r;
}

extern "C" struct ggml_cgraph *ggml_new_graph(struct ggml_context *ctx) {
    ggml_cgraph *g = new ggml_cgraph;
    ctx->graphs.push_back(g);
    return g;
}

extern "C" struct ggml_cgraph *ggml_new_graph_custom(struct ggml_context *ctx, size_t, bool) { return ggml_new_graph(ctx); }

static void visit(ggml_cgraph *g, ggml_tensor *t) {
    if (std::find(g->nodes.begin(), g->nodes.end(), t) != g->nodes.end()) return;
    if (std::find(g->leafs.begin(), g->leafs.end(), t) != g->leafs.end()) return;
    for (int i = 0; i < GGML_MAX_SRC; i++)
        if (t->src[i]) visit(g, t->src[i]);
    if (t->op == GGML_OP_NONE) g->leafs.push_back(t);
    else g->nodes.push_back(t);
}

extern "C" void ggml_build_forward_expand(struct ggml_cgraph *g, struct ggml_tensor *t) { visit(g, t); }

extern "C" struct ggml_tensor *ggml_graph_get_tensor(const struct ggml_cgraph *g, const char *name) {
    for (ggml_tensor *t : g->nodes)
        if (std::strcmp(t->name, name) == 0) return t;
    for (ggml_tensor *t : g->leafs)
        if (std::strcmp(t->name, name) == 0) return t;
    return nullptr;
}

extern "C" struct ggml_cgraph *ggml_compat_graph_view(struct ggml_cgraph *g, int i0, int i1) {
    ggml_cgraph *v = new ggml_cgraph;
    v->nodes.assign(g->nodes.begin() + i0, g->nodes.begin() + i1);
    v->leafs = g->leafs;
    v->parent = g->parent ? g->parent : g;
    return v;
}
extern "C" void ggml_compat_graph_view_free(struct ggml_cgraph *v) { delete v; }

extern "C" int ggml_node_get_use_count(const struct ggml_cgraph *g, int node_idx) {
    const ggml_tensor *t = g->nodes[node_idx];
    if (g->parent) g = g->parent;
    int n = 0;
    for (const ggml_tensor *u : g->nodes)
        for (int i = 0; i < GGML_MAX_SRC; i++)
            if (u->src[i] == t) n++;
    return n;
}
extern "C" int ggml_graph_n_nodes(struct ggml_cgraph *g) { return (int)g->nodes.size(); }
extern "C" struct ggml_tensor *ggml_graph_node(struct ggml_cgraph *g, int i) {
    if (i < 0) i += (int)g->nodes.size();
    return g->nodes[i];
}

// ---------------------------------------------------------------------------
// buffers, buffer types, backends, devices, registry
// ---------------------------------------------------------------------------
extern "C" ggml_backend_buffer_t ggml_backend_buffer_init(ggml_backend_buffer_type_t buft,
                                                           struct ggml_backend_buffer_i iface, void *context,
                                                           size_t size) {
    ggml_backend_buffer_t b = new ggml_backend_buffer;
    b->iface = iface;
    b->buft = buft;
    b->context = context;
    b->size = size;
    b->usage = GGML_BACKEND_BUFFER_USAGE_ANY;
    return b;
}

extern "C" const char *ggml_backend_buft_name(ggml_backend_buffer_type_t buft) { return buft->iface.get_name(buft); }
extern "C" ggml_backend_buffer_t ggml_backend_buft_alloc_buffer(ggml_backend_buffer_type_t buft, size_t size) {
    return buft->iface.alloc_buffer(buft, size);
}
extern "C" size_t ggml_backend_buft_get_alignment(ggml_backend_buffer_type_t buft) {
    return buft->iface.get_alignment(buft);
}
extern "C" size_t ggml_backend_buft_get_alloc_size(ggml_backend_buffer_type_t buft, const struct ggml_tensor *t) {
    return buft->iface.get_alloc_size ? buft->iface.get_alloc_size(buft, t) : ggml_nbytes(t);
}
extern "C" void ggml_backend_buffer_free(ggml_backend_buffer_t b) {
    if (!b) return;
    if (b->iface.free_buffer) b->iface.free_buffer(b);
    delete b;
}
extern "C" void *ggml_backend_buffer_get_base(ggml_backend_buffer_t b) { return b->iface.get_base(b); }
extern "C" size_t ggml_backend_buffer_get_size(ggml_backend_buffer_t b) { return b->size; }
extern "C" ggml_backend_buffer_type_t ggml_backend_buffer_get_type(ggml_backend_buffer_t b) { return b->buft; }
extern "C" void ggml_backend_buffer_clear(ggml_backend_buffer_t b, uint8_t v) {
    if (b->iface.clear) b->iface.clear(b, v);
}
extern "C" enum ggml_status ggml_backend_tensor_alloc(ggml_backend_buffer_t b, struct ggml_tensor *t, void *addr) {
    t->buffer = b;
    t->data = addr;
    return b->iface.init_tensor ? b->iface.init_tensor(b, t) : GGML_STATUS_SUCCESS;
}

static ggml_backend_buffer_t buffer_of(const ggml_tensor *t) { return t->view_src ? t->view_src->buffer : t->buffer; }

extern "C" void ggml_backend_tensor_set(struct ggml_tensor *t, const void *data, size_t offset, size_t size) {
    ggml_backend_buffer_t b = buffer_of(t);
    if (!b || offset + size > ggml_nbytes(t)) {
        std::fprintf(stderr, "ggml_backend_tensor_set: tensor '%s' not allocated or write out of bounds\n", t->name);
        std::abort();
    }
    if (size) b->iface.set_tensor(b, t, data, offset, size);
}

extern "C" void ggml_backend_tensor_get(const struct ggml_tensor *t, void *data, size_t offset, size_t size) {
    ggml_backend_buffer_t b = buffer_of(t);
    if (!b || offset + size > ggml_nbytes(t)) {
        std::fprintf(stderr, "ggml_backend_tensor_get: tensor '%s' not allocated or read out of bounds\n", t->name);
        std::abort();
    }
    if (size) b->iface.get_tensor(b, t, data, offset, size);
}

extern "C" const char *ggml_backend_name(ggml_backend_t be) { return be ? be->iface.get_name(be) : "NULL"; }
extern "C" void ggml_backend_free(ggml_backend_t be) {
    if (be) be->iface.free(be);
}
extern "C" ggml_backend_dev_t ggml_backend_get_device(ggml_backend_t be) { return be->device; }
extern "C" ggml_backend_buffer_type_t ggml_backend_get_default_buffer_type(ggml_backend_t be) {
    return be->device->iface.get_buffer_type(be->device);
}
extern "C" size_t ggml_backend_get_alignment(ggml_backend_t be) {
    return ggml_backend_buft_get_alignment(ggml_backend_get_default_buffer_type(be));
}
extern "C" void ggml_backend_synchronize(ggml_backend_t be) {
    if (be->iface.synchronize) be->iface.synchronize(be);
}
extern "C" enum ggml_status ggml_backend_graph_compute(ggml_backend_t be, struct ggml_cgraph *g) {
    const enum ggml_status st = be->iface.graph_compute(be, g);
    ggml_backend_synchronize(be);
    return st;
}
extern "C" bool ggml_backend_supports_op(ggml_backend_t be, const struct ggml_tensor *op) {
    return be->device->iface.supports_op(be->device, op);
}

extern "C" const char *ggml_backend_dev_name(ggml_backend_dev_t d) { return d->iface.get_name(d); }
extern "C" const char *ggml_backend_dev_description(ggml_backend_dev_t d) { return d->iface.get_description(d); }
extern "C" void ggml_backend_dev_memory(ggml_backend_dev_t d, size_t *free, size_t *total) {
    d->iface.get_memory(d, free, total);
}
extern "C" enum ggml_backend_dev_type ggml_backend_dev_type(ggml_backend_dev_t d) { return d->iface.get_type(d); }
extern "C" void ggml_backend_dev_get_props(ggml_backend_dev_t d, struct ggml_backend_dev_props *p) {
    std::memset(p, 0, sizeof(*p));
    d->iface.get_props(d, p);
}
extern "C" ggml_backend_reg_t ggml_backend_dev_backend_reg(ggml_backend_dev_t d) { return d->reg; }
extern "C" ggml_backend_t ggml_backend_dev_init(ggml_backend_dev_t d, const char *params) {
    return d->iface.init_backend(d, params);
}
extern "C" ggml_backend_buffer_type_t ggml_backend_dev_buffer_type(ggml_backend_dev_t d) {
    return d->iface.get_buffer_type(d);
}
extern "C" bool ggml_backend_dev_supports_op(ggml_backend_dev_t d, const struct ggml_tensor *op) {
    return d->iface.supports_op(d, op);
}
extern "C" bool ggml_backend_dev_supports_buft(ggml_backend_dev_t d, ggml_backend_buffer_type_t buft) {
    return d->iface.supports_buft(d, buft);
}

static std::vector<ggml_backend_reg_t> &registry() {
    static std::vector<ggml_backend_reg_t> regs;
    return regs;
}
extern "C" const char *ggml_backend_reg_name(ggml_backend_reg_t r) { return r->iface.get_name(r); }
extern "C" size_t ggml_backend_reg_dev_count(ggml_backend_reg_t r) { return r->iface.get_device_count(r); }
extern "C" ggml_backend_dev_t ggml_backend_reg_dev_get(ggml_backend_reg_t r, size_t i) {
    return r->iface.get_device(r, i);
}
extern "C" void *ggml_backend_reg_get_proc_address(ggml_backend_reg_t r, const char *name) {
    return r->iface.get_proc_address ? r->iface.get_proc_address(r, name) : nullptr;
}
extern "C" void ggml_backend_register(ggml_backend_reg_t r) {
    if (r && std::find(registry().begin(), registry().end(), r) == registry().end()) registry().push_back(r);
}
extern "C" size_t ggml_backend_reg_count(void) { return registry().size(); }
extern "C" ggml_backend_reg_t ggml_backend_reg_get(size_t i) { return registry().at(i); }
extern "C" size_t ggml_backend_dev_count(void) {
    size_t n = 0;
    for (auto r : registry()) n += ggml_backend_reg_dev_count(r);
    return n;
}
extern "C" ggml_backend_dev_t ggml_backend_dev_get(size_t i) {
    for (auto r : registry()) {
        const size_t n = ggml_backend_reg_dev_count(r);
        if (i < n) return ggml_backend_reg_dev_get(r, i);
        i -= n;
    }
    return nullptr;
}

// Allocate every not-yet-placed tensor of `ctx` in one buffer of the backend's
// default buffer type, each at an aligned offset sized by get_alloc_size.
extern "C" ggml_backend_buffer_t ggml_backend_alloc_ctx_tensors(struct ggml_context *ctx, ggml_backend_t be) {
    ggml_backend_buffer_type_t buft = ggml_backend_get_default_buffer_type(be);
    const size_t align = ggml_backend_buft_get_alignment(buft);
    auto pad = [&](size_t x) { return (x + align - 1) / align * align; };
    size_t total = 0;
    for (ggml_tensor *t : ctx->tensors)
        if (!t->data && !t->view_src) total += pad(ggml_backend_buft_get_alloc_size(buft, t));
    if (total == 0) return nullptr;
    ggml_backend_buffer_t b = ggml_backend_buft_alloc_buffer(buft, total);
    if (!b) return nullptr;
    char *base = (char *)ggml_backend_buffer_get_base(b);
    size_t off = 0;
    for (ggml_tensor *t : ctx->tensors) {
        if (t->data || t->view_src) continue;
        if (ggml_backend_tensor_alloc(b, t, base + off) != GGML_STATUS_SUCCESS) {
            ggml_backend_buffer_free(b);
            return nullptr;
        }
        off += pad(ggml_backend_buft_get_alloc_size(buft, t));
    }
    for (ggml_tensor *t : ctx->tensors) {
        if (t->view_src && !t->buffer) {
            t->buffer = t->view_src->buffer;
            t->data = (char *)t->view_src->data + t->view_offs;
        }
    }
    return b;
}
