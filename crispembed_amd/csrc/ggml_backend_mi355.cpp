// ggml_backend_mi355.cpp -- ggml backend that runs CrispEmbed's graphs on MI355X.
//
// Interface tables follow ggml-backend-impl.h.  The backend executes MUL_MAT on
// quantized weights (mq.h) and the other ops of the encoder graph
// (src/crispembed.cpp:1043-1468) through mq_ops.h: GET_ROWS, ADD / SUB / MUL / DIV,
// NORM / RMS_NORM, UNARY (GELU_ERF, GELU, SILU, RELU), CPY / CONT / DUP, ROPE
// (ggml_rope_ext, normal and NEOX), FLASH_ATTN_EXT, MUL_MAT_ID (mixture-of-experts on 3-D
// expert weights), SOFT_MAX, ARGSORT, REPEAT and MUL_MAT with an F32 first operand (the MoE
// block's router and expert mix), plus the metadata-only view ops.  Anything else is refused by
// supports_op, and ggml_backend_sched keeps it on the CPU backend, which is how
// CrispEmbed already falls back for ops a GPU backend rejects (src/crispembed.cpp:700-723).
//
// graph_compute fuses chains whose intermediate results have no other reader
// (ggml_node_get_use_count == 1) and are not graph outputs:
//   MUL_MAT [-> ADD(bias)], with the MUL_MATs after it on the same activation
//                                                  one grouped GEMM, biases added by its store
//   GET_ROWS, GET_ROWS, ADD [, GET_ROWS, ADD]      the embedding sum in one pass
//   FLASH_ATTN_EXT -> (views) -> MUL_MAT(Q8_0)     the attention also quantizes its result
//                                                  for the projection (mq_op_flash_attn_q8_0)
//   [ADD(residual) ->] NORM|RMS_NORM -> MUL(w) [-> ADD(b)]
//                                                  one row pass (mq_op_norm); before a Q8_0
//                                                  MUL_MAT it also quantizes the result for it
//                                                  (mq_op_norm_q8_0)
//   MUL_MAT -> ADD(bias) -> UNARY(GELU_ERF) -> MUL_MAT(Q8_0) [-> ADD(bias)]
//                                                  the first GEMM quantizes gelu(y + bias) for
//                                                  the second; the FFN intermediate is never written
//   ADD(bias) -> UNARY(GELU_ERF) -> MUL_MAT [-> ADD(bias)]
//                                                  bias and GELU applied while the activation
//                                                  is quantized for the mat-mul
// and MUL_MATs that read the same activation with the same weight type and shape
// one after another quantize it once.  MQ_GGML_NO_FUSION=1 runs every node on its own.
//
// Threading: like every ggml backend, one backend instance must be driven by one
// thread at a time (src/core/gpu_backend_pref.h:180-185); each instance owns one
// HIP stream (default priority) and one activation workspace.
#include <hip/hip_runtime.h>

#include <cstdio>
#include <cstdlib>
#include <algorithm>
#include <atomic>
#include <cstring>
#include <mutex>
#include <string>
#include <vector>

#include "ggml-backend-impl.h"
#include "ggml-impl.h"
#include "ggml-mi355.h"
#include "ggml.h"
#include "mq.h"
#include "mq_ops.h"

namespace {

void hip_check(hipError_t e, const char *what) {
    if (e != hipSuccess) {
        std::fprintf(stderr, "ggml-mi355: %s failed: %s\n", what, hipGetErrorString(e));
        std::abort();  // void ggml buffer callbacks cannot report errors (ggml's GGML_ABORT convention)
    }
}

struct DeviceCtx {
    int ordinal = 0;
    std::string name, description;
    ggml_backend_buffer_type buft{};
    ggml_backend_device dev{};
};

struct BufferCtx {
    int ordinal = 0;
    void *base = nullptr;
    size_t size = 0;
};

struct BackendCtx {
    int ordinal = 0;
    hipStream_t stream = nullptr;
    void *ws = nullptr;
    size_t ws_bytes = 0;
    std::string name;
    // what the workspace holds: the quantized activation of tensor ws_x for weight type
    // ws_type at ws_m x ws_k (ws_x NULL: nothing reusable)
    const ggml_tensor *ws_x = nullptr;
    int ws_type = -1, ws_path = 0;
    int64_t ws_m = 0, ws_k = 0;
    // the FLASH_ATTN_EXT node whose K/V fragments a q/k/v GEMM already stored at ws + kv_frag_off
    const ggml_tensor *kv_ready_for = nullptr;
    size_t kv_frag_off = 0;
    // HIP graph of the last graph computed twice in a row (its key: graph_key), replayed while
    // the same graph keeps coming back; seen_key is the graph computed eagerly last
    hipGraphExec_t gexec = nullptr;
    uint64_t gkey = 0, seen_key = 0;
    bool capturing = false;
    // q / k norm and rotation left to the attention: FLASH_ATTN_EXT node qk_fa reads q and k as
    // qk_q / qk_k (the inputs of their RMS_NORM -> MUL -> ROPE chains) with the norm weights
    // qk_qw / qk_kw and the rope cache cs
    const ggml_tensor *qk_fa = nullptr;
    mq_view qk_q{}, qk_k{};
    const float *qk_qw = nullptr, *qk_kw = nullptr;
    float qk_eps = 0.f;
    // the rope cache (cs_bytes of device memory) of the graph being computed, for the ROPE
    // parameters, positions and frequency factors cs_key names (empty: none yet)
    float *cs = nullptr;
    size_t cs_bytes = 0;
    std::vector<int64_t> cs_key;
    // the block lists (mq_op_mask_blocks, in mb_bytes of device memory) of FLASH_ATTN_EXT mask
    // mb_mask in the graph being computed: built at the first attention that reads the mask with
    // the shapes mb_key names, reused by the later ones (a decoder's every layer) until a node
    // writes the mask's bytes (mb_mask NULL: none)
    void *mb = nullptr;
    size_t mb_bytes = 0;
    const ggml_tensor *mb_mask = nullptr;
    std::vector<int64_t> mb_key;
    // the segment structure (mq_op_mask_segments) of mask sg_mask with the shapes sg_key in the
    // graph being computed: sg_len (0: none, the lists or the mask itself serve), found once
    // per graph, in sg_buf (sg_bytes of device scratch)
    void *sg_buf = nullptr;
    size_t sg_bytes = 0;
    const ggml_tensor *sg_mask = nullptr;
    std::vector<int64_t> sg_key;
    int64_t sg_len = 0;
    // whether mask mz_mask (shapes mz_key) adds nothing to the scores (mq_op_mask_is_zero), found
    // once per graph; mz_buf: its 4-byte flag on the device
    void *mz_buf = nullptr;
    const ggml_tensor *mz_mask = nullptr;
    std::vector<int64_t> mz_key;
    bool mz_zero = false;
    // ggml_backend_mi355_set_act_observer
    ggml_backend_mi355_act_observer act_cb = nullptr;
    void *act_user = nullptr;
    // gate|up weight images (the gate weight's rows, then the up weight's, planes built) of the
    // gated FFNs computed so far, for the gate|up GEMM that forms silu(gate) * up in its store;
    // each valid while no weight has been written since it was built (gen = weight_gen())
    struct GluImage {
        const void *gate, *up;
        uint64_t gen;
        void *img;
    };
    std::vector<GluImage> glu;
    // normed rows this graph left unwritten: their only readers are K-quant GEMMs that take the
    // Q8_K copy the norm left in the workspace (a reader that misses it fails loudly)
    std::vector<const ggml_tensor *> unwritten;
};

// Bumped by every write into a weight image (set_tensor, memset_tensor, cpy_tensor, clear, and
// the free of a buffer, whose addresses a later weight may reuse): derived copies of weights
// built before it are stale.
std::atomic<uint64_t> g_weight_gen{1};
uint64_t weight_gen() { return g_weight_gen.load(std::memory_order_acquire); }
void weights_written() { g_weight_gen.fetch_add(1, std::memory_order_acq_rel); }

std::vector<DeviceCtx *> &devices();
ggml_backend_reg &the_reg();

int mq_type_of(enum ggml_type t) {
    switch (t) {
        case GGML_TYPE_Q8_0: return MQ_TYPE_Q8_0;
        case GGML_TYPE_Q4_K: return MQ_TYPE_Q4_K;
        case GGML_TYPE_Q6_K: return MQ_TYPE_Q6_K;
        case GGML_TYPE_F16: return MQ_TYPE_F16;
        default: return -1;
    }
}

// any tensor type the graph ops read or write
int mq_type_any(enum ggml_type t) {
    switch (t) {
        case GGML_TYPE_F32: return MQ_TYPE_F32;
        case GGML_TYPE_I32: return MQ_TYPE_I32;
        default: return mq_type_of(t);
    }
}

// ggml metadata of a tensor as an mq_view.  Before allocation (supports_op) the view
// offset stands in for the address, so alignment checks see what allocation keeps
// (buffers and tensor offsets are 256-byte aligned).
mq_view view_of(const ggml_tensor *t) {
    mq_view v;
    v.data = t->data ? t->data : (void *)(uintptr_t)t->view_offs;
    v.type = mq_type_any(t->type);
    for (int i = 0; i < 4; i++) v.ne[i] = t->ne[i], v.nb[i] = t->nb[i];
    return v;
}

float op_param_f32(const ggml_tensor *t, int i) {
    float f;
    std::memcpy(&f, &t->op_params[i], sizeof(float));
    return f;
}

int unary_of(const ggml_tensor *t) {
    switch (ggml_get_unary_op(t)) {
        case GGML_UNARY_OP_GELU_ERF: return MQ_UNARY_GELU_ERF;
        case GGML_UNARY_OP_GELU: return MQ_UNARY_GELU;
        case GGML_UNARY_OP_SILU: return MQ_UNARY_SILU;
        case GGML_UNARY_OP_RELU: return MQ_UNARY_RELU;
        default: return -1;
    }
}

int binary_of(enum ggml_op op) {
    switch (op) {
        case GGML_OP_ADD: return MQ_BIN_ADD;
        case GGML_OP_SUB: return MQ_BIN_SUB;
        case GGML_OP_MUL: return MQ_BIN_MUL;
        case GGML_OP_DIV: return MQ_BIN_DIV;
        default: return -1;
    }
}

// A tensor whose allocation is a weight image: a supported weight type, 2-D,
// contiguous, not a view.  (F16 tensors qualify too: their image is the fp16
// rows plus the tiled copy the MFMA GEMM reads.)
bool is_image(const ggml_tensor *t) {
    const int mt = mq_type_of(t->type);
    return mt >= 0 && t->view_src == nullptr && t->ne[3] == 1 && ggml_is_contiguous(t) && mq_supports(mt, t->ne[0]) &&
           t->ne[1] > 0 && t->ne[2] > 0;
}

// A 3-D weight [k, n, n_exp] (the experts of MUL_MAT_ID) is allocated as n_exp weight images
// of image_bytes each, expert e at data + e * image_bytes; a 2-D weight is one image.  The
// GGUF byte offsets of set_tensor / get_tensor are mapped to the expert images, so readback
// still returns the GGUF bytes.
size_t image_bytes(const ggml_tensor *t) { return mq_weight_image_bytes(mq_type_of(t->type), t->ne[1], t->ne[0]); }

class DeviceGuard {
   public:
    explicit DeviceGuard(int dev) {
        hip_check(hipGetDevice(&prev_), "hipGetDevice");
        if (prev_ != dev) hip_check(hipSetDevice(dev), "hipSetDevice");
        dev_ = dev;
    }
    ~DeviceGuard() {
        if (prev_ != dev_) (void)hipSetDevice(prev_);
    }

   private:
    int prev_ = 0, dev_ = 0;
};

// ---------------------------------------------------------------- buffer ----
void buf_free(ggml_backend_buffer_t b) {
    BufferCtx *c = (BufferCtx *)b->context;
    DeviceGuard g(c->ordinal);
    (void)hipFree(c->base);
    delete c;
    weights_written();
}

void *buf_base(ggml_backend_buffer_t b) { return ((BufferCtx *)b->context)->base; }

enum ggml_status buf_init_tensor(ggml_backend_buffer_t, ggml_tensor *) { return GGML_STATUS_SUCCESS; }

// planes of the rows of expert e touched by GGUF bytes [offset, offset + size) of that expert
void rebuild_planes(ggml_tensor *t, int64_t e, size_t offset, size_t size) {
    const int mt = mq_type_of(t->type);
    const size_t rs = ggml_row_size(t->type, t->ne[0]);
    const int64_t r0 = (int64_t)(offset / rs), r1 = (int64_t)((offset + size + rs - 1) / rs);
    char *img = (char *)t->data + (size_t)e * image_bytes(t);
    weights_written();
    if (mq_weight_prepare(mt, img, t->ne[1], t->ne[0], r0, r1, nullptr) != 0) {
        std::fprintf(stderr, "ggml-mi355: weight preparation of '%s' failed: %s\n", t->name, mq_last_error());
        std::abort();
    }
    hip_check(hipStreamSynchronize(nullptr), "hipStreamSynchronize");
}

// Calls f(device address, tensor byte offset, bytes, expert) for the pieces of the tensor's
// byte range [offset, offset + size): one piece for plain tensors, one per expert image
// touched for weight images.
template <typename F>
void for_each_piece(ggml_tensor *t, size_t offset, size_t size, F f) {
    if (!is_image(t)) {
        f((char *)t->data + offset, (size_t)0, size, (int64_t)0, offset);
        return;
    }
    const size_t raw = ggml_row_size(t->type, t->ne[0]) * (size_t)t->ne[1], ib = image_bytes(t);
    size_t done = 0;
    while (done < size) {
        const size_t at = offset + done;
        const int64_t e = (int64_t)(at / raw);
        const size_t local = at - (size_t)e * raw, n = std::min(size - done, raw - local);
        f((char *)t->data + (size_t)e * ib + local, done, n, e, local);
        done += n;
    }
}

void buf_set_tensor(ggml_backend_buffer_t b, ggml_tensor *t, const void *data, size_t offset, size_t size) {
    BufferCtx *c = (BufferCtx *)b->context;
    DeviceGuard g(c->ordinal);
    for_each_piece(t, offset, size, [&](char *dev, size_t src_off, size_t n, int64_t e, size_t local) {
        hip_check(hipMemcpy(dev, (const char *)data + src_off, n, hipMemcpyHostToDevice), "hipMemcpy H2D");
        if (is_image(t)) rebuild_planes(t, e, local, n);
    });
}

void buf_get_tensor(ggml_backend_buffer_t b, const ggml_tensor *t, void *data, size_t offset, size_t size) {
    BufferCtx *c = (BufferCtx *)b->context;
    DeviceGuard g(c->ordinal);
    // hipMemcpy on the null stream waits for work queued on the (blocking) backend streams
    for_each_piece((ggml_tensor *)t, offset, size, [&](char *dev, size_t dst_off, size_t n, int64_t, size_t) {
        hip_check(hipMemcpy((char *)data + dst_off, dev, n, hipMemcpyDeviceToHost), "hipMemcpy D2H");
    });
}

void buf_memset_tensor(ggml_backend_buffer_t b, ggml_tensor *t, uint8_t value, size_t offset, size_t size) {
    BufferCtx *c = (BufferCtx *)b->context;
    DeviceGuard g(c->ordinal);
    for_each_piece(t, offset, size, [&](char *dev, size_t, size_t n, int64_t e, size_t local) {
        hip_check(hipMemset(dev, value, n), "hipMemset");
        if (is_image(t)) rebuild_planes(t, e, local, n);
    });
}

bool buf_cpy_tensor(ggml_backend_buffer_t b, const ggml_tensor *src, ggml_tensor *dst) {
    const ggml_backend_buffer_t sb = src->view_src ? src->view_src->buffer : src->buffer;
    if (!sb || sb->iface.free_buffer != buf_free) return false;  // only device-to-device within this backend
    BufferCtx *c = (BufferCtx *)b->context;
    DeviceGuard g(c->ordinal);
    if (is_image(src) != is_image(dst)) return false;  // layouts differ: the caller copies through the host
    if (is_image(dst)) {  // same type and shape: the whole images, planes included
        if (src->type != dst->type || src->ne[0] != dst->ne[0] || src->ne[1] != dst->ne[1] || src->ne[2] != dst->ne[2])
            return false;
        hip_check(hipMemcpy(dst->data, src->data, image_bytes(dst) * (size_t)dst->ne[2], hipMemcpyDeviceToDevice),
                  "hipMemcpy D2D");
        weights_written();
        return true;
    }
    hip_check(hipMemcpy(dst->data, src->data, ggml_nbytes(src), hipMemcpyDeviceToDevice), "hipMemcpy D2D");
    return true;
}

void buf_clear(ggml_backend_buffer_t b, uint8_t value) {
    BufferCtx *c = (BufferCtx *)b->context;
    DeviceGuard g(c->ordinal);
    hip_check(hipMemset(c->base, value, c->size), "hipMemset");
    hip_check(hipDeviceSynchronize(), "hipDeviceSynchronize");
    weights_written();
}

const ggml_backend_buffer_i kBufferIface = {
    buf_free, buf_base, buf_init_tensor, buf_memset_tensor, buf_set_tensor, buf_get_tensor, buf_cpy_tensor,
    buf_clear, nullptr,
};

// ----------------------------------------------------------- buffer type ----
const char *buft_name(ggml_backend_buffer_type_t buft) { return ((DeviceCtx *)buft->context)->name.c_str(); }

ggml_backend_buffer_t buft_alloc(ggml_backend_buffer_type_t buft, size_t size) {
    DeviceCtx *d = (DeviceCtx *)buft->context;
    DeviceGuard g(d->ordinal);
    void *p = nullptr;
    if (hipMalloc(&p, size ? size : 256) != hipSuccess) {
        (void)hipGetLastError();  // a failed allocation must not surface as the next launch's error
        std::fprintf(stderr, "ggml-mi355: failed to allocate %zu bytes on %s\n", size, d->name.c_str());
        return nullptr;  // the loader reports and fails (src/core/gguf_loader.cpp:408-415)
    }
    BufferCtx *c = new BufferCtx;
    c->ordinal = d->ordinal;
    c->base = p;
    c->size = size;
    return ggml_backend_buffer_init(buft, kBufferIface, c, size);
}

size_t buft_alignment(ggml_backend_buffer_type_t) { return 256; }  // weight images and workspaces need 256
size_t buft_max_size(ggml_backend_buffer_type_t) { return SIZE_MAX; }

size_t buft_alloc_size(ggml_backend_buffer_type_t, const ggml_tensor *t) {
    if (is_image(t)) return image_bytes(t) * (size_t)t->ne[2];
    return ggml_nbytes(t);
}

bool buft_is_host(ggml_backend_buffer_type_t) { return false; }

const ggml_backend_buffer_type_i kBuftIface = {buft_name, buft_alloc, buft_alignment, buft_max_size, buft_alloc_size,
                                               buft_is_host};

// --------------------------------------------------------------- backend ----
const char *be_name(ggml_backend_t be) { return ((BackendCtx *)be->context)->name.c_str(); }

void be_free(ggml_backend_t be) {
    BackendCtx *c = (BackendCtx *)be->context;
    {
        DeviceGuard g(c->ordinal);
        (void)hipStreamSynchronize(c->stream);
        if (c->gexec) (void)hipGraphExecDestroy(c->gexec);
        if (c->ws) (void)hipFree(c->ws);
        if (c->cs) (void)hipFree(c->cs);
        if (c->mb) (void)hipFree(c->mb);
        if (c->sg_buf) (void)hipFree(c->sg_buf);
        if (c->mz_buf) (void)hipFree(c->mz_buf);
        for (const BackendCtx::GluImage &gi : c->glu) (void)hipFree(gi.img);
        (void)hipStreamDestroy(c->stream);
    }
    delete c;
    delete be;
}

void be_synchronize(ggml_backend_t be) {
    BackendCtx *c = (BackendCtx *)be->context;
    DeviceGuard g(c->ordinal);
    hip_check(hipStreamSynchronize(c->stream), "hipStreamSynchronize");
}

bool is_view_op(enum ggml_op op) {
    return op == GGML_OP_NONE || op == GGML_OP_RESHAPE || op == GGML_OP_VIEW || op == GGML_OP_PERMUTE ||
           op == GGML_OP_TRANSPOSE;
}

// Rows of src1 / dst can be walked as one matrix of ne11*ne12*ne13 rows when
// their batch strides continue the row stride.
bool rows_flat(const ggml_tensor *t) {
    return t->nb[2] == t->nb[1] * (size_t)t->ne[1] && t->nb[3] == t->nb[2] * (size_t)t->ne[2];
}

bool ensure_ws(BackendCtx *c, size_t need) {
    if (need <= c->ws_bytes) return true;
    if (c->capturing) return false;  // no allocation under capture: the caller runs eagerly instead
    c->ws_x = nullptr;
    hip_check(hipStreamSynchronize(c->stream), "hipStreamSynchronize");
    if (c->gexec) {  // the captured graph holds the old workspace's address
        (void)hipGraphExecDestroy(c->gexec);
        c->gexec = nullptr;
        c->gkey = c->seen_key = 0;
    }
    if (c->ws) (void)hipFree(c->ws);
    c->ws = nullptr;
    c->ws_bytes = 0;
    if (hipMalloc(&c->ws, need) != hipSuccess) {
        (void)hipGetLastError();  // a failed allocation must not surface as the next launch's error
        c->ws = nullptr;
        std::fprintf(stderr, "ggml-mi355: workspace allocation of %zu bytes failed\n", need);
        return false;
    }
    c->ws_bytes = need;
    return true;
}

// Quantizes activation x (M rows of K floats, row stride in x->nb[1]) for weight type mt into
// the workspace, unless it is already there.  Returns an mq status.
int quantize_x(BackendCtx *c, const ggml_tensor *x, int mt, int64_t M, int64_t K, int path) {
    // Q4_K and Q6_K read the same tiled Q8_K activation
    const auto kq = [](int t) { return t == MQ_TYPE_Q4_K || t == MQ_TYPE_Q6_K; };
    const bool same = c->ws_type == mt || (path == MQ_PATH_GEMM && kq(c->ws_type) && kq(mt));
    if (c->ws_x == x && same && c->ws_m == M && c->ws_k == K && c->ws_path == path) return 0;
    if (std::find(c->unwritten.begin(), c->unwritten.end(), x) != c->unwritten.end()) {
        std::fprintf(stderr, "ggml-mi355: '%s' was left unwritten for the GEMMs that read its quantized copy, "
                     "which is gone (MQ_GGML_WRITE_NORMS=1 writes it)\n", x->name);
        return MQ_EINVAL;
    }
    c->ws_x = nullptr;
    if (!ensure_ws(c, mq_workspace_bytes(mt, M, K))) return MQ_ENOMEM;
    const int rc = mq_quantize_act_ex(mt, (const float *)x->data, (int64_t)(x->nb[1] / 4), M, K, nullptr, MQ_PRE_NONE,
                                      c->ws, c->ws_bytes, path, c->stream);
    if (rc == 0) c->ws_x = x, c->ws_type = mt, c->ws_m = M, c->ws_k = K, c->ws_path = path;
    return rc;
}

// The activation observer: the quantized activation `act` (mq_quantize_act_ex's layout for
// type mt, path) that the product at `node` is about to read, after the stream has finished
// writing it.
void observe_act(BackendCtx *c, const ggml_tensor *node, int mt, int64_t M, int64_t K, int path, const void *act) {
    if (!c->act_cb) return;
    hip_check(hipStreamSynchronize(c->stream), "hipStreamSynchronize");
    c->act_cb(node, mt, path, act, mq_workspace_bytes(mt, M, K), M, K, c->act_user);
}

// Decode-sized products on K-quant weights take mq_mul_mat_gemv: the GEMV quantizes its own
// activation, one launch instead of two (unless the activation is already quantized in the
// workspace, or a graph is being captured: that form may allocate on its first large input).
bool gemv_fused(const BackendCtx *c, const ggml_tensor *x, int mt, int64_t M, int64_t K, int path) {
    return path == MQ_PATH_GEMV && (mt == MQ_TYPE_Q4_K || mt == MQ_TYPE_Q6_K) && M <= 8 && K <= 6144 &&
           !c->capturing && !c->act_cb && c->ws_x != x && ((uintptr_t)x->data & 15) == 0 && (x->nb[1] / 4) % 4 == 0 &&
           std::getenv("MQ_GGML_NO_FUSION") == nullptr;
}

// y = x w^T (+ bias) into dst, for dst rows that continue one another (any row stride)
enum ggml_status mul_mat_flat(BackendCtx *c, const ggml_tensor *w, const ggml_tensor *x, ggml_tensor *dst,
                              const float *bias, const ggml_tensor *named) {
    const int mt = mq_type_of(w->type);
    const int64_t K = w->ne[0], N = w->ne[1], M = x->ne[1] * x->ne[2] * x->ne[3];
    const int path = mq_mul_mat_path(mt, N, K, M);
    if (gemv_fused(c, x, mt, M, K, path)) {
        const void *wi[1] = {w->data};
        const int64_t nn[1] = {N}, ld[1] = {(int64_t)(dst->nb[1] / 4)};
        float *yy[1] = {(float *)dst->data};
        const float *bb[1] = {bias};
        const int rc = mq_mul_mat_gemv(mt, 1, wi, nn, K, (const float *)x->data, (int64_t)(x->nb[1] / 4), nullptr, 0,
                                       MQ_PRE_NONE, M, yy, ld, bb, c->stream);
        if (rc != 0) {
            std::fprintf(stderr, "ggml-mi355: MUL_MAT '%s' failed: %s\n", named->name, mq_last_error());
            return rc == MQ_ENOMEM ? GGML_STATUS_ALLOC_FAILED : GGML_STATUS_FAILED;
        }
        return GGML_STATUS_SUCCESS;
    }
    int rc = quantize_x(c, x, mt, M, K, path);
    if (rc == 0) {
        observe_act(c, named, mt, M, K, path, c->ws);
        rc = mq_mul_mat_q_ex(mt, w->data, N, K, c->ws, M, (float *)dst->data, (int64_t)(dst->nb[1] / 4), bias, path,
                             c->stream);
    }
    if (rc != 0) {
        std::fprintf(stderr, "ggml-mi355: MUL_MAT '%s' failed: %s\n", named->name, mq_last_error());
        return rc == MQ_ENOMEM ? GGML_STATUS_ALLOC_FAILED : GGML_STATUS_FAILED;
    }
    return GGML_STATUS_SUCCESS;
}

enum ggml_status mul_mat(BackendCtx *c, ggml_tensor *dst) {
    const ggml_tensor *w = dst->src[0];
    const ggml_tensor *x = dst->src[1];
    if (rows_flat(x) && rows_flat(dst)) return mul_mat_flat(c, w, x, dst, nullptr, dst);
    // batches whose strides do not continue the rows: one mat-mul per (i2, i3)
    const int mt = mq_type_of(w->type);
    const int64_t K = w->ne[0], N = w->ne[1], M = x->ne[1];
    c->ws_x = nullptr;
    if (!ensure_ws(c, mq_workspace_bytes(mt, M, K))) return GGML_STATUS_ALLOC_FAILED;
    for (int64_t i3 = 0; i3 < x->ne[3]; i3++) {
        for (int64_t i2 = 0; i2 < x->ne[2]; i2++) {
            const float *xp = (const float *)((const char *)x->data + i2 * x->nb[2] + i3 * x->nb[3]);
            float *yp = (float *)((char *)dst->data + i2 * dst->nb[2] + i3 * dst->nb[3]);
            const int rc = mq_mul_mat(mt, w->data, N, K, xp, (int64_t)(x->nb[1] / 4), M, yp,
                                      (int64_t)(dst->nb[1] / 4), c->ws, c->ws_bytes, c->stream);
            if (rc != 0) {
                std::fprintf(stderr, "ggml-mi355: MUL_MAT '%s' failed: %s\n", dst->name, mq_last_error());
                return GGML_STATUS_FAILED;
            }
        }
    }
    return GGML_STATUS_SUCCESS;
}

enum ggml_status op_status(int rc, const ggml_tensor *node) {
    if (rc == 0) return GGML_STATUS_SUCCESS;
    std::fprintf(stderr, "ggml-mi355: %s '%s' failed: %s\n", ggml_op_name(node->op), node->name, mq_last_error());
    return GGML_STATUS_FAILED;
}

// a contiguous F32 vector of n floats, broadcast over rows (a norm weight or a bias)
bool is_row_vector(const ggml_tensor *t, int64_t n) {
    return t && t->type == GGML_TYPE_F32 && t->ne[0] == n && t->ne[1] == 1 && t->ne[2] == 1 && t->ne[3] == 1 &&
           t->nb[0] == sizeof(float);
}

// node i's result is read only by node i + 1 and is not a graph output
bool feeds_only_next(ggml_cgraph *cg, int i) {
    const ggml_tensor *t = ggml_graph_node(cg, i);
    return !(t->flags & GGML_TENSOR_FLAG_OUTPUT) && ggml_node_get_use_count(cg, i) == 1;
}

bool same_shape(const ggml_tensor *a, const ggml_tensor *b) {
    for (int i = 0; i < GGML_MAX_DIMS; i++)
        if (a->ne[i] != b->ne[i]) return false;
    return true;
}

bool flat_mul_mat(const ggml_tensor *mm);

// Node idx is the last node of the graph that computes anything (only views follow).  A
// MUL_MAT there may be observed: with an eval callback (the imatrix collector,
// src/imatrix.cpp:57-99, installed at src/crispembed.cpp:723) the scheduler computes the graph in
// pieces that end at each MUL_MAT it observes and then reads that MUL_MAT's src1.  So no fusion
// may leave the src1 of such a MUL_MAT unwritten.
bool last_compute_node(ggml_cgraph *cg, int idx, int n) {
    for (int j = idx + 1; j < n; j++) {
        const ggml_tensor *t = ggml_graph_node(cg, j);
        if (!ggml_is_empty(t) && !is_view_op(t->op)) return false;
    }
    return true;
}

// GET_ROWS(t0, i0), GET_ROWS(t1, i1), ADD [, GET_ROWS(t2, i2), ADD] from node i (the embedding
// sum), every intermediate read only by the next ADD: one mq_op_get_rows_sum.  Returns the
// nodes consumed.
int try_fuse_rows_sum(BackendCtx *c, ggml_cgraph *cg, int i, int n, enum ggml_status &st) {
    if (i + 2 >= n) return 0;
    ggml_tensor *g0 = ggml_graph_node(cg, i), *g1 = ggml_graph_node(cg, i + 1), *a1 = ggml_graph_node(cg, i + 2);
    auto gather_ok = [](const ggml_tensor *g) {
        return g->op == GGML_OP_GET_ROWS && g->src[0]->type == GGML_TYPE_F32 && g->src[1]->type == GGML_TYPE_I32;
    };
    auto single = [&](int idx) {
        return !(ggml_graph_node(cg, idx)->flags & GGML_TENSOR_FLAG_OUTPUT) && ggml_node_get_use_count(cg, idx) == 1;
    };
    if (!gather_ok(g0) || !gather_ok(g1) || a1->op != GGML_OP_ADD || a1->src[0] != g0 || a1->src[1] != g1 ||
        !single(i) || !single(i + 1))
        return 0;
    ggml_tensor *last = a1, *g2 = nullptr;
    int used = 3;
    if (i + 4 < n && single(i + 2)) {
        ggml_tensor *x2 = ggml_graph_node(cg, i + 3), *a2 = ggml_graph_node(cg, i + 4);
        if (gather_ok(x2) && a2->op == GGML_OP_ADD && a2->src[0] == a1 && a2->src[1] == x2 && single(i + 3)) {
            g2 = x2;
            last = a2;
            used = 5;
        }
    }
    if (!same_shape(last, g0) || !same_shape(g1, g0) || (g2 && !same_shape(g2, g0))) return 0;
    const mq_view t0 = view_of(g0->src[0]), t1 = view_of(g1->src[0]), i0 = view_of(g0->src[1]),
                  i1 = view_of(g1->src[1]), d = view_of(last);
    mq_view t2{}, i2{};
    if (g2) t2 = view_of(g2->src[0]), i2 = view_of(g2->src[1]);
    const mq_view *tabs[3] = {&t0, &t1, &t2}, *ids[3] = {&i0, &i1, &i2};
    const int rc = mq_op_get_rows_sum(g2 ? 3 : 2, tabs, ids, &d, c->stream);
    if (rc != 0) return 0;  // a layout this op does not take: the nodes run on their own
    st = GGML_STATUS_SUCCESS;
    return used;
}

bool overlaps(const ggml_tensor *a, const ggml_tensor *b);
const ggml_tensor *view_root(const ggml_tensor *t);

// RMS_NORM -> MUL(w [hd]) -> ROPE (NEOX over all hd dimensions) at node j, each result read only
// by the next node: the decoder's per-head q or k norm and rotation.  Returns the ROPE node.
ggml_tensor *qk_chain(ggml_cgraph *cg, int j, int n) {
    if (j + 2 >= n) return nullptr;
    ggml_tensor *nrm = ggml_graph_node(cg, j), *mul = ggml_graph_node(cg, j + 1), *rp = ggml_graph_node(cg, j + 2);
    if (nrm->op != GGML_OP_RMS_NORM || mul->op != GGML_OP_MUL || rp->op != GGML_OP_ROPE) return nullptr;
    if (mul->src[0] != nrm || rp->src[0] != mul || !feeds_only_next(cg, j) || !feeds_only_next(cg, j + 1))
        return nullptr;
    const int64_t hd = nrm->ne[0];
    if ((hd != 32 && hd != 64 && hd != 128) || rp->op_params[1] != hd || rp->op_params[2] != MQ_ROPE_NEOX)
        return nullptr;
    if (nrm->src[0]->type != GGML_TYPE_F32 || !is_row_vector(mul->src[1], hd) ||
        ((uintptr_t)mul->src[1]->data & 3) || (rp->flags & GGML_TENSOR_FLAG_OUTPUT))
        return nullptr;
    return rp;
}

// ggml_permute(t, 0, 2, 1, 3) of exactly t (judged by shape and strides)
bool is_head_permute(const ggml_tensor *p, const ggml_tensor *t) {
    return p && p->op == GGML_OP_PERMUTE && p->view_src == t && p->view_offs == 0 && p->ne[0] == t->ne[0] &&
           p->ne[1] == t->ne[2] && p->ne[2] == t->ne[1] && p->ne[3] == t->ne[3] && p->nb[0] == t->nb[0] &&
           p->nb[1] == t->nb[2] && p->nb[2] == t->nb[1] && p->nb[3] == t->nb[3];
}

// The q chain (qk_chain) at node i whose rotated q reaches a FLASH_ATTN_EXT only as its q
// (through the head permute), with k's chain further on feeding the same attention as its k,
// both with the same positions, ROPE parameters and eps: the six nodes are left to the
// attention (mq_op_flash_attn_qk_norm_rope reads q and k before the norms), and the rope cache
// of the positions is computed here (once per graph for the same positions and parameters).
// Returns the nodes consumed at i (3; k's are marked in done) or 0.
int try_defer_qk_norm_rope(BackendCtx *c, ggml_cgraph *cg, int i, int n, std::vector<char> &done) {
    ggml_tensor *rq = qk_chain(cg, i, n);
    if (!rq || c->qk_fa) return 0;
    int f = i + 3;
    while (f < n && ggml_graph_node(cg, f)->op != GGML_OP_FLASH_ATTN_EXT) f++;
    if (f >= n) return 0;
    ggml_tensor *fa = ggml_graph_node(cg, f);
    if (!is_head_permute(fa->src[0], rq)) return 0;
    ggml_tensor *rk = nullptr;
    int jk = i + 3;
    for (; jk < f; jk++)
        if ((rk = qk_chain(cg, jk, n)) && is_head_permute(fa->src[1], rk)) break;
    if (jk >= f) return 0;
    const ggml_tensor *nq = ggml_graph_node(cg, i), *nk = ggml_graph_node(cg, jk);
    const ggml_tensor *xq = nq->src[0], *xk = nk->src[0];
    if (std::memcmp(rq->op_params, rk->op_params, 15 * sizeof(int32_t)) != 0 || rq->src[1] != rk->src[1] ||
        rq->src[2] != rk->src[2] || op_param_f32(nq, 0) != op_param_f32(nk, 0) || fa->src[0]->ne[1] != fa->src[1]->ne[1])
        return 0;
    // nothing else reads the rotated q or k; no node that runs before the attention, nor the
    // attention's result, overwrites the chains' inputs (their buffers are free for reuse once
    // the RMS_NORM nodes have run, as the graph's allocator sees it)
    for (int u = i + 3; u < n; u++) {
        const ggml_tensor *t = ggml_graph_node(cg, u);
        if (t == fa || is_view_op(t->op)) continue;
        for (int si = 0; si < GGML_MAX_SRC; si++) {
            const ggml_tensor *r = view_root(t->src[si]);
            if (r && (r == rq || r == rk)) return 0;
        }
        // (k's chain is skipped; the products that compute q's and k's inputs may still follow)
        if (u < f && !(u >= jk && u < jk + 3) && !ggml_is_empty(t) &&
            ((t != view_root(xq) && overlaps(t, xq)) || (t != view_root(xk) && overlaps(t, xk))))
            return 0;
    }
    if (overlaps(fa, xq) || overlaps(fa, xk)) return 0;
    // q and k as the attention takes them: [hd, T, n_head, B], the head permute of the inputs
    auto permuted = [](const ggml_tensor *x) {
        mq_view v = view_of(x);
        std::swap(v.ne[1], v.ne[2]);
        std::swap(v.nb[1], v.nb[2]);
        return v;
    };
    const mq_view q = permuted(xq), k = permuted(xk), v = view_of(fa->src[2]), d = view_of(fa);
    mq_view m{};
    if (fa->src[3]) m = view_of(fa->src[3]);
    if (!mq_op_supported(MQ_OP_FLASH_ATTN, 0, &q, &k, &v, fa->src[3] ? &m : nullptr, &d)) return 0;
    // the rope cache: T positions x hd floats
    const int64_t T = rq->src[1]->ne[0], hd = nq->ne[0];
    if (T != q.ne[1]) return 0;
    std::vector<int64_t> key(rq->op_params, rq->op_params + 15);
    key.push_back((int64_t)(uintptr_t)rq->src[1]->data);
    key.push_back((int64_t)(uintptr_t)(rq->src[2] ? rq->src[2]->data : nullptr));
    key.push_back(T);
    if (key != c->cs_key) {
        const size_t need = (size_t)T * hd * sizeof(float);
        if (need > c->cs_bytes) {
            if (c->capturing) return 0;  // no allocation under capture: the nodes run on their own
            hip_check(hipStreamSynchronize(c->stream), "hipStreamSynchronize");
            if (c->gexec) {  // the captured graph holds the old table's address
                (void)hipGraphExecDestroy(c->gexec);
                c->gexec = nullptr;
                c->gkey = c->seen_key = 0;
            }
            if (c->cs) (void)hipFree(c->cs);
            c->cs = nullptr, c->cs_bytes = 0;
            if (hipMalloc((void **)&c->cs, need) != hipSuccess) {
                (void)hipGetLastError();
                c->cs = nullptr;
                return 0;
            }
            c->cs_bytes = need;
        }
        const mq_view pos = view_of(rq->src[1]);
        mq_view ff{};
        if (rq->src[2]) ff = view_of(rq->src[2]);
        const int32_t *ip = rq->op_params;
        if (mq_op_rope_cache(&pos, rq->src[2] ? &ff : nullptr, ip[1], ip[4], op_param_f32(rq, 5), op_param_f32(rq, 6),
                             op_param_f32(rq, 7), op_param_f32(rq, 8), op_param_f32(rq, 9), op_param_f32(rq, 10), c->cs,
                             c->stream) != 0)
            return 0;
        c->cs_key = key;
    }
    c->qk_fa = fa;
    c->qk_q = q, c->qk_k = k;
    c->qk_qw = (const float *)ggml_graph_node(cg, i + 1)->src[1]->data;
    c->qk_kw = (const float *)ggml_graph_node(cg, jk + 1)->src[1]->data;
    c->qk_eps = op_param_f32(nq, 0);
    done[jk] = done[jk + 1] = done[jk + 2] = 1;
    return 3;
}

// The block lists of mask mt (view m) for the attention of q and k: built once per graph and
// reused while the mask's bytes and the shapes stay (see BackendCtx::mb); NULL where the
// attention takes none, under capture before a buffer exists, or with MQ_GGML_NO_MASK_BLOCKS=1.
const void *mask_blocks(BackendCtx *c, const ggml_tensor *mt, const mq_view &q, const mq_view &k, const mq_view &m) {
    if (std::getenv("MQ_GGML_NO_MASK_BLOCKS")) return nullptr;
    const size_t need = mq_op_mask_blocks_bytes(&q, &k, &m);
    if (need == 0) return nullptr;
    std::vector<int64_t> key = {(int64_t)(uintptr_t)mt->data, q.ne[1], q.ne[2], q.ne[3], k.ne[1]};
    key.insert(key.end(), mt->ne, mt->ne + 4);
    key.insert(key.end(), mt->nb, mt->nb + 4);
    if (c->mb_mask == mt && key == c->mb_key) return c->mb;
    c->mb_mask = nullptr;
    if (need > c->mb_bytes) {
        if (c->capturing) return nullptr;  // no allocation under capture: the attention classifies itself
        hip_check(hipStreamSynchronize(c->stream), "hipStreamSynchronize");
        if (c->gexec) {  // the captured graph holds the old lists' address
            (void)hipGraphExecDestroy(c->gexec);
            c->gexec = nullptr;
            c->gkey = c->seen_key = 0;
        }
        if (c->mb) (void)hipFree(c->mb);
        c->mb = nullptr, c->mb_bytes = 0;
        if (hipMalloc(&c->mb, need) != hipSuccess) {
            (void)hipGetLastError();
            c->mb = nullptr;
            return nullptr;
        }
        c->mb_bytes = need;
    }
    if (mq_op_mask_blocks(&q, &k, &m, c->mb, c->mb_bytes, c->stream) != 0) return nullptr;
    c->mb_mask = mt, c->mb_key = key;
    return c->mb;
}

// The segment length of mask mt (view m) for the attention of q and k when the mask is exactly
// block-diagonal causal over segments of a multiple of 32 positions (a batched decoder's mask,
// decoder_encode_tokens_batch): found once per graph (a pass over the mask and a readback, which
// synchronizes the stream) and reused while the mask's bytes and the shapes stay; 0 otherwise,
// under capture, for masks the attention would not give block lists (small ones), or with
// MQ_GGML_NO_MASK_SEGMENTS=1.
int64_t mask_segments(BackendCtx *c, const ggml_tensor *mt, const mq_view &q, const mq_view &k, const mq_view &m) {
    if (std::getenv("MQ_GGML_NO_MASK_SEGMENTS") || c->capturing || q.ne[1] < 256) return 0;
    const size_t need = mq_op_mask_segments_bytes(&q, &k, &m);
    if (need == 0 || mq_op_mask_blocks_bytes(&q, &k, &m) == 0) return 0;
    std::vector<int64_t> key = {(int64_t)(uintptr_t)mt->data, q.ne[1], k.ne[1]};
    key.insert(key.end(), mt->ne, mt->ne + 4);
    key.insert(key.end(), mt->nb, mt->nb + 4);
    if (c->sg_mask == mt && key == c->sg_key) return c->sg_len;
    c->sg_mask = nullptr;
    if (need > c->sg_bytes) {
        hip_check(hipStreamSynchronize(c->stream), "hipStreamSynchronize");
        if (c->sg_buf) (void)hipFree(c->sg_buf);
        c->sg_buf = nullptr, c->sg_bytes = 0;
        if (hipMalloc(&c->sg_buf, need) != hipSuccess) {
            (void)hipGetLastError();
            c->sg_buf = nullptr;
            return 0;
        }
        c->sg_bytes = need;
    }
    int64_t S = 0;
    if (mq_op_mask_segments(&q, &k, &m, c->sg_buf, c->sg_bytes, &S, c->stream) != 0 || S % 32 != 0) S = 0;
    c->sg_mask = mt, c->sg_key = key, c->sg_len = S;
    return S;
}

// Whether mask tensor mt adds nothing to the scores of this attention (every value it reads +-0:
// an equal-length batch's padding mask), found once per graph with one flag read back; false
// under capture (no synchronization there) and with MQ_GGML_MASK_ALWAYS=1.
bool mask_zero(BackendCtx *c, const ggml_tensor *mt, const mq_view &q, const mq_view &k, const mq_view &m) {
    if (c->capturing || std::getenv("MQ_GGML_MASK_ALWAYS")) return false;
    std::vector<int64_t> key = {(int64_t)(uintptr_t)mt->data, q.ne[1], k.ne[1]};
    key.insert(key.end(), mt->ne, mt->ne + 4);
    key.insert(key.end(), mt->nb, mt->nb + 4);
    if (c->mz_mask == mt && key == c->mz_key) return c->mz_zero;
    c->mz_mask = nullptr;
    if (!c->mz_buf && hipMalloc(&c->mz_buf, 256) != hipSuccess) {
        (void)hipGetLastError();
        c->mz_buf = nullptr;
        return false;
    }
    int z = 0;
    if (mq_op_mask_is_zero(&q, &k, &m, c->mz_buf, 256, &z, c->stream) != 0) z = 0;
    c->mz_mask = mt, c->mz_key = key, c->mz_zero = z != 0;
    return c->mz_zero;
}

// The attention of FLASH_ATTN_EXT node fa: with q and k before their norm and rotation when those
// chains were left to it (c->qk_fa), else on its operands; per causal segment when the mask is a
// batched decoder's, else with the mask's block lists where the attention takes them; with its
// rows also quantized into act (act_bytes) for a projection on act_type weights when act is given.
int attn_call(BackendCtx *c, const ggml_tensor *fa, void *ws, size_t ws_bytes, void *act, size_t act_bytes,
              int act_type, int flags) {
    const mq_view v = view_of(fa->src[2]), d = view_of(fa);
    mq_view m{};
    if (fa->src[3]) m = view_of(fa->src[3]);
    const bool qk = c->qk_fa == fa;
    c->qk_fa = nullptr;
    const mq_view q = qk ? c->qk_q : view_of(fa->src[0]), k = qk ? c->qk_k : view_of(fa->src[1]);
    int64_t seg = 0;
    const void *blocks = nullptr;
    // a mask of zeros adds nothing: the attention runs unmasked (the same scores)
    const bool masked = fa->src[3] && !mask_zero(c, fa->src[3], q, k, m);
    if (masked && !(flags & MQ_ATTN_KV_READY)) seg = mask_segments(c, fa->src[3], q, k, m);
    if (masked && seg == 0) blocks = mask_blocks(c, fa->src[3], q, k, m);
    return mq_op_flash_attn_blocks(&q, &k, &v, masked ? &m : nullptr, &d, op_param_f32(fa, 0),
                                   qk ? c->qk_qw : nullptr, qk ? c->qk_kw : nullptr, qk ? c->qk_eps : 0.f,
                                   qk ? c->cs : nullptr, blocks, seg, ws, ws_bytes, act, act_bytes, act_type,
                                   qk ? 0 : flags, c->stream);
}

// [ADD(x, r) ->] NORM|RMS_NORM -> MUL(w) [-> ADD(b)] starting at node i: returns the number of
// nodes consumed (0: no match)
int try_fuse_norm(BackendCtx *c, ggml_cgraph *cg, int i, int n, enum ggml_status &st) {
    ggml_tensor *first = ggml_graph_node(cg, i);
    const ggml_tensor *res = nullptr;
    int j = i;
    // the residual sum has other readers (a pre-norm layer's residual stream): it is written too,
    // which the K-quant form below does
    bool add_shared = false;
    if (first->op == GGML_OP_ADD) {  // the residual sum feeding the norm
        if (i + 1 >= n) return 0;
        add_shared = !feeds_only_next(cg, i);
        const ggml_tensor *nx = ggml_graph_node(cg, i + 1);
        if ((nx->op != GGML_OP_NORM && nx->op != GGML_OP_RMS_NORM) || nx->src[0] != first) return 0;
        if (first->type != GGML_TYPE_F32 || !same_shape(first->src[0], first) || !same_shape(first->src[1], first))
            return 0;
        res = first->src[1];
        j = i + 1;
    }
    ggml_tensor *nrm = ggml_graph_node(cg, j);
    if (j + 1 >= n || !feeds_only_next(cg, j)) return 0;
    ggml_tensor *mul = ggml_graph_node(cg, j + 1);
    if (mul->op != GGML_OP_MUL || mul->src[0] != nrm || !is_row_vector(mul->src[1], nrm->ne[0])) return 0;
    const int kind0 = nrm->op == GGML_OP_NORM ? MQ_NORM_LAYER : MQ_NORM_RMS;
    // RMS_NORM -> MUL(w) -> ROPE: the decoder's per-head q / k norm and rotation in one pass
    if (!res && kind0 == MQ_NORM_RMS && j + 2 < n && feeds_only_next(cg, j + 1)) {
        ggml_tensor *rp = ggml_graph_node(cg, j + 2);
        const int32_t *ip = rp->op_params;
        if (rp->op == GGML_OP_ROPE && rp->src[0] == mul && ip[1] == 128 && ip[2] == MQ_ROPE_NEOX &&
            mul->ne[0] == 128 && ((uintptr_t)mul->src[1]->data & 3) == 0) {
            const mq_view x = view_of(nrm->src[0]), p = view_of(rp->src[1]), d = view_of(rp);
            mq_view f{};
            if (rp->src[2]) f = view_of(rp->src[2]);
            const int rc = mq_op_rms_norm_rope(&x, op_param_f32(nrm, 0), (const float *)mul->src[1]->data, &p,
                                               rp->src[2] ? &f : nullptr, &d, ip[1], ip[2], ip[4], op_param_f32(rp, 5),
                                               op_param_f32(rp, 6), op_param_f32(rp, 7), op_param_f32(rp, 8),
                                               op_param_f32(rp, 9), op_param_f32(rp, 10), c->stream);
            if (rc == 0) return (j - i) + 3;
            // shapes the fused op does not take run as the separate nodes
        }
    }
    ggml_tensor *last = mul;
    const float *b = nullptr;
    if (j + 2 < n && feeds_only_next(cg, j + 1)) {
        ggml_tensor *add = ggml_graph_node(cg, j + 2);
        if (add->op == GGML_OP_ADD && add->src[0] == mul && is_row_vector(add->src[1], nrm->ne[0])) {
            last = add;
            b = (const float *)add->src[1]->data;
        }
    }
    const int kind = nrm->op == GGML_OP_NORM ? MQ_NORM_LAYER : MQ_NORM_RMS;
    const mq_view x = view_of(res ? first->src[0] : nrm->src[0]), d = view_of(last);
    mq_view r{};
    if (res) r = view_of(res);
    if (!mq_op_supported(MQ_OP_NORM, kind, &x, res ? &r : nullptr, nullptr, nullptr, &d)) return 0;
    const int used = (j - i) + (last == mul ? 2 : 3);
    const float eps = op_param_f32(nrm, 0), *w = (const float *)mul->src[1]->data;
    // The next node that is not a view: when it is a Q8_0 MUL_MAT on the GEMM path reading this
    // result, the norm also leaves the result quantized in the workspace for it (mq_op_norm_q8_0),
    // and the activation cache lets that MUL_MAT (and its siblings) skip the quantizer.
    int nx = i + used;
    while (nx < n && (ggml_is_empty(ggml_graph_node(cg, nx)) || is_view_op(ggml_graph_node(cg, nx)->op))) nx++;
    const ggml_tensor *mm = nx < n ? ggml_graph_node(cg, nx) : nullptr;
    const int64_t K = last->ne[0], M = last->ne[1] * last->ne[2] * last->ne[3];
    auto dense = [K](const ggml_tensor *t) {
        return !t || (t->nb[0] == sizeof(float) && t->nb[1] == (size_t)K * sizeof(float) && rows_flat(t) &&
                      ((uintptr_t)t->data & 15) == 0);
    };
    // a K-quant MUL_MAT on the GEMM path reading an RMS norm's result (the decoder's attn / ffn
    // norms before q/k/v and gate/up): mq_op_norm_q8_K leaves it quantized to Q8_K, and writes
    // the residual sum when that has other readers
    const int mmt = (mm && mm->op == GGML_OP_MUL_MAT) ? mq_type_of(mm->src[0]->type) : -1;
    if (mm && (mmt == MQ_TYPE_Q4_K || mmt == MQ_TYPE_Q6_K) && mm->src[1] == last && flat_mul_mat(mm) &&
        kind == MQ_NORM_RMS && !b && K % 256 == 0 && K <= 2048 && dense(last) && dense(res) &&
        dense(res ? first->src[0] : nrm->src[0]) && (!add_shared || dense(first)) && ((uintptr_t)w & 15) == 0 &&
        mq_mul_mat_path(mmt, mm->src[0]->ne[1], K, M) == MQ_PATH_GEMM && ensure_ws(c, mq_workspace_bytes(mmt, M, K))) {
        mq_view sv{};
        if (add_shared) sv = view_of(first);
        c->ws_x = nullptr;
        // The normed rows themselves are left unwritten when every reader (all of the tensor's
        // uses, counted over the whole graph) is a K-quant MUL_MAT on the GEMM path taking them
        // as src1 -- they read the Q8_K copy -- and no observer or graph output wants the floats.
        bool skip_h = !c->act_cb && !(last->flags & GGML_TENSOR_FLAG_OUTPUT) && !std::getenv("MQ_GGML_WRITE_NORMS");
        if (skip_h) {
            int uses = 0;
            for (int jj = i + used; jj < n && skip_h; jj++) {
                const ggml_tensor *t = ggml_graph_node(cg, jj);
                bool reads = t->view_src == last;
                for (int q = 0; q < GGML_MAX_SRC; q++) reads = reads || t->src[q] == last;
                if (!reads) continue;
                const int tt = t->op == GGML_OP_MUL_MAT ? mq_type_of(t->src[0]->type) : -1;
                skip_h = (tt == MQ_TYPE_Q4_K || tt == MQ_TYPE_Q6_K) && t->src[1] == last && t->src[0] != last &&
                         flat_mul_mat(t) && t->src[0]->ne[0] == K && !last_compute_node(cg, jj, n) &&
                         mq_mul_mat_path(tt, t->src[0]->ne[1], K, M) == MQ_PATH_GEMM;
                uses++;
            }
            skip_h = skip_h && uses > 0 && uses == ggml_node_get_use_count(cg, i + used - 1);
        }
        const int rc = mq_op_norm_q8_K(kind, &x, res ? &r : nullptr, add_shared ? &sv : nullptr, skip_h ? nullptr : &d,
                                       eps, w, c->ws, c->ws_bytes, c->stream);
        if (rc == 0) c->ws_x = last, c->ws_type = mmt, c->ws_m = M, c->ws_k = K, c->ws_path = MQ_PATH_GEMM;
        if (rc == 0 && skip_h) c->unwritten.push_back(last);
        st = op_status(rc, nrm);
        return used;
    }
    if (add_shared) return 0;
    if (mm && mm->op == GGML_OP_MUL_MAT && mm->src[1] == last && mm->src[0]->type == GGML_TYPE_Q8_0 &&
        flat_mul_mat(mm) && K % 128 == 0 && K <= 1024 && dense(last) && dense(res) &&
        dense(res ? first->src[0] : nrm->src[0]) && ((uintptr_t)w & 15) == 0 && ((uintptr_t)b & 15) == 0 &&
        mq_mul_mat_path(MQ_TYPE_Q8_0, mm->src[0]->ne[1], K, M) == MQ_PATH_GEMM &&
        ensure_ws(c, mq_workspace_bytes(MQ_TYPE_Q8_0, M, K))) {
        const int rc = mq_op_norm_q8_0(kind, &x, res ? &r : nullptr, &d, eps, w, b, c->ws, c->ws_bytes, c->stream);
        if (rc == 0) c->ws_x = last, c->ws_type = MQ_TYPE_Q8_0, c->ws_m = M, c->ws_k = K, c->ws_path = MQ_PATH_GEMM;
        st = op_status(rc, nrm);
        return used;
    }
    st = op_status(mq_op_norm(kind, &x, res ? &r : nullptr, &d, eps, w, b, c->stream), nrm);
    return used;
}

// a MUL_MAT whose activation and result rows can be walked as one matrix
bool flat_mul_mat(const ggml_tensor *mm) {
    const ggml_tensor *x = mm->src[1];
    if (mq_type_of(mm->src[0]->type) < 0) return false;  // F32 weights: the small-product op
    return x->type == GGML_TYPE_F32 && x->nb[0] == sizeof(float) && x->nb[1] % sizeof(float) == 0 && rows_flat(x) &&
           rows_flat(mm) && mm->nb[0] == sizeof(float) && mm->nb[1] % sizeof(float) == 0;
}

// ADD(x, bias) -> UNARY(GELU_ERF) -> MUL_MAT(w, .) [-> ADD(., bias2)]: quantize
// gelu_erf(x + bias) straight into the mat-mul's activation workspace
int try_fuse_bias_gelu_mul_mat(BackendCtx *c, ggml_cgraph *cg, int i, int n, enum ggml_status &st) {
    ggml_tensor *add = ggml_graph_node(cg, i);
    if (i + 2 >= n || !feeds_only_next(cg, i) || !feeds_only_next(cg, i + 1)) return 0;
    ggml_tensor *gelu = ggml_graph_node(cg, i + 1), *mm = ggml_graph_node(cg, i + 2);
    if (gelu->op != GGML_OP_UNARY || ggml_get_unary_op(gelu) != GGML_UNARY_OP_GELU_ERF || gelu->src[0] != add) return 0;
    if (mm->op != GGML_OP_MUL_MAT || mm->src[1] != gelu) return 0;
    if (last_compute_node(cg, i + 2, n)) return 0;  // an observer may read the GELU result
    const ggml_tensor *x = add->src[0], *w = mm->src[0];
    const int64_t K = w->ne[0], N = w->ne[1];
    if (add->type != GGML_TYPE_F32 || x->type != GGML_TYPE_F32 || !is_row_vector(add->src[1], K) || x->ne[0] != K ||
        !same_shape(x, add))
        return 0;
    if (x->nb[0] != sizeof(float) || x->nb[1] % sizeof(float) || !rows_flat(x) || !flat_mul_mat(mm)) return 0;
    ggml_tensor *dst = mm;
    const float *bias2 = nullptr;
    if (i + 3 < n && feeds_only_next(cg, i + 2)) {
        ggml_tensor *a2 = ggml_graph_node(cg, i + 3);
        if (a2->op == GGML_OP_ADD && a2->src[0] == mm && is_row_vector(a2->src[1], N) && flat_mul_mat(mm) &&
            rows_flat(a2) && a2->nb[0] == sizeof(float) && a2->nb[1] % sizeof(float) == 0) {
            dst = a2;
            bias2 = (const float *)a2->src[1]->data;
        }
    }
    const int mt = mq_type_of(w->type);
    const int64_t M = x->ne[1] * x->ne[2] * x->ne[3];
    c->ws_x = nullptr;
    if (!ensure_ws(c, mq_workspace_bytes(mt, M, K))) {
        st = GGML_STATUS_ALLOC_FAILED;
        return 3;
    }
    const int path = mq_mul_mat_path(mt, N, K, M);
    int rc = mq_quantize_act_ex(mt, (const float *)x->data, (int64_t)(x->nb[1] / 4), M, K,
                                (const float *)add->src[1]->data, MQ_PRE_GELU_ERF, c->ws, c->ws_bytes, path, c->stream);
    if (rc == 0) {
        c->ws_x = gelu, c->ws_type = mt, c->ws_m = M, c->ws_k = K, c->ws_path = path;
        observe_act(c, mm, mt, M, K, path, c->ws);
        rc = mq_mul_mat_q_ex(mt, w->data, N, K, c->ws, M, (float *)dst->data, (int64_t)(dst->nb[1] / 4), bias2, path,
                             c->stream);
    }
    st = op_status(rc, mm);
    return dst == mm ? 3 : 4;
}

// MUL_MAT(w1, x) -> ADD(., bias) -> UNARY(GELU_ERF) -> MUL_MAT(w2, .) [-> ADD(., bias2)] with
// both products on the GEMM path (the encoder FFN) and a Q8_0 w2, or Q4_K / Q6_K w1 and w2 at
// the sizes the Q8_K-output GEMM accepts: the first GEMM adds the bias, applies GELU-erf and
// quantizes its own output for the second (mq_mul_mat_q_requant, the same bytes the activation
// quantizer would write), so the FFN's intermediate is never written.  The quantized
// intermediate sits in the workspace after x's quantized activation.
int try_fuse_ffn(BackendCtx *c, ggml_cgraph *cg, int i, int n, enum ggml_status &st) {
    if (i + 3 >= n || !feeds_only_next(cg, i) || !feeds_only_next(cg, i + 1) || !feeds_only_next(cg, i + 2)) return 0;
    ggml_tensor *mm1 = ggml_graph_node(cg, i), *add = ggml_graph_node(cg, i + 1);
    ggml_tensor *gelu = ggml_graph_node(cg, i + 2), *mm2 = ggml_graph_node(cg, i + 3);
    if (add->op != GGML_OP_ADD || add->src[0] != mm1 || add->type != GGML_TYPE_F32 || !same_shape(add, mm1)) return 0;
    if (gelu->op != GGML_OP_UNARY || ggml_get_unary_op(gelu) != GGML_UNARY_OP_GELU_ERF || gelu->src[0] != add) return 0;
    if (mm2->op != GGML_OP_MUL_MAT || mm2->src[1] != gelu || !flat_mul_mat(mm1) || !flat_mul_mat(mm2)) return 0;
    if (last_compute_node(cg, i + 3, n)) return 0;  // an observer may read the GELU result
    const ggml_tensor *w1 = mm1->src[0], *x = mm1->src[1], *w2 = mm2->src[0];
    const int64_t K1 = w1->ne[0], N1 = w1->ne[1], N2 = w2->ne[1];
    if (w2->ne[0] != N1 || !is_row_vector(add->src[1], N1)) return 0;
    const int mt1 = mq_type_of(w1->type), mt2 = mq_type_of(w2->type);
    const int64_t M = x->ne[1] * x->ne[2] * x->ne[3];
    if (!mq_mul_mat_q_requant_supported(mt1, mt2, M, N1)) return 0;
    if (mq_mul_mat_path(mt1, N1, K1, M) != MQ_PATH_GEMM || mq_mul_mat_path(mt2, N2, N1, M) != MQ_PATH_GEMM)
        return 0;
    ggml_tensor *dst = mm2;
    const float *bias2 = nullptr;
    if (i + 4 < n && feeds_only_next(cg, i + 3)) {
        ggml_tensor *a2 = ggml_graph_node(cg, i + 4);
        if (a2->op == GGML_OP_ADD && a2->src[0] == mm2 && is_row_vector(a2->src[1], N2) && rows_flat(a2) &&
            a2->nb[0] == sizeof(float) && a2->nb[1] % sizeof(float) == 0) {
            dst = a2;
            bias2 = (const float *)a2->src[1]->data;
        }
    }
    const size_t off = (mq_workspace_bytes(mt1, M, K1) + 255) & ~(size_t)255;
    if (!ensure_ws(c, off + mq_workspace_bytes(mt2, M, N1))) {
        st = GGML_STATUS_ALLOC_FAILED;
        return dst == mm2 ? 4 : 5;
    }
    void *ws2 = (char *)c->ws + off;
    int rc = quantize_x(c, x, mt1, M, K1, MQ_PATH_GEMM);
    if (rc == 0) {
        observe_act(c, mm1, mt1, M, K1, MQ_PATH_GEMM, c->ws);
        rc = mq_mul_mat_q_requant(mt1, w1->data, N1, K1, c->ws, M, (const float *)add->src[1]->data, MQ_PRE_GELU_ERF,
                                  mt2, ws2, c->ws_bytes - off, c->stream);
    }
    if (rc == 0) {
        observe_act(c, mm2, mt2, M, N1, MQ_PATH_GEMM, ws2);
        rc = mq_mul_mat_q_ex(mt2, w2->data, N2, N1, ws2, M, (float *)dst->data, (int64_t)(dst->nb[1] / 4), bias2,
                             MQ_PATH_GEMM, c->stream);
    }
    st = op_status(rc, mm1);
    return dst == mm2 ? 4 : 5;
}

// The gate|up image of gate weight wg and up weight wu (same type, n_ff x k each): built on first
// use from their GGUF rows (gate rows, then up rows, then the planes), rebuilt once a weight has
// been written since.  NULL under capture when it is not built yet (no allocation there).
void *glu_image(BackendCtx *c, const ggml_tensor *wg, const ggml_tensor *wu) {
    const uint64_t gen = weight_gen();
    for (size_t j = 0; j < c->glu.size(); j++) {
        BackendCtx::GluImage &gi = c->glu[j];
        if (gi.gate != wg->data || gi.up != wu->data) continue;
        if (gi.gen == gen) return gi.img;
        if (c->capturing) return nullptr;
        hip_check(hipStreamSynchronize(c->stream), "hipStreamSynchronize");  // queued work may read it
        (void)hipFree(gi.img);
        c->glu.erase(c->glu.begin() + (long)j);
        break;
    }
    if (c->capturing) return nullptr;
    const int mt = mq_type_of(wg->type);
    const int64_t nff = wg->ne[1], k = wg->ne[0];
    const size_t raw = ggml_row_size(wg->type, k) * (size_t)nff;
    void *img = nullptr;
    if (hipMalloc(&img, mq_weight_image_bytes(mt, 2 * nff, k)) != hipSuccess) {
        (void)hipGetLastError();
        return nullptr;
    }
    hip_check(hipMemcpyAsync(img, wg->data, raw, hipMemcpyDeviceToDevice, c->stream), "hipMemcpyAsync D2D");
    hip_check(hipMemcpyAsync((char *)img + raw, wu->data, raw, hipMemcpyDeviceToDevice, c->stream),
              "hipMemcpyAsync D2D");
    if (mq_weight_prepare(mt, img, 2 * nff, k, 0, 2 * nff, c->stream) != 0) {
        hip_check(hipStreamSynchronize(c->stream), "hipStreamSynchronize");
        (void)hipFree(img);
        return nullptr;
    }
    c->glu.push_back({wg->data, wu->data, gen, img});
    return img;
}

// MUL_MAT(w_gate, x) -> UNARY(SILU) -> MUL_MAT(w_up, x) -> MUL(silu, up), the gated FFN of
// src/decoder_embed.cpp:793-801 with separate gate and up weights, on the GEMM path at the sizes
// the gate|up GEMM takes (mq_mul_mat_q_swiglu): one GEMM over the gate|up image forms
// silu(gate) * up in its store, straight into the MUL's tensor; gate, its SiLU and up are never
// written (each has no other reader).  The product's values are those of the separate nodes.
int try_fuse_glu(BackendCtx *c, ggml_cgraph *cg, int i, int n, enum ggml_status &st) {
    if (i + 3 >= n) return 0;
    ggml_tensor *gate = ggml_graph_node(cg, i), *silu = ggml_graph_node(cg, i + 1);
    ggml_tensor *up = ggml_graph_node(cg, i + 2), *mul = ggml_graph_node(cg, i + 3);
    if (silu->op != GGML_OP_UNARY || ggml_get_unary_op(silu) != GGML_UNARY_OP_SILU || silu->src[0] != gate) return 0;
    if (up->op != GGML_OP_MUL_MAT || mul->op != GGML_OP_MUL) return 0;
    if (!((mul->src[0] == silu && mul->src[1] == up) || (mul->src[0] == up && mul->src[1] == silu))) return 0;
    // (with an activation observer installed the nodes run as they stand: its callers compare
    // the products' inputs and outputs node by node)
    if (!feeds_only_next(cg, i) || !feeds_only_next(cg, i + 1) || ggml_node_get_use_count(cg, i + 2) != 1 ||
        (up->flags & GGML_TENSOR_FLAG_OUTPUT) || i + 4 >= n || c->act_cb)
        return 0;
    const ggml_tensor *wg = gate->src[0], *wu = up->src[0], *x = gate->src[1];
    if (up->src[1] != x || !flat_mul_mat(gate) || !flat_mul_mat(up) || wg->type != wu->type || wg->ne[0] != wu->ne[0] ||
        wg->ne[1] != wu->ne[1] || !is_image(wg) || !is_image(wu) || wg->ne[2] != 1 || wu->ne[2] != 1)
        return 0;
    const int mt = mq_type_of(wg->type);
    const int64_t nff = wg->ne[1], K = wg->ne[0], M = x->ne[1] * x->ne[2] * x->ne[3];
    if ((mt != MQ_TYPE_Q4_K && mt != MQ_TYPE_Q6_K) || !same_shape(mul, gate) || mul->type != GGML_TYPE_F32 ||
        mul->nb[0] != sizeof(float) || !rows_flat(mul) || mul->nb[1] % sizeof(float) != 0)
        return 0;
    if (mq_mul_mat_path(mt, 2 * nff, K, M) != MQ_PATH_GEMM || !mq_mul_mat_q_swiglu_supported(mt, nff, M)) return 0;
    void *img = glu_image(c, wg, wu);
    if (!img) return 0;
    int rc = quantize_x(c, x, mt, M, K, MQ_PATH_GEMM);
    if (rc == 0)
        rc = mq_mul_mat_q_swiglu(mt, img, nff, K, c->ws, M, (float *)mul->data, (int64_t)(mul->nb[1] / 4), c->stream);
    st = op_status(rc, gate);
    return 4;
}

// UNARY(SILU)(gate) -> MUL_MAT(w_up, x) -> MUL(silu, up) -> MUL_MAT(w_down, product), the gated FFN
// of src/decoder_embed.cpp:793-802 with separate gate and up weights: the up projection runs as
// usual, then the down projection's activation is silu(gate) * up formed by its quantizer
// (mq_quantize_act_silu_mul), or for a decode-sized K-quant down projection inside its GEMV
// (mq_mul_mat_gemv, MQ_PRE_SILU_MUL).  Neither the SiLU's nor the product's tensor is written:
// both have no other reader, and the down projection must not be the graph's last node (an
// observer reads its src1).
enum ggml_status compute_node(BackendCtx *c, ggml_tensor *node);

int try_fuse_silu_mul(BackendCtx *c, ggml_cgraph *cg, int i, int n, const std::vector<char> &done,
                      enum ggml_status &st) {
    ggml_tensor *silu = ggml_graph_node(cg, i);
    if (ggml_get_unary_op(silu) != GGML_UNARY_OP_SILU || i + 3 >= n) return 0;
    ggml_tensor *up = ggml_graph_node(cg, i + 1), *mul = ggml_graph_node(cg, i + 2), *down = ggml_graph_node(cg, i + 3);
    if (up->op != GGML_OP_MUL_MAT || mul->op != GGML_OP_MUL || down->op != GGML_OP_MUL_MAT || down->src[1] != mul) return 0;
    if (!((mul->src[0] == silu && mul->src[1] == up) || (mul->src[0] == up && mul->src[1] == silu))) return 0;
    if (!feeds_only_next(cg, i) || ggml_node_get_use_count(cg, i + 1) != 1 || (up->flags & GGML_TENSOR_FLAG_OUTPUT) ||
        !feeds_only_next(cg, i + 2) || last_compute_node(cg, i + 3, n))
        return 0;
    const ggml_tensor *gate = silu->src[0];
    for (const ggml_tensor *t : {gate, (const ggml_tensor *)up, (const ggml_tensor *)silu, (const ggml_tensor *)mul})
        if (t->type != GGML_TYPE_F32 || !same_shape(t, gate) || t->nb[0] != sizeof(float) || !rows_flat(t)) return 0;
    if (gate->nb[1] != up->nb[1] || gate->nb[1] % sizeof(float) != 0 || !flat_mul_mat(up) || !flat_mul_mat(down)) return 0;
    const ggml_tensor *wd = down->src[0];
    const int mt = mq_type_of(wd->type);
    const int64_t K = wd->ne[0], N = wd->ne[1], M = mul->ne[1] * mul->ne[2] * mul->ne[3], ld = (int64_t)(gate->nb[1] / 4);
    if (mul->ne[0] != K || !mq_supports(mt, K)) return 0;
    const int path = mq_mul_mat_path(mt, N, K, M);
    const bool gemv = path == MQ_PATH_GEMV && (mt == MQ_TYPE_Q4_K || mt == MQ_TYPE_Q6_K) && M <= 8 && K <= 6144 &&
                      !c->capturing && !c->act_cb && ((uintptr_t)gate->data & 15) == 0 && ((uintptr_t)up->data & 15) == 0 && ld % 4 == 0;
    if (!done[i + 1]) {  // (done: computed already, grouped with the gate projection)
        st = compute_node(c, up);
        if (st != GGML_STATUS_SUCCESS) return 4;
    }
    int rc;
    if (gemv) {
        const void *wi[1] = {wd->data};
        const int64_t nn[1] = {N}, ldy[1] = {(int64_t)(down->nb[1] / 4)};
        float *yy[1] = {(float *)down->data};
        const float *bb[1] = {nullptr};
        rc = mq_mul_mat_gemv(mt, 1, wi, nn, K, (const float *)gate->data, ld, (const float *)up->data, ld,
                             MQ_PRE_SILU_MUL, M, yy, ldy, bb, c->stream);
    } else {
        c->ws_x = nullptr;  // the workspace receives the product
        if (!ensure_ws(c, mq_workspace_bytes(mt, M, K))) {
            st = GGML_STATUS_ALLOC_FAILED;
            return 4;
        }
        rc = mq_quantize_act_silu_mul(mt, (const float *)gate->data, (const float *)up->data, ld, M, K, c->ws,
                                      c->ws_bytes, path, c->stream);
        if (rc == 0) {
            c->ws_x = mul, c->ws_type = mt, c->ws_m = M, c->ws_k = K, c->ws_path = path;
            st = mul_mat_flat(c, wd, mul, down, nullptr, down);
            return 4;
        }
    }
    st = op_status(rc, down);
    return 4;
}

// FLASH_ATTN_EXT whose result (after view nodes, as rows of n_head * head_dim) is read by a
// Q8_0, Q4_K or Q6_K MUL_MAT on the GEMM path (the output projection): the attention also leaves
// it quantized for that MUL_MAT (Q8_0, or Q8_K for the K-quants: by the attention kernel's own
// store where its form has one, else by the quantizer right after it) and the activation cache
// lets the MUL_MAT skip the quantizer.  The quantized rows sit at the workspace start, the K/V
// fragments after them.
int try_fuse_attn(BackendCtx *c, ggml_cgraph *cg, int i, int n, enum ggml_status &st) {
    ggml_tensor *node = ggml_graph_node(cg, i);
    int nx = i + 1;
    while (nx < n && (ggml_is_empty(ggml_graph_node(cg, nx)) || is_view_op(ggml_graph_node(cg, nx)->op))) nx++;
    if (nx >= n) return 0;
    const ggml_tensor *mm = ggml_graph_node(cg, nx);
    const int mt = mm->op == GGML_OP_MUL_MAT ? mq_type_of(mm->src[0]->type) : -1;
    if ((mt != MQ_TYPE_Q8_0 && mt != MQ_TYPE_Q4_K && mt != MQ_TYPE_Q6_K) || !flat_mul_mat(mm)) return 0;
    const ggml_tensor *x = mm->src[1];
    if (x != node && (x->view_src != node || x->view_offs != 0)) return 0;
    const int64_t K = x->ne[0], M = x->ne[1] * x->ne[2] * x->ne[3];
    if (K != node->ne[0] * node->ne[1] || M != node->ne[2] * node->ne[3] || K % (mt == MQ_TYPE_Q8_0 ? 128 : 256) != 0 ||
        x->nb[1] != (size_t)K * sizeof(float) || node->nb[1] != (size_t)node->ne[0] * sizeof(float) ||
        node->nb[2] != (size_t)K * sizeof(float) || node->nb[3] != node->nb[2] * (size_t)node->ne[2])
        return 0;
    if (mq_mul_mat_path(mt, mm->src[0]->ne[1], K, M) != MQ_PATH_GEMM) return 0;
    const mq_view k = view_of(node->src[1]);
    const size_t act = (mq_workspace_bytes(mt, M, K) + 255) & ~(size_t)255;
    const bool ready = c->kv_ready_for == node;  // K/V fragments stored by the q/k/v GEMM
    const size_t foff = ready ? c->kv_frag_off : act;
    c->kv_ready_for = nullptr;
    c->ws_x = nullptr;
    if ((ready && foff < act) || !ensure_ws(c, foff + mq_op_flash_attn_workspace_bytes(&k))) {
        st = GGML_STATUS_ALLOC_FAILED;
        return 1;
    }
    const int rc = attn_call(c, node, (char *)c->ws + foff, c->ws_bytes - foff, c->ws, act, mt,
                             ready ? MQ_ATTN_KV_READY : 0);
    if (rc == 0) c->ws_x = x, c->ws_type = mt, c->ws_m = M, c->ws_k = K, c->ws_path = MQ_PATH_GEMM;
    st = op_status(rc, node);
    return 1;
}

// A MUL_MAT of a group and the bias ADD fused into its store (add_idx < 0: none).
// true when the bytes of tensor a and tensor b overlap
bool overlaps(const ggml_tensor *a, const ggml_tensor *b) {
    const char *a0 = (const char *)a->data, *b0 = (const char *)b->data;
    return a0 && b0 && a0 < b0 + ggml_nbytes(b) && b0 < a0 + ggml_nbytes(a);
}

struct MulMatMember {
    ggml_tensor *mm, *dst;
    const float *bias;
    int idx, add_idx;
};

// MUL_MAT j with the ADD(., bias) that follows it, when the ADD can go into the store.  Left
// alone when the ADD starts a bias -> GELU_ERF -> MUL_MAT chain (that fusion saves more).
MulMatMember mul_mat_member(ggml_cgraph *cg, int j, int n) {
    ggml_tensor *mm = ggml_graph_node(cg, j);
    MulMatMember m{mm, mm, nullptr, j, -1};
    if (j + 1 >= n || !feeds_only_next(cg, j)) return m;
    ggml_tensor *add = ggml_graph_node(cg, j + 1);
    if (add->op != GGML_OP_ADD || add->src[0] != mm || !is_row_vector(add->src[1], mm->src[0]->ne[1])) return m;
    if (!rows_flat(add) || add->nb[0] != sizeof(float) || add->nb[1] % sizeof(float)) return m;
    if (j + 3 < n && feeds_only_next(cg, j + 1)) {
        const ggml_tensor *u = ggml_graph_node(cg, j + 2), *m2 = ggml_graph_node(cg, j + 3);
        if (u->op == GGML_OP_UNARY && ggml_get_unary_op(u) == GGML_UNARY_OP_GELU_ERF && u->src[0] == add &&
            m2->op == GGML_OP_MUL_MAT && m2->src[1] == u)
            return m;
    }
    m.dst = add;
    m.bias = (const float *)add->src[1]->data;
    m.add_idx = j + 1;
    return m;
}

// MUL_MAT [-> ADD(bias)] at node i and the MUL_MATs after it (within 32 nodes) that read the same
// activation with the same weight type and k (q, k and v of a layer; a gated FFN's gate and up):
// one activation quantization and one grouped launch.  Returns the nodes
// consumed from i on; the later members (and their ADDs) are marked in `done`.
const ggml_tensor *view_root(const ggml_tensor *t) {
    while (t && t->view_src) t = t->view_src;
    return t;
}

// The FLASH_ATTN_EXT that is the next non-view node after a q, k, v group and the only reader of
// k's and v's results (through reshape / permute views of ggml's [head_dim, T, n_kv_head, B]
// form over dense rows), or NULL.  Sets T, head_dim and n_kv_head.
const ggml_tensor *qkv_attention(ggml_cgraph *cg, const MulMatMember *mem, int nm, int n, int64_t M, int &T, int &hd,
                                 int &nkv) {
    if (nm != 3) return nullptr;
    int j = (mem[2].add_idx >= 0 ? mem[2].add_idx : mem[2].idx) + 1;
    while (j < n && (ggml_is_empty(ggml_graph_node(cg, j)) || is_view_op(ggml_graph_node(cg, j)->op))) j++;
    if (j >= n) return nullptr;
    const ggml_tensor *fa = ggml_graph_node(cg, j);
    if (fa->op != GGML_OP_FLASH_ATTN_EXT) return nullptr;
    for (int g = 1; g <= 2; g++) {
        const ggml_tensor *r = mem[g].dst, *t = fa->src[g];
        const int idx = mem[g].add_idx >= 0 ? mem[g].add_idx : mem[g].idx;
        if (view_root(t) != r || t->data != r->data || (r->flags & GGML_TENSOR_FLAG_OUTPUT) ||
            ggml_node_get_use_count(cg, idx) != 1)
            return nullptr;
        if (t->ne[0] != 32 && t->ne[0] != 64 && t->ne[0] != 128) return nullptr;
        if (t->ne[1] % 32 != 0 || t->ne[1] * t->ne[3] != M || t->ne[0] * t->ne[2] != r->ne[0]) return nullptr;
        if (t->nb[0] != sizeof(float) || t->nb[1] != r->nb[1] || r->nb[1] != (size_t)r->ne[0] * sizeof(float) ||
            t->nb[2] != (size_t)t->ne[0] * sizeof(float) || t->nb[3] != t->nb[1] * (size_t)t->ne[1])
            return nullptr;
    }
    if (fa->src[1]->ne[0] != fa->src[2]->ne[0] || fa->src[1]->ne[2] != fa->src[2]->ne[2]) return nullptr;
    // nothing else reads k or v, through any view
    for (int q = mem[0].idx + 1; q < n; q++) {
        const ggml_tensor *u = ggml_graph_node(cg, q);
        if (u == fa || is_view_op(u->op)) continue;
        for (int si = 0; si < GGML_MAX_SRC; si++) {
            const ggml_tensor *r = view_root(u->src[si]);
            if (r && (r == mem[1].dst || r == mem[2].dst) && u != mem[1].dst && u != mem[2].dst) return nullptr;
        }
    }
    T = (int)fa->src[1]->ne[1], hd = (int)fa->src[1]->ne[0], nkv = (int)fa->src[1]->ne[2];
    return fa;
}

int try_group_mul_mat(BackendCtx *c, ggml_cgraph *cg, int i, int n, std::vector<char> &done, enum ggml_status &st) {
    ggml_tensor *mm = ggml_graph_node(cg, i);
    if (!flat_mul_mat(mm)) return 0;
    const ggml_tensor *x = mm->src[1], *w0 = mm->src[0];
    MulMatMember mem[4];
    int nm = 0;
    mem[nm++] = mul_mat_member(cg, i, n);
    // Later members may also sit behind other nodes (a decoder's q is normed and rotated before
    // its k product).  Such a member is computed ahead of those nodes, which is safe when none of
    // them reads or writes the member's output bytes (ggml-alloc may have given them memory the
    // member's output reuses) or writes the activation's bytes.
    std::vector<const ggml_tensor *> between;
    auto clashes = [&](const MulMatMember &m) {
        for (const ggml_tensor *b : between) {
            if (overlaps(b, m.mm) || overlaps(b, m.dst) || overlaps(b, x)) return true;
            for (int k = 0; k < GGML_MAX_SRC; k++)
                if (b->src[k] && (overlaps(b->src[k], m.mm) || overlaps(b->src[k], m.dst))) return true;
        }
        return false;
    };
    const int scan_end = std::min(n, i + 32);
    for (int j = (mem[0].add_idx >= 0 ? mem[0].add_idx : i) + 1; j < scan_end && nm < 4; j++) {
        ggml_tensor *t = ggml_graph_node(cg, j);
        if (is_view_op(t->op) || ggml_is_empty(t)) continue;
        if (t->op != GGML_OP_MUL_MAT || done[j] || t->src[1] != x || t->src[0]->type != w0->type ||
            t->src[0]->ne[0] != w0->ne[0] || !flat_mul_mat(t)) {
            if (t->op == GGML_OP_FLASH_ATTN_EXT || t->op == GGML_OP_MUL_MAT_ID) break;  // workspace users
            between.push_back(t);
            continue;
        }
        const MulMatMember m = mul_mat_member(cg, j, n);
        if (!between.empty() && clashes(m)) break;
        mem[nm] = m;
        if (mem[nm].add_idx >= 0) j = mem[nm].add_idx;
        nm++;
    }
    if (nm == 1 && mem[0].add_idx < 0) return 0;  // a lone MUL_MAT: the plain path
    const int mt = mq_type_of(w0->type);
    const int64_t K = w0->ne[0], M = x->ne[1] * x->ne[2] * x->ne[3];
    const void *w[4];
    int64_t nn[4], ldy[4];
    float *y[4];
    const float *b[4];
    for (int g = 0; g < nm; g++) {
        w[g] = mem[g].mm->src[0]->data;
        nn[g] = mem[g].mm->src[0]->ne[1];
        y[g] = (float *)mem[g].dst->data;
        ldy[g] = (int64_t)(mem[g].dst->nb[1] / sizeof(float));
        b[g] = mem[g].bias;
    }
    int64_t n_all = 0;
    for (int g = 0; g < nm; g++) n_all += nn[g];
    const int path = mq_mul_mat_path(mt, n_all, K, M);
    int rc = 1;
    int T = 0, hd = 0, nkv = 0;
    const ggml_tensor *fa = path == MQ_PATH_GEMM ? qkv_attention(cg, mem, nm, n, M, T, hd, nkv) : nullptr;
    if (fa) {
        // k and v go straight into the attention's fragments, after the quantized activations
        const mq_view kv = view_of(fa->src[1]);
        const size_t a1 = mq_workspace_bytes(mt, M, K), a2 = mq_workspace_bytes(MQ_TYPE_Q8_0, M, fa->ne[0] * fa->ne[1]);
        const size_t off = ((a1 > a2 ? a1 : a2) + 255) & ~(size_t)255, fb = mq_op_flash_attn_workspace_bytes(&kv);
        if (ensure_ws(c, off + fb)) {
            rc = quantize_x(c, x, mt, M, K, path);
            if (rc == 0)
                for (int g = 0; g < nm; g++) observe_act(c, mem[g].mm, mt, M, K, path, c->ws);
            if (rc == 0)
                rc = mq_mul_mat_q_qkv(mt, w, nn, K, c->ws, M, y[0], ldy[0], b, T, hd, nkv, (char *)c->ws + off, fb,
                                      c->stream);
            if (rc == 0) c->kv_ready_for = fa, c->kv_frag_off = off;
        }
    }
    if (rc == 1 && nm <= 3 && gemv_fused(c, x, mt, M, K, path))
        rc = mq_mul_mat_gemv(mt, nm, w, nn, K, (const float *)x->data, (int64_t)(x->nb[1] / 4), nullptr, 0, MQ_PRE_NONE,
                             M, y, ldy, b, c->stream);
    if (rc == 1) {
        rc = quantize_x(c, x, mt, M, K, path);
        if (rc == 0)
            for (int g = 0; g < nm; g++) observe_act(c, mem[g].mm, mt, M, K, path, c->ws);
        if (rc == 0) rc = mq_mul_mat_q_group(mt, nm, w, nn, K, c->ws, M, y, ldy, b, path, c->stream);
    }
    if (rc != 0) {
        std::fprintf(stderr, "ggml-mi355: MUL_MAT '%s' (%d grouped) failed: %s\n", mm->name, nm, mq_last_error());
        st = rc == MQ_ENOMEM ? GGML_STATUS_ALLOC_FAILED : GGML_STATUS_FAILED;
    }
    for (int g = 1; g < nm; g++) {
        done[mem[g].idx] = 1;
        if (mem[g].add_idx >= 0) done[mem[g].add_idx] = 1;
    }
    return mem[0].add_idx >= 0 ? 2 : 1;
}

enum ggml_status compute_node(BackendCtx *c, ggml_tensor *node) {
    switch (node->op) {
        case GGML_OP_MUL_MAT:
            if (node->src[0]->type == GGML_TYPE_F32) {  // the small F32 products (router, expert mix)
                const mq_view a = view_of(node->src[0]), b = view_of(node->src[1]), d = view_of(node);
                return op_status(mq_op_mul_mat_f32(&a, &b, &d, c->stream), node);
            }
            return mul_mat(c, node);
        case GGML_OP_GET_ROWS: {
            const mq_view a = view_of(node->src[0]), b = view_of(node->src[1]), d = view_of(node);
            return op_status(mq_op_get_rows(&a, &b, &d, c->stream), node);
        }
        case GGML_OP_ADD:
        case GGML_OP_SUB:
        case GGML_OP_MUL:
        case GGML_OP_DIV: {
            const mq_view a = view_of(node->src[0]), b = view_of(node->src[1]), d = view_of(node);
            return op_status(mq_op_binary(binary_of(node->op), &a, &b, &d, c->stream), node);
        }
        case GGML_OP_NORM:
        case GGML_OP_RMS_NORM: {
            const mq_view x = view_of(node->src[0]), d = view_of(node);
            return op_status(mq_op_norm(node->op == GGML_OP_NORM ? MQ_NORM_LAYER : MQ_NORM_RMS, &x, nullptr, &d,
                                        op_param_f32(node, 0), nullptr, nullptr, c->stream),
                             node);
        }
        case GGML_OP_UNARY: {
            const mq_view x = view_of(node->src[0]), d = view_of(node);
            return op_status(mq_op_unary(unary_of(node), &x, &d, c->stream), node);
        }
        case GGML_OP_CPY:
        case GGML_OP_CONT:
        case GGML_OP_DUP: {
            // CPY writes into its second source (the result is a view of it)
            const mq_view s = view_of(node->src[0]), d = view_of(node->op == GGML_OP_CPY ? node->src[1] : node);
            return op_status(mq_op_cpy(&s, &d, c->stream), node);
        }
        case GGML_OP_SOFT_MAX: {
            const mq_view x = view_of(node->src[0]), d = view_of(node);
            mq_view m{};
            if (node->src[1]) m = view_of(node->src[1]);
            return op_status(mq_op_soft_max(&x, node->src[1] ? &m : nullptr, &d, op_param_f32(node, 0), c->stream), node);
        }
        case GGML_OP_ARGSORT: {
            const mq_view x = view_of(node->src[0]), d = view_of(node);
            return op_status(mq_op_argsort(&x, &d, node->op_params[0] == GGML_SORT_ORDER_DESC ? MQ_SORT_DESC : MQ_SORT_ASC,
                                           c->stream),
                             node);
        }
        case GGML_OP_REPEAT: {
            const mq_view x = view_of(node->src[0]), d = view_of(node);
            return op_status(mq_op_repeat(&x, &d, c->stream), node);
        }
        case GGML_OP_MUL_MAT_ID: {
            // routed on the device (no stream sync, capturable); MQ_GGML_MOE_HOST=1: the ids read
            // back to the host and one product per used expert
            const ggml_tensor *as = node->src[0];
            const mq_view b = view_of(node->src[1]), ids = view_of(node->src[2]), d = view_of(node);
            const int mt = mq_type_of(as->type), n_exp = (int)as->ne[2];
            const int64_t rows = ids.ne[0] * ids.ne[1];
            c->ws_x = nullptr;
            const char *he = std::getenv("MQ_GGML_MOE_HOST");
            if (!(he && std::atoi(he) != 0) && n_exp <= 1024) {  // the device routing's limit
                if (!ensure_ws(c, mq_op_mul_mat_id_device_workspace_bytes(mt, n_exp, as->ne[1], as->ne[0], rows)))
                    return GGML_STATUS_ALLOC_FAILED;
                return op_status(mq_op_mul_mat_id_device(mt, as->data, image_bytes(as), n_exp, as->ne[1], as->ne[0], &b,
                                                         &ids, &d, c->ws, c->ws_bytes, c->stream),
                                 node);
            }
            if (!ensure_ws(c, mq_op_mul_mat_id_workspace_bytes(mt, as->ne[1], as->ne[0], rows)))
                return GGML_STATUS_ALLOC_FAILED;
            return op_status(mq_op_mul_mat_id(mt, as->data, image_bytes(as), n_exp, as->ne[1], as->ne[0], &b, &ids, &d,
                                              c->ws, c->ws_bytes, c->stream),
                             node);
        }
        case GGML_OP_ROPE: {
            const mq_view x = view_of(node->src[0]), p = view_of(node->src[1]), d = view_of(node);
            mq_view f{};
            if (node->src[2]) f = view_of(node->src[2]);
            const int32_t *ip = node->op_params;
            return op_status(mq_op_rope(&x, &p, node->src[2] ? &f : nullptr, &d, ip[1], ip[2], ip[4],
                                        op_param_f32(node, 5), op_param_f32(node, 6), op_param_f32(node, 7),
                                        op_param_f32(node, 8), op_param_f32(node, 9), op_param_f32(node, 10), c->stream),
                             node);
        }
        case GGML_OP_FLASH_ATTN_EXT: {
            const mq_view k = view_of(node->src[1]);
            const bool ready = c->kv_ready_for == node;  // K/V fragments stored by the q/k/v GEMM
            const size_t foff = ready ? c->kv_frag_off : 0;
            c->kv_ready_for = nullptr;
            c->ws_x = nullptr;
            if (!ensure_ws(c, foff + mq_op_flash_attn_workspace_bytes(&k))) return GGML_STATUS_ALLOC_FAILED;
            return op_status(attn_call(c, node, (char *)c->ws + foff, c->ws_bytes - foff, nullptr, 0, MQ_TYPE_Q8_0,
                                       ready ? MQ_ATTN_KV_READY : 0),
                             node);
        }
        default:
            std::fprintf(stderr, "ggml-mi355: op %s reached graph_compute but is not supported\n",
                         ggml_op_name(node->op));
            return GGML_STATUS_FAILED;
    }
}

enum ggml_status run_nodes(BackendCtx *c, ggml_cgraph *cg) {
    const int n = ggml_graph_n_nodes(cg);
    const bool fuse = std::getenv("MQ_GGML_NO_FUSION") == nullptr;
    c->ws_x = nullptr;  // the inputs may have been rewritten since the last graph
    c->kv_ready_for = nullptr;
    c->qk_fa = nullptr;
    c->cs_key.clear();  // and the positions
    c->mb_mask = c->sg_mask = c->mz_mask = nullptr;  // and the masks
    c->unwritten.clear();
    std::vector<char> done(n, 0);  // nodes already computed as part of an earlier group
    for (int i = 0; i < n; i++) {
        ggml_tensor *node = ggml_graph_node(cg, i);
        if (done[i] || ggml_is_empty(node) || is_view_op(node->op)) {
            // a product computed ahead with an earlier group wrote its bytes then
            if (done[i] && !is_view_op(node->op)) {
                if (c->mb_mask && overlaps(node, c->mb_mask)) c->mb_mask = nullptr;
                if (c->sg_mask && overlaps(node, c->sg_mask)) c->sg_mask = nullptr;
                if (c->mz_mask && overlaps(node, c->mz_mask)) c->mz_mask = nullptr;
            }
            continue;
        }
        enum ggml_status st = GGML_STATUS_SUCCESS;
        int used = 0;
        // The workspace's quantized activation (ws_x) stays reusable across nodes that neither use
        // the workspace nor write ws_x's bytes: the q, k and v products of one normed activation,
        // or its gate and up products, quantize it once although elementwise nodes run between
        // them.  The nodes that use the workspace drop or replace it themselves.
        if (!fuse) c->ws_x = nullptr;
        const ggml_tensor *ws_before = c->ws_x;
        if (fuse) {
            switch (node->op) {
                case GGML_OP_MUL_MAT:
                    if (!std::getenv("MQ_GGML_NO_GLU")) used = try_fuse_glu(c, cg, i, n, st);
                    if (!used) used = try_fuse_ffn(c, cg, i, n, st);
                    if (!used) used = try_group_mul_mat(c, cg, i, n, done, st);
                    break;
                case GGML_OP_NORM:
                case GGML_OP_RMS_NORM:
                    if (!std::getenv("MQ_GGML_NO_QK_ATTN")) used = try_defer_qk_norm_rope(c, cg, i, n, done);
                    if (!used) used = try_fuse_norm(c, cg, i, n, st);
                    break;
                case GGML_OP_FLASH_ATTN_EXT: used = try_fuse_attn(c, cg, i, n, st); break;
                case GGML_OP_GET_ROWS: used = try_fuse_rows_sum(c, cg, i, n, st); break;
                case GGML_OP_UNARY: used = try_fuse_silu_mul(c, cg, i, n, done, st); break;
                case GGML_OP_ADD:
                    used = try_fuse_norm(c, cg, i, n, st);
                    if (!used) used = try_fuse_bias_gelu_mul_mat(c, cg, i, n, st);
                    break;
                default: break;
            }
        }
        if (used == 0) {
            st = compute_node(c, node);
            used = 1;
        }
        if (st != GGML_STATUS_SUCCESS) return st;
        if (c->ws_x && c->ws_x == ws_before)
            for (int j = i; j < i + used; j++) {
                const ggml_tensor *t = ggml_graph_node(cg, j);
                if (!is_view_op(t->op) && overlaps(t, c->ws_x)) {
                    c->ws_x = nullptr;
                    break;
                }
            }
        for (int j = i; j < i + used && (c->mb_mask || c->sg_mask || c->mz_mask); j++) {
            const ggml_tensor *t = ggml_graph_node(cg, j);
            if (is_view_op(t->op)) continue;
            if (c->mb_mask && overlaps(t, c->mb_mask)) c->mb_mask = nullptr;
            if (c->sg_mask && overlaps(t, c->sg_mask)) c->sg_mask = nullptr;
            if (c->mz_mask && overlaps(t, c->mz_mask)) c->mz_mask = nullptr;
        }
        i += used - 1;
    }
    c->ws_x = nullptr;
    return GGML_STATUS_SUCCESS;
}

// What a captured launch sequence depends on: every node's op, type, shape, strides,
// op_params and the addresses it reads and writes (the input data may change; the addresses
// may not), and the knobs that change the launches.  FNV-1a.
uint64_t graph_key(ggml_cgraph *cg) {
    uint64_t h = 1469598103934665603ull;
    auto mix = [&](const void *p, size_t n) {
        const unsigned char *b = (const unsigned char *)p;
        for (size_t i = 0; i < n; i++) h = (h ^ b[i]) * 1099511628211ull;
    };
    const int n = ggml_graph_n_nodes(cg);
    mix(&n, sizeof n);
    const uint64_t wgen = weight_gen();  // copies of weights (the gate|up images) follow their writes
    mix(&wgen, sizeof wgen);
    for (int i = 0; i < n; i++) {
        const ggml_tensor *t = ggml_graph_node(cg, i);
        mix(&t->op, sizeof t->op);
        mix(&t->type, sizeof t->type);
        mix(t->ne, sizeof t->ne);
        mix(t->nb, sizeof t->nb);
        mix(t->op_params, sizeof t->op_params);
        mix(&t->data, sizeof t->data);
        mix(&t->flags, sizeof t->flags);
        for (int j = 0; j < GGML_MAX_SRC; j++) {
            const void *d = t->src[j] ? t->src[j]->data : nullptr;
            mix(&d, sizeof d);
        }
    }
    for (const char *k : {"MQ_GGML_NO_FUSION", "MQ_GEMM_CFG", "MQ_ATTN_SPLIT", "MQ_GEMV_WGS", "MQ_GEMV_PF",
                          "MQ_FORCE_GEMV_MAX_M", "MQ_Q8_0_VARIANT", "MQ_GGML_NO_MASK_BLOCKS", "MQ_ATTN_SPLIT_WAVES",
                          "MQ_GGML_NO_MASK_SEGMENTS", "MQ_GGML_MOE_HOST", "MQ_GGML_NO_GLU",
                          "MQ_GGML_WRITE_NORMS", "MQ_GGML_MASK_ALWAYS"}) {
        const char *v = std::getenv(k);
        if (v) mix(v, std::strlen(v));
        mix("|", 1);
    }
    return h;
}

// With MQ_GGML_GRAPH=1: eager on a graph's first call (which also sizes the workspace),
// captured into a HIP graph on its second consecutive call, replayed from then on while the
// same graph comes back.  Off by default: on MI355X / ROCm 7.2 a replayed graph runs its
// kernels no faster than the stream does (each small dependent kernel costs ~4.5 us either
// way, measured on 16-token MiniLM graphs), and ~6 % slower on 32 x 128 batches.
enum ggml_status be_graph_compute(ggml_backend_t be, ggml_cgraph *cg) {
    BackendCtx *c = (BackendCtx *)be->context;
    DeviceGuard g(c->ordinal);
    const char *ge = std::getenv("MQ_GGML_GRAPH");
    if (!ge || std::atoi(ge) == 0) return run_nodes(c, cg);
    const uint64_t key = graph_key(cg);
    if (c->gexec && key == c->gkey) {
        const hipError_t e = hipGraphLaunch(c->gexec, c->stream);
        if (e == hipSuccess) return GGML_STATUS_SUCCESS;
        std::fprintf(stderr, "ggml-mi355: hipGraphLaunch failed (%s); running eagerly\n", hipGetErrorString(e));
        (void)hipGraphExecDestroy(c->gexec);
        c->gexec = nullptr;
        c->gkey = c->seen_key = 0;
        return run_nodes(c, cg);
    }
    if (key != c->seen_key) {
        c->seen_key = key;
        return run_nodes(c, cg);
    }
    // the same graph a second time: capture it
    if (hipStreamBeginCapture(c->stream, hipStreamCaptureModeThreadLocal) != hipSuccess) return run_nodes(c, cg);
    c->capturing = true;
    const enum ggml_status st = run_nodes(c, cg);
    c->capturing = false;
    hipGraph_t graph = nullptr;
    const hipError_t ec = hipStreamEndCapture(c->stream, &graph);
    hipGraphExec_t exec = nullptr;
    const bool ok = st == GGML_STATUS_SUCCESS && ec == hipSuccess && graph &&
                    hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0) == hipSuccess;
    if (graph) (void)hipGraphDestroy(graph);
    if (!ok) {  // nothing ran: replay the graph eagerly and try capturing next time
        if (exec) (void)hipGraphExecDestroy(exec);
        (void)hipGetLastError();
        c->seen_key = 0;
        return run_nodes(c, cg);
    }
    if (c->gexec) (void)hipGraphExecDestroy(c->gexec);
    c->gexec = exec;
    c->gkey = key;
    const hipError_t e = hipGraphLaunch(c->gexec, c->stream);
    return e == hipSuccess ? GGML_STATUS_SUCCESS : GGML_STATUS_FAILED;
}

ggml_guid *backend_guid() {
    static ggml_guid guid = {0x4d, 0x49, 0x33, 0x35, 0x35, 0x58, 0x2d, 0x67,
                             0x66, 0x78, 0x39, 0x35, 0x30, 0x2d, 0x6d, 0x71};  // "MI355X-gfx950-mq"
    return &guid;
}

const ggml_backend_i kBackendIface = {
    be_name, be_free, nullptr, nullptr, nullptr, be_synchronize, nullptr, nullptr, nullptr, nullptr,
    be_graph_compute, nullptr, nullptr, nullptr,
};

// ---------------------------------------------------------------- device ----
const char *dev_name(ggml_backend_dev_t d) { return ((DeviceCtx *)d->context)->name.c_str(); }
const char *dev_desc(ggml_backend_dev_t d) { return ((DeviceCtx *)d->context)->description.c_str(); }

void dev_memory(ggml_backend_dev_t d, size_t *free, size_t *total) {
    DeviceGuard g(((DeviceCtx *)d->context)->ordinal);
    *free = *total = 0;
    (void)hipMemGetInfo(free, total);
}

enum ggml_backend_dev_type dev_type(ggml_backend_dev_t) { return GGML_BACKEND_DEVICE_TYPE_GPU; }

void dev_props(ggml_backend_dev_t d, ggml_backend_dev_props *p) {
    p->name = dev_name(d);
    p->description = dev_desc(d);
    p->type = GGML_BACKEND_DEVICE_TYPE_GPU;
    p->device_id = nullptr;
    dev_memory(d, &p->memory_free, &p->memory_total);
    p->caps = {false, false, false, false};  // no async copies, host buffers, host-pointer buffers or events
}

ggml_backend_t dev_init(ggml_backend_dev_t d, const char *) {
    DeviceCtx *dc = (DeviceCtx *)d->context;
    DeviceGuard g(dc->ordinal);
    BackendCtx *c = new BackendCtx;
    c->ordinal = dc->ordinal;
    c->name = dc->name;
    if (hipStreamCreate(&c->stream) != hipSuccess) {
        delete c;
        return nullptr;
    }
    ggml_backend *be = new ggml_backend;
    be->guid = backend_guid();
    be->iface = kBackendIface;
    be->device = d;
    be->context = c;
    return be;
}

ggml_backend_buffer_type_t dev_buft(ggml_backend_dev_t d) { return &((DeviceCtx *)d->context)->buft; }

bool dev_supports_buft(ggml_backend_dev_t d, ggml_backend_buffer_type_t buft) {
    return buft == &((DeviceCtx *)d->context)->buft;
}

bool in_this_device(ggml_backend_dev_t d, const ggml_tensor *t) {
    const ggml_backend_buffer_t b = t->view_src ? t->view_src->buffer : t->buffer;
    return !b || b->buft == &((DeviceCtx *)d->context)->buft;
}

bool supports_mul_mat(ggml_backend_dev_t d, const ggml_tensor *op) {
    const ggml_tensor *w = op->src[0], *x = op->src[1];
    if (!w || !x) return false;
    const int mt = mq_type_of(w->type);
    if (mt < 0 || x->type != GGML_TYPE_F32 || op->type != GGML_TYPE_F32) return false;
    if (w->ne[2] != 1 || w->ne[3] != 1 || w->view_src != nullptr || !ggml_is_contiguous(w)) return false;
    if (!mq_supports(mt, w->ne[0])) return false;
    if (x->nb[0] != sizeof(float) || op->nb[0] != sizeof(float)) return false;
    if (x->nb[1] % sizeof(float) || op->nb[1] % sizeof(float)) return false;
    // the weight must live in this device's buffers (that is where its planes are)
    if (w->buffer && w->buffer->buft != &((DeviceCtx *)d->context)->buft) return false;
    return true;
}

bool dev_supports_op(ggml_backend_dev_t d, const ggml_tensor *op) {
    if (is_view_op(op->op)) return true;
    mq_view v[5], dst = view_of(op);
    const mq_view *p[5] = {nullptr, nullptr, nullptr, nullptr, nullptr};
    for (int i = 0; i < 5; i++)
        if (op->src[i]) {
            v[i] = view_of(op->src[i]);
            if (v[i].type < 0) return false;
            p[i] = &v[i];
        }
    if (dst.type < 0) return false;
    switch (op->op) {
        case GGML_OP_MUL_MAT:
            if (op->src[0] && op->src[0]->type == GGML_TYPE_F32)
                return mq_op_supported(MQ_OP_MUL_MAT_F32, 0, p[0], p[1], nullptr, nullptr, &dst);
            return supports_mul_mat(d, op);
        case GGML_OP_SOFT_MAX:
            // no ALiBi slopes, no attention sinks
            if (op_param_f32(op, 1) != 0.0f || op->src[2]) return false;
            return mq_op_supported(MQ_OP_SOFT_MAX, 0, p[0], p[1], nullptr, nullptr, &dst);
        case GGML_OP_ARGSORT:
            return mq_op_supported(MQ_OP_ARGSORT, op->op_params[0] == GGML_SORT_ORDER_DESC ? MQ_SORT_DESC : MQ_SORT_ASC,
                                   p[0], nullptr, nullptr, nullptr, &dst);
        case GGML_OP_REPEAT: return mq_op_supported(MQ_OP_REPEAT, 0, p[0], nullptr, nullptr, nullptr, &dst);
        case GGML_OP_GET_ROWS:
            // a weight table must be in this device's memory (the GGUF bytes at its start)
            return in_this_device(d, op->src[0]) && mq_op_supported(MQ_OP_GET_ROWS, 0, p[0], p[1], nullptr, nullptr, &dst);
        case GGML_OP_ADD:
        case GGML_OP_SUB:
        case GGML_OP_MUL:
        case GGML_OP_DIV: return mq_op_supported(MQ_OP_BINARY, binary_of(op->op), p[0], p[1], nullptr, nullptr, &dst);
        case GGML_OP_NORM: return mq_op_supported(MQ_OP_NORM, MQ_NORM_LAYER, p[0], nullptr, nullptr, nullptr, &dst);
        case GGML_OP_RMS_NORM: return mq_op_supported(MQ_OP_NORM, MQ_NORM_RMS, p[0], nullptr, nullptr, nullptr, &dst);
        case GGML_OP_UNARY:
            return unary_of(op) >= 0 && mq_op_supported(MQ_OP_UNARY, unary_of(op), p[0], nullptr, nullptr, nullptr, &dst);
        case GGML_OP_CPY: return mq_op_supported(MQ_OP_CPY, 0, p[0], nullptr, nullptr, nullptr, p[1]);
        case GGML_OP_CONT:
        case GGML_OP_DUP: return mq_op_supported(MQ_OP_CPY, 0, p[0], nullptr, nullptr, nullptr, &dst);
        case GGML_OP_MUL_MAT_ID: {
            // expert weights: a 3-D weight image set in this device's buffers; b [k, 1|n_used, T],
            // ids [n_used, T], dst [n, n_used, T], F32 rows contiguous
            const ggml_tensor *as = op->src[0], *b = op->src[1], *ids = op->src[2];
            if (!as || !b || !ids || !is_image(as) || !in_this_device(d, as)) return false;
            if (b->type != GGML_TYPE_F32 || ids->type != GGML_TYPE_I32 || op->type != GGML_TYPE_F32) return false;
            const int64_t n_used = ids->ne[0], T = ids->ne[1];
            if (b->ne[0] != as->ne[0] || (b->ne[1] != 1 && b->ne[1] != n_used) || b->ne[2] != T || b->ne[3] != 1 ||
                ids->ne[2] != 1 || op->ne[0] != as->ne[1] || op->ne[1] != n_used || op->ne[2] != T)
                return false;
            return b->nb[0] == sizeof(float) && b->nb[1] % 16 == 0 && b->nb[2] % 16 == 0 && b->view_offs % 16 == 0 &&
                   ids->nb[0] == sizeof(int32_t) && op->nb[0] == sizeof(float);
        }
        case GGML_OP_ROPE: {
            const int n_dims = op->op_params[1], mode = op->op_params[2];
            if (n_dims <= 0 || n_dims % 2 || n_dims > op->src[0]->ne[0]) return false;
            return mq_op_supported(MQ_OP_ROPE, mode, p[0], p[1], p[2], nullptr, &dst);
        }
        case GGML_OP_FLASH_ATTN_EXT:
            // no ALiBi slopes, no logit soft-capping, no attention sinks
            if (op_param_f32(op, 1) != 0.0f || op_param_f32(op, 2) != 0.0f || op->src[4]) return false;
            return mq_op_supported(MQ_OP_FLASH_ATTN, 0, p[0], p[1], p[2], p[3], &dst);
        default: return false;
    }
}

bool dev_offload_op(ggml_backend_dev_t, const ggml_tensor *) { return false; }

const ggml_backend_device_i kDeviceIface = {
    dev_name, dev_desc,           dev_memory,      dev_type,       dev_props, dev_init, dev_buft, nullptr, nullptr,
    dev_supports_op, dev_supports_buft, dev_offload_op, nullptr, nullptr, nullptr,
};

// -------------------------------------------------------------- registry ----
std::vector<DeviceCtx *> &devices() {
    static std::vector<DeviceCtx *> devs;
    static std::once_flag once;
    std::call_once(once, [] {
        int n = 0;
        if (hipGetDeviceCount(&n) != hipSuccess) n = 0;
        for (int i = 0; i < n; i++) {
            hipDeviceProp_t prop;
            if (hipGetDeviceProperties(&prop, i) != hipSuccess) continue;
            if (std::strncmp(prop.gcnArchName, "gfx950", 6) != 0) continue;
            DeviceCtx *d = new DeviceCtx;
            d->ordinal = i;
            d->name = "MI355X" + std::to_string(devs.size());
            d->description = std::string(prop.name) + " (" + prop.gcnArchName + ", " +
                             std::to_string(prop.multiProcessorCount) + " CUs)";
            d->buft.iface = kBuftIface;
            d->buft.context = d;
            d->dev.iface = kDeviceIface;
            d->dev.reg = &the_reg();
            d->dev.context = d;
            d->buft.device = &d->dev;
            devs.push_back(d);
        }
    });
    return devs;
}

const char *reg_name(ggml_backend_reg_t) { return "MI355X"; }
size_t reg_count(ggml_backend_reg_t) { return devices().size(); }
ggml_backend_dev_t reg_dev(ggml_backend_reg_t, size_t i) { return i < devices().size() ? &devices()[i]->dev : nullptr; }
void *reg_proc(ggml_backend_reg_t, const char *) { return nullptr; }  // no set_n_threads: GPU kernels, not CPU threads

ggml_backend_reg &the_reg() {
    static ggml_backend_reg reg = {GGML_BACKEND_API_VERSION, {reg_name, reg_count, reg_dev, reg_proc}, nullptr};
    return reg;
}

}  // namespace

extern "C" {

ggml_backend_reg_t ggml_backend_mi355_reg(void) { return &the_reg(); }

int ggml_backend_mi355_get_device_count(void) { return (int)devices().size(); }

ggml_backend_buffer_type_t ggml_backend_mi355_buffer_type(int device) {
    if (device < 0 || device >= (int)devices().size()) return nullptr;
    return &devices()[device]->buft;
}

ggml_backend_t ggml_backend_mi355_init(int device) {
    if (device < 0 || device >= (int)devices().size()) return nullptr;
    return dev_init(&devices()[device]->dev, nullptr);
}

bool ggml_backend_is_mi355(ggml_backend_t backend) {
    return backend && backend->guid == backend_guid();
}

// The two symbols ggml's loader resolves in a backend library built for dynamic loading:
// ggml_backend_load takes the registry from ggml_backend_init (and checks its api_version),
// ggml_backend_load_best ranks candidate libraries by ggml_backend_score, 0 meaning "cannot run
// here".  This library can run wherever a gfx950 device is visible.
ggml_backend_reg_t ggml_backend_init(void) { return &the_reg(); }

int ggml_backend_score(void) { return devices().empty() ? 0 : 1; }

void ggml_backend_mi355_set_act_observer(ggml_backend_t backend, ggml_backend_mi355_act_observer cb, void *user) {
    if (!ggml_backend_is_mi355(backend)) return;
    BackendCtx *c = (BackendCtx *)backend->context;
    c->act_cb = cb, c->act_user = user;
}

}  // extern "C"
