// ggml_backend_mi355.cpp -- ggml backend that runs GGML_OP_MUL_MAT on MI355X.
//
// Interface tables follow ggml-backend-impl.h.  The backend executes only
// MUL_MAT (plus the metadata-only view ops); ggml_backend_sched keeps every
// other op on the CPU backend, which is how CrispEmbed already falls back for
// ops a GPU backend rejects (src/crispembed.cpp:700-723).
//
// Threading: like every ggml backend, one backend instance must be driven by one
// thread at a time (src/core/gpu_backend_pref.h:180-185); each instance owns one
// HIP stream (default priority) and one activation workspace.
#include <hip/hip_runtime.h>

#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <string>
#include <vector>

#include "ggml-backend-impl.h"
#include "ggml-mi355.h"
#include "ggml.h"
#include "mq.h"

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
};

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

// A tensor whose allocation is a weight image: a supported weight type, 2-D,
// contiguous, not a view.  (F16 tensors qualify too: their image is the fp16
// rows plus the tiled copy the MFMA GEMM reads.)
bool is_image(const ggml_tensor *t) {
    const int mt = mq_type_of(t->type);
    return mt >= 0 && t->view_src == nullptr && t->ne[2] == 1 && t->ne[3] == 1 && ggml_is_contiguous(t) &&
           mq_supports(mt, t->ne[0]) && t->ne[1] > 0;
}

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
}

void *buf_base(ggml_backend_buffer_t b) { return ((BufferCtx *)b->context)->base; }

enum ggml_status buf_init_tensor(ggml_backend_buffer_t, ggml_tensor *) { return GGML_STATUS_SUCCESS; }

void rebuild_planes(BufferCtx *c, ggml_tensor *t, size_t offset, size_t size) {
    if (!is_image(t)) return;
    const int mt = mq_type_of(t->type);
    const size_t rs = ggml_row_size(t->type, t->ne[0]);
    const int64_t r0 = (int64_t)(offset / rs), r1 = (int64_t)((offset + size + rs - 1) / rs);
    if (mq_weight_prepare(mt, t->data, t->ne[1], t->ne[0], r0, r1, nullptr) != 0) {
        std::fprintf(stderr, "ggml-mi355: weight preparation of '%s' failed: %s\n", t->name, mq_last_error());
        std::abort();
    }
    hip_check(hipStreamSynchronize(nullptr), "hipStreamSynchronize");
    (void)c;
}

void buf_set_tensor(ggml_backend_buffer_t b, ggml_tensor *t, const void *data, size_t offset, size_t size) {
    BufferCtx *c = (BufferCtx *)b->context;
    DeviceGuard g(c->ordinal);
    hip_check(hipMemcpy((char *)t->data + offset, data, size, hipMemcpyHostToDevice), "hipMemcpy H2D");
    rebuild_planes(c, t, offset, size);
}

void buf_get_tensor(ggml_backend_buffer_t b, const ggml_tensor *t, void *data, size_t offset, size_t size) {
    BufferCtx *c = (BufferCtx *)b->context;
    DeviceGuard g(c->ordinal);
    // hipMemcpy on the null stream waits for work queued on the (blocking) backend streams
    hip_check(hipMemcpy(data, (const char *)t->data + offset, size, hipMemcpyDeviceToHost), "hipMemcpy D2H");
}

void buf_memset_tensor(ggml_backend_buffer_t b, ggml_tensor *t, uint8_t value, size_t offset, size_t size) {
    BufferCtx *c = (BufferCtx *)b->context;
    DeviceGuard g(c->ordinal);
    hip_check(hipMemset((char *)t->data + offset, value, size), "hipMemset");
    rebuild_planes(c, t, offset, size);
}

bool buf_cpy_tensor(ggml_backend_buffer_t b, const ggml_tensor *src, ggml_tensor *dst) {
    const ggml_backend_buffer_t sb = src->view_src ? src->view_src->buffer : src->buffer;
    if (!sb || sb->iface.free_buffer != buf_free) return false;  // only device-to-device within this backend
    BufferCtx *c = (BufferCtx *)b->context;
    DeviceGuard g(c->ordinal);
    const size_t n = ggml_nbytes(src);
    hip_check(hipMemcpy(dst->data, src->data, n, hipMemcpyDeviceToDevice), "hipMemcpy D2D");
    rebuild_planes(c, dst, 0, n);
    return true;
}

void buf_clear(ggml_backend_buffer_t b, uint8_t value) {
    BufferCtx *c = (BufferCtx *)b->context;
    DeviceGuard g(c->ordinal);
    hip_check(hipMemset(c->base, value, c->size), "hipMemset");
    hip_check(hipDeviceSynchronize(), "hipDeviceSynchronize");
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
    if (is_image(t)) return mq_weight_image_bytes(mq_type_of(t->type), t->ne[1], t->ne[0]);
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
        if (c->ws) (void)hipFree(c->ws);
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

enum ggml_status mul_mat(BackendCtx *c, ggml_tensor *dst) {
    const ggml_tensor *w = dst->src[0];
    const ggml_tensor *x = dst->src[1];
    const int mt = mq_type_of(w->type);
    const int64_t K = w->ne[0], N = w->ne[1];
    const bool flat = rows_flat(x) && rows_flat(dst);
    const int64_t M = flat ? x->ne[1] * x->ne[2] * x->ne[3] : x->ne[1];
    const size_t need = mq_workspace_bytes(mt, M, K);
    if (need > c->ws_bytes) {
        hip_check(hipStreamSynchronize(c->stream), "hipStreamSynchronize");
        if (c->ws) (void)hipFree(c->ws);
        c->ws = nullptr;
        c->ws_bytes = 0;
        if (hipMalloc(&c->ws, need) != hipSuccess) {
            c->ws = nullptr;
            std::fprintf(stderr, "ggml-mi355: workspace allocation of %zu bytes failed\n", need);
            return GGML_STATUS_ALLOC_FAILED;
        }
        c->ws_bytes = need;
    }
    const int64_t nbat2 = flat ? 1 : x->ne[2], nbat3 = flat ? 1 : x->ne[3];
    for (int64_t i3 = 0; i3 < nbat3; i3++) {
        for (int64_t i2 = 0; i2 < nbat2; i2++) {
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

enum ggml_status be_graph_compute(ggml_backend_t be, ggml_cgraph *cg) {
    BackendCtx *c = (BackendCtx *)be->context;
    DeviceGuard g(c->ordinal);
    const int n = ggml_graph_n_nodes(cg);
    for (int i = 0; i < n; i++) {
        ggml_tensor *node = ggml_graph_node(cg, i);
        if (ggml_is_empty(node) || is_view_op(node->op)) continue;
        if (node->op != GGML_OP_MUL_MAT) {
            std::fprintf(stderr, "ggml-mi355: op %s reached graph_compute but is not supported\n",
                         ggml_op_name(node->op));
            return GGML_STATUS_FAILED;
        }
        const enum ggml_status st = mul_mat(c, node);
        if (st != GGML_STATUS_SUCCESS) return st;
    }
    return GGML_STATUS_SUCCESS;  // enqueued; ggml_backend_graph_compute synchronizes
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

bool dev_supports_op(ggml_backend_dev_t d, const ggml_tensor *op) {
    if (is_view_op(op->op)) return true;
    if (op->op != GGML_OP_MUL_MAT) return false;
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

}  // extern "C"
