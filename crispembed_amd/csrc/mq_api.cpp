// mq_api.cpp -- the extern "C" entry points of libmq.so (declared in include/mq.h).
//
// Argument checking happens here, on the host, before any launch: every kernel
// assumes the shapes validated below (k a multiple of the block size, m <= 8 for
// the GEMV, 16-byte aligned planes), so no kernel is ever launched on a shape it
// would index out of bounds.
#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <map>
#include <mutex>
#include <string>

#include "mq_internal.h"

namespace mq {
namespace host {
size_t quantize_chunk(int type, const float *src, void *dst, int64_t nrows, int64_t k);
}
int set_error(int code, const char *fmt, ...) __attribute__((format(printf, 2, 3)));
}  // namespace mq

using namespace mq;

namespace {

thread_local std::string g_err;

int fail(int code, const char *fmt, ...) __attribute__((format(printf, 2, 3)));
int fail(int code, const char *fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof(buf), fmt, ap);
    va_end(ap);
    g_err = buf;
    return code;
}

}  // namespace

// error reporting shared with the other host files of the library (mq_bert.cpp)
int mq::set_error(int code, const char *fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof(buf), fmt, ap);
    va_end(ap);
    g_err = buf;
    return code;
}

namespace {

int hip_fail(hipError_t e, const char *what) {
    return fail(MQ_EHIP, "%s: %s", what, hipGetErrorString(e));
}

// env knobs: unset, "" or "0" mean off (the reference's core_env::on semantics,
// src/core/env_gate.h:25-42); numeric knobs parse the value
int env_int(const char *name, int dflt) {
    const char *v = std::getenv(name);
    if (!v || !*v) return dflt;
    char *end = nullptr;
    const long x = std::strtol(v, &end, 10);
    return (end && *end == 0) ? (int)x : dflt;
}

int g_gemv_max_m = -1;
int g_q8_0_variant = -1;

struct Workspace {
    void *ptr = nullptr;
    size_t bytes = 0;
};
// mq_mul_mat's internal activation buffers (workspace == NULL), one per (device, stream): work
// queued on one stream never shares its quantized activations with another stream's
std::mutex g_ws_mu;
std::map<std::pair<int, void *>, Workspace> g_ws;

bool type_ok(int t) {
    return t == MQ_TYPE_Q8_0 || t == MQ_TYPE_Q4_K || t == MQ_TYPE_Q6_K || t == MQ_TYPE_F16;
}

int check_weight_shape(int type, int64_t n, int64_t k) {
    if (!type_ok(type)) return fail(MQ_EUNSUPPORTED, "weight type %d is not Q8_0/Q4_K/Q6_K/F16", type);
    if (n <= 0 || k <= 0) return fail(MQ_EINVAL, "bad shape n=%lld k=%lld", (long long)n, (long long)k);
    if (!mq_supports(type, k))
        return fail(MQ_EUNSUPPORTED, "k=%lld is not a multiple of the %s block", (long long)k,
                    type == MQ_TYPE_F16 ? "32-value F16" : "quant");
    if (n > INT32_MAX || k > INT32_MAX || n * k > ((int64_t)1 << 40))
        return fail(MQ_EINVAL, "tensor too large n=%lld k=%lld", (long long)n, (long long)k);
    return MQ_OK;
}

bool is_aligned(const void *p, size_t a) { return ((uintptr_t)p % a) == 0; }

// The library's own activation workspace for work queued on `stream` of the current device, grown
// (hipMalloc) to at least `need` bytes.
int stream_workspace(size_t need, void *stream, void **ws, size_t *bytes) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return hip_fail(e, "hipGetDevice");
    std::lock_guard<std::mutex> lk(g_ws_mu);
    Workspace &w = g_ws[{dev, stream}];
    if (w.bytes < need) {
        // the old buffer may still be read by work queued earlier on this stream
        e = hipStreamSynchronize((hipStream_t)stream);
        if (e != hipSuccess) return hip_fail(e, "hipStreamSynchronize");
        if (w.ptr) (void)hipFree(w.ptr);
        w.ptr = nullptr;
        w.bytes = 0;
        e = hipMalloc(&w.ptr, need);
        if (e != hipSuccess) {
            (void)hipGetLastError();  // a failed allocation must not surface as the next launch's error
            w.ptr = nullptr;
            return fail(MQ_ENOMEM, "hipMalloc(%zu) for the activation workspace failed", need);
        }
        w.bytes = need;
    }
    *ws = w.ptr;
    *bytes = w.bytes;
    return MQ_OK;
}

}  // namespace

extern "C" {

const char *mq_last_error(void) { return g_err.c_str(); }

int mq_release_workspace(void *stream) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return hip_fail(e, "hipGetDevice");
    std::lock_guard<std::mutex> lk(g_ws_mu);
    auto it = g_ws.find({dev, stream});
    if (it == g_ws.end()) return MQ_OK;
    e = hipStreamSynchronize((hipStream_t)stream);  // work queued on the stream may still read it
    if (e != hipSuccess) return hip_fail(e, "hipStreamSynchronize");
    if (it->second.ptr) (void)hipFree(it->second.ptr);
    g_ws.erase(it);
    return MQ_OK;
}

int mq_init(void) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return hip_fail(e, "hipGetDevice");
    hipDeviceProp_t prop;
    e = hipGetDeviceProperties(&prop, dev);
    if (e != hipSuccess) return hip_fail(e, "hipGetDeviceProperties");
    if (std::strncmp(prop.gcnArchName, "gfx950", 6) != 0)
        return fail(MQ_ENODEV, "device %d is %s, this library is built for gfx950", dev, prop.gcnArchName);
    return MQ_OK;
}

int mq_measure_mfma_i8(int iters, double *tops, void *stream) {
    if (iters <= 0 || !tops) return fail(MQ_EINVAL, "mq_measure_mfma_i8: iters > 0 and tops required");
    int dev = 0, ncu = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e == hipSuccess) e = hipDeviceGetAttribute(&ncu, hipDeviceAttributeMultiprocessorCount, dev);
    if (e != hipSuccess) return hip_fail(e, "device query");
    hipStream_t s = (hipStream_t)stream;
    int *out = nullptr;
    hipEvent_t e0 = nullptr, e1 = nullptr;
    float ms = 0.f;
    e = hipMalloc(&out, (size_t)ncu * 256 * sizeof(int));
    if (e != hipSuccess) {
        (void)hipGetLastError();
        return fail(MQ_ENOMEM, "hipMalloc for the probe output failed");
    }
    if ((e = hipEventCreate(&e0)) == hipSuccess && (e = hipEventCreate(&e1)) == hipSuccess &&
        (e = mq::launch_mfma_probe(iters, out, ncu, s)) == hipSuccess &&  // warm-up: clocks, code object
        (e = hipEventRecord(e0, s)) == hipSuccess && (e = mq::launch_mfma_probe(iters, out, ncu, s)) == hipSuccess &&
        (e = hipEventRecord(e1, s)) == hipSuccess && (e = hipEventSynchronize(e1)) == hipSuccess)
        e = hipEventElapsedTime(&ms, e0, e1);
    if (e0) (void)hipEventDestroy(e0);
    if (e1) (void)hipEventDestroy(e1);
    (void)hipFree(out);
    if (e != hipSuccess) return hip_fail(e, "MFMA probe");
    *tops = 2.0 * 32 * 32 * 32 * 8 * (double)iters * 4 * ncu / (ms * 1e-3) / 1e12;
    return MQ_OK;
}

int mq_gemv_max_m(void) {
    if (g_gemv_max_m < 0) {
        int v = env_int("MQ_FORCE_GEMV_MAX_M", 8);
        g_gemv_max_m = v < 0 ? 0 : (v > 8 ? 8 : v);
    }
    return g_gemv_max_m;
}

int mq_q8_0_variant(void) {
    if (g_q8_0_variant < 0) {
        const int v = env_int("MQ_Q8_0_VARIANT", MQ_Q8_0_X86);
        g_q8_0_variant = (v == MQ_Q8_0_NEON || v == MQ_Q8_0_REF) ? v : MQ_Q8_0_X86;
    }
    return g_q8_0_variant;
}

int mq_set_q8_0_variant(int variant) {
    if (variant != MQ_Q8_0_X86 && variant != MQ_Q8_0_NEON && variant != MQ_Q8_0_REF)
        return fail(MQ_EINVAL, "unknown Q8_0 variant %d", variant);
    g_q8_0_variant = variant;
    return MQ_OK;
}

int64_t mq_blck_size(int type) { return blck_size(type); }
size_t mq_type_size(int type) { return type_size(type); }
size_t mq_row_size(int type, int64_t k) { return row_size(type, k); }

int mq_vec_dot_type(int type) {
    switch (type) {
        case MQ_TYPE_Q8_0: return MQ_TYPE_Q8_0;
        case MQ_TYPE_Q4_K:
        case MQ_TYPE_Q6_K: return MQ_TYPE_Q8_K;
        case MQ_TYPE_F16: return MQ_TYPE_F16;
        default: return -1;
    }
}

int mq_supports(int type, int64_t k) {
    if (k <= 0) return 0;
    switch (type) {
        case MQ_TYPE_Q8_0: return k % QK8_0 == 0;
        case MQ_TYPE_Q4_K:
        case MQ_TYPE_Q6_K: return k % QK_K == 0;
        case MQ_TYPE_F16: return k % 32 == 0;
        default: return 0;
    }
}

size_t mq_quantize_chunk(int type, const float *src_host, void *dst_host, int64_t nrows, int64_t k) {
    const size_t r = host::quantize_chunk(type, src_host, dst_host, nrows, k);
    if (r == 0 && nrows > 0) fail(MQ_EINVAL, "mq_quantize_chunk: bad type %d or k=%lld", type, (long long)k);
    return r;
}

int mq_quantize_q8_0(const float *x, int64_t ldx, void *y, int64_t nrows, int64_t k, int variant, void *stream) {
    if (!x || !y || nrows < 0 || k <= 0 || k % QK8_0 || ldx < k)
        return fail(MQ_EINVAL, "mq_quantize_q8_0: bad arguments");
    if (variant != MQ_Q8_0_X86 && variant != MQ_Q8_0_NEON && variant != MQ_Q8_0_REF)
        return fail(MQ_EINVAL, "mq_quantize_q8_0: unknown variant %d", variant);
    if (!is_aligned(y, 2)) return fail(MQ_EINVAL, "mq_quantize_q8_0: y must be 2-byte aligned");
    const hipError_t e = launch_quantize_q8_0_gguf(x, ldx, y, nrows, k, variant, (hipStream_t)stream);
    return e == hipSuccess ? MQ_OK : hip_fail(e, "mq_quantize_q8_0");
}

int mq_quantize_q8_K(const float *x, int64_t ldx, void *y, int64_t nrows, int64_t k, void *stream) {
    if (!x || !y || nrows < 0 || k <= 0 || k % QK_K || ldx < k)
        return fail(MQ_EINVAL, "mq_quantize_q8_K: bad arguments");
    if (!is_aligned(y, 4)) return fail(MQ_EINVAL, "mq_quantize_q8_K: y must be 4-byte aligned");
    const hipError_t e = launch_quantize_q8_K_gguf(x, ldx, y, nrows, k, (hipStream_t)stream);
    return e == hipSuccess ? MQ_OK : hip_fail(e, "mq_quantize_q8_K");
}

int mq_quantize_f16(const float *x, int64_t ldx, void *y, int64_t nrows, int64_t k, void *stream) {
    if (!x || !y || nrows < 0 || k <= 0 || k % 4 || ldx < k) return fail(MQ_EINVAL, "mq_quantize_f16: bad arguments");
    if (!is_aligned(y, 2)) return fail(MQ_EINVAL, "mq_quantize_f16: y must be 2-byte aligned");
    const hipError_t e = launch_quantize_f16(x, ldx, y, nrows, k, (hipStream_t)stream);
    return e == hipSuccess ? MQ_OK : hip_fail(e, "mq_quantize_f16");
}

int mq_dequantize(int type, const void *w, float *y, int64_t nrows, int64_t k, int fused, void *stream) {
    if (!w || !y || nrows < 0 || k <= 0) return fail(MQ_EINVAL, "mq_dequantize: bad arguments");
    if (type != MQ_TYPE_F16 && type != MQ_TYPE_Q8_0 && type != MQ_TYPE_Q4_K && type != MQ_TYPE_Q6_K &&
        type != MQ_TYPE_Q8_K)
        return fail(MQ_EUNSUPPORTED, "mq_dequantize: type %d", type);
    if (k % blck_size(type)) return fail(MQ_EINVAL, "mq_dequantize: k=%lld not a multiple of the block", (long long)k);
    if (!is_aligned(w, 4)) return fail(MQ_EINVAL, "mq_dequantize: w must be 4-byte aligned");
    const hipError_t e = launch_dequantize(type, w, y, nrows, k, fused, (hipStream_t)stream);
    return e == hipSuccess ? MQ_OK : hip_fail(e, "mq_dequantize");
}

size_t mq_gguf_bytes(int type, int64_t n, int64_t k) { return weight_planes(type, n, k).gguf; }
size_t mq_gguf_bytes_aligned(int type, int64_t n, int64_t k) { return align256(weight_planes(type, n, k).gguf); }
size_t mq_weight_image_bytes(int type, int64_t n, int64_t k) {
    if (!type_ok(type) || n <= 0 || k <= 0 || !mq_supports(type, k)) return 0;
    return weight_planes(type, n, k).total;
}

int mq_weight_prepare(int type, void *image, int64_t n, int64_t k, int64_t row0, int64_t row1, void *stream) {
    int rc = check_weight_shape(type, n, k);
    if (rc) return rc;
    if (!image || !is_aligned(image, 256)) return fail(MQ_EINVAL, "mq_weight_prepare: image must be 256-byte aligned");
    if (row0 < 0) row0 = 0;
    if (row1 > n) row1 = n;
    const hipError_t e = launch_weight_prepare(type, image, n, k, row0, row1, (hipStream_t)stream);
    return e == hipSuccess ? MQ_OK : hip_fail(e, "mq_weight_prepare");
}

size_t mq_workspace_bytes(int type, int64_t m, int64_t k) {
    if (!type_ok(type) || m < 0 || k <= 0) return 0;
    return act_workspace_bytes(type, m, k);
}

// The path MQ_PATH_AUTO takes when n is known: the GEMV up to mq_gemv_max_m rows, and up to 32
// rows (in 8-row launches, each streaming the weight) while the GEMM's 128x128 tile grid would
// have fewer than 64 workgroups -- narrow layers of short inputs, where the GEMM's few
// workgroups each walk the whole of K.
int mq_mul_mat_path(int type, int64_t n, int64_t k, int64_t m) {
    (void)type;
    (void)k;
    if (m <= mq_gemv_max_m()) return MQ_PATH_GEMV;
    if (mq_gemv_max_m() >= 8 && m <= GEMV_MAX_M && ((m + 127) / 128) * ((n + 127) / 128) < 64) return MQ_PATH_GEMV;
    return MQ_PATH_GEMM;
}

static int resolve_path(int path, int64_t m) {
    if (path == MQ_PATH_AUTO) path = (m <= mq_gemv_max_m()) ? MQ_PATH_GEMV : MQ_PATH_GEMM;
    if (path == MQ_PATH_GEMV && m > GEMV_MAX_M)
        return fail(MQ_EINVAL, "GEMV path takes m <= %d (m=%lld)", GEMV_MAX_M, (long long)m);
    if (path != MQ_PATH_GEMV && path != MQ_PATH_GEMM) return fail(MQ_EINVAL, "unknown path %d", path);
    return path;
}

int mq_quantize_act(int type, const float *x, int64_t ldx, int64_t m, int64_t k, void *workspace,
                    size_t workspace_bytes, int path, void *stream) {
    return mq_quantize_act_ex(type, x, ldx, m, k, nullptr, MQ_PRE_NONE, workspace, workspace_bytes, path, stream);
}

int mq_quantize_act_ex(int type, const float *x, int64_t ldx, int64_t m, int64_t k, const float *bias, int op,
                       void *workspace, size_t workspace_bytes, int path, void *stream) {
    if (!type_ok(type)) return fail(MQ_EUNSUPPORTED, "weight type %d is not Q8_0/Q4_K/Q6_K/F16", type);
    if (!mq_supports(type, k)) return fail(MQ_EUNSUPPORTED, "k=%lld not supported for type %d", (long long)k, type);
    if (!x || !workspace || m < 0 || m > INT32_MAX || ldx < k) return fail(MQ_EINVAL, "mq_quantize_act: bad arguments");
    if (op != MQ_PRE_NONE && op != MQ_PRE_GELU_ERF && op != MQ_PRE_SILU_MUL)
        return fail(MQ_EINVAL, "mq_quantize_act: unknown prologue op %d", op);
    if (op == MQ_PRE_SILU_MUL && ldx < 2 * k)
        return fail(MQ_EINVAL, "mq_quantize_act: MQ_PRE_SILU_MUL reads 2k = %lld values per row, ldx = %lld",
                    (long long)(2 * k), (long long)ldx);
    if (!is_aligned(workspace, 256)) return fail(MQ_EINVAL, "mq_quantize_act: workspace must be 256-byte aligned");
    if (m == 0) return MQ_OK;
    path = resolve_path(path, m);
    if (path < 0) return path;
    const bool tiled = (path == MQ_PATH_GEMM);
    const size_t need = tiled ? act_planes(type, m, k, true).total : gemv_ws_bytes(type, m, k);
    if (workspace_bytes < need)
        return fail(MQ_EINVAL, "mq_quantize_act: workspace %zu bytes < %zu needed", workspace_bytes, need);
    const hipError_t e =
        launch_quantize_act_planar(type, x, ldx, workspace, m, k, mq_q8_0_variant(), tiled, (hipStream_t)stream, op, bias);
    return e == hipSuccess ? MQ_OK : hip_fail(e, "activation quantization");
}

int mq_quantize_act_silu_mul(int type, const float *gate, const float *up, int64_t ld, int64_t m, int64_t k,
                             void *workspace, size_t workspace_bytes, int path, void *stream) {
    if (!type_ok(type)) return fail(MQ_EUNSUPPORTED, "weight type %d is not Q8_0/Q4_K/Q6_K/F16", type);
    if (!mq_supports(type, k)) return fail(MQ_EUNSUPPORTED, "k=%lld not supported for type %d", (long long)k, type);
    if (!gate || !up || !workspace || m < 0 || m > INT32_MAX || ld < k)
        return fail(MQ_EINVAL, "mq_quantize_act_silu_mul: bad arguments");
    if (!is_aligned(workspace, 256)) return fail(MQ_EINVAL, "mq_quantize_act_silu_mul: workspace must be 256-byte aligned");
    if (m == 0) return MQ_OK;
    path = resolve_path(path, m);
    if (path < 0) return path;
    const bool tiled = (path == MQ_PATH_GEMM);
    const size_t need = tiled ? act_planes(type, m, k, true).total : gemv_ws_bytes(type, m, k);
    if (workspace_bytes < need)
        return fail(MQ_EINVAL, "mq_quantize_act_silu_mul: workspace %zu bytes < %zu needed", workspace_bytes, need);
    const hipError_t e = launch_quantize_act_planar(type, gate, ld, workspace, m, k, mq_q8_0_variant(), tiled,
                                                    (hipStream_t)stream, MQ_PRE_SILU_MUL, nullptr, up);
    return e == hipSuccess ? MQ_OK : hip_fail(e, "activation quantization");
}

int mq_mul_mat_q_ex(int type, const void *w_image, int64_t n, int64_t k, const void *workspace, int64_t m, float *y,
                    int64_t ldy, const float *bias, int path, void *stream) {
    int rc = check_weight_shape(type, n, k);
    if (rc) return rc;
    if (!w_image || !workspace || !y || m < 0 || m > INT32_MAX || ldy < n) return fail(MQ_EINVAL, "mq_mul_mat_q: bad arguments");
    if (!is_aligned(w_image, 256) || !is_aligned(workspace, 256))
        return fail(MQ_EINVAL, "mq_mul_mat_q: weight image and workspace must be 256-byte aligned");
    if (m == 0) return MQ_OK;
    path = resolve_path(path, m);
    if (path < 0) return path;
    const hipError_t e = (path == MQ_PATH_GEMV)
                             ? launch_gemv(type, w_image, n, k, workspace, m, y, ldy, (hipStream_t)stream, bias)
                             : launch_gemm(type, w_image, n, k, workspace, m, y, ldy, (hipStream_t)stream, bias);
    return e == hipSuccess ? MQ_OK : hip_fail(e, path == MQ_PATH_GEMV ? "gemv" : "gemm");
}

int mq_mul_mat_q_requant(int type, const void *w_image, int64_t n, int64_t k, const void *workspace, int64_t m,
                         const float *bias, int op, int out_type, void *out_workspace, size_t out_workspace_bytes,
                         void *stream) {
    int rc = check_weight_shape(type, n, k);
    if (rc) return rc;
    const bool q8k = out_type == MQ_TYPE_Q4_K || out_type == MQ_TYPE_Q6_K;
    if (out_type != MQ_TYPE_Q8_0 && !q8k)
        return fail(MQ_EUNSUPPORTED, "mq_mul_mat_q_requant: the output type must be Q8_0, Q4_K or Q6_K");
    if (op != MQ_PRE_NONE && op != MQ_PRE_GELU_ERF)
        return fail(MQ_EINVAL, "mq_mul_mat_q_requant: op must be MQ_PRE_NONE or MQ_PRE_GELU_ERF");
    if (n % KSTAGE != 0) return fail(MQ_EINVAL, "mq_mul_mat_q_requant: n must be a multiple of %d", KSTAGE);
    if (!w_image || !workspace || !out_workspace || m < 0 || m > INT32_MAX)
        return fail(MQ_EINVAL, "mq_mul_mat_q_requant: bad arguments");
    if (!is_aligned(w_image, 256) || !is_aligned(workspace, 256) || !is_aligned(out_workspace, 256))
        return fail(MQ_EINVAL, "mq_mul_mat_q_requant: weight image and workspaces must be 256-byte aligned");
    if (m == 0) return MQ_OK;
    if (q8k && !gemm_requant_q8k_fits(type, m, n))
        return fail(MQ_EUNSUPPORTED,
                    "mq_mul_mat_q_requant: Q8_K output needs Q4_K/Q6_K weights, n a multiple of 256 and >= 256 "
                    "workgroups of 128 x 256 (type %d, m = %lld, n = %lld)",
                    type, (long long)m, (long long)n);
    const size_t need = act_planes(out_type, m, n, true).total;
    if (out_workspace_bytes < need)
        return fail(MQ_EINVAL, "mq_mul_mat_q_requant: output workspace of %zu bytes, %zu needed", out_workspace_bytes,
                    need);
    const hipError_t e = launch_gemm_requant(type, w_image, n, k, workspace, m, bias, op, mq_q8_0_variant(), out_type,
                                             out_workspace, (hipStream_t)stream);
    return e == hipSuccess ? MQ_OK : hip_fail(e, "gemm");
}

int mq_mul_mat_q_requant_supported(int type, int out_type, int64_t m, int64_t n) {
    if (!type_ok(type) || m <= 0 || m > INT32_MAX || n <= 0 || n % KSTAGE != 0) return 0;
    if (out_type == MQ_TYPE_Q8_0) return 1;
    if (out_type == MQ_TYPE_Q4_K || out_type == MQ_TYPE_Q6_K) return gemm_requant_q8k_fits(type, m, n) ? 1 : 0;
    return 0;
}

int mq_mul_mat_q_swiglu_supported(int type, int64_t n_ff, int64_t m) {
    if (!type_ok(type) || n_ff <= 0 || n_ff > INT32_MAX / 2 || m <= 0 || m > INT32_MAX) return 0;
    return gemm_swiglu_fits(m, n_ff) ? 1 : 0;
}

int mq_mul_mat_q_swiglu(int type, const void *w_image, int64_t n_ff, int64_t k, const void *workspace, int64_t m,
                        float *y, int64_t ldy, void *stream) {
    if (n_ff <= 0 || n_ff > INT32_MAX / 2) return fail(MQ_EINVAL, "mq_mul_mat_q_swiglu: bad n_ff");
    int rc = check_weight_shape(type, 2 * n_ff, k);
    if (rc) return rc;
    if (!w_image || !workspace || !y || m < 0 || m > INT32_MAX || ldy < n_ff)
        return fail(MQ_EINVAL, "mq_mul_mat_q_swiglu: bad arguments");
    if (!is_aligned(w_image, 256) || !is_aligned(workspace, 256))
        return fail(MQ_EINVAL, "mq_mul_mat_q_swiglu: weight image and workspace must be 256-byte aligned");
    if (m == 0) return MQ_OK;
    if (!gemm_swiglu_fits(m, n_ff))
        return fail(MQ_EUNSUPPORTED, "mq_mul_mat_q_swiglu: m = %lld, n_ff = %lld runs as mul_mat + quantizer prologue",
                    (long long)m, (long long)n_ff);
    const hipError_t e = launch_gemm_swiglu(type, w_image, n_ff, k, workspace, m, y, ldy, (hipStream_t)stream);
    return e == hipSuccess ? MQ_OK : hip_fail(e, "gemm");
}

int mq_mul_mat_q_qkv(int type, const void *const *w_images, const int64_t *n, int64_t k, const void *workspace,
                     int64_t m, float *y_q, int64_t ldy_q, const float *const *bias, int T, int head_dim,
                     int n_kv_head, void *kv_frags, size_t kv_frags_bytes, void *stream) {
    if (!w_images || !n || !y_q || !kv_frags || !workspace)
        return fail(MQ_EINVAL, "mq_mul_mat_q_qkv: NULL weights, n, y_q, workspace or kv_frags");
    for (int g = 0; g < 3; g++) {
        const int rc = check_weight_shape(type, n[g], k);
        if (rc) return rc;
        if (!w_images[g] || !is_aligned(w_images[g], 256))
            return fail(MQ_EINVAL, "mq_mul_mat_q_qkv: weight image %d missing or not 256-byte aligned", g);
    }
    if (head_dim != 32 && head_dim != 64 && head_dim != 128)
        return fail(MQ_EUNSUPPORTED, "mq_mul_mat_q_qkv: head_dim must be 32, 64 or 128");
    if (n_kv_head <= 0 || n[1] != (int64_t)n_kv_head * head_dim || n[2] != n[1])
        return fail(MQ_EINVAL, "mq_mul_mat_q_qkv: k and v must have n_kv_head * head_dim rows");
    if (T <= 0 || T % 32 != 0 || m <= 0 || m % T != 0 || m > INT32_MAX)
        return fail(MQ_EINVAL, "mq_mul_mat_q_qkv: m must be whole sequences of T tokens, T a multiple of 32");
    if (ldy_q < n[0] || !is_aligned(workspace, 256) || ((uintptr_t)kv_frags & 15))
        return fail(MQ_EINVAL, "mq_mul_mat_q_qkv: bad ldy_q or alignment");
    const size_t need = attn_workspace_bytes((int)(m / T), T, n_kv_head, head_dim);
    if (kv_frags_bytes < need)
        return fail(MQ_EINVAL, "mq_mul_mat_q_qkv: kv_frags of %zu bytes, %zu needed", kv_frags_bytes, need);
    const hipError_t e = launch_gemm_qkv(type, w_images, n, k, workspace, m, y_q, ldy_q, bias, T, head_dim, n_kv_head,
                                         kv_frags, (hipStream_t)stream);
    return e == hipSuccess ? MQ_OK : hip_fail(e, "gemm");
}

int mq_mul_mat_q_group(int type, int n_groups, const void *const *w_images, const int64_t *n, int64_t k,
                       const void *workspace, int64_t m, float *const *y, const int64_t *ldy, const float *const *bias,
                       int path, void *stream) {
    if (n_groups < 1 || n_groups > 4 || !w_images || !n || !y || !ldy)
        return fail(MQ_EINVAL, "mq_mul_mat_q_group: 1 to 4 groups with weights, n, y and ldy");
    for (int g = 0; g < n_groups; g++) {
        const int rc = check_weight_shape(type, n[g], k);
        if (rc) return rc;
        if (!w_images[g] || !y[g] || ldy[g] < n[g] || !is_aligned(w_images[g], 256))
            return fail(MQ_EINVAL, "mq_mul_mat_q_group: group %d: bad weight image, output or ldy", g);
    }
    if (!workspace || m < 0 || m > INT32_MAX || !is_aligned(workspace, 256))
        return fail(MQ_EINVAL, "mq_mul_mat_q_group: bad workspace or m");
    if (m == 0) return MQ_OK;
    path = resolve_path(path, m);
    if (path < 0) return path;
    if (path == MQ_PATH_GEMV && n_groups <= 3) {  // K-quants at m <= 8: one stream launch over all weights
        const hipError_t e = launch_gemv_group(type, n_groups, w_images, n, k, workspace, m, y, ldy, bias,
                                               (hipStream_t)stream);
        return e == hipSuccess ? MQ_OK : hip_fail(e, "gemv");
    }
    if (path == MQ_PATH_GEMV) {  // weight-streaming: one launch per weight costs nothing extra
        for (int g = 0; g < n_groups; g++) {
            const hipError_t e = launch_gemv(type, w_images[g], n[g], k, workspace, m, y[g], ldy[g], (hipStream_t)stream,
                                             bias ? bias[g] : nullptr);
            if (e != hipSuccess) return hip_fail(e, "gemv");
        }
        return MQ_OK;
    }
    const hipError_t e = launch_gemm_group(type, n_groups, w_images, n, k, workspace, m, y, ldy, bias, (hipStream_t)stream);
    return e == hipSuccess ? MQ_OK : hip_fail(e, "gemm");
}

int mq_mul_mat_gemv(int type, int n_groups, const void *const *w_images, const int64_t *n, int64_t k, const float *x,
                    int64_t ldx, const float *x2, int64_t ldx2, int op, int64_t m, float *const *y, const int64_t *ldy,
                    const float *const *bias, void *stream) {
    if (n_groups < 1 || n_groups > 3 || !w_images || !n || !y || !ldy || !x)
        return fail(MQ_EINVAL, "mq_mul_mat_gemv: 1 to 3 groups with weights, n, y, ldy and x");
    for (int g = 0; g < n_groups; g++) {
        const int rc = check_weight_shape(type, n[g], k);
        if (rc) return rc;
        if (!w_images[g] || !y[g] || ldy[g] < n[g] || !is_aligned(w_images[g], 256))
            return fail(MQ_EINVAL, "mq_mul_mat_gemv: group %d: bad weight image, output or ldy", g);
    }
    if (op != MQ_PRE_NONE && op != MQ_PRE_SILU_MUL) return fail(MQ_EINVAL, "mq_mul_mat_gemv: op must be MQ_PRE_NONE or MQ_PRE_SILU_MUL");
    if (op == MQ_PRE_SILU_MUL && (!x2 || ldx2 < k)) return fail(MQ_EINVAL, "mq_mul_mat_gemv: MQ_PRE_SILU_MUL needs x2");
    if (m < 0 || ldx < k) return fail(MQ_EINVAL, "mq_mul_mat_gemv: bad m or ldx");
    if (m == 0) return MQ_OK;
    if (!gemv_fused_ok(type, n_groups, k, m))
        return fail(MQ_EUNSUPPORTED, "mq_mul_mat_gemv: K-quant weights, m <= %d and k <= 6144 only", GEMV_CHUNK);
    if (!is_aligned(x, 16) || (ldx & 3) || (x2 && (!is_aligned(x2, 16) || (ldx2 & 3))))
        return fail(MQ_EINVAL, "mq_mul_mat_gemv: x / x2 must be 16-byte aligned with row strides a multiple of 4");
    // Every workgroup quantizes the whole activation it reads: that pays (a launch saved) while it
    // is a few superblock-rows, SiLU rows costing about three plain ones.  Measured on MI355X
    // (HIP-graph replay, us): q|k|v, m = 8: 5.2 fused / 6.0 two launches; down (k 6144, SiLU):
    // m = 1 7.4 / 7.7, m = 2 8.8 / 8.0.  Past that the activation is quantized once, into the
    // stream's internal workspace, and read by the GEMV: the same bytes, the same results.
    // MQ_GEMV_FUSED: 1 always quantizes inside the GEMV, 0 never (where the layout allows)
    const int force = env_int("MQ_GEMV_FUSED", -1);
    const bool side_by_side = op != MQ_PRE_SILU_MUL || (x2 == x + k && ldx2 == ldx);
    const bool two_step = force == 0 || (force < 0 && m * (k / QK_K) * (op == MQ_PRE_SILU_MUL ? 3 : 1) > 100);
    if (two_step && side_by_side) {
        void *ws = nullptr;
        size_t wsb = 0;
        int rc = stream_workspace(act_workspace_bytes(type, m, k), stream, &ws, &wsb);
        if (!rc) rc = mq_quantize_act_ex(type, x, ldx, m, k, nullptr, op, ws, wsb, MQ_PATH_GEMV, stream);
        if (!rc) rc = mq_mul_mat_q_group(type, n_groups, w_images, n, k, ws, m, y, ldy, bias, MQ_PATH_GEMV, stream);
        return rc;
    }
    const hipError_t e = launch_gemv_group_f32(type, n_groups, w_images, n, k, x, ldx, op == MQ_PRE_SILU_MUL ? x2 : nullptr,
                                               ldx2, op, m, y, ldy, bias, (hipStream_t)stream);
    return e == hipSuccess ? MQ_OK : hip_fail(e, "gemv");
}

int mq_mul_mat_q(int type, const void *w_image, int64_t n, int64_t k, const void *workspace, int64_t m, float *y,
                 int64_t ldy, int path, void *stream) {
    return mq_mul_mat_q_ex(type, w_image, n, k, workspace, m, y, ldy, nullptr, path, stream);
}

int mq_mul_mat_ex(int type, const void *w_image, int64_t n, int64_t k, const float *x, int64_t ldx, int64_t m,
                  float *y, int64_t ldy, void *workspace, size_t workspace_bytes, int path, void *stream) {
    int rc = check_weight_shape(type, n, k);
    if (rc) return rc;
    if (!w_image || !x || !y) return fail(MQ_EINVAL, "mq_mul_mat: NULL pointer");
    if (m < 0 || m > INT32_MAX || ldx < k || ldy < n) return fail(MQ_EINVAL, "mq_mul_mat: bad m/ldx/ldy");
    if (m == 0) return MQ_OK;
    if (!is_aligned(w_image, 256)) return fail(MQ_EINVAL, "mq_mul_mat: weight image must be 256-byte aligned");
    if (path == MQ_PATH_AUTO) path = mq_mul_mat_path(type, n, k, m);
    path = resolve_path(path, m);
    if (path < 0) return path;
    const size_t need = act_workspace_bytes(type, m, k);
    void *ws = workspace;
    if (ws) {
        if (workspace_bytes < need)
            return fail(MQ_EINVAL, "mq_mul_mat: workspace %zu bytes < %zu needed", workspace_bytes, need);
    } else {
        rc = stream_workspace(need, stream, &ws, &workspace_bytes);
        if (rc) return rc;
    }
    rc = mq_quantize_act(type, x, ldx, m, k, ws, workspace_bytes, path, stream);
    if (rc) return rc;
    return mq_mul_mat_q(type, w_image, n, k, ws, m, y, ldy, path, stream);
}

int mq_mul_mat(int type, const void *w_image, int64_t n, int64_t k, const float *x, int64_t ldx, int64_t m, float *y,
               int64_t ldy, void *workspace, size_t workspace_bytes, void *stream) {
    return mq_mul_mat_ex(type, w_image, n, k, x, ldx, m, y, ldy, workspace, workspace_bytes, MQ_PATH_AUTO, stream);
}

}  // extern "C"

namespace {

// The quantized activations of mq_mul_mat_noalloc: a file-scope device array, so the call needs
// no allocation.  Each GPU holds its own copy at its own address, found once per device with
// hipGetSymbolAddress (the array's name is only a host-side stand-in for the device address).
static __device__ __align__(256) uint8_t scratch[MQ_NOALLOC_SCRATCH_BYTES];

std::mutex g_scratch_mu;
void *g_scratch[64];  // per HIP device ordinal: the device address of `scratch`

int scratch_ptr(void **out) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return hip_fail(e, "hipGetDevice");
    if (dev < 0 || dev >= 64) return fail(MQ_EINVAL, "device ordinal %d", dev);
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    if (!g_scratch[dev]) {
        void *p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !p) return hip_fail(e != hipSuccess ? e : hipErrorInvalidSymbol, "hipGetSymbolAddress");
        g_scratch[dev] = p;
    }
    *out = g_scratch[dev];
    return MQ_OK;
}

}  // namespace

extern "C" {

int mq_mul_mat_noalloc(int type, const void *w_image, int64_t n, int64_t k, const float *x, int64_t ldx, int64_t m,
                       float *y, int64_t ldy, int path, void *stream) {
    int rc = check_weight_shape(type, n, k);
    if (rc) return rc;
    if (!w_image || !x || !y) return fail(MQ_EINVAL, "mq_mul_mat_noalloc: NULL pointer");
    if (m < 0 || m > INT32_MAX || ldx < k || ldy < n) return fail(MQ_EINVAL, "mq_mul_mat_noalloc: bad m/ldx/ldy");
    if (m == 0) return MQ_OK;
    if (!is_aligned(w_image, 256)) return fail(MQ_EINVAL, "mq_mul_mat_noalloc: weight image must be 256-byte aligned");
    if (path == MQ_PATH_AUTO) path = mq_mul_mat_path(type, n, k, m);
    path = resolve_path(path, m);
    if (path < 0) return path;
    const size_t need = act_workspace_bytes(type, m, k);
    if (need > (size_t)MQ_NOALLOC_SCRATCH_BYTES)
        return fail(MQ_EINVAL, "mq_mul_mat_noalloc: m=%lld x k=%lld needs %zu bytes of activations, more than the %u-byte "
                    "scratch array", (long long)m, (long long)k, need, (unsigned)MQ_NOALLOC_SCRATCH_BYTES);
    void *ws = nullptr;
    rc = scratch_ptr(&ws);
    if (rc) return rc;
    // every byte the kernels read is written first by the quantizer (pad rows and pad K bytes
    // included), so the previous call's contents need no clearing
    rc = mq_quantize_act(type, x, ldx, m, k, ws, MQ_NOALLOC_SCRATCH_BYTES, path, stream);
    if (rc) return rc;
    return mq_mul_mat_q(type, w_image, n, k, ws, m, y, ldy, path, stream);
}

}  // extern "C"
