// mq_runner.h -- device buffers and weight uploads shared by the model runners
// (mq_bert.cpp, mq_decoder.cpp).  Host code; errors go through mq::set_error.
#pragma once
#include <hip/hip_runtime.h>

#include <vector>

#include "../../include/mq.h"

namespace mq {
int set_error(int code, const char *fmt, ...) __attribute__((format(printf, 2, 3)));  // mq_api.cpp

// A device allocation that only grows.
struct DevBuf {
    void *p = nullptr;
    size_t bytes = 0;
    DevBuf() = default;
    DevBuf(const DevBuf &) = delete;
    DevBuf &operator=(const DevBuf &) = delete;
    DevBuf(DevBuf &&o) noexcept : p(o.p), bytes(o.bytes) { o.p = nullptr, o.bytes = 0; }
    ~DevBuf() {
        if (p) (void)hipFree(p);
    }
    bool ensure(size_t n) {
        if (n <= bytes) return true;
        if (p) (void)hipFree(p);
        p = nullptr;
        bytes = 0;
        if (hipMalloc(&p, n) != hipSuccess) {
            (void)hipGetLastError();  // a failed allocation must not surface as the next launch's error
            return false;
        }
        bytes = n;
        return true;
    }
    float *f() const { return (float *)p; }
};

// A prepared weight image of n x k.
struct Linear {
    DevBuf img;
    int64_t n = 0, k = 0;
};

inline int upload(DevBuf &d, const void *src, size_t bytes) {
    if (!src) return set_error(MQ_EINVAL, "NULL host tensor");
    if (!d.ensure(bytes)) return set_error(MQ_ENOMEM, "hipMalloc(%zu) failed", bytes);
    if (hipMemcpy(d.p, src, bytes, hipMemcpyHostToDevice) != hipSuccess)
        return set_error(MQ_EHIP, "hipMemcpy of %zu bytes failed", bytes);
    return MQ_OK;
}

// The GGUF rows of one or more weights with the same k, concatenated in order into one
// prepared image (rows are independent dot products, so one mul_mat over the
// concatenation equals the separate mul_mats side by side in its output columns).
inline int upload_linear(Linear &L, int type, const std::vector<const void *> &parts, const std::vector<int64_t> &rows,
                         int64_t k) {
    const size_t rs = mq_row_size(type, k);
    if (rs == 0 || parts.size() != rows.size()) return set_error(MQ_EINVAL, "bad weight type %d / k %lld", type, (long long)k);
    int64_t n = 0;
    for (int64_t r : rows) n += r;
    const size_t img = mq_weight_image_bytes(type, n, k);
    if (!L.img.ensure(img)) return set_error(MQ_ENOMEM, "hipMalloc(%zu) failed", img);
    size_t off = 0;
    for (size_t i = 0; i < parts.size(); i++) {
        if (!parts[i]) return set_error(MQ_EINVAL, "NULL weight");
        if (hipMemcpy((char *)L.img.p + off, parts[i], rows[i] * rs, hipMemcpyHostToDevice) != hipSuccess)
            return set_error(MQ_EHIP, "hipMemcpy of weights failed");
        off += rows[i] * rs;
    }
    L.n = n;
    L.k = k;
    const int rc = mq_weight_prepare(type, L.img.p, n, k, 0, n, nullptr);
    if (rc) return rc;
    return hipDeviceSynchronize() == hipSuccess ? MQ_OK : set_error(MQ_EHIP, "weight preparation failed");
}

inline int hip_rc(hipError_t e, const char *what) {
    return e == hipSuccess ? MQ_OK : set_error(MQ_EHIP, "%s: %s", what, hipGetErrorString(e));
}

}  // namespace mq
