// mq_decoder_run.cpp -- native decoder-embedder runner on the quantized MUL_MAT path (mq_decoder.h).
//
// Per layer (pre-norm Qwen3 block, src/decoder_embed.cpp:718-814):
//   Hn   = rms_norm(X) * attn_norm                  (fused with the previous residual ADD)
//   qkv  = Hn . [Wq; Wk; Wv]^T                      one mul_mat over the concatenated rows
//   A    = causal GQA attention(rope(rms_norm_head(q) * q_norm),
//                               rope(rms_norm_head(k) * k_norm), v)
//          the per-head norms and rotations applied as the attention kernels load q and k
//   X    = X + A . Wo^T;  Hn = rms_norm(X) * ffn_norm
//   gu   = Hn . [Wgate; Wup]^T                      one mul_mat, gate and up side by side
//   X    = X + (silu(gate) * up) . Wdown^T          the product formed in the gate|up GEMM's
//                                                   store (large batches) or by the quantizer
// then the output RMS norm of the pooled rows and L2 normalisation.
#include <hip/hip_runtime.h>

#include <cstdlib>

#include <cmath>
#include <cstring>
#include <mutex>
#include <vector>

#include "../../include/mq.h"
#include "../../include/mq_decoder.h"
#include "mq_internal.h"
#include "mq_runner.h"

namespace mq {
hipError_t launch_add_rmsnorm(const float *y, const float *res, const int32_t *ids, const float *tok, int n_vocab,
                              const float *w, float eps, float *xout, float *hout, int64_t rows, int H, hipStream_t s);
hipError_t launch_qk_norm_rope(float *qkv, int64_t ld, const float *qw, const float *kw, float eps, int nq, int nkv,
                               int hd, int T, float theta_base, int64_t rows, float2 *cs, hipStream_t s);
size_t attn_workspace_bytes(int B, int T, int nkv, int hd);
hipError_t launch_rope_table(float2 *cs, int T, int hd, float theta_base, hipStream_t s);
hipError_t launch_attn_frag(const float *qkv, int64_t ld, float *out, int64_t ldo, int B, int T, int nq, int nkv,
                            int hd, float scale, int causal, const float *qw, const float *kw, float eps,
                            const float2 *cs, void *ws, hipStream_t s, void *q_ws = nullptr,
                            int q_type = MQ_TYPE_Q8_0, bool q_only = false);
hipError_t launch_last_rmsnorm_l2(const float *x, const float *w, float eps, float *out, int B, int T, int H,
                                  hipStream_t s);
hipError_t launch_mean_pool_l2(const float *x, float *out, int B, int T, int H, hipStream_t s);  // mq_encoder.hip
}  // namespace mq

using namespace mq;

namespace {
struct DecLayer {
    Linear qkv, o, gu, down;
    DevBuf attn_norm, ffn_norm, q_norm, k_norm;
    bool has_qn = false, has_kn = false;
};
}  // namespace

struct mq_decoder {
    mq_decoder_hparams hp{};
    DevBuf tok, out_norm;
    std::vector<DecLayer> layers;
    DevBuf x, h, qkv, att, y, gu, ws, rope, kvf;
    mq_decoder_observer obs = nullptr;
    void *obs_user = nullptr;
};

extern "C" int mq_decoder_set_observer(mq_decoder *m, mq_decoder_observer cb, void *user) {
    if (!m) return set_error(MQ_EINVAL, "NULL runner");
    m->obs = cb;
    m->obs_user = user;
    return MQ_OK;
}

extern "C" mq_decoder *mq_decoder_create(const mq_decoder_hparams *hp) {
    if (!hp || hp->n_layer <= 0 || hp->n_embd <= 0 || hp->n_head <= 0 || hp->n_kv_head <= 0 ||
        hp->n_head % hp->n_kv_head != 0 || hp->n_ff <= 0 || hp->n_vocab <= 0 || !(hp->rms_norm_eps > 0.f) ||
        !(hp->rope_theta > 0.f) || (hp->pooling != 1 && hp->pooling != 2)) {
        set_error(MQ_EINVAL, "bad decoder hyper-parameters");
        return nullptr;
    }
    if (hp->head_dim != 64 && hp->head_dim != 128) {
        set_error(MQ_EUNSUPPORTED, "head_dim %d (this runner takes 64 or 128)", hp->head_dim);
        return nullptr;
    }
    if (hp->n_embd > 4096) {
        set_error(MQ_EUNSUPPORTED, "n_embd %d > 4096", hp->n_embd);
        return nullptr;
    }
    const int q_dim = hp->n_head * hp->head_dim;
    if (!mq_supports(hp->wtype, hp->n_embd) || !mq_supports(hp->wtype, hp->n_ff) || !mq_supports(hp->wtype, q_dim)) {
        set_error(MQ_EUNSUPPORTED, "weight type %d does not tile k = %d / %d / %d", hp->wtype, hp->n_embd, hp->n_ff,
                  q_dim);
        return nullptr;
    }
    mq_decoder *m = new mq_decoder();
    m->hp = *hp;
    m->layers.resize(hp->n_layer);
    return m;
}

extern "C" void mq_decoder_free(mq_decoder *m) { delete m; }

extern "C" int mq_decoder_set_embeddings(mq_decoder *m, const float *tok, const float *out_norm) {
    if (!m || !tok || !out_norm) return set_error(MQ_EINVAL, "NULL embedding table / output norm");
    const size_t H = (size_t)m->hp.n_embd * sizeof(float);
    int rc;
    if ((rc = upload(m->tok, tok, H * m->hp.n_vocab))) return rc;
    return upload(m->out_norm, out_norm, H);
}

extern "C" int mq_decoder_set_layer(mq_decoder *m, int il, const void *wq, const void *wk, const void *wv,
                                    const void *wo, const void *wgate, const void *wup, const void *wdown,
                                    const float *attn_norm, const float *ffn_norm, const float *q_norm,
                                    const float *k_norm) {
    if (!m || il < 0 || il >= m->hp.n_layer) return set_error(MQ_EINVAL, "bad layer index %d", il);
    if (!attn_norm || !ffn_norm) return set_error(MQ_EINVAL, "NULL norm weight");
    DecLayer &L = m->layers[il];
    const mq_decoder_hparams &hp = m->hp;
    const int t = hp.wtype;
    const int64_t H = hp.n_embd, F = hp.n_ff, qd = (int64_t)hp.n_head * hp.head_dim,
                  kvd = (int64_t)hp.n_kv_head * hp.head_dim;
    const size_t f4 = sizeof(float);
    int rc;
    if ((rc = upload_linear(L.qkv, t, {wq, wk, wv}, {qd, kvd, kvd}, H))) return rc;
    if ((rc = upload_linear(L.o, t, {wo}, {H}, qd))) return rc;
    if ((rc = upload_linear(L.gu, t, {wgate, wup}, {F, F}, H))) return rc;
    if ((rc = upload_linear(L.down, t, {wdown}, {H}, F))) return rc;
    if ((rc = upload(L.attn_norm, attn_norm, H * f4))) return rc;
    if ((rc = upload(L.ffn_norm, ffn_norm, H * f4))) return rc;
    L.has_qn = q_norm != nullptr;
    L.has_kn = k_norm != nullptr;
    if (q_norm && (rc = upload(L.q_norm, q_norm, hp.head_dim * f4))) return rc;
    if (k_norm && (rc = upload(L.k_norm, k_norm, hp.head_dim * f4))) return rc;
    return MQ_OK;
}

extern "C" int mq_decoder_encode(mq_decoder *m, const int32_t *ids, int B, int T, float *out, float *hidden,
                                 void *stream) {
    if (!m || !ids || !out || B <= 0 || T <= 0) return set_error(MQ_EINVAL, "bad encode arguments");
    const mq_decoder_hparams &hp = m->hp;
    for (const DecLayer &L : m->layers)
        if (!L.qkv.img.p) return set_error(MQ_EINVAL, "layer weights not set");
    if (!m->tok.p) return set_error(MQ_EINVAL, "embeddings not set");
    const int64_t rows = (int64_t)B * T, H = hp.n_embd, F = hp.n_ff;
    const int hd = hp.head_dim, nq = hp.n_head, nkv = hp.n_kv_head;
    const int64_t qd = (int64_t)nq * hd, ldqkv = qd + 2 * (int64_t)nkv * hd;
    const int t = hp.wtype;
    const size_t f4 = sizeof(float);
    const size_t wsb = std::max({mq_workspace_bytes(t, rows, H), mq_workspace_bytes(t, rows, qd),
                                 mq_workspace_bytes(t, rows, F)});
    if (!m->x.ensure(rows * H * f4) || !m->h.ensure(rows * H * f4) || !m->qkv.ensure(rows * ldqkv * f4) ||
        !m->att.ensure(rows * qd * f4) || !m->y.ensure(rows * H * f4) || !m->gu.ensure(rows * 2 * F * f4) ||
        !m->ws.ensure(wsb) || !m->rope.ensure((size_t)T * (hd / 2) * sizeof(float2)) ||
        !m->kvf.ensure(attn_workspace_bytes(B, T, nkv, hd)))
        return set_error(MQ_ENOMEM, "activation buffers for %lld rows", (long long)rows);
    hipStream_t s = (hipStream_t)stream;
    const float eps = hp.rms_norm_eps;
    float *X = hidden ? hidden : m->x.f();
    float *Hn = m->h.f();
    int rc;
    // the observer sees a tensor once the work producing it is done
    auto observe = [&](const char *name, int il, const float *x, int64_t cols, bool quantized) {
        if (!m->obs) return MQ_OK;
        if (hipStreamSynchronize(s) != hipSuccess) return set_error(MQ_EHIP, "stream synchronisation failed");
        m->obs(name, il, x, rows, cols, quantized ? m->ws.p : nullptr, quantized ? m->ws.bytes : 0, m->obs_user);
        return MQ_OK;
    };
    // a mat-mul of an fp32 input, quantized first (and observed under `name` when set)
    auto mm = [&](const Linear &L, const float *in, int64_t ldin, float *y, const char *name = nullptr, int il = 0) {
        const int path = mq_mul_mat_path(t, L.n, L.k, rows);
        int r = mq_quantize_act(t, in, ldin, rows, L.k, m->ws.p, m->ws.bytes, path, s);
        if (!r && name) r = observe(name, il, in, L.k, true);
        return r ? r : mq_mul_mat_q(t, L.img.p, L.n, L.k, m->ws.p, rows, y, L.n, path, s);
    };
    // X = token_embd[ids]; Hn = rms_norm(X) * attn_norm[0]
    if ((rc = hip_rc(launch_add_rmsnorm(nullptr, nullptr, ids, m->tok.f(), hp.n_vocab, m->layers[0].attn_norm.f(), eps, X, Hn, rows,
                                        (int)H, s),
                     "embedding")))
        return rc;
    if ((rc = hip_rc(launch_rope_table((float2 *)m->rope.p, T, hd, hp.rope_theta, s), "rope table"))) return rc;
    // K-quant weights with the qkv and gate|up products on the GEMM path: the residual + RMS norm
    // also leaves its result as their Q8_K activation (launch_add_rmsnorm_q8_K), so Hn is not
    // quantized again.  hn_q: the workspace holds Hn quantized.
    const bool norm_q = (t == MQ_TYPE_Q4_K || t == MQ_TYPE_Q6_K) && H % 256 == 0 && H <= 2048 &&
                        !m->layers.empty() && mq_mul_mat_path(t, m->layers[0].qkv.n, H, rows) == MQ_PATH_GEMM &&
                        mq_mul_mat_path(t, m->layers[0].gu.n, H, rows) == MQ_PATH_GEMM &&
                        std::getenv("MQ_DECODER_NORM_PASS") == nullptr;
    bool hn_q = false;
    auto mm_hn = [&](const Linear &L, float *y, const char *name, int il) {  // a product of Hn
        if (!hn_q) return mm(L, Hn, H, y, name, il);
        int r = observe(name, il, Hn, H, true);
        return r ? r : mq_mul_mat_q(t, L.img.p, L.n, L.k, m->ws.p, rows, y, L.n, MQ_PATH_GEMM, s);
    };
    auto add_norm = [&](const float *w, const char *what, bool last) {  // X += y; Hn = rms_norm(X) * w
        if (norm_q) {  // inside the stack Hn is read only in its quantized form: not written (unless observed)
            hn_q = true;
            return hip_rc(launch_add_rmsnorm_q8_K(m->y.f(), X, w, eps, X, (last || m->obs) ? Hn : nullptr, rows, (int)H,
                                                  m->ws.p, s),
                          what);
        }
        return hip_rc(launch_add_rmsnorm(m->y.f(), X, nullptr, nullptr, 0, w, eps, X, Hn, rows, (int)H, s), what);
    };
    // K-quant o projections on the GEMM path read the attention rows as the attention stores
    // them quantized (Q8_K; launch_attn quantizes its fp32 output itself where its kernel
    // cannot); MQ_DECODER_ATTN_QPASS=1 keeps the separate quantizer
    const bool att_q = (t == MQ_TYPE_Q4_K || t == MQ_TYPE_Q6_K) && qd % 256 == 0 && !m->layers.empty() &&
                       mq_mul_mat_path(t, m->layers[0].o.n, qd, rows) == MQ_PATH_GEMM &&
                       std::getenv("MQ_DECODER_ATTN_QPASS") == nullptr;
    // the gate|up GEMM forms silu(gate) * up in its store where the shape allows (not while
    // observed: the observer reads gate and up); MQ_DECODER_NO_GLU=1 keeps the two-step form
    const bool glu = !m->obs && !m->layers.empty() && gemm_swiglu_fits(rows, F) &&
                     mq_mul_mat_path(t, m->layers[0].gu.n, H, rows) == MQ_PATH_GEMM &&
                     std::getenv("MQ_DECODER_NO_GLU") == nullptr;
    for (size_t il = 0; il < m->layers.size(); il++) {
        const DecLayer &L = m->layers[il];
        if ((rc = mm_hn(L.qkv, m->qkv.f(), "attn_norm", (int)il))) return rc;
        hn_q = false;
        if ((rc = hip_rc(launch_attn_frag(m->qkv.f(), ldqkv, m->att.f(), qd, B, T, nq, nkv, hd,
                                          1.0f / sqrtf((float)hd), hp.causal, L.has_qn ? L.q_norm.f() : nullptr,
                                          L.has_kn ? L.k_norm.f() : nullptr, eps, (const float2 *)m->rope.p,
                                          m->kvf.p, s, att_q ? m->ws.p : nullptr, t, att_q && !m->obs),
                         "attention")))
            return rc;
        if (att_q) {  // the attention left its rows quantized in the workspace
            if ((rc = observe("attn_out", (int)il, m->att.f(), qd, true))) return rc;
            if ((rc = mq_mul_mat_q(t, L.o.img.p, L.o.n, L.o.k, m->ws.p, rows, m->y.f(), L.o.n, MQ_PATH_GEMM, s)))
                return rc;
        } else if ((rc = mm(L.o, m->att.f(), qd, m->y.f(), "attn_out", (int)il))) {
            return rc;
        }
        // X += A Wo^T; Hn = rms_norm(X) * ffn_norm
        if ((rc = add_norm(L.ffn_norm.f(), "attention residual", false))) return rc;
        const int dpath = mq_mul_mat_path(t, L.down.n, L.down.k, rows);
        if (glu) {
            // silu(gate) * up formed in the gate|up GEMM's store (F columns), then quantized as is
            if (!hn_q && (rc = mq_quantize_act(t, Hn, H, rows, H, m->ws.p, m->ws.bytes, MQ_PATH_GEMM, s))) return rc;
            hn_q = false;
            if ((rc = mq_mul_mat_q_swiglu(t, L.gu.img.p, F, H, m->ws.p, rows, m->gu.f(), F, s))) return rc;
            if ((rc = mq_quantize_act(t, m->gu.f(), F, rows, F, m->ws.p, m->ws.bytes, dpath, s))) return rc;
        } else {
            if ((rc = mm_hn(L.gu, m->gu.f(), "ffn_norm", (int)il))) return rc;
            hn_q = false;
            // down projection of silu(gate) * up, the product formed inside the quantizer
            if ((rc = mq_quantize_act_ex(t, m->gu.f(), 2 * F, rows, F, nullptr, MQ_PRE_SILU_MUL, m->ws.p,
                                         m->ws.bytes, dpath, s)))
                return rc;
            if ((rc = observe("ffn_gate_up", (int)il, m->gu.f(), 2 * F, true))) return rc;
        }
        if ((rc = mq_mul_mat_q(t, L.down.img.p, L.down.n, L.down.k, m->ws.p, rows, m->y.f(), H, dpath, s)))
            return rc;
        // X += FFN; Hn = rms_norm(X) * (next layer's attn_norm, or the output norm)
        const float *wn = (il + 1 < m->layers.size()) ? m->layers[il + 1].attn_norm.f() : m->out_norm.f();
        if ((rc = add_norm(wn, "ffn residual", il + 1 == m->layers.size()))) return rc;
        if ((rc = observe("l_out", (int)il, X, H, false))) return rc;
    }
    // mean pooling averages the output-normed rows (Hn); last-token pooling norms the last row
    if (hp.pooling == 1) return hip_rc(launch_mean_pool_l2(Hn, out, B, T, (int)H, s), "pooling");
    return hip_rc(launch_last_rmsnorm_l2(X, m->out_norm.f(), eps, out, B, T, (int)H, s), "pooling");
}

extern "C" int mq_qk_norm_rope(float *qkv, int64_t ld, const float *q_norm, const float *k_norm, float eps, int n_head,
                               int n_kv_head, int head_dim, int T, float theta, int64_t rows, void *stream) {
    if (!qkv || n_head <= 0 || n_kv_head <= 0 || T <= 0 || rows < 0 || !(theta > 0.f) ||
        ld < (int64_t)(n_head + 2 * n_kv_head) * head_dim)
        return set_error(MQ_EINVAL, "mq_qk_norm_rope: bad arguments");
    if (head_dim != 64 && head_dim != 128) return set_error(MQ_EUNSUPPORTED, "head_dim %d (64 or 128)", head_dim);
    // the angle table lives in a per-process buffer that only grows; the caller's stream is
    // synchronised before it is replaced, and calls that overlap on two streams must not
    // use different T or head_dim
    // (never freed: it may outlive the HIP runtime at process exit)
    static std::mutex mu;
    static DevBuf *table = new DevBuf();
    std::lock_guard<std::mutex> lk(mu);
    const size_t need = (size_t)T * (head_dim / 2) * sizeof(float2);
    if (need > table->bytes) {
        if (hipDeviceSynchronize() != hipSuccess) return set_error(MQ_EHIP, "hipDeviceSynchronize failed");
        if (!table->ensure(need)) return set_error(MQ_ENOMEM, "hipMalloc(%zu) failed", need);
    }
    return hip_rc(launch_qk_norm_rope(qkv, ld, q_norm, k_norm, eps, n_head, n_kv_head, head_dim, T, theta, rows,
                                      (float2 *)table->p, (hipStream_t)stream),
                  "q/k norm + rope");
}

extern "C" size_t mq_attention_workspace_bytes(int B, int T, int n_kv_head, int head_dim) {
    if (B <= 0 || T <= 0 || n_kv_head <= 0 || (head_dim != 64 && head_dim != 128)) return 0;
    return attn_workspace_bytes(B, T, n_kv_head, head_dim);
}

extern "C" int mq_attention(const float *qkv, int64_t ld, float *out, int64_t ldo, int B, int T, int n_head,
                            int n_kv_head, int head_dim, float scale, int causal, void *workspace,
                            size_t workspace_bytes, void *stream) {
    if (!qkv || !out || B <= 0 || T <= 0 || n_head <= 0 || n_kv_head <= 0 || n_head % n_kv_head != 0 ||
        ld % 4 != 0 || ((uintptr_t)qkv & 15) != 0 || ld < (int64_t)(n_head + 2 * n_kv_head) * head_dim ||
        ldo < (int64_t)n_head * head_dim)
        return set_error(MQ_EINVAL, "mq_attention: bad arguments");
    if (head_dim != 64 && head_dim != 128) return set_error(MQ_EUNSUPPORTED, "head_dim %d (64 or 128)", head_dim);
    const size_t need = attn_workspace_bytes(B, T, n_kv_head, head_dim);
    if (!workspace || ((uintptr_t)workspace & 15) != 0 || workspace_bytes < need)
        return set_error(MQ_EINVAL, "mq_attention: workspace of %zu bytes (16-byte aligned) needed, %zu given", need,
                         workspace_bytes);
    return hip_rc(launch_attn_frag(qkv, ld, out, ldo, B, T, n_head, n_kv_head, head_dim, scale, causal, nullptr,
                                   nullptr, 0.f, nullptr, workspace, (hipStream_t)stream),
                  "attention");
}

extern "C" int mq_decoder_get_hparams(const mq_decoder *m, mq_decoder_hparams *hp) {
    if (!m || !hp) return set_error(MQ_EINVAL, "NULL runner or output");
    *hp = m->hp;
    return MQ_OK;
}
