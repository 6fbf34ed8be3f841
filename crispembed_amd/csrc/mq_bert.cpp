// mq_bert.cpp -- native BERT-encoder runner on the quantized MUL_MAT path (mq_bert.h).
//
// Per layer (post-LN BERT, src/crispembed.cpp:1159-1436):
//   qkv  = X . [Wq; Wk; Wv]^T        one mul_mat: the three weights' GGUF rows are
//                                    concatenated into one [3H x H] image (rows are
//                                    independent dot products, so this is exact)
//   A    = attention(qkv + b_qkv)    fp32, scale 1/sqrt(head_dim), full mask
//   X    = LN1(X + A . Wo^T + bo)
//   Hh   = gelu_erf(X . W1^T + b1)
//   X    = LN2(X + Hh . W2^T + b2)
// then mean pooling and L2 normalisation.  Device memory comes from hipMalloc; the
// activation buffers grow to the largest B*T seen.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdlib>
#include <cstring>
#include <vector>

#include "../../include/mq.h"
#include "../../include/mq_bert.h"
#include "../../include/mq_ops.h"
#include "mq_internal.h"
#include "mq_runner.h"

namespace mq {
hipError_t launch_embed_ln(const int32_t *ids, const int32_t *types, const float *word, const float *pos,
                           const float *type, const float *lw, const float *lb, float eps, float *out, int64_t rows,
                           int T, int H, int n_vocab, int n_type, hipStream_t s);
hipError_t launch_bias_res_ln(const float *y, const float *bias, const float *res, const float *lw, const float *lb,
                              float eps, float *out, int64_t rows, int H, hipStream_t s);
hipError_t launch_attention(const float *qkv, const float *bqkv, float *out, int B, int T, int H, int nh,
                            hipStream_t s);
hipError_t launch_mean_pool_l2(const float *x, float *out, int B, int T, int H, hipStream_t s);
}  // namespace mq

using namespace mq;

namespace {

struct Layer {
    Linear qkv, o, fc1, fc2;
    DevBuf bqkv, bo, b1, b2, ln1w, ln1b, ln2w, ln2b;
};

}  // namespace

struct mq_bert {
    mq_bert_hparams hp{};
    DevBuf tok, pos, type, lnw, lnb;
    std::vector<Layer> layers;
    DevBuf x, qkv, att, y, ff, ws, ws2, aws;
    int64_t rows_cap = 0;
};

extern "C" mq_bert *mq_bert_create(const mq_bert_hparams *hp) {
    if (!hp || hp->n_layer <= 0 || hp->n_embd <= 0 || hp->n_head <= 0 || hp->n_embd % hp->n_head != 0 ||
        hp->n_ff <= 0 || hp->n_vocab <= 0 || hp->n_max_pos <= 0 || hp->n_type < 0) {
        set_error(MQ_EINVAL, "bad BERT hyper-parameters");
        return nullptr;
    }
    if (!mq_supports(hp->wtype, hp->n_embd) || !mq_supports(hp->wtype, hp->n_ff)) {
        set_error(MQ_EUNSUPPORTED, "weight type %d does not tile k = %d / %d", hp->wtype, hp->n_embd, hp->n_ff);
        return nullptr;
    }
    mq_bert *m = new mq_bert();
    m->hp = *hp;
    m->layers.resize(hp->n_layer);
    return m;
}

extern "C" void mq_bert_free(mq_bert *m) { delete m; }

extern "C" int mq_bert_set_embeddings(mq_bert *m, const float *tok, const float *pos, const float *type,
                                      const float *ln_w, const float *ln_b) {
    if (!m || !tok || !pos || !ln_w || !ln_b || (m->hp.n_type > 0 && !type))
        return set_error(MQ_EINVAL, "NULL embedding table");
    const size_t H = (size_t)m->hp.n_embd * sizeof(float);
    int rc;
    if ((rc = upload(m->tok, tok, H * m->hp.n_vocab))) return rc;
    if ((rc = upload(m->pos, pos, H * m->hp.n_max_pos))) return rc;
    if (m->hp.n_type > 0 && (rc = upload(m->type, type, H * m->hp.n_type))) return rc;
    if ((rc = upload(m->lnw, ln_w, H))) return rc;
    return upload(m->lnb, ln_b, H);
}

extern "C" int mq_bert_set_layer(mq_bert *m, int il, const void *wq, const void *wk, const void *wv, const void *wo,
                                 const void *w1, const void *w2, const float *bq, const float *bk, const float *bv,
                                 const float *bo, const float *b1, const float *b2, const float *ln1_w,
                                 const float *ln1_b, const float *ln2_w, const float *ln2_b) {
    if (!m || il < 0 || il >= m->hp.n_layer) return set_error(MQ_EINVAL, "bad layer index %d", il);
    if (!bq || !bk || !bv || !bo || !b1 || !b2 || !ln1_w || !ln1_b || !ln2_w || !ln2_b)
        return set_error(MQ_EINVAL, "NULL bias / LayerNorm parameter");
    Layer &L = m->layers[il];
    const int t = m->hp.wtype;
    const int64_t H = m->hp.n_embd, F = m->hp.n_ff;
    int rc;
    if ((rc = upload_linear(L.qkv, t, {wq, wk, wv}, {H, H, H}, H))) return rc;
    if ((rc = upload_linear(L.o, t, {wo}, {H}, H))) return rc;
    if ((rc = upload_linear(L.fc1, t, {w1}, {F}, H))) return rc;
    if ((rc = upload_linear(L.fc2, t, {w2}, {H}, F))) return rc;
    std::vector<float> bqkv(3 * H);
    std::memcpy(bqkv.data(), bq, H * sizeof(float));
    std::memcpy(bqkv.data() + H, bk, H * sizeof(float));
    std::memcpy(bqkv.data() + 2 * H, bv, H * sizeof(float));
    if ((rc = upload(L.bqkv, bqkv.data(), 3 * H * sizeof(float)))) return rc;
    if ((rc = upload(L.bo, bo, H * sizeof(float)))) return rc;
    if ((rc = upload(L.b1, b1, F * sizeof(float)))) return rc;
    if ((rc = upload(L.b2, b2, H * sizeof(float)))) return rc;
    if ((rc = upload(L.ln1w, ln1_w, H * sizeof(float)))) return rc;
    if ((rc = upload(L.ln1b, ln1_b, H * sizeof(float)))) return rc;
    if ((rc = upload(L.ln2w, ln2_w, H * sizeof(float)))) return rc;
    return upload(L.ln2b, ln2_b, H * sizeof(float));
}

extern "C" int mq_bert_encode(mq_bert *m, const int32_t *ids, const int32_t *types, int B, int T, float *out,
                              float *hidden, void *stream) {
    if (!m || !ids || !out || B <= 0 || T <= 0) return set_error(MQ_EINVAL, "bad encode arguments");
    const mq_bert_hparams &hp = m->hp;
    if (T > hp.n_max_pos) return set_error(MQ_EINVAL, "T = %d exceeds n_max_pos = %d", T, hp.n_max_pos);
    for (const Layer &L : m->layers)
        if (!L.qkv.img.p) return set_error(MQ_EINVAL, "layer weights not set");
    if (!m->tok.p) return set_error(MQ_EINVAL, "embeddings not set");
    const int64_t rows = (int64_t)B * T, H = hp.n_embd, F = hp.n_ff;
    const int t = hp.wtype;
    const size_t f4 = sizeof(float);
    const size_t wsb = std::max({mq_workspace_bytes(t, rows, H), mq_workspace_bytes(t, rows, F)});
    // FFN on the GEMM path: the FFN-up GEMM adds its bias, applies GELU-erf and quantizes its
    // own output for the FFN-down GEMM (mq_mul_mat_q_requant: Q8_0, or Q8_K for the K-quants at
    // the sizes its 128 x 256 tiles fill the GPU), into the second workspace
    const bool kquant = t == MQ_TYPE_Q4_K || t == MQ_TYPE_Q6_K;
    const bool ffn_fused = ((t == MQ_TYPE_Q8_0 && F % 128 == 0) || (kquant && gemm_requant_q8k_fits(t, rows, F))) &&
                           mq_mul_mat_path(t, F, H, rows) == MQ_PATH_GEMM && mq_mul_mat_path(t, H, F, rows) == MQ_PATH_GEMM;
    const size_t wsb2 = ffn_fused ? mq_workspace_bytes(t, rows, F) : 0;
    if (!m->x.ensure(rows * H * f4) || !m->qkv.ensure(rows * 3 * H * f4) || !m->att.ensure(rows * H * f4) ||
        !m->y.ensure(rows * H * f4) || !m->ff.ensure(rows * F * f4) || !m->ws.ensure(wsb) ||
        (ffn_fused && !m->ws2.ensure(wsb2)))
        return set_error(MQ_ENOMEM, "activation buffers for %lld rows", (long long)rows);
    hipStream_t s = (hipStream_t)stream;
    const float eps = hp.layer_norm_eps;
    float *X = hidden ? hidden : m->x.f();
    int rc;
    if ((rc = hip_rc(launch_embed_ln(ids, hp.n_type > 0 ? types : nullptr, m->tok.f(), m->pos.f(),
                                     hp.n_type > 0 ? m->type.f() : nullptr, m->lnw.f(), m->lnb.f(), eps, X, rows, T,
                                     (int)H, hp.n_vocab, hp.n_type, s),
                     "embeddings")))
        return rc;
    auto mm = [&](const Linear &L, const float *in, float *y) {
        return mq_mul_mat(t, L.img.p, L.n, L.k, in, L.k, rows, y, L.n, m->ws.p, m->ws.bytes, s);
    };
    // Q8_0 with every product on the GEMM path: each post-LN norm also leaves its result
    // quantized for the GEMM that reads it (mq_op_norm_q8_0), the o and FFN-down biases go into
    // the GEMM stores, and the FFN intermediate never leaves the FFN-up GEMM (above).
    // Attention there is the fragment attention of FLASH_ATTN_EXT on strided views of the qkv
    // rows (the q/k/v biases added by the qkv GEMM's store).
    const int hd = (int)(H / hp.n_head);
    const bool norm_fused = t == MQ_TYPE_Q8_0 && ffn_fused && H % 128 == 0 && H <= 1024 && (hd == 32 || hd == 64 || hd == 128) &&
                            mq_mul_mat_path(t, 3 * H, H, rows) == MQ_PATH_GEMM &&
                            mq_mul_mat_path(t, H, H, rows) == MQ_PATH_GEMM;
    if (norm_fused) {
        auto strided = [&](float *p, int64_t ld) {  // [hd, T, n_head, B] over rows of ld floats
            mq_view v{};
            v.data = p;
            v.type = MQ_TYPE_F32;
            v.ne[0] = hd, v.ne[1] = T, v.ne[2] = hp.n_head, v.ne[3] = B;
            v.nb[0] = 4, v.nb[1] = 4 * ld, v.nb[2] = 4 * (size_t)hd, v.nb[3] = 4 * ld * T;
            return v;
        };
        const mq_view qv = strided(m->qkv.f(), 3 * H), kv = strided(m->qkv.f() + H, 3 * H),
                      vv = strided(m->qkv.f() + 2 * H, 3 * H);
        mq_view ov{};  // [hd, n_head, T, B]: rows of H floats
        ov.data = m->att.f();
        ov.type = MQ_TYPE_F32;
        ov.ne[0] = hd, ov.ne[1] = hp.n_head, ov.ne[2] = T, ov.ne[3] = B;
        ov.nb[0] = 4, ov.nb[1] = 4 * (size_t)hd, ov.nb[2] = 4 * H, ov.nb[3] = 4 * H * T;
        if (!m->aws.ensure(mq_op_flash_attn_workspace_bytes(&kv)))
            return set_error(MQ_ENOMEM, "attention workspace for %lld rows", (long long)rows);
        const float ascale = 1.0f / std::sqrt((float)hd);
        // whole 32-key blocks per sequence: K / V straight from the qkv GEMM into the fragments
        const bool kv_direct = T % 32 == 0 && std::getenv("MQ_BERT_KV_PASS") == nullptr;
        AttnArgs attn;
        attn.q = m->qkv.f(), attn.k = m->qkv.f() + H, attn.v = m->qkv.f() + 2 * H;
        attn.q_st = attn.k_st = attn.v_st = 3 * H;
        attn.q_sh = attn.k_sh = attn.v_sh = hd;
        attn.q_sb = attn.k_sb = attn.v_sb = 3 * H * T;
        attn.out = m->att.f();
        attn.o_st = H, attn.o_sh = hd, attn.o_sb = H * T;
        attn.B = B, attn.Tq = T, attn.Tk = T, attn.nq = hp.n_head, attn.nkv = hp.n_head, attn.hd = hd;
        attn.scale = ascale;
        attn.ws = m->aws.p;
        attn.q_ws = m->ws.p;
        attn.q_var = mq_q8_0_variant();
        attn.kv_ready = true;
        attn.q_only = true;  // the o projection reads the attention rows quantized only
        mq_view xv{};
        xv.data = X;
        xv.type = MQ_TYPE_F32;
        xv.ne[0] = H, xv.ne[1] = rows, xv.ne[2] = 1, xv.ne[3] = 1;
        xv.nb[0] = 4, xv.nb[1] = 4 * H, xv.nb[2] = xv.nb[3] = 4 * H * rows;
        mq_view yv = xv;
        yv.data = m->y.f();
        const int G = MQ_PATH_GEMM;
        if ((rc = mq_quantize_act_ex(t, X, H, rows, H, nullptr, MQ_PRE_NONE, m->ws.p, m->ws.bytes, G, s))) return rc;
        for (const Layer &L : m->layers) {  // m->ws holds X quantized at the top of each layer
            if (kv_direct) {
                // the qkv GEMM writes K and V as the attention's operand fragments; the attention
                // stores its rows as the o projection's Q8_0 activation
                if ((rc = hip_rc(launch_gemm_kv(t, L.qkv.img.p, L.qkv.n, L.qkv.k, m->ws.p, rows, m->qkv.f(), L.qkv.n,
                                                L.bqkv.f(), (int)H, T, hd, hp.n_head, m->aws.p, s),
                                 "qkv gemm")) ||
                    (rc = hip_rc(launch_attn(attn, s), "attention")))
                    return rc;
            } else if ((rc = mq_mul_mat_q_ex(t, L.qkv.img.p, L.qkv.n, L.qkv.k, m->ws.p, rows, m->qkv.f(), L.qkv.n,
                                             L.bqkv.f(), G, s)) ||
                       (rc = mq_op_flash_attn_q8_0(&qv, &kv, &vv, nullptr, &ov, ascale, m->aws.p, m->aws.bytes,
                                                   m->ws.p, m->ws.bytes, s))) {
                return rc;
            }
            if ((rc = mq_mul_mat_q_ex(t, L.o.img.p, L.o.n, L.o.k, m->ws.p, rows, m->y.f(), L.o.n, L.bo.f(), G, s)) ||
                (rc = mq_op_norm_q8_0(MQ_NORM_LAYER, &xv, &yv, &xv, eps, L.ln1w.f(), L.ln1b.f(), m->ws.p, m->ws.bytes,
                                      s)) ||
                (rc = mq_mul_mat_q_requant(t, L.fc1.img.p, L.fc1.n, L.fc1.k, m->ws.p, rows, L.b1.f(), MQ_PRE_GELU_ERF,
                                           MQ_TYPE_Q8_0, m->ws2.p, m->ws2.bytes, s)) ||
                (rc = mq_mul_mat_q_ex(t, L.fc2.img.p, L.fc2.n, L.fc2.k, m->ws2.p, rows, m->y.f(), L.fc2.n, L.b2.f(), G,
                                      s)) ||
                (rc = mq_op_norm_q8_0(MQ_NORM_LAYER, &xv, &yv, &xv, eps, L.ln2w.f(), L.ln2b.f(), m->ws.p, m->ws.bytes,
                                      s)))
                return rc;
        }
        return hip_rc(launch_mean_pool_l2(X, out, B, T, (int)H, s), "pooling");
    }
    for (const Layer &L : m->layers) {
        if ((rc = mm(L.qkv, X, m->qkv.f()))) return rc;
        if ((rc = hip_rc(launch_attention(m->qkv.f(), L.bqkv.f(), m->att.f(), B, T, (int)H, hp.n_head, s), "attention")))
            return rc;
        if ((rc = mm(L.o, m->att.f(), m->y.f()))) return rc;
        if ((rc = hip_rc(launch_bias_res_ln(m->y.f(), L.bo.f(), X, L.ln1w.f(), L.ln1b.f(), eps, X, rows, (int)H, s),
                         "attention residual")))
            return rc;
        if (ffn_fused) {
            if ((rc = mq_quantize_act_ex(t, X, H, rows, H, nullptr, MQ_PRE_NONE, m->ws.p, m->ws.bytes, MQ_PATH_GEMM,
                                         s)) ||
                (rc = mq_mul_mat_q_requant(t, L.fc1.img.p, L.fc1.n, L.fc1.k, m->ws.p, rows, L.b1.f(), MQ_PRE_GELU_ERF,
                                           t, m->ws2.p, m->ws2.bytes, s)) ||
                (rc = mq_mul_mat_q(t, L.fc2.img.p, L.fc2.n, L.fc2.k, m->ws2.p, rows, m->y.f(), L.fc2.n, MQ_PATH_GEMM,
                                   s)))
                return rc;
        } else {
            if ((rc = mm(L.fc1, X, m->ff.f()))) return rc;
            // FFN-up bias and GELU-erf are applied by the FFN-down activation quantizer
            if ((rc = mq_quantize_act_ex(t, m->ff.f(), F, rows, F, L.b1.f(), MQ_PRE_GELU_ERF, m->ws.p, m->ws.bytes,
                                         MQ_PATH_AUTO, s)))
                return rc;
            if ((rc = mq_mul_mat_q(t, L.fc2.img.p, L.fc2.n, L.fc2.k, m->ws.p, rows, m->y.f(), L.fc2.n, MQ_PATH_AUTO, s)))
                return rc;
        }
        if ((rc = hip_rc(launch_bias_res_ln(m->y.f(), L.b2.f(), X, L.ln2w.f(), L.ln2b.f(), eps, X, rows, (int)H, s),
                         "ffn residual")))
            return rc;
    }
    return hip_rc(launch_mean_pool_l2(X, out, B, T, (int)H, s), "pooling");
}

extern "C" int mq_bert_get_hparams(const mq_bert *m, mq_bert_hparams *hp) {
    if (!m || !hp) return set_error(MQ_EINVAL, "NULL runner or output");
    *hp = m->hp;
    return MQ_OK;
}
