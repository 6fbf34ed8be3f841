// mq_gguf_load.cpp -- GGUF -> runner loaders (mq_bert_load, mq_decoder_load; mq_gguf.h).
//
// Hyper-parameters are resolved through the same key lists, in the same order, as CrispEmbed's
// loaders (first key present wins): the BERT list of src/crispembed.cpp:437-470 (bert.*, then
// xlmr.*, then <general.architecture>.*), and decoder.<suffix> then <arch>.<suffix> of
// src/decoder_embed.cpp:96-175.  Tensor names accept both CrispEmbed's own (enc.N.*, dec.N.*)
// and the llama.cpp-style (blk.N.*) spellings the reference accepts, and the layer count is
// taken from the highest layer index present, as the reference does.
#include <cmath>
#include <cstdio>
#include <cstring>
#include <string>
#include <vector>

#include "../../include/mq.h"
#include "../../include/mq_gguf.h"
#include "mq_internal.h"

namespace mq {
int set_error(int code, const char *fmt, ...) __attribute__((format(printf, 2, 3)));  // mq_api.cpp
namespace host {
bool dequantize_rows(int type, const void *src, float *dst, int64_t nrows, int64_t k);  // mq_host_quant.cpp
}
}  // namespace mq
using mq::set_error;

namespace {

struct File {
    mq_gguf *g = nullptr;
    std::string path;
    explicit File(const char *p) : g(mq_gguf_open(p)), path(p ? p : "") {}
    ~File() { mq_gguf_close(g); }
};

struct TInfo {
    int64_t idx = -1;
    int type = 0, n_dims = 0;
    int64_t ne[4] = {1, 1, 1, 1};
    const void *data = nullptr;
};

TInfo tensor(const mq_gguf *g, const std::vector<std::string> &names) {
    TInfo t;
    for (const std::string &n : names) {
        t.idx = mq_gguf_find_tensor(g, n.c_str());
        if (t.idx >= 0) break;
    }
    if (t.idx >= 0) {
        mq_gguf_tensor_info(g, t.idx, &t.type, &t.n_dims, t.ne, nullptr, nullptr);
        t.data = mq_gguf_tensor_data(g, t.idx);
    }
    return t;
}

bool has_u32(const mq_gguf *g, const std::string &k) {
    const int64_t i = mq_gguf_find_key(g, k.c_str());
    if (i < 0) return false;
    const int t = mq_gguf_kv_type(g, i);
    return t != MQ_GGUF_FLOAT32 && t != MQ_GGUF_FLOAT64 && t != MQ_GGUF_BOOL && t != MQ_GGUF_STRING &&
           t != MQ_GGUF_ARRAY;
}
bool has_f32(const mq_gguf *g, const std::string &k) {
    const int64_t i = mq_gguf_find_key(g, k.c_str());
    return i >= 0 && (mq_gguf_kv_type(g, i) == MQ_GGUF_FLOAT32 || mq_gguf_kv_type(g, i) == MQ_GGUF_FLOAT64);
}
// first key of the list that is present (with a convertible type) wins
int first_u32(const mq_gguf *g, const std::vector<std::string> &keys, int def) {
    for (const std::string &k : keys)
        if (has_u32(g, k)) return (int)mq_gguf_get_u32(g, k.c_str(), 0);
    return def;
}
float first_f32(const mq_gguf *g, const std::vector<std::string> &keys, float def) {
    for (const std::string &k : keys)
        if (has_f32(g, k)) return mq_gguf_get_f32(g, k.c_str(), def);
    return def;
}

// highest layer index + 1 among tensors named <prefix>N.
int count_layers(const mq_gguf *g, const std::vector<std::string> &prefixes) {
    int n = 0;
    for (int64_t i = 0; i < mq_gguf_n_tensors(g); i++) {
        const char *name = mq_gguf_tensor_name(g, i);
        for (const std::string &p : prefixes) {
            if (std::strncmp(name, p.c_str(), p.size()) != 0) continue;
            int v = 0;
            const char *c = name + p.size();
            bool digits = false;
            while (*c >= '0' && *c <= '9') v = v * 10 + (*c++ - '0'), digits = true;
            if (digits && *c == '.' && v + 1 > n) n = v + 1;
        }
    }
    return n;
}

// an fp32 copy of a whole table (any type the host dequantizer decodes)
bool table_f32(const TInfo &t, int64_t rows, int64_t k, std::vector<float> &out) {
    out.resize((size_t)rows * k);
    return mq::host::dequantize_rows(t.type, t.data, out.data(), rows, k);
}

bool is_linear_type(int t) {
    return t == MQ_TYPE_Q8_0 || t == MQ_TYPE_Q4_K || t == MQ_TYPE_Q6_K || t == MQ_TYPE_F16;
}

// checks a linear weight [k in, n out] of the model's type; sets wtype from the first one
bool linear_ok(const TInfo &t, int64_t k, int64_t n, int &wtype, const char *name, const std::string &path) {
    if (t.idx < 0) return set_error(MQ_EINVAL, "GGUF '%s': missing %s", path.c_str(), name), false;
    if (t.n_dims != 2 || t.ne[0] != k || t.ne[1] != n)
        return set_error(MQ_EINVAL, "GGUF '%s': %s has shape [%lld, %lld], expected [%lld, %lld]", path.c_str(), name,
                         (long long)t.ne[0], (long long)t.ne[1], (long long)k, (long long)n),
               false;
    if (!is_linear_type(t.type))
        return set_error(MQ_EUNSUPPORTED, "GGUF '%s': %s has ggml type %d (Q8_0, Q4_K, Q6_K or F16 is run)", path.c_str(),
                         name, t.type),
               false;
    if (wtype < 0) wtype = t.type;
    if (t.type != wtype)
        return set_error(MQ_EUNSUPPORTED, "GGUF '%s': %s has type %d, other linear weights %d (one type per model)",
                         path.c_str(), name, t.type, wtype),
               false;
    return true;
}

// an fp32 vector of n values (F32 or F16), or `fill` when absent and allowed
bool vec_f32(const TInfo &t, int64_t n, std::vector<float> &out, const char *name, const std::string &path,
             bool optional = false, float fill = 0.0f) {
    if (t.idx < 0) {
        if (!optional) return set_error(MQ_EINVAL, "GGUF '%s': missing %s", path.c_str(), name), false;
        out.assign((size_t)n, fill);
        return true;
    }
    if (t.ne[0] * t.ne[1] * t.ne[2] * t.ne[3] != n || (t.type != MQ_TYPE_F32 && t.type != MQ_TYPE_F16))
        return set_error(MQ_EINVAL, "GGUF '%s': %s is not an F32/F16 vector of %lld", path.c_str(), name, (long long)n),
               false;
    out.resize((size_t)n);
    return mq::host::dequantize_rows(t.type, t.data, out.data(), 1, n);
}

}  // namespace

extern "C" mq_bert *mq_bert_load(const char *path) {
    File f(path);
    const mq_gguf *g = f.g;
    if (!g) return nullptr;
    const std::string arch = mq_gguf_get_str(g, "general.architecture", "");
    auto ak = [&](const char *k) { return arch + "." + k; };
    mq_bert_hparams hp{};
    hp.n_embd = first_u32(g, {"bert.hidden_size", "bert.embedding_length", "xlmr.embedding_length", ak("embedding_length"),
                              ak("hidden_size")}, 384);
    hp.n_head = first_u32(g, {"bert.num_attention_heads", "bert.attention.head_count", "xlmr.attention.head_count",
                              ak("attention.head_count")}, 12);
    hp.n_layer = first_u32(g, {"bert.num_hidden_layers", "bert.block_count", "xlmr.block_count", ak("block_count")}, 6);
    hp.n_ff = first_u32(g, {"bert.intermediate_size", "bert.feed_forward_length", "xlmr.feed_forward_length",
                            ak("feed_forward_length")}, 1536);
    hp.n_vocab = first_u32(g, {"bert.vocab_size", ak("vocab_size")}, 30522);
    hp.n_max_pos = first_u32(g, {"bert.max_position_embeddings", "bert.context_length", "xlmr.context_length",
                                 ak("context_length")}, 512);
    hp.layer_norm_eps = first_f32(g, {"bert.layer_norm_eps", "bert.attention.layer_norm_epsilon",
                                      "xlmr.attention.layer_norm_epsilon", ak("attention.layer_norm_epsilon")}, 1e-12f);
    // pooling: bert.pooling_method (0 mean, 1 cls, 2 last), else Ollama's pooling_type - 1
    int pool = (int)mq_gguf_get_u32(g, "bert.pooling_method", 0xffffffffu);
    if (pool < 0 || mq_gguf_find_key(g, "bert.pooling_method") < 0) {
        const int pt = first_u32(g, {"bert.pooling_type", "xlmr.pooling_type", ak("pooling_type")}, -1);
        pool = pt > 0 ? pt - 1 : 0;
    }
    if (pool != 0) return set_error(MQ_EUNSUPPORTED, "GGUF '%s': pooling method %d (mean pooling is run)", path, pool), nullptr;
    if (mq_gguf_get_u32(g, "bert.pre_ln", 0) != 0 || arch == "modern-bert")
        return set_error(MQ_EUNSUPPORTED, "GGUF '%s': pre-LN encoder (the post-LN BERT graph is run)", path), nullptr;
    if (mq_gguf_get_u32(g, "bert.position_offset", mq_gguf_get_u32(g, "xlmr.position_offset", 0)) != 0)
        return set_error(MQ_EUNSUPPORTED, "GGUF '%s': position offset (RoBERTa / XLM-R positions)", path), nullptr;
    const std::string ffn_act = mq_gguf_get_str(g, "bert.ffn_act", "");
    if (!ffn_act.empty() && ffn_act != "gelu")
        return set_error(MQ_EUNSUPPORTED, "GGUF '%s': ffn activation '%s' (GELU-erf is run)", path, ffn_act.c_str()), nullptr;
    if (first_u32(g, {"bert.num_experts", ak("expert_count")}, 0) > 0)
        return set_error(MQ_EUNSUPPORTED, "GGUF '%s': mixture-of-experts FFN", path), nullptr;

    const TInfo tok = tensor(g, {"token_embd.weight"}), pos = tensor(g, {"position_embd.weight"}),
                typ = tensor(g, {"token_type_embd.weight", "token_types.weight"}),
                lnw = tensor(g, {"embd_ln.weight", "token_embd_norm.weight"}),
                lnb = tensor(g, {"embd_ln.bias", "token_embd_norm.bias"});
    if (tok.idx < 0) return set_error(MQ_EINVAL, "GGUF '%s': missing token_embd.weight", path), nullptr;
    if (pos.idx < 0 || tensor(g, {"rel_embd.weight"}).idx >= 0)
        return set_error(MQ_EUNSUPPORTED, "GGUF '%s': no absolute position embeddings (RoPE / relative-position encoder)",
                         path),
               nullptr;
    // shapes win over metadata, as in the reference (token_embd is [n_embd, n_vocab])
    hp.n_embd = (int)tok.ne[0];
    hp.n_vocab = (int)tok.ne[1];
    hp.n_max_pos = (int)pos.ne[1];
    hp.n_type = typ.idx >= 0 ? (int)typ.ne[1] : 0;
    const int counted = count_layers(g, {"enc.", "blk."});
    if (counted > 0) hp.n_layer = counted;
    if (pos.ne[0] != hp.n_embd || (typ.idx >= 0 && typ.ne[0] != hp.n_embd))
        return set_error(MQ_EINVAL, "GGUF '%s': embedding tables of different widths", path), nullptr;
    const int64_t H = hp.n_embd, F = hp.n_ff;

    // linear weights: one type for the model
    int wtype = -1;
    for (int il = 0; il < hp.n_layer; il++) {
        const std::string e = "enc." + std::to_string(il) + ".", b = "blk." + std::to_string(il) + ".";
        if (tensor(g, {e + "ffn_gate.weight", b + "ffn_gate.weight", e + "ffn_up_gate.weight", b + "ffn_up_gate.weight"}).idx >= 0)
            return set_error(MQ_EUNSUPPORTED, "GGUF '%s': gated FFN (the GELU FFN is run)", path), nullptr;
        const TInfo qkv = tensor(g, {e + "attn.qkv.weight", b + "attn_qkv.weight"});
        if (qkv.idx >= 0) {
            if (!linear_ok(qkv, H, 3 * H, wtype, "attn.qkv.weight", f.path)) return nullptr;
        } else {
            if (!linear_ok(tensor(g, {e + "attn.q.weight", b + "attn_q.weight"}), H, H, wtype, "attn.q.weight", f.path) ||
                !linear_ok(tensor(g, {e + "attn.k.weight", b + "attn_k.weight"}), H, H, wtype, "attn.k.weight", f.path) ||
                !linear_ok(tensor(g, {e + "attn.v.weight", b + "attn_v.weight"}), H, H, wtype, "attn.v.weight", f.path))
                return nullptr;
        }
        const TInfo fc1 = tensor(g, {e + "ffn.fc1.weight", b + "ffn_up.weight"});
        if (fc1.idx >= 0 && fc1.n_dims == 2) {
            if (il == 0 && fc1.ne[1] != F) hp.n_ff = (int)fc1.ne[1];  // shapes win over metadata
        }
        if (!linear_ok(tensor(g, {e + "attn.o.weight", b + "attn_output.weight"}), H, H, wtype, "attn.o.weight", f.path) ||
            !linear_ok(fc1, H, hp.n_ff, wtype, "ffn.fc1.weight", f.path) ||
            !linear_ok(tensor(g, {e + "ffn.fc2.weight", b + "ffn_down.weight"}), hp.n_ff, H, wtype, "ffn.fc2.weight", f.path))
            return nullptr;
    }
    hp.wtype = wtype;
    mq_bert *m = mq_bert_create(&hp);
    if (!m) return nullptr;
    auto bail = [&]() -> mq_bert * {
        mq_bert_free(m);
        return nullptr;
    };
    {
        std::vector<float> vt, vp, vy, vw, vb;
        if (!table_f32(tok, hp.n_vocab, H, vt) || !table_f32(pos, hp.n_max_pos, H, vp) ||
            (hp.n_type > 0 && !table_f32(typ, hp.n_type, H, vy)))
            return set_error(MQ_EUNSUPPORTED, "GGUF '%s': embedding table type not decoded (F32, F16, Q8_0, Q4_K, Q6_K)",
                             path),
                   bail();
        if (!vec_f32(lnw, H, vw, "embd_ln.weight", f.path) || !vec_f32(lnb, H, vb, "embd_ln.bias", f.path)) return bail();
        if (mq_bert_set_embeddings(m, vt.data(), vp.data(), hp.n_type > 0 ? vy.data() : nullptr, vw.data(), vb.data()))
            return bail();
    }
    const size_t rs = mq_row_size(wtype, H);
    for (int il = 0; il < hp.n_layer; il++) {
        const std::string e = "enc." + std::to_string(il) + ".", b = "blk." + std::to_string(il) + ".";
        const TInfo qkv = tensor(g, {e + "attn.qkv.weight", b + "attn_qkv.weight"});
        const void *wq, *wk, *wv;
        std::vector<float> bq, bk, bv, bo, b1, b2, l1w, l1b, l2w, l2b;
        if (qkv.idx >= 0) {  // fused q|k|v rows
            wq = qkv.data;
            wk = (const uint8_t *)qkv.data + H * rs;
            wv = (const uint8_t *)qkv.data + 2 * H * rs;
            std::vector<float> bqkv;
            if (!vec_f32(tensor(g, {e + "attn.qkv.bias", b + "attn_qkv.bias"}), 3 * H, bqkv, "attn.qkv.bias", f.path, true))
                return bail();
            bq.assign(bqkv.begin(), bqkv.begin() + H);
            bk.assign(bqkv.begin() + H, bqkv.begin() + 2 * H);
            bv.assign(bqkv.begin() + 2 * H, bqkv.end());
        } else {
            wq = tensor(g, {e + "attn.q.weight", b + "attn_q.weight"}).data;
            wk = tensor(g, {e + "attn.k.weight", b + "attn_k.weight"}).data;
            wv = tensor(g, {e + "attn.v.weight", b + "attn_v.weight"}).data;
            if (!vec_f32(tensor(g, {e + "attn.q.bias", b + "attn_q.bias"}), H, bq, "attn.q.bias", f.path, true) ||
                !vec_f32(tensor(g, {e + "attn.k.bias", b + "attn_k.bias"}), H, bk, "attn.k.bias", f.path, true) ||
                !vec_f32(tensor(g, {e + "attn.v.bias", b + "attn_v.bias"}), H, bv, "attn.v.bias", f.path, true))
                return bail();
        }
        const void *wo = tensor(g, {e + "attn.o.weight", b + "attn_output.weight"}).data;
        const void *w1 = tensor(g, {e + "ffn.fc1.weight", b + "ffn_up.weight"}).data;
        const void *w2 = tensor(g, {e + "ffn.fc2.weight", b + "ffn_down.weight"}).data;
        if (!vec_f32(tensor(g, {e + "attn.o.bias", b + "attn_output.bias"}), H, bo, "attn.o.bias", f.path, true) ||
            !vec_f32(tensor(g, {e + "ffn.fc1.bias", b + "ffn_up.bias"}), hp.n_ff, b1, "ffn.fc1.bias", f.path, true) ||
            !vec_f32(tensor(g, {e + "ffn.fc2.bias", b + "ffn_down.bias"}), H, b2, "ffn.fc2.bias", f.path, true) ||
            !vec_f32(tensor(g, {e + "ln1.weight", b + "attn_output_norm.weight", b + "attn_norm.weight"}), H, l1w,
                     "ln1.weight", f.path) ||
            !vec_f32(tensor(g, {e + "ln1.bias", b + "attn_output_norm.bias", b + "attn_norm.bias"}), H, l1b, "ln1.bias",
                     f.path) ||
            !vec_f32(tensor(g, {e + "ln2.weight", b + "layer_output_norm.weight", b + "ffn_norm.weight"}), H, l2w,
                     "ln2.weight", f.path) ||
            !vec_f32(tensor(g, {e + "ln2.bias", b + "layer_output_norm.bias", b + "ffn_norm.bias"}), H, l2b, "ln2.bias",
                     f.path))
            return bail();
        if (mq_bert_set_layer(m, il, wq, wk, wv, wo, w1, w2, bq.data(), bk.data(), bv.data(), bo.data(), b1.data(),
                              b2.data(), l1w.data(), l1b.data(), l2w.data(), l2b.data()))
            return bail();
    }
    return m;
}

extern "C" mq_decoder *mq_decoder_load(const char *path) {
    File f(path);
    const mq_gguf *g = f.g;
    if (!g) return nullptr;
    const std::string arch = mq_gguf_get_str(g, "general.architecture", "");
    std::string pfx = "decoder";
    if (arch == "gemma3" || arch == "gemma-embedding" || arch == "qwen3" || arch == "ministral3" || arch == "llama")
        pfx = arch;
    // decoder.<suffix>, then <arch>.<suffix>
    auto u32 = [&](const char *suffix, int def) {
        return first_u32(g, {std::string("decoder.") + suffix, pfx + "." + suffix}, def);
    };
    auto f32 = [&](const char *suffix, float def) {
        return first_f32(g, {std::string("decoder.") + suffix, pfx + "." + suffix}, def);
    };
    mq_decoder_hparams hp{};
    hp.n_vocab = u32("vocab_size", 0);
    hp.n_embd = u32("hidden_size", u32("embedding_length", 1024));
    hp.n_head = u32("num_attention_heads", u32("attention.head_count", 16));
    hp.n_kv_head = u32("num_key_value_heads", u32("attention.head_count_kv", hp.n_head));
    hp.n_layer = u32("num_hidden_layers", u32("block_count", 28));
    hp.n_ff = u32("intermediate_size", u32("feed_forward_length", 3072));
    hp.rms_norm_eps = f32("rms_norm_eps", f32("attention.layer_norm_rms_epsilon", 1e-6f));
    hp.rope_theta = f32("rope_theta", f32("rope.freq_base", 10000.0f));
    hp.causal = u32("is_bidirectional", 0) != 0 ? 0 : 1;
    int pm = u32("pooling_method", -1);
    if (pm < 0) {
        const int pt = u32("pooling_type", 3);  // Ollama {1 mean, 2 cls, 3 last}
        pm = pt == 3 ? 2 : pt == 1 ? 1 : 2;
    }
    hp.pooling = pm;
    hp.head_dim = u32("head_dim", u32("attention.key_length", 0));
    if (arch == "gemma3" || arch == "gemma-embedding" || u32("gemma_norm", 0) != 0)
        return set_error(MQ_EUNSUPPORTED, "GGUF '%s': Gemma-style decoder (the Qwen3 graph is run)", path), nullptr;
    if (u32("activation", 0) != 0)
        return set_error(MQ_EUNSUPPORTED, "GGUF '%s': FFN activation %d (SwiGLU is run)", path, u32("activation", 0)), nullptr;
    if (u32("rope_scaling_type", u32("rope.scaling_type", 0)) != 0 || f32("rope_theta_local", f32("rope.freq_base_local", 0.f)) != 0.f ||
        u32("global_attn_every_n_layers", u32("attention.sliding_window_layer_period", 0)) != 0)
        return set_error(MQ_EUNSUPPORTED, "GGUF '%s': RoPE scaling or sliding-window attention", path), nullptr;
    if (f32("attn_scale", f32("attention.key_length_scale", 0.f)) != 0.f || f32("embed_scale", 1.f) != 1.f)
        return set_error(MQ_EUNSUPPORTED, "GGUF '%s': non-default attention or embedding scale", path), nullptr;
    if (u32("normalize_embeddings", 1) == 0)
        return set_error(MQ_EUNSUPPORTED, "GGUF '%s': unnormalised embeddings (L2-normalised output is run)", path), nullptr;
    if (mq_gguf_find_key(g, "decoder.mrope_section") >= 0)
        return set_error(MQ_EUNSUPPORTED, "GGUF '%s': multimodal RoPE sections", path), nullptr;
    if (hp.pooling != 1 && hp.pooling != 2)
        return set_error(MQ_EUNSUPPORTED, "GGUF '%s': pooling method %d (mean or last token is run)", path, hp.pooling), nullptr;

    const TInfo tok = tensor(g, {"token_embd.weight"}), onorm = tensor(g, {"output_norm.weight", "final_norm.weight"});
    if (tok.idx < 0 || tok.n_dims != 2) return set_error(MQ_EINVAL, "GGUF '%s': missing token_embd.weight", path), nullptr;
    hp.n_vocab = (int)tok.ne[1];
    hp.n_embd = (int)tok.ne[0];
    const int counted = count_layers(g, {"dec.", "blk."});
    if (counted > 0) hp.n_layer = counted;
    if (tensor(g, {"dense.0.weight"}).idx >= 0)
        return set_error(MQ_EUNSUPPORTED, "GGUF '%s': post-pooling dense projection", path), nullptr;
    if (hp.head_dim == 0 && hp.n_head > 0) hp.head_dim = hp.n_embd / hp.n_head;
    const int64_t H = hp.n_embd, qd = (int64_t)hp.n_head * hp.head_dim, kvd = (int64_t)hp.n_kv_head * hp.head_dim;
    int wtype = -1;
    for (int il = 0; il < hp.n_layer; il++) {
        const std::string d = "dec." + std::to_string(il) + ".", b = "blk." + std::to_string(il) + ".";
        auto t2 = [&](const char *s1, const char *s2) { return tensor(g, {d + s1, b + s2}); };
        if (t2("attn.q.bias", "attn_q.bias").idx >= 0 || t2("attn.k.bias", "attn_k.bias").idx >= 0 ||
            t2("attn.v.bias", "attn_v.bias").idx >= 0 || t2("attn.o.bias", "attn_output.bias").idx >= 0)
            return set_error(MQ_EUNSUPPORTED, "GGUF '%s': attention projection biases", path), nullptr;
        if (t2("post_attn_norm.weight", "post_attention_norm.weight").idx >= 0 ||
            t2("pre_ffn_norm.weight", "pre_ffn_norm.weight").idx >= 0 ||
            t2("post_ffn_norm.weight", "post_ffw_norm.weight").idx >= 0)
            return set_error(MQ_EUNSUPPORTED, "GGUF '%s': sandwich norms", path), nullptr;
        const TInfo gate = t2("ffn.gate.weight", "ffn_gate.weight");
        if (il == 0 && gate.idx >= 0 && gate.n_dims == 2) hp.n_ff = (int)gate.ne[1];  // shapes win
        if (!linear_ok(t2("attn.q.weight", "attn_q.weight"), H, qd, wtype, "attn.q.weight", f.path) ||
            !linear_ok(t2("attn.k.weight", "attn_k.weight"), H, kvd, wtype, "attn.k.weight", f.path) ||
            !linear_ok(t2("attn.v.weight", "attn_v.weight"), H, kvd, wtype, "attn.v.weight", f.path) ||
            !linear_ok(t2("attn.o.weight", "attn_output.weight"), qd, H, wtype, "attn.o.weight", f.path) ||
            !linear_ok(gate, H, hp.n_ff, wtype, "ffn.gate.weight", f.path) ||
            !linear_ok(t2("ffn.up.weight", "ffn_up.weight"), H, hp.n_ff, wtype, "ffn.up.weight", f.path) ||
            !linear_ok(t2("ffn.down.weight", "ffn_down.weight"), hp.n_ff, H, wtype, "ffn.down.weight", f.path))
            return nullptr;
    }
    hp.wtype = wtype;
    mq_decoder *m = mq_decoder_create(&hp);
    if (!m) return nullptr;
    auto bail = [&]() -> mq_decoder * {
        mq_decoder_free(m);
        return nullptr;
    };
    {
        std::vector<float> vt, vn;
        if (!table_f32(tok, hp.n_vocab, H, vt))
            return set_error(MQ_EUNSUPPORTED, "GGUF '%s': token_embd type %d not decoded", path, tok.type), bail();
        if (!vec_f32(onorm, H, vn, "output_norm.weight", f.path)) return bail();
        if (mq_decoder_set_embeddings(m, vt.data(), vn.data())) return bail();
    }
    for (int il = 0; il < hp.n_layer; il++) {
        const std::string d = "dec." + std::to_string(il) + ".", b = "blk." + std::to_string(il) + ".";
        auto t2 = [&](const char *s1, const char *s2) { return tensor(g, {d + s1, b + s2}); };
        std::vector<float> an, fn, qn, kn;
        const TInfo tq = t2("attn.q_norm.weight", "attn_q_norm.weight"), tk = t2("attn.k_norm.weight", "attn_k_norm.weight");
        if (!vec_f32(t2("attn_norm.weight", "attn_norm.weight"), H, an, "attn_norm.weight", f.path) ||
            !vec_f32(t2("ffn_norm.weight", "ffn_norm.weight"), H, fn, "ffn_norm.weight", f.path) ||
            (tq.idx >= 0 && !vec_f32(tq, hp.head_dim, qn, "attn.q_norm.weight", f.path)) ||
            (tk.idx >= 0 && !vec_f32(tk, hp.head_dim, kn, "attn.k_norm.weight", f.path)))
            return bail();
        if (mq_decoder_set_layer(m, il, t2("attn.q.weight", "attn_q.weight").data, t2("attn.k.weight", "attn_k.weight").data,
                                 t2("attn.v.weight", "attn_v.weight").data, t2("attn.o.weight", "attn_output.weight").data,
                                 t2("ffn.gate.weight", "ffn_gate.weight").data, t2("ffn.up.weight", "ffn_up.weight").data,
                                 t2("ffn.down.weight", "ffn_down.weight").data, an.data(), fn.data(),
                                 tq.idx >= 0 ? qn.data() : nullptr, tk.idx >= 0 ? kn.data() : nullptr))
            return bail();
    }
    return m;
}
