// test-decoder-graph-mi355 -- CrispEmbed's decoder-embedder graph for the Qwen3 family, built
// with ggml's graph API as src/decoder_embed.cpp builds it (:680-830: GET_ROWS embedding, per
// layer RMS_NORM x attn_norm, q/k/v MUL_MAT, RESHAPE_3D, per-head RMS_NORM x q_norm / k_norm,
// ROPE_EXT NEOX on pos_ids, PERMUTE, FLASH_ATTN_EXT with the causal F16 mask (none for
// bidirectional models), the output projection, residual ADD, RMS_NORM x ffn_norm, SiLU(gate) *
// up, the down projection and residual ADD; then the output RMS norm), one sequence of T
// tokens, computed entirely by the MI355X backend.
//
// usage: test-decoder-graph-mi355 model.gguf T ids.i32 out.f32 [--iters N]
//   out: the normed last hidden state [H, T] as float32.  Prints one JSON line.
#include <chrono>
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <map>
#include <string>
#include <vector>

#include "ggml-backend.h"
#include "ggml-mi355.h"
#include "ggml.h"
#include "mq_gguf.h"

static std::vector<char> read_file(const char *path) {
    std::vector<char> v;
    FILE *f = std::fopen(path, "rb");
    if (!f) return v;
    std::fseek(f, 0, SEEK_END);
    v.resize((size_t)std::ftell(f));
    std::fseek(f, 0, SEEK_SET);
    if (std::fread(v.data(), 1, v.size(), f) != v.size()) v.clear();
    std::fclose(f);
    return v;
}

static int fail(const char *msg) {
    std::printf("{\"ok\": false, \"error\": \"%s\"}\n", msg);
    return 1;
}

int main(int argc, char **argv) {
    if (argc < 5) return fail("usage: model.gguf T ids out [--iters N]");
    const char *path = argv[1];
    const int T = std::atoi(argv[2]);
    int iters = 0;
    for (int i = 5; i < argc; i++)
        if (!std::strcmp(argv[i], "--iters") && i + 1 < argc) iters = std::atoi(argv[++i]);
    std::vector<char> ids_raw = read_file(argv[3]);
    if (T <= 0 || ids_raw.size() != (size_t)T * 4) return fail("bad T or ids file size");

    ggml_backend_register(ggml_backend_mi355_reg());
    ggml_backend_t be = ggml_backend_mi355_init(0);
    if (!be) return fail("no MI355X device");

    mq_gguf *g = mq_gguf_open(path);
    if (!g) return fail("cannot open the GGUF");
    const char *a = "qwen3";
    auto key = [&](const char *k) { return std::string(a) + "." + k; };
    const int n_layer = (int)mq_gguf_get_u32(g, key("block_count").c_str(), 0);
    const int H = (int)mq_gguf_get_u32(g, key("embedding_length").c_str(), 0);
    const int nh = (int)mq_gguf_get_u32(g, key("attention.head_count").c_str(), 0);
    const int nkv = (int)mq_gguf_get_u32(g, key("attention.head_count_kv").c_str(), 0);
    const int hd = (int)mq_gguf_get_u32(g, key("attention.key_length").c_str(), 0);
    const float eps = mq_gguf_get_f32(g, key("attention.layer_norm_rms_epsilon").c_str(), 1e-6f);
    const float theta = mq_gguf_get_f32(g, key("rope.freq_base").c_str(), 1e6f);
    const bool causal = mq_gguf_get_u32(g, "decoder.is_bidirectional", 0) == 0;
    if (n_layer <= 0 || H <= 0 || nh <= 0 || nkv <= 0 || hd <= 0) return fail("missing hyper-parameters");

    const int64_t nt = mq_gguf_n_tensors(g);
    ggml_init_params wp = {ggml_tensor_overhead() * (size_t)(nt + 8), nullptr, true};
    ggml_context *wctx = ggml_init(wp);
    std::map<std::string, ggml_tensor *> W;
    for (int64_t i = 0; i < nt; i++) {
        int type, nd;
        int64_t ne[4];
        size_t off, nbytes;
        mq_gguf_tensor_info(g, i, &type, &nd, ne, &off, &nbytes);
        ggml_tensor *t = ggml_new_tensor_4d(wctx, (ggml_type)type, ne[0], ne[1], ne[2], ne[3]);
        ggml_set_name(t, mq_gguf_tensor_name(g, i));
        W[mq_gguf_tensor_name(g, i)] = t;
    }
    ggml_backend_buffer_t wbuf = ggml_backend_alloc_ctx_tensors(wctx, be);
    if (!wbuf) return fail("weight buffer allocation failed");
    for (int64_t i = 0; i < nt; i++) {
        ggml_tensor *t = W[mq_gguf_tensor_name(g, i)];
        ggml_backend_tensor_set(t, mq_gguf_tensor_data(g, i), 0, ggml_nbytes(t));
    }
    auto get = [&](const std::string &n) -> ggml_tensor * {
        auto it = W.find(n);
        return it == W.end() ? nullptr : it->second;
    };

    ggml_init_params gp = {ggml_tensor_overhead() * (size_t)(n_layer * 64 + 64) + ggml_graph_overhead(), nullptr, true};
    ggml_context *gctx = ggml_init(gp);
    ggml_tensor *ids = ggml_new_tensor_1d(gctx, GGML_TYPE_I32, T);
    ggml_set_name(ids, "inp_tokens");
    ggml_set_input(ids);
    ggml_tensor *pos = ggml_new_tensor_1d(gctx, GGML_TYPE_I32, T);
    ggml_set_name(pos, "pos_ids");
    ggml_set_input(pos);
    ggml_tensor *mask = nullptr;
    if (causal) {
        mask = ggml_new_tensor_2d(gctx, GGML_TYPE_F16, T, T);
        ggml_set_name(mask, "causal_mask");
        ggml_set_input(mask);
    }
    auto rms_norm = [&](ggml_tensor *x, ggml_tensor *w) { return ggml_mul(gctx, ggml_rms_norm(gctx, x, eps), w); };
    ggml_tensor *cur = ggml_get_rows(gctx, get("token_embd.weight"), ids);
    for (int il = 0; il < n_layer; il++) {
        const std::string p = "dec." + std::to_string(il) + ".";
        ggml_tensor *residual = cur;
        cur = rms_norm(cur, get(p + "attn_norm.weight"));
        ggml_tensor *Q = ggml_mul_mat(gctx, get(p + "attn.q.weight"), cur);
        ggml_tensor *K = ggml_mul_mat(gctx, get(p + "attn.k.weight"), cur);
        ggml_tensor *V = ggml_mul_mat(gctx, get(p + "attn.v.weight"), cur);
        Q = ggml_reshape_3d(gctx, Q, hd, nh, T);
        K = ggml_reshape_3d(gctx, K, hd, nkv, T);
        V = ggml_reshape_3d(gctx, V, hd, nkv, T);
        if (get(p + "attn.q_norm.weight")) Q = rms_norm(Q, get(p + "attn.q_norm.weight"));
        if (get(p + "attn.k_norm.weight")) K = rms_norm(K, get(p + "attn.k_norm.weight"));
        Q = ggml_rope_ext(gctx, Q, pos, nullptr, hd, GGML_ROPE_TYPE_NEOX, 0, theta, 1.0f, 0.0f, 1.0f, 0.0f, 0.0f);
        K = ggml_rope_ext(gctx, K, pos, nullptr, hd, GGML_ROPE_TYPE_NEOX, 0, theta, 1.0f, 0.0f, 1.0f, 0.0f, 0.0f);
        Q = ggml_permute(gctx, Q, 0, 2, 1, 3);
        K = ggml_permute(gctx, K, 0, 2, 1, 3);
        V = ggml_permute(gctx, V, 0, 2, 1, 3);
        ggml_tensor *attn = ggml_flash_attn_ext(gctx, Q, K, V, mask, 1.0f / std::sqrt((float)hd), 0.0f, 0.0f);
        attn = ggml_reshape_2d(gctx, attn, (int64_t)nh * hd, T);
        attn = ggml_mul_mat(gctx, get(p + "attn.o.weight"), attn);
        cur = ggml_add(gctx, residual, attn);
        residual = cur;
        cur = rms_norm(cur, get(p + "ffn_norm.weight"));
        ggml_tensor *gate = ggml_silu(gctx, ggml_mul_mat(gctx, get(p + "ffn.gate.weight"), cur));
        ggml_tensor *up = ggml_mul_mat(gctx, get(p + "ffn.up.weight"), cur);
        ggml_tensor *ffn = ggml_mul_mat(gctx, get(p + "ffn.down.weight"), ggml_mul(gctx, gate, up));
        cur = ggml_add(gctx, residual, ffn);
    }
    cur = rms_norm(cur, get("output_norm.weight"));
    ggml_set_name(cur, "decoder_out");
    ggml_set_output(cur);
    ggml_cgraph *gf = ggml_new_graph(gctx);
    ggml_build_forward_expand(gf, cur);

    int unsupported = 0;
    for (int i = 0; i < ggml_graph_n_nodes(gf); i++)
        if (!ggml_backend_supports_op(be, ggml_graph_node(gf, i))) {
            std::fprintf(stderr, "unsupported node %d: %s %s\n", i, ggml_op_name(ggml_graph_node(gf, i)->op),
                         ggml_graph_node(gf, i)->name);
            unsupported++;
        }
    ggml_backend_buffer_t gbuf = ggml_backend_alloc_ctx_tensors(gctx, be);
    if (!gbuf) return fail("graph buffer allocation failed");
    std::vector<int32_t> pv(T);
    for (int t = 0; t < T; t++) pv[t] = t;
    ggml_backend_tensor_set(ids, ids_raw.data(), 0, (size_t)T * 4);
    ggml_backend_tensor_set(pos, pv.data(), 0, (size_t)T * 4);
    if (mask) {  // 0 where key <= query, -inf above the diagonal
        std::vector<uint16_t> m((size_t)T * T);
        for (int q = 0; q < T; q++)
            for (int k = 0; k < T; k++) m[(size_t)q * T + k] = k <= q ? 0x0000 : 0xFC00;
        ggml_backend_tensor_set(mask, m.data(), 0, m.size() * 2);
    }
    if (ggml_backend_graph_compute(be, gf) != GGML_STATUS_SUCCESS) return fail("graph_compute failed");
    std::vector<float> out((size_t)H * T);
    ggml_backend_tensor_get(cur, out.data(), 0, out.size() * sizeof(float));
    FILE *f = std::fopen(argv[4], "wb");
    if (!f || std::fwrite(out.data(), sizeof(float), out.size(), f) != out.size()) return fail("cannot write output");
    std::fclose(f);
    double ms = 0.0;
    if (iters > 0) {
        const auto t0 = std::chrono::steady_clock::now();
        for (int i = 0; i < iters; i++)
            if (ggml_backend_graph_compute(be, gf) != GGML_STATUS_SUCCESS) return fail("graph_compute failed");
        ms = std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - t0).count() / iters;
    }
    std::printf("{\"ok\": true, \"nodes\": %d, \"unsupported\": %d, \"ms_per_graph\": %.4f, \"iters\": %d}\n",
                ggml_graph_n_nodes(gf), unsupported, ms, iters);
    ggml_backend_buffer_free(gbuf);
    ggml_backend_buffer_free(wbuf);
    ggml_free(gctx);
    ggml_free(wctx);
    ggml_backend_free(be);
    mq_gguf_close(g);
    return 0;
}
