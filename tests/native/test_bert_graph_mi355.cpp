// test-bert-graph-mi355 -- CrispEmbed's BERT encoder graph, built with ggml's graph API as
// build_encoder_graph builds it (src/crispembed.cpp:1043-1468, the post-LN path: GET_ROWS
// embeddings + NORM/MUL/ADD, per layer q/k/v MUL_MAT + ADD (or one fused qkv MUL_MAT and three
// CONT(VIEW)s), RESHAPE_4D + PERMUTE, FLASH_ATTN_EXT with no mask or the per-item padding mask
// of encode_tokens_group_4d (src/crispembed.cpp:2052-2127), the output projection, residual
// ADD + layer norm, and the GELU_ERF FFN), computed entirely by the MI355X backend.
//
// usage: test-bert-graph-mi355 model.gguf B T ids.i32 types.i32 lens.i32 out.f32 [--fused-qkv] [--iters N]
//                              [--check-replay]
//   ids / types: B*T int32 (item-major, t fastest); lens: B int32 real lengths (all T: no mask);
//   out: the encoder_out tensor [H, B*T] as float32.  Prints one JSON line.
//   --observe: then computes the graph as ggml's scheduler does when an eval callback observes
//   every MUL_MAT (the imatrix collector, src/imatrix.cpp:57-99): in pieces that end at each
//   MUL_MAT, reading that MUL_MAT's src1 after its piece, with every graph tensor first filled
//   with NaN bytes; and once more node by node (MQ_GGML_NO_FUSION=1) as the reference.  Reports
//   how many observed src1 still hold NaN (unwritten), the largest relative difference of any
//   src1 and of the imatrix sums (sum of x^2 per column) against the node-by-node run.
//   --packed [--pack-maxtok N]: the reference's default GPU batching instead (encode_tokens_packed
//   with its greedy grouping, src/crispembed.cpp:1870-2008, 2192-2216): items are packed end to end,
//   in groups of at most N tokens (default 384; an item longer than N forms its own group), each
//   group one graph of T_g = its summed lengths with B = 1, positions restarting per item, and the
//   block-diagonal F16 mask "seg_mask" [T_g, T_g] (0 within an item, -inf elsewhere); a group of
//   one item is encode_tokens' graph (no mask).  out then holds the groups' rows one after another
//   (each item's real tokens only); --iters times all groups' graph_compute calls in sequence.
//   --check-replay: after the first (eager) compute, computes the graph for a second id set
//   (each id + 1; the backend captures it), then for the first set and the second again (the
//   captured graph replayed, with uploads and readbacks in between), and reports whether the
//   replays equal the first two results bit for bit; the second set's result goes to
//   <out>.second.
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

static double fin(double x) { return std::isfinite(x) ? x : 1e30; }  // JSON has no inf / nan

static uint16_t f16_bits(float x) {  // 0 and -inf only (the mask values)
    return std::isinf(x) ? 0xFC00 : 0x0000;
}

int main(int argc, char **argv) {
    if (argc < 8) return fail("usage: model.gguf B T ids types lens out [--fused-qkv] [--iters N]");
    const char *path = argv[1];
    const int B = std::atoi(argv[2]), T = std::atoi(argv[3]);
    bool fused_qkv = false, check_replay = false, observe = false, packed = false;
    int iters = 0, pack_maxtok = 384;
    for (int i = 8; i < argc; i++) {
        if (!std::strcmp(argv[i], "--packed")) packed = true;
        if (!std::strcmp(argv[i], "--pack-maxtok") && i + 1 < argc) pack_maxtok = std::atoi(argv[++i]);
        if (!std::strcmp(argv[i], "--fused-qkv")) fused_qkv = true;
        if (!std::strcmp(argv[i], "--check-replay")) check_replay = true;
        if (!std::strcmp(argv[i], "--observe")) observe = true;
        if (!std::strcmp(argv[i], "--iters") && i + 1 < argc) iters = std::atoi(argv[++i]);
    }
    const int TB = B * T;
    std::vector<char> ids_raw = read_file(argv[4]), types_raw = read_file(argv[5]), lens_raw = read_file(argv[6]);
    if (ids_raw.size() != (size_t)TB * 4 || types_raw.size() != (size_t)TB * 4 || lens_raw.size() != (size_t)B * 4)
        return fail("bad ids / types / lens file sizes");
    const int32_t *lens = (const int32_t *)lens_raw.data();
    bool padded = false;
    for (int b = 0; b < B; b++) padded |= lens[b] != T;

    ggml_backend_register(ggml_backend_mi355_reg());
    ggml_backend_t be = ggml_backend_mi355_init(0);
    if (!be) return fail("no MI355X device");

    mq_gguf *g = mq_gguf_open(path);
    if (!g) return fail("cannot open the GGUF");
    const int n_layer = (int)mq_gguf_get_u32(g, "bert.num_hidden_layers", 0);
    const int H = (int)mq_gguf_get_u32(g, "bert.hidden_size", 0);
    const int n_head = (int)mq_gguf_get_u32(g, "bert.num_attention_heads", 0);
    const float eps = mq_gguf_get_f32(g, "bert.layer_norm_eps", 1e-12f);
    const int hd = H / n_head;

    // weights: one context, one backend buffer, GGUF bytes uploaded with tensor_set
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
    // the fused q|k|v variant concatenates the three projections into one weight and bias
    ggml_tensor *qkv_w[64] = {}, *qkv_b[64] = {};
    if (fused_qkv) {
        for (int il = 0; il < n_layer; il++) {
            const std::string p = "enc." + std::to_string(il) + ".attn.";
            const ggml_tensor *q = W[p + "q.weight"];
            qkv_w[il] = ggml_new_tensor_2d(wctx, q->type, q->ne[0], 3 * q->ne[1]);
            qkv_b[il] = ggml_new_tensor_1d(wctx, GGML_TYPE_F32, 3 * q->ne[1]);
        }
    }
    ggml_backend_buffer_t wbuf = ggml_backend_alloc_ctx_tensors(wctx, be);
    if (!wbuf) return fail("weight buffer allocation failed");
    for (int64_t i = 0; i < nt; i++) {
        ggml_tensor *t = W[mq_gguf_tensor_name(g, i)];
        ggml_backend_tensor_set(t, mq_gguf_tensor_data(g, i), 0, ggml_nbytes(t));
    }
    if (fused_qkv) {
        for (int il = 0; il < n_layer; il++) {
            const std::string p = "enc." + std::to_string(il) + ".attn.";
            size_t ow = 0, ob = 0;
            for (const char *x : {"q", "k", "v"}) {
                const int64_t iw = mq_gguf_find_tensor(g, (p + x + ".weight").c_str());
                const int64_t ib = mq_gguf_find_tensor(g, (p + x + ".bias").c_str());
                const size_t nw = ggml_nbytes(W[p + x + ".weight"]), nbb = ggml_nbytes(W[p + x + ".bias"]);
                ggml_backend_tensor_set(qkv_w[il], mq_gguf_tensor_data(g, iw), ow, nw);
                ggml_backend_tensor_set(qkv_b[il], mq_gguf_tensor_data(g, ib), ob, nbb);
                ow += nw, ob += nbb;
            }
        }
    }

    // the graph (build_encoder_graph's standard post-LN path) for Bg items of Tg tokens; mask_kind
    // 0: none, 1: the per-item padding mask [Tg, Tg, 1, Bg], 2: the packed seg_mask [Tg, Tg]
    struct EncGraph {
        ggml_context *ctx;
        ggml_cgraph *gf;
        ggml_tensor *tok_ids, *pos_ids, *type_ids, *mask, *out;
    };
    auto build_graph = [&](int Bg, int Tg, int mask_kind) {
        EncGraph e{};
        const int TBg = Bg * Tg;
        ggml_init_params gp = {ggml_tensor_overhead() * (size_t)(n_layer * 64 + 64) + ggml_graph_overhead(), nullptr,
                               true};
        ggml_context *gctx = e.ctx = ggml_init(gp);
        e.tok_ids = ggml_new_tensor_1d(gctx, GGML_TYPE_I32, TBg);
        ggml_set_name(e.tok_ids, "tok_ids");
        ggml_set_input(e.tok_ids);
        e.pos_ids = ggml_new_tensor_1d(gctx, GGML_TYPE_I32, TBg);
        ggml_set_name(e.pos_ids, "pos_ids");
        ggml_set_input(e.pos_ids);
        e.type_ids = ggml_new_tensor_1d(gctx, GGML_TYPE_I32, TBg);
        ggml_set_name(e.type_ids, "type_ids");
        ggml_set_input(e.type_ids);
        if (mask_kind == 1) {
            e.mask = ggml_new_tensor_4d(gctx, GGML_TYPE_F16, Tg, Tg, 1, Bg);
            ggml_set_name(e.mask, "pad_mask");
            ggml_set_input(e.mask);
        } else if (mask_kind == 2) {
            e.mask = ggml_new_tensor_2d(gctx, GGML_TYPE_F16, Tg, Tg);
            ggml_set_name(e.mask, "seg_mask");
            ggml_set_input(e.mask);
        }
        ggml_tensor *cur = ggml_get_rows(gctx, W["token_embd.weight"], e.tok_ids);
        cur = ggml_add(gctx, cur, ggml_get_rows(gctx, W["position_embd.weight"], e.pos_ids));
        cur = ggml_add(gctx, cur, ggml_get_rows(gctx, W["token_type_embd.weight"], e.type_ids));
        cur = ggml_norm(gctx, cur, eps);
        cur = ggml_mul(gctx, cur, W["embd_ln.weight"]);
        cur = ggml_add(gctx, cur, W["embd_ln.bias"]);
        for (int il = 0; il < n_layer; il++) {
            const std::string p = "enc." + std::to_string(il) + ".";
            auto w = [&](const char *n) { return W[p + n]; };
            ggml_tensor *inp = cur, *Q, *K, *V;
            if (fused_qkv) {
                ggml_tensor *qkv = ggml_add(gctx, ggml_mul_mat(gctx, qkv_w[il], cur), qkv_b[il]);
                Q = ggml_cont(gctx, ggml_view_2d(gctx, qkv, H, TBg, 3 * H * sizeof(float), 0));
                K = ggml_cont(gctx, ggml_view_2d(gctx, qkv, H, TBg, 3 * H * sizeof(float), H * sizeof(float)));
                V = ggml_cont(gctx, ggml_view_2d(gctx, qkv, H, TBg, 3 * H * sizeof(float), 2 * H * sizeof(float)));
            } else {
                Q = ggml_add(gctx, ggml_mul_mat(gctx, w("attn.q.weight"), cur), w("attn.q.bias"));
                K = ggml_add(gctx, ggml_mul_mat(gctx, w("attn.k.weight"), cur), w("attn.k.bias"));
                V = ggml_add(gctx, ggml_mul_mat(gctx, w("attn.v.weight"), cur), w("attn.v.bias"));
            }
            Q = ggml_permute(gctx, ggml_reshape_4d(gctx, Q, hd, n_head, Tg, Bg), 0, 2, 1, 3);
            K = ggml_permute(gctx, ggml_reshape_4d(gctx, K, hd, n_head, Tg, Bg), 0, 2, 1, 3);
            V = ggml_permute(gctx, ggml_reshape_4d(gctx, V, hd, n_head, Tg, Bg), 0, 2, 1, 3);
            ggml_tensor *attn = ggml_flash_attn_ext(gctx, Q, K, V, e.mask, 1.0f / std::sqrt((float)hd), 0.0f, 0.0f);
            attn = ggml_reshape_2d(gctx, attn, H, TBg);
            attn = ggml_add(gctx, ggml_mul_mat(gctx, w("attn.o.weight"), attn), w("attn.o.bias"));
            cur = ggml_add(gctx, inp, attn);
            cur = ggml_norm(gctx, cur, eps);
            cur = ggml_mul(gctx, cur, w("ln1.weight"));
            cur = ggml_add(gctx, cur, w("ln1.bias"));
            ggml_tensor *ffn = ggml_add(gctx, ggml_mul_mat(gctx, w("ffn.fc1.weight"), cur), w("ffn.fc1.bias"));
            ffn = ggml_gelu_erf(gctx, ffn);
            ffn = ggml_add(gctx, ggml_mul_mat(gctx, w("ffn.fc2.weight"), ffn), w("ffn.fc2.bias"));
            cur = ggml_add(gctx, cur, ffn);
            cur = ggml_norm(gctx, cur, eps);
            cur = ggml_mul(gctx, cur, w("ln2.weight"));
            cur = ggml_add(gctx, cur, w("ln2.bias"));
        }
        ggml_set_name(cur, "encoder_out");
        ggml_set_output(cur);
        e.gf = ggml_new_graph(gctx);
        ggml_build_forward_expand(e.gf, cur);
        e.out = cur;
        return e;
    };
    auto count_unsupported = [&](ggml_cgraph *gf) {  // every node must be claimed by the backend
        int u = 0;
        for (int i = 0; i < ggml_graph_n_nodes(gf); i++)
            if (!ggml_backend_supports_op(be, ggml_graph_node(gf, i))) {
                std::fprintf(stderr, "unsupported node %d: %s %s\n", i, ggml_op_name(ggml_graph_node(gf, i)->op),
                             ggml_graph_node(gf, i)->name);
                u++;
            }
        return u;
    };

    if (packed) {  // encode_tokens_packed over the greedy groups
        const int32_t *ids_in = (const int32_t *)ids_raw.data(), *types_in = (const int32_t *)types_raw.data();
        struct Group {
            EncGraph e;
            ggml_backend_buffer_t buf;
            int i0, i1, T;
        };
        std::vector<Group> groups;
        int unsupported = 0, nodes = 0;
        for (int i = 0; i < B;) {
            int j = i, tsum = 0;
            while (j < B && !(j > i && tsum + lens[j] > pack_maxtok)) tsum += lens[j++];
            Group gr{build_graph(1, tsum, j - i > 1 ? 2 : 0), nullptr, i, j, tsum};
            unsupported += count_unsupported(gr.e.gf);
            nodes += ggml_graph_n_nodes(gr.e.gf);
            gr.buf = ggml_backend_alloc_ctx_tensors(gr.e.ctx, be);
            if (!gr.buf) return fail("graph buffer allocation failed");
            std::vector<int32_t> tok, pos, typ;
            std::vector<uint16_t> m;
            if (gr.e.mask) m.assign((size_t)tsum * tsum, 0xFC00);
            for (int b = i, s0 = 0; b < j; s0 += lens[b], b++)
                for (int t = 0; t < lens[b]; t++) {
                    tok.push_back(ids_in[(size_t)b * T + t]), typ.push_back(types_in[(size_t)b * T + t]);
                    pos.push_back(t);
                    if (gr.e.mask)
                        for (int k = 0; k < lens[b]; k++) m[(size_t)(s0 + t) * tsum + s0 + k] = 0x0000;
                }
            ggml_backend_tensor_set(gr.e.tok_ids, tok.data(), 0, tok.size() * 4);
            ggml_backend_tensor_set(gr.e.pos_ids, pos.data(), 0, pos.size() * 4);
            ggml_backend_tensor_set(gr.e.type_ids, typ.data(), 0, typ.size() * 4);
            if (gr.e.mask) ggml_backend_tensor_set(gr.e.mask, m.data(), 0, m.size() * 2);
            groups.push_back(gr);
            i = j;
        }
        std::vector<float> out;
        for (const Group &gr : groups) {
            if (ggml_backend_graph_compute(be, gr.e.gf) != GGML_STATUS_SUCCESS) return fail("graph_compute failed");
            const size_t at = out.size();
            out.resize(at + (size_t)H * gr.T);
            ggml_backend_tensor_get(gr.e.out, out.data() + at, 0, (size_t)H * gr.T * sizeof(float));
        }
        FILE *f = std::fopen(argv[7], "wb");
        if (!f || std::fwrite(out.data(), sizeof(float), out.size(), f) != out.size()) return fail("cannot write output");
        std::fclose(f);
        double ms = 0.0;
        if (iters > 0) {
            const auto t0 = std::chrono::steady_clock::now();
            for (int it = 0; it < iters; it++)
                for (const Group &gr : groups)
                    if (ggml_backend_graph_compute(be, gr.e.gf) != GGML_STATUS_SUCCESS) return fail("graph_compute failed");
            ggml_backend_synchronize(be);
            ms = std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - t0).count() / iters;
        }
        std::string sizes;
        for (const Group &gr : groups) sizes += (sizes.empty() ? "" : ", ") + std::to_string(gr.T);
        std::printf("{\"ok\": true, \"nodes\": %d, \"unsupported\": %d, \"ms_per_graph\": %.4f, \"iters\": %d, "
                    "\"groups\": %zu, \"group_tokens\": [%s]}\n",
                    nodes, unsupported, ms, iters, groups.size(), sizes.c_str());
        for (Group &gr : groups) {
            ggml_backend_buffer_free(gr.buf);
            ggml_free(gr.e.ctx);
        }
        ggml_backend_buffer_free(wbuf);
        ggml_free(wctx);
        ggml_backend_free(be);
        mq_gguf_close(g);
        return 0;
    }

    const EncGraph eg = build_graph(B, T, padded && B > 1 ? 1 : 0);
    ggml_context *gctx = eg.ctx;
    ggml_cgraph *gf = eg.gf;
    ggml_tensor *tok_ids = eg.tok_ids, *pos_ids = eg.pos_ids, *type_ids = eg.type_ids, *pad_mask = eg.mask, *cur = eg.out;
    const int unsupported = count_unsupported(gf);
    ggml_backend_buffer_t gbuf = ggml_backend_alloc_ctx_tensors(gctx, be);
    if (!gbuf) return fail("graph buffer allocation failed");

    std::vector<int32_t> pos(TB);
    for (int b = 0; b < B; b++)
        for (int t = 0; t < T; t++) pos[(size_t)b * T + t] = t;
    auto set_inputs = [&]() {
        ggml_backend_tensor_set(tok_ids, ids_raw.data(), 0, (size_t)TB * 4);
        ggml_backend_tensor_set(type_ids, types_raw.data(), 0, (size_t)TB * 4);
        ggml_backend_tensor_set(pos_ids, pos.data(), 0, (size_t)TB * 4);
        if (pad_mask) {
            std::vector<uint16_t> m((size_t)B * T * T);
            for (int b = 0; b < B; b++)
                for (int q = 0; q < T; q++)
                    for (int k = 0; k < T; k++)
                        m[((size_t)b * T + q) * T + k] = f16_bits(k < lens[b] ? 0.f : -INFINITY);
            ggml_backend_tensor_set(pad_mask, m.data(), 0, m.size() * 2);
        }
    };
    set_inputs();

    if (ggml_backend_graph_compute(be, gf) != GGML_STATUS_SUCCESS) return fail("graph_compute failed");
    std::vector<float> out((size_t)H * TB);
    ggml_backend_tensor_get(cur, out.data(), 0, out.size() * sizeof(float));
    FILE *f = std::fopen(argv[7], "wb");
    if (!f || std::fwrite(out.data(), sizeof(float), out.size(), f) != out.size()) return fail("cannot write output");
    std::fclose(f);

    int replay_identical = -1;
    if (check_replay) {
        std::vector<int32_t> ids2(TB);
        const int32_t *ids1 = (const int32_t *)ids_raw.data();
        for (int i = 0; i < TB; i++) ids2[i] = ids1[i] + 1;
        std::vector<float> o2(out.size()), o3(out.size()), o4(out.size());
        auto run = [&](const void *ids, std::vector<float> &dst) {
            ggml_backend_tensor_set(tok_ids, ids, 0, (size_t)TB * 4);
            if (ggml_backend_graph_compute(be, gf) != GGML_STATUS_SUCCESS) return false;
            ggml_backend_tensor_get(cur, dst.data(), 0, dst.size() * sizeof(float));
            return true;
        };
        if (!run(ids2.data(), o2) || !run(ids1, o3) || !run(ids2.data(), o4)) return fail("graph_compute failed");
        replay_identical = std::memcmp(o3.data(), out.data(), out.size() * 4) == 0 &&
                           std::memcmp(o4.data(), o2.data(), out.size() * 4) == 0;
        const std::string p2 = std::string(argv[7]) + ".second";
        FILE *f2 = std::fopen(p2.c_str(), "wb");
        if (!f2 || std::fwrite(o2.data(), sizeof(float), o2.size(), f2) != o2.size()) return fail("cannot write output");
        std::fclose(f2);
        ggml_backend_tensor_set(tok_ids, ids1, 0, (size_t)TB * 4);
    }
    // imatrix-style observation of every MUL_MAT's src1 (see --observe above)
    int observed = 0, src1_nan = -1;
    double src1_max_rel = -1.0, imatrix_max_rel = -1.0, out_max_rel = -1.0;
    if (observe) {
        const int n = ggml_graph_n_nodes(gf);
        std::vector<int> mms;
        for (int i = 0; i < n; i++)
            if (ggml_graph_node(gf, i)->op == GGML_OP_MUL_MAT) mms.push_back(i);
        auto read_src1 = [&](int i, std::vector<float> &v) {
            const ggml_tensor *x = ggml_graph_node(gf, i)->src[1];
            v.resize(ggml_nbytes(x) / sizeof(float));
            ggml_backend_tensor_get(x, v.data(), 0, ggml_nbytes(x));
        };
        std::vector<std::vector<float>> seen(mms.size()), ref(mms.size());
        ggml_backend_buffer_clear(gbuf, 0xFF);  // 0xFFFFFFFF is a NaN: an unwritten src1 shows
        set_inputs();
        int i0 = 0;
        for (size_t j = 0; j < mms.size(); j++) {
            ggml_cgraph *v = ggml_compat_graph_view(gf, i0, mms[j] + 1);
            const enum ggml_status st = ggml_backend_graph_compute(be, v);
            ggml_compat_graph_view_free(v);
            if (st != GGML_STATUS_SUCCESS) return fail("graph_compute of an observed piece failed");
            read_src1(mms[j], seen[j]);
            i0 = mms[j] + 1;
        }
        ggml_cgraph *tail = ggml_compat_graph_view(gf, i0, n);
        const enum ggml_status st_tail = ggml_backend_graph_compute(be, tail);
        ggml_compat_graph_view_free(tail);
        if (st_tail != GGML_STATUS_SUCCESS) return fail("graph_compute of the last piece failed");
        std::vector<float> obs_out(out.size());
        ggml_backend_tensor_get(cur, obs_out.data(), 0, obs_out.size() * sizeof(float));
        // the reference: node by node, every intermediate written
        ggml_backend_buffer_clear(gbuf, 0xFF);
        set_inputs();
        setenv("MQ_GGML_NO_FUSION", "1", 1);
        const enum ggml_status st_ref = ggml_backend_graph_compute(be, gf);
        unsetenv("MQ_GGML_NO_FUSION");
        if (st_ref != GGML_STATUS_SUCCESS) return fail("node-by-node graph_compute failed");
        for (size_t j = 0; j < mms.size(); j++) read_src1(mms[j], ref[j]);
        observed = (int)mms.size();
        src1_nan = 0;
        src1_max_rel = imatrix_max_rel = 0.0;
        for (size_t j = 0; j < mms.size(); j++) {
            const std::vector<float> &a = seen[j], &r = ref[j];
            const int64_t ne0 = ggml_graph_node(gf, mms[j])->src[1]->ne[0];
            bool nan = false;
            double mx = 0.0, d = 0.0;
            std::vector<double> sa(ne0, 0.0), sr(ne0, 0.0);  // imatrix: sum of x^2 per column
            for (size_t e = 0; e < a.size(); e++) {
                nan |= std::isnan(a[e]) || std::isnan(r[e]);
                mx = std::fmax(mx, std::fabs((double)r[e]));
                d = std::fmax(d, std::fabs((double)a[e] - (double)r[e]));
                sa[e % ne0] += (double)a[e] * a[e];
                sr[e % ne0] += (double)r[e] * r[e];
            }
            src1_nan += nan;
            src1_max_rel = std::fmax(src1_max_rel, nan ? INFINITY : d / (mx > 0 ? mx : 1.0));
            double smx = 0.0, sd = 0.0;
            for (int64_t c = 0; c < ne0; c++) {
                smx = std::fmax(smx, sr[c]);
                sd = std::fmax(sd, std::fabs(sa[c] - sr[c]));
            }
            imatrix_max_rel = std::fmax(imatrix_max_rel, nan ? INFINITY : sd / (smx > 0 ? smx : 1.0));
        }
        double omx = 0.0, od = 0.0;
        for (size_t e = 0; e < out.size(); e++) {
            omx = std::fmax(omx, std::fabs((double)out[e]));
            od = std::fmax(od, std::fabs((double)obs_out[e] - (double)out[e]));
        }
        out_max_rel = std::isnan(od) ? INFINITY : od / (omx > 0 ? omx : 1.0);
        set_inputs();
    }
    double ms = 0.0;
    if (iters > 0) {
        const auto t0 = std::chrono::steady_clock::now();
        for (int i = 0; i < iters; i++)
            if (ggml_backend_graph_compute(be, gf) != GGML_STATUS_SUCCESS) return fail("graph_compute failed");
        ms = std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - t0).count() / iters;
    }
    std::printf("{\"ok\": true, \"nodes\": %d, \"unsupported\": %d, \"ms_per_graph\": %.4f, \"iters\": %d, "
                "\"replay_identical\": %d, \"observed\": %d, \"src1_nan\": %d, \"src1_max_rel\": %.3g, "
                "\"imatrix_max_rel\": %.3g, \"out_max_rel\": %.3g}\n",
                ggml_graph_n_nodes(gf), unsupported, ms, iters, replay_identical, observed, src1_nan, fin(src1_max_rel),
                fin(imatrix_max_rel), fin(out_max_rel));
    ggml_backend_buffer_free(gbuf);
    ggml_backend_buffer_free(wbuf);
    ggml_free(gctx);
    ggml_free(wctx);
    ggml_backend_free(be);
    mq_gguf_close(g);
    return 0;
}
