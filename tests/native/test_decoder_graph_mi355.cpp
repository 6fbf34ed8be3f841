// test-decoder-graph-mi355 -- CrispEmbed's decoder-embedder graph for the Qwen3 family, built
// with ggml's graph API as src/decoder_embed.cpp builds it (:680-830: GET_ROWS embedding, per
// layer RMS_NORM x attn_norm, q/k/v MUL_MAT, RESHAPE_3D, per-head RMS_NORM x q_norm / k_norm,
// ROPE_EXT NEOX on pos_ids, PERMUTE, FLASH_ATTN_EXT with the F16 mask (none for a bidirectional
// model's single sequence), the output projection, residual ADD, RMS_NORM x ffn_norm,
// SiLU(gate) * up, the down projection and residual ADD; then the output RMS norm), computed
// entirely by the MI355X backend.
//
// usage: test-decoder-graph-mi355 model.gguf T ids.i32 out.f32 [--batch B] [--lens lens.i32]
//                                 [--iters N] [--act-check] [--dump rows.i32 dir] [--observe]
//   Without --batch (or B = 1): one sequence of T tokens (decoder_encode_tokens).
//   --batch B: ids.i32 holds B items of T slots (item b's tokens at b * T, its length lens[b] from
//   lens.i32, default T), laid out as decoder_encode_tokens_batch lays them out
//   (src/decoder_embed.cpp:1322-1443): with a common prefix of at least 4 tokens and a causal
//   model, [prefix | suffix_0 padded | suffix_1 padded | ...] with positions continuing the
//   prefix, else [item_0 padded | item_1 padded | ...] with positions restarting per item; one
//   T_total x T_total F16 mask (0 where a query may see a key: causal within its item and to the
//   prefix, a padding position only itself; -inf elsewhere) shared by every layer.
//   out: the normed last hidden state [H, T_total] as float32.  Prints one JSON line (with the
//   layout: T_total, prefix, slot).
//   --act-check: sets the backend's activation observer (ggml_backend_mi355_set_act_observer)
//   and compares every quantized activation a product reads with the oracle's quantization of
//   the graph's own fp32 src1 (for the down projection, whose src1 SiLU(gate) * up the backend
//   forms inside the quantizer, of silu(gate) * up from the gate and up tensors with the host
//   expf): quants, scales and the Q4_K min-term operands, every row.  Reports rows that differ
//   (must be none outside the down projection) and the down projection's fraction of equal quants.
//   --dump rows.i32 dir: for the token rows listed in rows.i32, writes per layer il the fp32
//   rows of attn_norm / attn_out / ffn_norm / gate / up / l_out (dir/<name>_<il>.f32), and with
//   --act-check the quantized activations the products read (dir/act_<name>_<il>.i8 quants and
//   .f32 scales) -- the teacher-forcing inputs of the Python test.
//   --observe: then computes the graph as ggml's scheduler does when an eval callback observes
//   every MUL_MAT (the imatrix collector, src/imatrix.cpp:57-99, installed on the decoder's
//   scheduler at src/crispembed.cpp:2483): in pieces that end at each MUL_MAT, reading its src1
//   after its piece, every graph tensor first filled with NaN bytes; and once more node by node
//   (MQ_GGML_NO_FUSION=1) as the reference.  Reports the observed src1 that still hold NaN, the
//   largest relative difference of any src1 and of the imatrix sums of x^2 per column, and of
//   the output against the unobserved run (and each item's last-token cosine between them); with
//   --act-check the observed run's quantized activations are checked as well (obs_act_*).
#include <chrono>
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <map>
#include <string>
#include <vector>

#include <hip/hip_runtime_api.h>

#include "ggml-backend.h"
#include "ggml-mi355.h"
#include "ggml.h"
#include "ggml_oracle.h"
#include "mq.h"
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

static bool write_file(const std::string &path, const void *p, size_t n) {
    FILE *f = std::fopen(path.c_str(), "wb");
    if (!f) return false;
    const bool ok = std::fwrite(p, 1, n, f) == n;
    return std::fclose(f) == 0 && ok;
}

static int fail(const char *msg) {
    std::printf("{\"ok\": false, \"error\": \"%s\"}\n", msg);
    return 1;
}

static double fin(double x) { return std::isfinite(x) ? x : 1e30; }  // JSON has no inf / nan

static std::vector<float> get_f32(const ggml_tensor *t) {
    std::vector<float> v(ggml_nbytes(t) / sizeof(float));
    ggml_backend_tensor_get(t, v.data(), 0, ggml_nbytes(t));
    return v;
}

// ---------------------------------------------------------------- activation check ----
// The GEMM-path activation layout (mq_quantize_act_ex, MQ_PATH_GEMM), restated from its
// definition in include/mq.h: quants in 1 KB fragments -- lane L of fragment (row tile rt, 32-byte
// K chunk kc) holds row 32 rt + L % 32, bytes 32 kc + 16 (L / 32) .. + 16 -- over m_pad = m rounded
// up to 256 rows and kb_pad = K bytes rounded up to 128; then (256-byte aligned) the scales as
// float planes [block][m_pad]; for Q8_K then the min-term operands: per (row tile, superblock) 64
// lanes x 8 halves, lane r % 32 holding B_j & 63 and lane 32 + r % 32 holding 64 (B_j >> 6) for
// the 8 sub-block sums B_j of row r.
static size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

struct Layer {  // the tensors of one layer that the dump writes
    ggml_tensor *attn_norm, *attn_out, *ffn_norm, *gate, *up, *l_out, *q, *o, *gmm, *down;
};

struct ActCheck {
    std::map<const ggml_tensor *, std::pair<int, std::string>> role;  // product -> (layer, activation)
    const std::vector<int32_t> *rows = nullptr;                      // dump rows
    std::string dir;
    int calls = 0, checked = 0, unchecked = 0, silu_calls = 0;
    int64_t rows_checked = 0, rows_bad = 0;
    double silu_min_same = 1.0;
    std::string first_bad;
    const void *last_act = nullptr;
    const ggml_tensor *last_src1 = nullptr;
    bool io_error = false;
};

static bool is_silu(const ggml_tensor *t) {
    return t && t->op == GGML_OP_UNARY && ggml_get_unary_op(t) == GGML_UNARY_OP_SILU;
}

static void act_observer(const ggml_tensor *node, int type, int path, const void *act, size_t act_bytes, int64_t M,
                         int64_t K, void *user) {
    ActCheck &ck = *(ActCheck *)user;
    ck.calls++;
    const ggml_tensor *x = node->src[1];
    if (act == ck.last_act && x == ck.last_src1) return;  // a grouped member: the same activation
    ck.last_act = act, ck.last_src1 = x;
    if (path != MQ_PATH_GEMM || (type != MQ_TYPE_Q4_K && type != MQ_TYPE_Q6_K && type != MQ_TYPE_Q8_0)) {
        ck.unchecked++;
        return;
    }
    // the fp32 input the product quantizes
    std::vector<float> xin;
    const ggml_tensor *mul = x;
    const bool silu_mul = mul->op == GGML_OP_MUL && (is_silu(mul->src[0]) || is_silu(mul->src[1]));
    if (silu_mul) {
        const ggml_tensor *s = is_silu(mul->src[0]) ? mul->src[0] : mul->src[1];
        const ggml_tensor *u = s == mul->src[0] ? mul->src[1] : mul->src[0];
        const std::vector<float> g = get_f32(s->src[0]), up = get_f32(u);
        xin.resize(g.size());
        for (size_t e = 0; e < g.size(); e++) xin[e] = g[e] / (1.0f + std::exp(-g[e])) * up[e];  // ggml_silu_f32
    } else {
        xin = get_f32(x);
    }
    if ((int64_t)xin.size() != M * K) {
        ck.unchecked++;
        return;
    }
    std::vector<uint8_t> img(act_bytes);
    if (hipMemcpy(img.data(), act, act_bytes, hipMemcpyDeviceToHost) != hipSuccess) {
        ck.io_error = true;
        return;
    }
    const bool q8k = type != MQ_TYPE_Q8_0;
    const int64_t bs = q8k ? 256 : 32, nblk = K / bs;
    const size_t rsz = or_row_size(q8k ? OR_TYPE_Q8_K : OR_TYPE_Q8_0, K);
    std::vector<uint8_t> ref((size_t)M * rsz);
    or_quantize_act_rows(type, xin.data(), K, ref.data(), M, K, mq_q8_0_variant());
    const int64_t m_pad = (M + 255) / 256 * 256, kb_pad = (K + 127) / 128 * 128;
    const size_t xd = align256((size_t)m_pad * kb_pad), xmin = align256(xd + (size_t)nblk * m_pad * 4);
    const int8_t *q = (const int8_t *)img.data();
    const float *d = (const float *)(img.data() + xd);
    const uint16_t *fr = (const uint16_t *)(img.data() + xmin);
    // the quants row-major: fragment (rt, kc) lane l -> row 32 rt + l % 32, bytes 32 kc + 16 (l / 32)
    std::vector<int8_t> qr((size_t)M * K);
    for (int64_t rt = 0; rt < (M + 31) / 32; rt++)
        for (int64_t kc = 0; kc < K / 32; kc++)
            for (int l = 0; l < 64; l++) {
                const int64_t r = rt * 32 + l % 32;
                if (r < M) std::memcpy(&qr[(size_t)r * K + kc * 32 + 16 * (l / 32)], q + ((rt * (kb_pad / 32) + kc) * 64 + l) * 16, 16);
            }
    int64_t same = 0;
    for (int64_t r = 0; r < M; r++) {
        bool bad = false;
        const uint8_t *rb = ref.data() + (size_t)r * rsz;
        const int8_t *rq = &qr[(size_t)r * K];
        for (int64_t j = 0; j < nblk; j++) {
            const float rd = d[j * m_pad + r];
            float dw;
            const int8_t *qw;
            if (q8k) {
                const or_block_q8_K *blk = (const or_block_q8_K *)rb + j;
                dw = blk->d, qw = blk->qs;
                for (int sb = 0; sb < 8; sb++) {  // min-term operands from the oracle's sums
                    const int Bj = blk->bsums[2 * sb] + blk->bsums[2 * sb + 1];
                    const uint16_t lo = or_fp32_to_fp16((float)(Bj & 63)), hi = or_fp32_to_fp16((float)(64 * (Bj >> 6)));
                    const size_t base = (((size_t)(r / 32) * nblk + j) * 64) * 8;
                    if (fr[base + (r % 32) * 8 + sb] != lo || fr[base + (32 + r % 32) * 8 + sb] != hi) bad = true;
                }
            } else {
                const or_block_q8_0 *blk = (const or_block_q8_0 *)rb + j;
                dw = or_fp16_to_fp32(blk->d), qw = blk->qs;
            }
            uint32_t a, b2;
            std::memcpy(&a, &rd, 4), std::memcpy(&b2, &dw, 4);
            if (a != b2) bad = true;
            if (std::memcmp(rq + j * bs, qw, (size_t)bs) == 0) {
                same += bs;
            } else {
                bad = true;
                for (int64_t e = 0; e < bs; e++) same += rq[j * bs + e] == qw[e];
            }
        }
        if (bad) {
            ck.rows_bad += !silu_mul;
            if (!silu_mul && ck.first_bad.empty()) {
                char buf[160];
                std::snprintf(buf, sizeof buf, "%s row %lld", node->name, (long long)r);
                ck.first_bad = buf;
            }
        }
    }
    ck.checked++;
    ck.rows_checked += M;
    {
        auto r = ck.role.find(node);
        std::fprintf(stderr, "act-check %s layer %d: %lld rows x %lld, %lld bad so far\n",
                     r == ck.role.end() ? node->name : r->second.second.c_str(), r == ck.role.end() ? -1 : r->second.first,
                     (long long)M, (long long)K, (long long)ck.rows_bad);
    }
    if (silu_mul) {
        ck.silu_calls++;
        ck.silu_min_same = std::fmin(ck.silu_min_same, (double)same / (double)(M * K));
    }
    // the activation of the dump rows, as the product reads it
    auto it = ck.role.find(node);
    if (ck.rows && it != ck.role.end()) {
        const std::vector<int32_t> &rows = *ck.rows;
        std::vector<int8_t> oq((size_t)rows.size() * K);
        std::vector<float> od((size_t)rows.size() * nblk);
        for (size_t i = 0; i < rows.size(); i++) {
            const int64_t r = rows[i];
            std::memcpy(&oq[i * K], &qr[(size_t)r * K], (size_t)K);
            for (int64_t j = 0; j < nblk; j++) od[i * nblk + j] = d[j * m_pad + r];
        }
        const std::string stem = ck.dir + "/act_" + it->second.second + "_" + std::to_string(it->second.first);
        if (!write_file(stem + ".i8", oq.data(), oq.size()) || !write_file(stem + ".f32", od.data(), od.size() * 4))
            ck.io_error = true;
    }
}

int main(int argc, char **argv) {
    if (argc < 5) return fail("usage: model.gguf T ids out [--batch B] [--lens f] [--iters N] [--act-check] ...");
    const char *path = argv[1];
    const int T = std::atoi(argv[2]);
    int iters = 0, B = 1;
    bool observe = false, act_check = false;
    const char *lens_path = nullptr, *rows_path = nullptr, *dump_dir = nullptr;
    for (int i = 5; i < argc; i++) {
        if (!std::strcmp(argv[i], "--iters") && i + 1 < argc) iters = std::atoi(argv[++i]);
        else if (!std::strcmp(argv[i], "--batch") && i + 1 < argc) B = std::atoi(argv[++i]);
        else if (!std::strcmp(argv[i], "--lens") && i + 1 < argc) lens_path = argv[++i];
        else if (!std::strcmp(argv[i], "--observe")) observe = true;
        else if (!std::strcmp(argv[i], "--act-check")) act_check = true;
        else if (!std::strcmp(argv[i], "--dump") && i + 2 < argc) rows_path = argv[++i], dump_dir = argv[++i];
        else return fail("unknown argument");
    }
    std::vector<char> ids_raw = read_file(argv[3]);
    if (T <= 0 || B <= 0 || ids_raw.size() != (size_t)B * T * 4) return fail("bad T / B or ids file size");
    const int32_t *ids_in = (const int32_t *)ids_raw.data();
    std::vector<int> lens(B, T);
    if (lens_path) {
        std::vector<char> l = read_file(lens_path);
        if (l.size() != (size_t)B * 4) return fail("bad lens file size");
        for (int b = 0; b < B; b++) {
            lens[b] = ((const int32_t *)l.data())[b];
            if (lens[b] < 1 || lens[b] > T) return fail("lens out of range");
        }
    }

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

    // ---- token layout, positions and mask (src/decoder_embed.cpp:1297-1443) ----
    int P = 0, slot = T, T_total = T;
    bool use_prefix = false, use_mask = causal;
    std::vector<int32_t> tok, pos;
    std::vector<uint16_t> mask;  // F16: 0x0000 = 0, 0xFC00 = -inf
    if (B == 1) {                // the single-text path: causal mask over the sequence
        T_total = slot = lens[0];
        tok.assign(ids_in, ids_in + T_total);
        for (int t = 0; t < T_total; t++) pos.push_back(t);
        if (causal) {
            mask.assign((size_t)T_total * T_total, 0xFC00);
            for (int q = 0; q < T_total; q++)
                for (int k = 0; k <= q; k++) mask[(size_t)q * T_total + k] = 0x0000;
        }
    } else {
        int min_len = lens[0];
        for (int b = 1; b < B; b++) min_len = std::min(min_len, lens[b]);
        for (; P < min_len; P++) {  // detect_common_prefix
            bool match = true;
            for (int b = 1; b < B && match; b++) match = ids_in[(size_t)b * T + P] == ids_in[P];
            if (!match) break;
        }
        use_prefix = P >= 4 && causal;
        int S_max = 0, T_max = 0;
        for (int b = 0; b < B; b++) S_max = std::max(S_max, lens[b] - (P >= 4 ? P : 0)), T_max = std::max(T_max, lens[b]);
        slot = use_prefix ? S_max : T_max;
        if (!use_prefix) P = 0;
        T_total = use_prefix ? P + S_max * B : T_max * B;
        tok.assign(T_total, 0);
        pos.assign(T_total, 0);
        mask.assign((size_t)T_total * T_total, 0xFC00);
        auto open = [&](int q, int k) { mask[(size_t)q * T_total + k] = 0x0000; };
        if (use_prefix) {
            for (int t = 0; t < P; t++) {
                tok[t] = ids_in[t], pos[t] = t;
                for (int k = 0; k <= t; k++) open(t, k);
            }
            for (int b = 0; b < B; b++) {
                const int base = P + b * S_max, sl = lens[b] - P;
                for (int s = 0; s < sl; s++) {
                    tok[base + s] = ids_in[(size_t)b * T + P + s], pos[base + s] = P + s;
                    for (int k = 0; k < P; k++) open(base + s, k);
                    for (int k = 0; k <= s; k++) open(base + s, base + k);
                }
                for (int s = sl; s < S_max; s++) open(base + s, base + s);
            }
        } else {
            for (int b = 0; b < B; b++) {
                for (int t = 0; t < lens[b]; t++) {
                    tok[b * T_max + t] = ids_in[(size_t)b * T + t], pos[b * T_max + t] = t;
                    for (int k = 0; k < (causal ? t + 1 : lens[b]); k++) open(b * T_max + t, b * T_max + k);
                }
                for (int t = lens[b]; t < T_max; t++) open(b * T_max + t, b * T_max + t);
            }
        }
        use_mask = true;
    }

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

    const size_t graph_size = std::max(4096, n_layer * 50 + 256);  // as decoder_encode_tokens_batch sizes it
    ggml_init_params gp = {ggml_tensor_overhead() * (size_t)(n_layer * 64 + 64) + ggml_graph_overhead_custom(graph_size, false),
                           nullptr, true};
    ggml_context *gctx = ggml_init(gp);
    ggml_tensor *ids = ggml_new_tensor_1d(gctx, GGML_TYPE_I32, T_total);
    ggml_set_name(ids, "inp_tokens");
    ggml_set_input(ids);
    ggml_tensor *pos_t = ggml_new_tensor_1d(gctx, GGML_TYPE_I32, T_total);
    ggml_set_name(pos_t, "pos_ids");
    ggml_set_input(pos_t);
    ggml_tensor *mask_t = nullptr;
    if (use_mask) {
        mask_t = ggml_new_tensor_2d(gctx, GGML_TYPE_F16, T_total, T_total);
        ggml_set_name(mask_t, "attn_mask");
        ggml_set_input(mask_t);
    }
    auto rms_norm = [&](ggml_tensor *x, ggml_tensor *w) { return ggml_mul(gctx, ggml_rms_norm(gctx, x, eps), w); };
    std::vector<Layer> layers(n_layer);
    ggml_tensor *cur = ggml_get_rows(gctx, get("token_embd.weight"), ids);
    for (int il = 0; il < n_layer; il++) {
        const std::string p = "dec." + std::to_string(il) + ".";
        Layer &Ly = layers[il];
        ggml_tensor *residual = cur;
        cur = Ly.attn_norm = rms_norm(cur, get(p + "attn_norm.weight"));
        ggml_tensor *Q = Ly.q = ggml_mul_mat(gctx, get(p + "attn.q.weight"), cur);
        ggml_tensor *K = ggml_mul_mat(gctx, get(p + "attn.k.weight"), cur);
        ggml_tensor *V = ggml_mul_mat(gctx, get(p + "attn.v.weight"), cur);
        Q = ggml_reshape_3d(gctx, Q, hd, nh, T_total);
        K = ggml_reshape_3d(gctx, K, hd, nkv, T_total);
        V = ggml_reshape_3d(gctx, V, hd, nkv, T_total);
        if (get(p + "attn.q_norm.weight")) Q = rms_norm(Q, get(p + "attn.q_norm.weight"));
        if (get(p + "attn.k_norm.weight")) K = rms_norm(K, get(p + "attn.k_norm.weight"));
        Q = ggml_rope_ext(gctx, Q, pos_t, nullptr, hd, GGML_ROPE_TYPE_NEOX, 0, theta, 1.0f, 0.0f, 1.0f, 0.0f, 0.0f);
        K = ggml_rope_ext(gctx, K, pos_t, nullptr, hd, GGML_ROPE_TYPE_NEOX, 0, theta, 1.0f, 0.0f, 1.0f, 0.0f, 0.0f);
        Q = ggml_permute(gctx, Q, 0, 2, 1, 3);
        K = ggml_permute(gctx, K, 0, 2, 1, 3);
        V = ggml_permute(gctx, V, 0, 2, 1, 3);
        ggml_tensor *attn = ggml_flash_attn_ext(gctx, Q, K, V, mask_t, 1.0f / std::sqrt((float)hd), 0.0f, 0.0f);
        attn = Ly.attn_out = ggml_reshape_2d(gctx, attn, (int64_t)nh * hd, T_total);
        attn = Ly.o = ggml_mul_mat(gctx, get(p + "attn.o.weight"), attn);
        cur = ggml_add(gctx, residual, attn);
        residual = cur;
        cur = Ly.ffn_norm = rms_norm(cur, get(p + "ffn_norm.weight"));
        ggml_tensor *gate = Ly.gate = Ly.gmm = ggml_mul_mat(gctx, get(p + "ffn.gate.weight"), cur);
        gate = ggml_silu(gctx, gate);
        ggml_tensor *up = Ly.up = ggml_mul_mat(gctx, get(p + "ffn.up.weight"), cur);
        ggml_tensor *ffn = Ly.down = ggml_mul_mat(gctx, get(p + "ffn.down.weight"), ggml_mul(gctx, gate, up));
        cur = Ly.l_out = ggml_add(gctx, residual, ffn);
    }
    cur = rms_norm(cur, get("output_norm.weight"));
    ggml_set_name(cur, "decoder_out");
    ggml_set_output(cur);
    ggml_cgraph *gf = ggml_new_graph_custom(gctx, graph_size, false);
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
    auto set_inputs = [&]() {
        ggml_backend_tensor_set(ids, tok.data(), 0, (size_t)T_total * 4);
        ggml_backend_tensor_set(pos_t, pos.data(), 0, (size_t)T_total * 4);
        if (mask_t) ggml_backend_tensor_set(mask_t, mask.data(), 0, mask.size() * 2);
    };
    set_inputs();

    std::vector<int32_t> dump_rows;
    if (rows_path) {
        std::vector<char> r = read_file(rows_path);
        dump_rows.assign((const int32_t *)r.data(), (const int32_t *)(r.data() + r.size()));
        for (int32_t v : dump_rows)
            if (v < 0 || v >= T_total) return fail("dump row out of range");
    }
    ActCheck ck;
    if (act_check) {
        for (int il = 0; il < n_layer; il++) {
            ck.role[layers[il].q] = {il, "attn_norm"};
            ck.role[layers[il].o] = {il, "attn_out"};
            ck.role[layers[il].gmm] = {il, "ffn_norm"};
            ck.role[layers[il].down] = {il, "ffn_gate_up"};
        }
        if (rows_path) ck.rows = &dump_rows, ck.dir = dump_dir;
        ggml_backend_mi355_set_act_observer(be, act_observer, &ck);
    }
    if (ggml_backend_graph_compute(be, gf) != GGML_STATUS_SUCCESS) return fail("graph_compute failed");
    ggml_backend_mi355_set_act_observer(be, nullptr, nullptr);
    if (ck.io_error) return fail("activation check: copy or write failed");
    std::vector<float> out = get_f32(cur);
    if (!write_file(argv[4], out.data(), out.size() * sizeof(float))) return fail("cannot write output");
    if (rows_path) {  // the teacher-forcing tensors of every layer, at the dump rows
        for (int il = 0; il < n_layer; il++) {
            const Layer &Ly = layers[il];
            const std::pair<const char *, ggml_tensor *> named[] = {{"attn_norm", Ly.attn_norm}, {"attn_out", Ly.attn_out},
                                                                    {"ffn_norm", Ly.ffn_norm},   {"gate", Ly.gate},
                                                                    {"up", Ly.up},               {"l_out", Ly.l_out}};
            for (const auto &nt2 : named) {
                const int64_t ne0 = nt2.second->ne[0];
                std::vector<float> v(dump_rows.size() * ne0);
                for (size_t i = 0; i < dump_rows.size(); i++)
                    ggml_backend_tensor_get(nt2.second, v.data() + i * ne0, (size_t)dump_rows[i] * nt2.second->nb[1],
                                            ne0 * sizeof(float));
                if (!write_file(std::string(dump_dir) + "/" + nt2.first + "_" + std::to_string(il) + ".f32", v.data(),
                                v.size() * 4))
                    return fail("cannot write a dump file");
            }
        }
    }

    // imatrix-style observation of every MUL_MAT's src1 (see --observe above)
    int observed = 0, src1_nan = -1;
    double src1_max_rel = -1.0, src1_max_rel_first = -1.0, src1_max_rel_norm0 = -1.0, imatrix_max_rel = -1.0,
           out_max_rel = -1.0, obs_pooled_cos_min = -1.0;
    ActCheck ck2;  // the observed run's own activations (with --act-check)
    if (observe) {
        const int n = ggml_graph_n_nodes(gf);
        std::vector<int> mms;
        for (int i = 0; i < n; i++)
            if (ggml_graph_node(gf, i)->op == GGML_OP_MUL_MAT) mms.push_back(i);
        // the reference first: node by node, every intermediate written; each distinct src1 kept
        ggml_backend_buffer_clear(gbuf, 0xFF);  // 0xFFFFFFFF is a NaN: an unwritten src1 shows
        set_inputs();
        setenv("MQ_GGML_NO_FUSION", "1", 1);
        const enum ggml_status st_ref = ggml_backend_graph_compute(be, gf);
        unsetenv("MQ_GGML_NO_FUSION");
        if (st_ref != GGML_STATUS_SUCCESS) return fail("node-by-node graph_compute failed");
        {
            const std::vector<float> nbn = get_f32(cur);
            double omx = 0.0, od = 0.0;
            for (size_t e = 0; e < out.size(); e++) {
                omx = std::fmax(omx, std::fabs((double)out[e]));
                od = std::fmax(od, std::fabs((double)nbn[e] - (double)out[e]));
            }
            std::fprintf(stderr, "node-by-node output against the fused run: max rel %.3g\n", od / omx);
        }
        std::map<const ggml_tensor *, std::vector<float>> ref;
        for (int i : mms) {
            const ggml_tensor *x = ggml_graph_node(gf, i)->src[1];
            if (!ref.count(x)) ref[x] = get_f32(x);
        }
        ggml_backend_buffer_clear(gbuf, 0xFF);
        set_inputs();
        if (act_check) {
            ck2.role = ck.role;
            ggml_backend_mi355_set_act_observer(be, act_observer, &ck2);
        }
        int i0 = 0;
        src1_nan = 0;
        src1_max_rel = src1_max_rel_first = imatrix_max_rel = 0.0;
        for (size_t j = 0; j < mms.size(); j++) {
            ggml_cgraph *v = ggml_compat_graph_view(gf, i0, mms[j] + 1);
            const enum ggml_status st = ggml_backend_graph_compute(be, v);
            ggml_compat_graph_view_free(v);
            if (st != GGML_STATUS_SUCCESS) return fail("graph_compute of an observed piece failed");
            const ggml_tensor *x = ggml_graph_node(gf, mms[j])->src[1];
            const std::vector<float> seen = get_f32(x), &r = ref[x];
            const int64_t ne0 = x->ne[0];
            bool nan = false;
            double mx = 0.0, d = 0.0;
            std::vector<double> sa(ne0, 0.0), sr(ne0, 0.0);  // imatrix: sum of x^2 per column
            for (size_t e = 0; e < seen.size(); e++) {
                nan |= std::isnan(seen[e]) || std::isnan(r[e]);
                mx = std::fmax(mx, std::fabs((double)r[e]));
                d = std::fmax(d, std::fabs((double)seen[e] - (double)r[e]));
                sa[e % ne0] += (double)seen[e] * seen[e];
                sr[e % ne0] += (double)r[e] * r[e];
            }
            src1_nan += nan;
            src1_max_rel = std::fmax(src1_max_rel, nan ? INFINITY : d / (mx > 0 ? mx : 1.0));
            if (j < 7)  // the first layer's products
                src1_max_rel_first = std::fmax(src1_max_rel_first, nan ? INFINITY : d / (mx > 0 ? mx : 1.0));
            if (j < 3)  // q / k / v of the first layer: the normed embeddings, before any quantization
                src1_max_rel_norm0 = std::fmax(src1_max_rel_norm0, nan ? INFINITY : d / (mx > 0 ? mx : 1.0));
            if (j < 14) {
                int64_t worst = 0;
                for (size_t e = 0; e < seen.size(); e++)
                    if (std::fabs((double)seen[e] - r[e]) > std::fabs((double)seen[worst] - r[worst])) worst = (int64_t)e;
                std::fprintf(stderr, "product %zu (%s, src1 %s op %s): max rel %.3g at element %lld (row %lld): %.8g vs %.8g\n",
                             j, ggml_graph_node(gf, mms[j])->src[0]->name, x->name, ggml_op_name(x->op),
                             d / (mx > 0 ? mx : 1.0), (long long)worst, (long long)(worst / ne0), seen[worst], r[worst]);
            }
            double smx = 0.0, sd = 0.0;
            for (int64_t c = 0; c < ne0; c++) {
                smx = std::fmax(smx, sr[c]);
                sd = std::fmax(sd, std::fabs(sa[c] - sr[c]));
            }
            imatrix_max_rel = std::fmax(imatrix_max_rel, nan ? INFINITY : sd / (smx > 0 ? smx : 1.0));
            i0 = mms[j] + 1;
            observed++;
            if (observed % 7 == 0) std::fprintf(stderr, "observed %d products, src1 max rel %.3g\n", observed, src1_max_rel);
        }
        ggml_cgraph *tail = ggml_compat_graph_view(gf, i0, n);
        const enum ggml_status st_tail = ggml_backend_graph_compute(be, tail);
        ggml_compat_graph_view_free(tail);
        if (st_tail != GGML_STATUS_SUCCESS) return fail("graph_compute of the last piece failed");
        ggml_backend_mi355_set_act_observer(be, nullptr, nullptr);
        if (ck2.io_error) return fail("activation check of the observed run: copy or write failed");
        const std::vector<float> obs_out = get_f32(cur);
        obs_pooled_cos_min = 1.0;  // each item's last token (last-token pooling), observed against unobserved
        for (int b = 0; b < B; b++) {
            const int64_t row = B == 1 ? T_total - 1 : (use_prefix ? P + (int64_t)b * slot + lens[b] - P - 1
                                                                   : (int64_t)b * slot + lens[b] - 1);
            double ab = 0.0, aa = 0.0, bb = 0.0;
            for (int e = 0; e < H; e++) {
                const double u = obs_out[row * H + e], v = out[row * H + e];
                ab += u * v, aa += u * u, bb += v * v;
            }
            obs_pooled_cos_min = std::fmin(obs_pooled_cos_min, ab / std::sqrt(aa * bb));
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
        if (ggml_backend_graph_compute(be, gf) != GGML_STATUS_SUCCESS) return fail("graph_compute failed");
        ggml_backend_synchronize(be);
        const auto t0 = std::chrono::steady_clock::now();
        for (int i = 0; i < iters; i++)
            if (ggml_backend_graph_compute(be, gf) != GGML_STATUS_SUCCESS) return fail("graph_compute failed");
        ggml_backend_synchronize(be);
        ms = std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - t0).count() / iters;
    }
    std::printf("{\"ok\": true, \"nodes\": %d, \"unsupported\": %d, \"ms_per_graph\": %.4f, \"iters\": %d, "
                "\"T_total\": %d, \"prefix\": %d, \"slot\": %d, \"act_calls\": %d, \"act_checked\": %d, "
                "\"act_unchecked\": %d, \"act_rows_checked\": %lld, \"act_rows_bad\": %lld, \"act_first_bad\": \"%s\", "
                "\"silu_calls\": %d, \"silu_min_same\": %.7f, \"observed\": %d, \"src1_nan\": %d, "
                "\"src1_max_rel\": %.3g, \"src1_max_rel_first\": %.3g, \"src1_max_rel_norm0\": %.3g, "
                "\"imatrix_max_rel\": %.3g, \"out_max_rel\": %.3g, \"obs_pooled_cos_min\": %.9f, "
                "\"obs_act_checked\": %d, \"obs_act_unchecked\": %d, \"obs_act_rows_bad\": %lld, "
                "\"obs_silu_min_same\": %.7f}\n",
                ggml_graph_n_nodes(gf), unsupported, ms, iters, T_total, use_prefix ? P : 0, slot, ck.calls, ck.checked,
                ck.unchecked, (long long)ck.rows_checked, (long long)ck.rows_bad, ck.first_bad.c_str(), ck.silu_calls,
                ck.silu_min_same, observed, src1_nan, fin(src1_max_rel), fin(src1_max_rel_first), fin(src1_max_rel_norm0),
                fin(imatrix_max_rel), fin(out_max_rel), obs_pooled_cos_min, ck2.checked, ck2.unchecked,
                (long long)ck2.rows_bad, ck2.silu_min_same);
    ggml_backend_buffer_free(gbuf);
    ggml_backend_buffer_free(wbuf);
    ggml_free(gctx);
    ggml_free(wctx);
    ggml_backend_free(be);
    mq_gguf_close(g);
    return 0;
}
