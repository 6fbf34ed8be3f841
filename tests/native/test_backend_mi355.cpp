// test-backend-mi355 -- runs GGML_OP_MUL_MAT graphs through the MI355X ggml
// backend exactly as a ggml host would (registry lookup by name, one backend
// buffer from ggml_backend_alloc_ctx_tensors, tensor_set of GGUF bytes,
// ggml_backend_graph_compute, tensor_get) and checks every result against the
// CPU oracle.  It follows the reference's backend smoke test
// (tests/test_backend_smoke.cpp: backend chosen by name, graph computed, JSON
// summary) with MUL_MAT graphs in place of the 16-element ADD.
//
// usage: test-backend-mi355 [backend-name-prefix] [--json]
#include <dlfcn.h>

#include <algorithm>
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <string>
#include <vector>

#include "ggml-backend-impl.h"  // ggml_backend_reg::api_version, as ggml_backend_load checks it
#include "ggml-backend.h"
#include "ggml-mi355.h"
#include "ggml.h"
#include "ggml_oracle.h"

static bool starts_with_ci(const char *s, const char *prefix) {
    for (; *prefix; ++s, ++prefix)
        if (!*s || std::tolower((unsigned char)*s) != std::tolower((unsigned char)*prefix)) return false;
    return true;
}

// first GPU device whose name starts with `pref` (the selection rule of
// crispasr_init_gpu_backend, src/core/gpu_backend_pref.h:117-132)
static ggml_backend_t init_by_name(const char *pref) {
    for (size_t i = 0; i < ggml_backend_dev_count(); ++i) {
        ggml_backend_dev_t dev = ggml_backend_dev_get(i);
        if (ggml_backend_dev_type(dev) != GGML_BACKEND_DEVICE_TYPE_GPU) continue;
        if (starts_with_ci(ggml_backend_dev_name(dev), pref)) return ggml_backend_dev_init(dev, nullptr);
    }
    return nullptr;
}

static uint64_t g_state = 0x1234567u;
static double uniform01() {
    uint64_t z = (g_state += 0x9E3779B97F4A7C15ull);
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    z ^= z >> 31;
    return ((z >> 11) + 1.0) * (1.0 / 9007199254740992.0);
}
static std::vector<float> normal(size_t n, double sd) {
    std::vector<float> v(n);
    for (size_t i = 0; i < n; i += 2) {
        const double r = std::sqrt(-2.0 * std::log(uniform01())), t = 2.0 * M_PI * uniform01();
        v[i] = (float)(sd * r * std::cos(t));
        if (i + 1 < n) v[i + 1] = (float)(sd * r * std::sin(t));
    }
    return v;
}

static double rel_err(const std::vector<float> &got, const std::vector<float> &ref) {
    double num = 0, den = 0;
    for (size_t i = 0; i < got.size(); i++) {
        num = std::fmax(num, std::fabs((double)got[i] - ref[i]));
        den = std::fmax(den, std::fabs((double)ref[i]));
    }
    return den > 0 ? num / den : num;
}

struct Result {
    int cases = 0;
    double max_err = 0;
    bool roundtrip = true, partial = true, batched = true, supports = true, computed = true, moe = true;
    bool sched = true, failures = true;
};

// One weight of `type` [K in, N out], activations [K, M] (ne2 batches), through the graph.
static void run_case(ggml_backend_t be, ggml_type type, int64_t K, int64_t N, int64_t M, int64_t B, Result &res) {
    ggml_init_params ip = {ggml_tensor_overhead() * 8 + ggml_graph_overhead(), nullptr, true};
    ggml_context *ctx = ggml_init(ip);
    ggml_tensor *W = ggml_new_tensor_2d(ctx, type, K, N);
    ggml_tensor *X = B > 1 ? ggml_new_tensor_3d(ctx, GGML_TYPE_F32, K, M, B) : ggml_new_tensor_2d(ctx, GGML_TYPE_F32, K, M);
    ggml_set_name(W, "w");
    ggml_set_name(X, "x");
    ggml_tensor *Y = ggml_mul_mat(ctx, W, X);
    ggml_set_output(Y);
    if (!ggml_backend_supports_op(be, Y)) {
        std::fprintf(stderr, "case %s K=%lld: supports_op refused\n", ggml_type_name(type), (long long)K);
        res.supports = false;
        ggml_free(ctx);
        return;
    }
    ggml_backend_buffer_t buf = ggml_backend_alloc_ctx_tensors(ctx, be);
    if (!buf) {
        res.computed = false;
        ggml_free(ctx);
        return;
    }
    const size_t rs = or_row_size((int)type, K);
    std::vector<float> wf = normal((size_t)(N * K), 0.02);
    std::vector<uint8_t> wq(rs * N);
    or_quantize_chunk((int)type, wf.data(), wq.data(), N, K);
    ggml_backend_tensor_set(W, wq.data(), 0, wq.size());
    std::vector<float> x = normal((size_t)(K * M * B), 1.0);
    ggml_backend_tensor_set(X, x.data(), 0, x.size() * 4);
    ggml_cgraph *gf = ggml_new_graph(ctx);
    ggml_build_forward_expand(gf, Y);

    auto check = [&](const std::vector<uint8_t> &wbytes, bool &flag) {
        if (ggml_backend_graph_compute(be, gf) != GGML_STATUS_SUCCESS) {
            res.computed = false;
            return;
        }
        std::vector<float> y((size_t)(N * M * B)), yref((size_t)(N * M * B));
        ggml_backend_tensor_get(Y, y.data(), 0, y.size() * 4);
        or_mul_mat((int)type, wbytes.data(), N, K, x.data(), K, M * B, yref.data(), N, 4, OR_Q8_0_X86);
        const double e = rel_err(y, yref);
        res.max_err = std::fmax(res.max_err, e);
        res.cases++;
        if (!(e <= 1e-4)) {
            flag = false;
            std::fprintf(stderr, "case %s K=%lld N=%lld M=%lld B=%lld: rel err %.3g\n", ggml_type_name(type),
                         (long long)K, (long long)N, (long long)M, (long long)B, e);
        }
    };
    bool ok = true;
    check(wq, ok);
    if (B > 1) res.batched = res.batched && ok;
    // get_tensor returns the uploaded GGUF bytes
    std::vector<uint8_t> back(wq.size());
    ggml_backend_tensor_get(W, back.data(), 0, back.size());
    if (back != wq) res.roundtrip = false;
    // partial write of rows [5, 13): the backend rebuilds the planes of those rows only
    if (N >= 13) {
        std::vector<float> wf2 = normal((size_t)(8 * K), 0.03);
        std::vector<uint8_t> rows(rs * 8);
        or_quantize_chunk((int)type, wf2.data(), rows.data(), 8, K);
        ggml_backend_tensor_set(W, rows.data(), 5 * rs, rows.size());
        std::memcpy(wq.data() + 5 * rs, rows.data(), rows.size());
        bool pok = true;
        check(wq, pok);
        res.partial = res.partial && pok;
    }
    ggml_backend_buffer_free(buf);
    ggml_free(ctx);
}

// GGML_OP_MUL_MAT_ID (src/crispembed.cpp:1365,1371): E experts [K, N] of `type` in one 3-D
// weight, activations X [K, nb1, T] (nb1 = 1: every slot reads its token's row), routing ids
// [n_used, T] as a view of a [E, T] tensor (the shape ggml_top_k leaves: the first n_used of
// each token's sorted expert list).  Checked against the oracle row by row; also the 3-D
// weight's GGUF-byte readback and a write spanning two experts.
static void run_case_id(ggml_backend_t be, ggml_type type, int64_t K, int64_t N, int64_t E, int64_t n_used,
                        int64_t T, bool bcast, Result &res) {
    ggml_init_params ip = {ggml_tensor_overhead() * 8 + ggml_graph_overhead(), nullptr, true};
    ggml_context *ctx = ggml_init(ip);
    const int64_t nb1 = bcast ? 1 : n_used;
    ggml_tensor *W = ggml_new_tensor_3d(ctx, type, K, N, E);
    ggml_tensor *X = ggml_new_tensor_3d(ctx, GGML_TYPE_F32, K, nb1, T);
    ggml_tensor *I = ggml_new_tensor_2d(ctx, GGML_TYPE_I32, E, T);
    ggml_tensor *ids = ggml_view_2d(ctx, I, n_used, T, I->nb[1], 0);
    ggml_tensor *Y = ggml_mul_mat_id(ctx, W, X, ids);
    if (!ggml_backend_supports_op(be, Y)) {
        std::fprintf(stderr, "mul_mat_id %s: supports_op refused\n", ggml_type_name(type));
        res.supports = false;
        ggml_free(ctx);
        return;
    }
    ggml_backend_buffer_t buf = ggml_backend_alloc_ctx_tensors(ctx, be);
    if (!buf) {
        res.computed = false;
        ggml_free(ctx);
        return;
    }
    const size_t rs = or_row_size((int)type, K);
    std::vector<float> wf = normal((size_t)(E * N * K), 0.02);
    std::vector<uint8_t> wq(rs * N * E);
    or_quantize_chunk((int)type, wf.data(), wq.data(), N * E, K);
    ggml_backend_tensor_set(W, wq.data(), 0, wq.size());
    std::vector<float> x = normal((size_t)(K * nb1 * T), 1.0);
    ggml_backend_tensor_set(X, x.data(), 0, x.size() * 4);
    std::vector<int32_t> route((size_t)(E * T));
    for (int64_t t = 0; t < T; t++) {  // a permutation of the experts per token
        for (int64_t e = 0; e < E; e++) route[t * E + e] = (int32_t)e;
        for (int64_t e = E - 1; e > 0; e--) std::swap(route[t * E + e], route[t * E + (int64_t)(uniform01() * (e + 1)) % (e + 1)]);
    }
    ggml_backend_tensor_set(I, route.data(), 0, route.size() * 4);
    ggml_cgraph *gf = ggml_new_graph(ctx);
    ggml_build_forward_expand(gf, Y);
    auto check = [&](bool &flag) {
        if (ggml_backend_graph_compute(be, gf) != GGML_STATUS_SUCCESS) {
            res.computed = false;
            return;
        }
        std::vector<float> y((size_t)(N * n_used * T)), yref(y.size());
        ggml_backend_tensor_get(Y, y.data(), 0, y.size() * 4);
        for (int64_t t = 0; t < T; t++)
            for (int64_t i = 0; i < n_used; i++) {
                const int32_t e = route[t * E + i];
                or_mul_mat((int)type, wq.data() + (size_t)e * N * rs, N, K, x.data() + (t * nb1 + i % nb1) * K, K, 1,
                           yref.data() + (t * n_used + i) * N, N, 1, OR_Q8_0_X86);
            }
        const double err = rel_err(y, yref);
        res.max_err = std::fmax(res.max_err, err);
        res.cases++;
        if (!(err <= 1e-4)) {
            flag = false;
            std::fprintf(stderr, "mul_mat_id %s K=%lld N=%lld E=%lld used=%lld T=%lld: rel err %.3g\n",
                         ggml_type_name(type), (long long)K, (long long)N, (long long)E, (long long)n_used, (long long)T,
                         err);
        }
    };
    bool ok = true;
    check(ok);
    std::vector<uint8_t> back(wq.size());
    ggml_backend_tensor_get(W, back.data(), 0, back.size());
    if (back != wq) {
        res.roundtrip = false;
        ok = false;
    }
    // rows N-3 .. N+2: the last rows of expert 0 and the first of expert 1
    std::vector<float> wf2 = normal((size_t)(6 * K), 0.03);
    std::vector<uint8_t> rows(rs * 6);
    or_quantize_chunk((int)type, wf2.data(), rows.data(), 6, K);
    ggml_backend_tensor_set(W, rows.data(), (N - 3) * rs, rows.size());
    std::memcpy(wq.data() + (N - 3) * rs, rows.data(), rows.size());
    check(ok);
    res.moe = res.moe && ok;
    ggml_backend_buffer_free(buf);
    ggml_free(ctx);
}

// The MoE FFN block exactly as build_encoder_graph builds it for Nomic-v2-style encoders
// (src/crispembed.cpp:1327-1382): F32 router MUL_MAT, SOFT_MAX, top-k (ARGSORT + view),
// GET_ROWS of the selected probabilities, REPEAT of the input over the k slots, MUL_MAT_ID
// (fc1), GELU_ERF, MUL_MAT_ID (fc2), CONT(PERMUTE), the F32 weighted-sum MUL_MAT and the bias
// ADD, every node on the backend.  Reference: the same steps on the host with the oracle's
// mat-muls (activations requantized as ggml does) and fp64 softmax / GELU.
static void run_moe_block(ggml_backend_t be, ggml_type type, Result &res) {
    const int64_t H = 256, F = 512, E = 8, KT = 2, TB = 48;
    ggml_init_params ip = {ggml_tensor_overhead() * 40 + ggml_graph_overhead(), nullptr, true};
    ggml_context *ctx = ggml_init(ip);
    ggml_tensor *cur = ggml_new_tensor_2d(ctx, GGML_TYPE_F32, H, TB);
    ggml_tensor *router = ggml_new_tensor_2d(ctx, GGML_TYPE_F32, H, E);
    ggml_tensor *fc1 = ggml_new_tensor_3d(ctx, type, H, F, E);
    ggml_tensor *fc2 = ggml_new_tensor_3d(ctx, type, F, H, E);
    ggml_tensor *bias = ggml_new_tensor_1d(ctx, GGML_TYPE_F32, H);
    ggml_tensor *logits = ggml_mul_mat(ctx, router, cur);
    ggml_tensor *probs = ggml_soft_max(ctx, logits);
    ggml_tensor *ids = ggml_top_k(ctx, probs, (int)KT);
    ggml_tensor *top_w = ggml_get_rows(ctx, ggml_reshape_3d(ctx, probs, 1, E, TB), ids);
    top_w = ggml_reshape_2d(ctx, top_w, KT, TB);
    ggml_tensor *slots = ggml_repeat(ctx, ggml_reshape_3d(ctx, cur, H, 1, TB), ggml_new_tensor_3d(ctx, GGML_TYPE_F32, H, KT, TB));
    ggml_tensor *up = ggml_gelu_erf(ctx, ggml_mul_mat_id(ctx, fc1, slots, ids));
    ggml_tensor *down = ggml_mul_mat_id(ctx, fc2, up, ids);
    ggml_tensor *down_p = ggml_cont(ctx, ggml_permute(ctx, down, 1, 0, 2, 3));
    ggml_tensor *ffn = ggml_mul_mat(ctx, ggml_reshape_3d(ctx, top_w, KT, 1, TB), down_p);
    ffn = ggml_add(ctx, ggml_reshape_2d(ctx, ffn, H, TB), bias);
    ggml_set_output(ffn);
    ggml_cgraph *gf = ggml_new_graph(ctx);
    ggml_build_forward_expand(gf, ffn);
    for (int i = 0; i < ggml_graph_n_nodes(gf); i++)
        if (!ggml_backend_supports_op(be, ggml_graph_node(gf, i))) {
            std::fprintf(stderr, "moe block: %s refused\n", ggml_op_name(ggml_graph_node(gf, i)->op));
            res.supports = res.moe = false;
        }
    ggml_backend_buffer_t buf = ggml_backend_alloc_ctx_tensors(ctx, be);
    if (!buf) {
        res.computed = false;
        ggml_free(ctx);
        return;
    }
    std::vector<float> x = normal((size_t)(H * TB), 1.0), rw = normal((size_t)(H * E), 0.2), bv = normal((size_t)H, 0.1);
    const size_t rs1 = or_row_size((int)type, H), rs2 = or_row_size((int)type, F);
    std::vector<float> w1f = normal((size_t)(E * F * H), 0.05), w2f = normal((size_t)(E * H * F), 0.05);
    std::vector<uint8_t> w1(rs1 * F * E), w2(rs2 * H * E);
    or_quantize_chunk((int)type, w1f.data(), w1.data(), F * E, H);
    or_quantize_chunk((int)type, w2f.data(), w2.data(), H * E, F);
    ggml_backend_tensor_set(cur, x.data(), 0, x.size() * 4);
    ggml_backend_tensor_set(router, rw.data(), 0, rw.size() * 4);
    ggml_backend_tensor_set(fc1, w1.data(), 0, w1.size());
    ggml_backend_tensor_set(fc2, w2.data(), 0, w2.size());
    ggml_backend_tensor_set(bias, bv.data(), 0, bv.size() * 4);
    if (ggml_backend_graph_compute(be, gf) != GGML_STATUS_SUCCESS) {
        res.computed = res.moe = false;
        ggml_backend_buffer_free(buf);
        ggml_free(ctx);
        return;
    }
    std::vector<float> y((size_t)(H * TB));
    ggml_backend_tensor_get(ffn, y.data(), 0, y.size() * 4);
    std::vector<float> yref(y.size());
    for (int64_t t = 0; t < TB; t++) {
        const float *xt = x.data() + t * H;
        std::vector<double> p(E);
        double mx = -1e300, sum = 0;
        for (int64_t e = 0; e < E; e++) {
            float acc = 0.f;  // the F32 router product in fp32, k order
            for (int64_t h = 0; h < H; h++) acc += rw[e * H + h] * xt[h];
            p[e] = acc;
            mx = std::fmax(mx, p[e]);
        }
        for (auto &v : p) sum += (v = std::exp(v - mx));
        std::vector<int> ord(E);
        for (int e = 0; e < E; e++) ord[e] = e;
        std::stable_sort(ord.begin(), ord.end(), [&](int a, int b) { return p[a] > p[b]; });
        for (int64_t h = 0; h < H; h++) yref[t * H + h] = bv[h];
        std::vector<double> acc(H, 0.0);
        for (int64_t i = 0; i < KT; i++) {
            const int e = ord[i];
            std::vector<float> u(F), dn(H);
            or_mul_mat((int)type, w1.data() + (size_t)e * F * rs1, F, H, xt, H, 1, u.data(), F, 1, OR_Q8_0_X86);
            for (auto &v : u) v = (float)(0.5 * v * (1.0 + std::erf(v / std::sqrt(2.0))));
            or_mul_mat((int)type, w2.data() + (size_t)e * H * rs2, H, F, u.data(), F, 1, dn.data(), H, 1, OR_Q8_0_X86);
            for (int64_t h = 0; h < H; h++) acc[h] += (p[e] / sum) * dn[h];
        }
        for (int64_t h = 0; h < H; h++) yref[t * H + h] = (float)(acc[h] + bv[h]);
    }
    const double err = rel_err(y, yref);
    res.cases++;
    // the bar of the GELU prologue: device erff vs the host's erf may move a requantized fc2
    // input by one step near a rounding boundary
    if (!(err <= 1e-3)) {
        res.moe = false;
        std::fprintf(stderr, "moe block %s: rel err %.3g\n", ggml_type_name(type), err);
    }
    std::fprintf(stderr, "moe block %s: rel err %.3g\n", ggml_type_name(type), err);
    ggml_backend_buffer_free(buf);
    ggml_free(ctx);
}

// The library's dynamic-loading entry points, looked up the way ggml_backend_load does: dlopen
// the backend library, dlsym ggml_backend_init (registry, api_version checked) and
// ggml_backend_score (0: cannot run here).  Returns the score, -1 on a missing or wrong symbol.
static int check_dl_entry_points() {
    Dl_info info;
    if (!dladdr((void *)&ggml_backend_mi355_reg, &info) || !info.dli_fname) return -1;
    void *h = dlopen(info.dli_fname, RTLD_NOW | RTLD_LOCAL);
    if (!h) return -1;
    auto init = (ggml_backend_reg_t (*)(void))dlsym(h, "ggml_backend_init");
    auto score = (int (*)(void))dlsym(h, "ggml_backend_score");
    int s = -1;
    if (init && score) {
        ggml_backend_reg_t reg = init();
        if (reg == ggml_backend_mi355_reg() && reg->api_version == GGML_BACKEND_API_VERSION &&
            std::strcmp(ggml_backend_reg_name(reg), "MI355X") == 0)
            s = score();
        // the score says whether the registry has a device
        if (s >= 0 && (s > 0) != (ggml_backend_reg_dev_count(reg) > 0)) s = -1;
    }
    dlclose(h);
    return s;
}

// A minimal ggml_backend_sched_graph_compute: the reference's scheduler (src/crispembed.cpp:
// 700-723, 1471-1483) gives every node the first backend whose supports_op claims it, cuts the
// graph into splits of consecutive nodes on one backend, copies a split's inputs produced on
// another backend into it, and fails the call when a split's compute is not SUCCESS.  Graph:
// Y2 = W2 (tanh(W1 X)); TANH is not claimed, so the splits are MUL_MAT (GPU) | TANH (host) |
// MUL_MAT (GPU).  The host split reads its input back with tensor_get and leaves its output
// where the next GPU split reads it (tensor_set), as sched's input copy does.  Checks: three
// splits, the set_n_threads proc lookup sched makes returns NULL, Y1 against the oracle, Y2
// against the oracle's product of W2 with the host's tanh of the GPU's Y1 (each at 1e-4).
static void run_sched_split(ggml_backend_t be, ggml_type type, int64_t M, Result &res) {
    const int64_t K = 512, N1 = 256, N2 = 96;
    ggml_init_params ip = {ggml_tensor_overhead() * 8 + ggml_graph_overhead(), nullptr, true};
    ggml_context *ctx = ggml_init(ip);
    ggml_tensor *W1 = ggml_new_tensor_2d(ctx, type, K, N1);
    ggml_tensor *W2 = ggml_new_tensor_2d(ctx, type, N1, N2);
    ggml_tensor *X = ggml_new_tensor_2d(ctx, GGML_TYPE_F32, K, M);
    ggml_tensor *Y1 = ggml_mul_mat(ctx, W1, X);
    ggml_tensor *T = ggml_unary(ctx, Y1, GGML_UNARY_OP_TANH);
    ggml_tensor *Y2 = ggml_mul_mat(ctx, W2, T);
    ggml_set_output(Y2);
    ggml_cgraph *gf = ggml_new_graph(ctx);
    ggml_build_forward_expand(gf, Y2);
    ggml_backend_buffer_t buf = ggml_backend_alloc_ctx_tensors(ctx, be);
    ggml_backend_dev_t dev = ggml_backend_get_device(be);
    if (!buf || ggml_backend_reg_get_proc_address(ggml_backend_dev_backend_reg(dev), "ggml_backend_set_n_threads")) {
        res.sched = false;
        if (buf) ggml_backend_buffer_free(buf);
        ggml_free(ctx);
        return;
    }
    std::vector<float> w1f = normal((size_t)(N1 * K), 0.05), w2f = normal((size_t)(N2 * N1), 0.05);
    std::vector<uint8_t> w1(or_row_size((int)type, K) * N1), w2(or_row_size((int)type, N1) * N2);
    or_quantize_chunk((int)type, w1f.data(), w1.data(), N1, K);
    or_quantize_chunk((int)type, w2f.data(), w2.data(), N2, N1);
    std::vector<float> x = normal((size_t)(K * M), 1.0);
    ggml_backend_tensor_set(W1, w1.data(), 0, w1.size());
    ggml_backend_tensor_set(W2, w2.data(), 0, w2.size());
    ggml_backend_tensor_set(X, x.data(), 0, x.size() * 4);
    const int n = ggml_graph_n_nodes(gf);
    int splits = 0;
    std::vector<float> th;
    for (int i0 = 0; i0 < n;) {
        const bool on_gpu = ggml_backend_supports_op(be, ggml_graph_node(gf, i0));
        int i1 = i0 + 1;
        while (i1 < n && ggml_backend_supports_op(be, ggml_graph_node(gf, i1)) == on_gpu) i1++;
        splits++;
        if (on_gpu) {
            ggml_cgraph *view = ggml_compat_graph_view(gf, i0, i1);
            const ggml_status st = ggml_backend_graph_compute(be, view);
            ggml_compat_graph_view_free(view);
            if (st != GGML_STATUS_SUCCESS) {
                res.sched = false;
                break;
            }
        } else {
            for (int i = i0; i < i1; i++) {  // this driver's host backend knows TANH only
                ggml_tensor *node = ggml_graph_node(gf, i), *src = node->src[0];
                if (node->op != GGML_OP_UNARY || ggml_get_unary_op(node) != GGML_UNARY_OP_TANH) {
                    res.sched = false;
                    break;
                }
                std::vector<float> v((size_t)ggml_nelements(src));
                ggml_backend_tensor_get(src, v.data(), 0, v.size() * 4);
                for (auto &e : v) e = std::tanh(e);
                ggml_backend_tensor_set(node, v.data(), 0, v.size() * 4);
                th = v;
            }
        }
        i0 = i1;
    }
    if (res.sched && splits == 3 && th.size() == (size_t)(N1 * M)) {
        std::vector<float> y1((size_t)(N1 * M)), y1ref(y1.size()), y2((size_t)(N2 * M)), y2ref(y2.size());
        ggml_backend_tensor_get(Y1, y1.data(), 0, y1.size() * 4);
        ggml_backend_tensor_get(Y2, y2.data(), 0, y2.size() * 4);
        or_mul_mat((int)type, w1.data(), N1, K, x.data(), K, M, y1ref.data(), N1, 4, OR_Q8_0_X86);
        or_mul_mat((int)type, w2.data(), N2, N1, th.data(), N1, M, y2ref.data(), N2, 4, OR_Q8_0_X86);
        const double e1 = rel_err(y1, y1ref), e2 = rel_err(y2, y2ref);
        res.max_err = std::fmax(res.max_err, std::fmax(e1, e2));
        res.cases += 2;
        if (!(e1 <= 1e-4) || !(e2 <= 1e-4)) {
            res.sched = false;
            std::fprintf(stderr, "sched split %s M=%lld: rel err %.3g / %.3g\n", ggml_type_name(type), (long long)M,
                         e1, e2);
        }
    } else {
        res.sched = false;
        std::fprintf(stderr, "sched split %s M=%lld: %d splits\n", ggml_type_name(type), (long long)M, splits);
    }
    ggml_backend_buffer_free(buf);
    ggml_free(ctx);
}

// Failure paths a host relies on: an allocation the device cannot hold returns NULL (the
// loader then fails cleanly, src/core/gguf_loader.cpp:408-415), a graph with a node the
// backend does not compute returns a status other than SUCCESS (the caller fails the call,
// src/crispembed.cpp:1483), and neither leaves the backend unusable: the next allocation and
// graph still succeed and are checked against the oracle.
static void run_failures(ggml_backend_t be, Result &res) {
    ggml_backend_buffer_type_t buft = ggml_backend_get_default_buffer_type(be);
    if (ggml_backend_buft_alloc_buffer(buft, (size_t)1 << 52) != nullptr) res.failures = false;
    {
        ggml_init_params ip = {ggml_tensor_overhead() * 4, nullptr, true};
        ggml_context *ctx = ggml_init(ip);
        ggml_new_tensor_2d(ctx, GGML_TYPE_F32, (int64_t)1 << 24, (int64_t)1 << 24);  // 1 PiB
        if (ggml_backend_alloc_ctx_tensors(ctx, be) != nullptr) res.failures = false;
        ggml_free(ctx);
    }
    {
        ggml_init_params ip = {ggml_tensor_overhead() * 4 + ggml_graph_overhead(), nullptr, true};
        ggml_context *ctx = ggml_init(ip);
        ggml_tensor *x = ggml_new_tensor_2d(ctx, GGML_TYPE_F32, 64, 4);
        ggml_tensor *t = ggml_unary(ctx, x, GGML_UNARY_OP_TANH);
        ggml_cgraph *gf = ggml_new_graph(ctx);
        ggml_build_forward_expand(gf, t);
        ggml_backend_buffer_t buf = ggml_backend_alloc_ctx_tensors(ctx, be);
        if (!buf) res.failures = false;
        else {
            std::vector<float> v(256, 0.5f);
            ggml_backend_tensor_set(x, v.data(), 0, v.size() * 4);
            if (ggml_backend_graph_compute(be, gf) == GGML_STATUS_SUCCESS) res.failures = false;
            ggml_backend_buffer_free(buf);
        }
        ggml_free(ctx);
    }
    Result after;
    run_case(be, GGML_TYPE_Q8_0, 384, 40, 77, 1, after);
    run_case(be, GGML_TYPE_Q4_K, 512, 40, 4, 1, after);
    if (!(after.computed && after.cases >= 2 && after.max_err <= 1e-4)) res.failures = false;
    res.cases += after.cases;
    res.max_err = std::fmax(res.max_err, after.max_err);
}

int main(int argc, char **argv) {
    const char *requested = "MI355X";
    bool json = false;
    for (int i = 1; i < argc; ++i) {
        if (std::strcmp(argv[i], "--json") == 0) json = true;
        else requested = argv[i];
    }
    const int dl_score = check_dl_entry_points();
    ggml_backend_register(ggml_backend_mi355_reg());  // the one-line host hook
    ggml_backend_t be = init_by_name(requested);
    if (!be) {
        std::fprintf(stderr, "test-backend-mi355: no GPU device matching '%s' (%zu devices registered)\n", requested,
                     ggml_backend_dev_count());
        if (json)
            std::printf("{\"requested\":\"%s\",\"device_available\":false,\"dl_score\":%d,\"correct\":false}\n",
                        requested, dl_score);
        return 1;
    }
    ggml_backend_dev_t dev = ggml_backend_get_device(be);
    Result res;
    const ggml_type types[] = {GGML_TYPE_Q8_0, GGML_TYPE_Q4_K, GGML_TYPE_Q6_K, GGML_TYPE_F16};
    for (ggml_type t : types) {
        const int64_t K = (t == GGML_TYPE_Q8_0) ? 384 : 512;
        for (int64_t M : {1, 4, 8, 77, 300}) run_case(be, t, K, 96, M, 1, res);
        run_case(be, t, K, 40, 7, 3, res);  // batched activations [K, 7, 3]
    }
    // mixture of experts: 8 experts, top-2, both activation layouts, GEMV- and GEMM-sized groups
    run_case_id(be, GGML_TYPE_Q8_0, 256, 96, 8, 2, 40, true, res);
    run_case_id(be, GGML_TYPE_Q4_K, 512, 64, 8, 2, 300, false, res);
    run_case_id(be, GGML_TYPE_Q6_K, 256, 40, 4, 3, 7, true, res);
    run_case_id(be, GGML_TYPE_F16, 128, 72, 6, 2, 90, false, res);
    run_moe_block(be, GGML_TYPE_Q8_0, res);
    run_moe_block(be, GGML_TYPE_Q4_K, res);
    // CPU-fallback splits (GEMM- and GEMV-sized) and the failure paths
    run_sched_split(be, GGML_TYPE_Q4_K, 40, res);
    run_sched_split(be, GGML_TYPE_Q4_K, 3, res);
    run_sched_split(be, GGML_TYPE_Q8_0, 40, res);
    run_failures(be, res);
    // supports_op must refuse what the kernels do not handle (CPU fallback)
    {
        ggml_init_params ip = {ggml_tensor_overhead() * 16 + ggml_graph_overhead(), nullptr, true};
        ggml_context *ctx = ggml_init(ip);
        ggml_tensor *wf32 = ggml_new_tensor_2d(ctx, GGML_TYPE_F32, 64, 8);
        ggml_tensor *wf16 = ggml_new_tensor_2d(ctx, GGML_TYPE_F16, 48, 8);  // k % 32 != 0
        ggml_tensor *wq = ggml_new_tensor_2d(ctx, GGML_TYPE_Q4_K, 256, 8);
        ggml_tensor *x64 = ggml_new_tensor_2d(ctx, GGML_TYPE_F32, 64, 3);
        ggml_tensor *x48 = ggml_new_tensor_2d(ctx, GGML_TYPE_F32, 48, 3);
        ggml_tensor *xh = ggml_new_tensor_2d(ctx, GGML_TYPE_F16, 256, 3);
        // F32 weights: the small products are claimed, large ones stay on the CPU
        if (!ggml_backend_supports_op(be, ggml_mul_mat(ctx, wf32, x64))) res.supports = false;
        ggml_tensor *wbig = ggml_new_tensor_2d(ctx, GGML_TYPE_F32, 4096, 4096);
        ggml_tensor *xbig = ggml_new_tensor_2d(ctx, GGML_TYPE_F32, 4096, 8);
        if (ggml_backend_supports_op(be, ggml_mul_mat(ctx, wbig, xbig))) res.supports = false;
        if (ggml_backend_supports_op(be, ggml_mul_mat(ctx, wf16, x48))) res.supports = false;
        if (ggml_backend_supports_op(be, ggml_mul_mat(ctx, wq, xh))) res.supports = false;
        // the encoder's elementwise ops are claimed for F32, refused for F16 operands or
        // shapes that do not broadcast
        if (!ggml_backend_supports_op(be, ggml_add(ctx, x64, x64))) res.supports = false;
        if (!ggml_backend_supports_op(be, ggml_gelu_erf(ctx, x64))) res.supports = false;
        if (ggml_backend_supports_op(be, ggml_add(ctx, xh, xh))) res.supports = false;
        if (ggml_backend_supports_op(be, ggml_add(ctx, x64, x48))) res.supports = false;
        if (ggml_backend_supports_op(be, ggml_unary(ctx, x64, GGML_UNARY_OP_TANH))) res.supports = false;
        ggml_free(ctx);
    }
    const bool correct = res.computed && res.roundtrip && res.partial && res.batched && res.supports && res.moe &&
                         res.sched && res.failures && dl_score > 0 && res.cases > 0 && res.max_err <= 1e-4;
    if (json)
        std::printf("{\"requested\":\"%s\",\"name\":\"%s\",\"description\":\"%s\",\"type\":%d,\"cases\":%d,"
                    "\"max_rel_err\":%.3g,\"roundtrip_ok\":%s,\"partial_write_ok\":%s,\"batched_ok\":%s,"
                    "\"supports_op_ok\":%s,\"moe_ok\":%s,\"sched_split_ok\":%s,\"failures_ok\":%s,\"dl_score\":%d,"
                    "\"computed\":%s,\"correct\":%s}\n",
                    requested, ggml_backend_dev_name(dev), ggml_backend_dev_description(dev),
                    (int)ggml_backend_dev_type(dev), res.cases, res.max_err, res.roundtrip ? "true" : "false",
                    res.partial ? "true" : "false", res.batched ? "true" : "false", res.supports ? "true" : "false",
                    res.moe ? "true" : "false", res.sched ? "true" : "false", res.failures ? "true" : "false", dl_score,
                    res.computed ? "true" : "false", correct ? "true" : "false");
    else
        std::printf("backend-mi355 name=%s cases=%d max_rel_err=%.3g correct=%d\n", ggml_backend_dev_name(dev),
                    res.cases, res.max_err, correct ? 1 : 0);
    ggml_backend_free(be);
    return correct ? 0 : 2;
}
