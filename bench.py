#!/usr/bin/env python3
"""Benchmark of the quantized MUL_MAT hot path on one MI355X.

Default workload (the headline): Q4_K mul_mat at the XLM-R-large / BGE-M3 FFN
shape -- up W[4096 x 1024] on X[8192 x 1024] (16 seq x 512 tokens) and down
W[1024 x 4096] on GELU(X)[8192 x 4096].  One step = both mul_mats, each with its
Q8_K activation quantization, inputs already resident in HBM.

value = whole-step int8 TOPS (2*M*N*K per mul_mat / step time).
roofline = the dominant kernel, the up GEMM (k_gemm<Q4_K>, M 8192 N 4096 K 1024), against
its binding roofline: the larger of its MFMA floor (ops at the 5.0 POP/s int8 peak) and its
HBM floor (GGUF weight + quantized X + fp32 Y bytes at 8 TB/s); the launch time is the mean of
HIP events on the launch stream.  The down GEMM is reported beside it (second_kernel), and
both also as a fraction of the int8 MFMA peak.
cpu_baseline = the restated ggml-cpu mul_mat (AVX-512 VNNI or AVX2 integer dots, threads =
the CPUs this job may use) on a bounded sample of token rows of the same workload.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu] [--no-extras]
                      [--only q8_0|e2e|graph|qwen3|qgraph|decode]
"""
import argparse
import ctypes
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "Q8_0/Q4_K mul_mat TOPS & % roofline; MiniLM-shape embeddings/sec, 1 GPU"
PEAK_INT8_TOPS = 5000.0   # MI355X dense int8 MFMA, 5.0 POP/s
PEAK_HBM_GBS = 8000.0     # MI355X HBM3E, 8 TB/s


def log(msg):
    print(msg, file=sys.stderr, flush=True)


class Dev:
    """Device-side state for one weight matrix and its activations."""

    def __init__(self, torch, L, mq, wtype, w_gguf, n, k, x, name):
        self.wtype, self.n, self.k, self.m = wtype, n, k, x.shape[0]
        size = L.mq_weight_image_bytes(wtype, n, k)
        self.img = torch.zeros(size + 256, dtype=torch.uint8, device="cuda")
        self.wp = self.img.data_ptr() + ((-self.img.data_ptr()) % 256)
        off = self.wp - self.img.data_ptr()
        self.img[off:off + w_gguf.size] = torch.from_numpy(w_gguf.ravel()).cuda()
        s = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
        mq.check(L.mq_weight_prepare(wtype, ctypes.c_void_p(self.wp), n, k, 0, n, s))
        self.x = torch.from_numpy(x).cuda()
        self.y = torch.empty((self.m, n), dtype=torch.float32, device="cuda")
        self.wsb = L.mq_workspace_bytes(wtype, self.m, k)
        self.ws = torch.empty(self.wsb + 256, dtype=torch.uint8, device="cuda")
        self.wsp = self.ws.data_ptr() + ((-self.ws.data_ptr()) % 256)
        self.name = name


def _measured_traffic(kernel, launch):
    """HBM bytes per launch of `kernel` (the `launch` entry: "up" or "down") from the committed
    rocprofv3 byte-counter runs (profiles/traffic.json: FETCH_SIZE and WRITE_SIZE per dispatch,
    each scaled by what the counter reads for a plain copy of known size)."""
    path = os.path.join(ROOT, "profiles", "traffic.json")
    try:
        t = json.load(open(path))
    except (OSError, ValueError):
        return None
    if t.get("kernel") != kernel:
        return None
    return t.get("launches", {}).get(launch, {}).get("bytes_per_launch")


def quantize_weights(L, wtype, wf):
    import numpy as np
    n, k = wf.shape
    out = np.empty(L.mq_row_size(wtype, k) * n, dtype=np.uint8)
    got = L.mq_quantize_chunk(wtype, wf.ctypes.data_as(ctypes.c_void_p), out.ctypes.data_as(ctypes.c_void_p), n, k)
    assert got == out.size
    return out


def bench_q4k_ffn(args, torch, L, mq, synth):
    import numpy as np
    M, H, F = 8192, 1024, 4096
    t0 = time.time()
    w_up = synth.normal("xlmr_ffn/W_up", (F, H), std=0.02)
    w_dn = synth.normal("xlmr_ffn/W_down", (H, F), std=0.02)
    x_up = synth.normal("xlmr_ffn/X_up", (M, H))
    x_dn = synth.gelu_erf(synth.normal("xlmr_ffn/X_down_pre", (M, F)))
    q_up = quantize_weights(L, mq.TYPE_Q4_K, w_up)
    q_dn = quantize_weights(L, mq.TYPE_Q4_K, w_dn)
    up = Dev(torch, L, mq, mq.TYPE_Q4_K, q_up, F, H, x_up, "up")
    dn = Dev(torch, L, mq, mq.TYPE_Q4_K, q_dn, H, F, x_dn, "down")
    torch.cuda.synchronize()
    log(f"[bench] inputs ready in {time.time() - t0:.1f}s")
    stream = torch.cuda.current_stream()
    s = ctypes.c_void_p(stream.cuda_stream)
    ops_up = 2.0 * M * F * H
    ops_dn = 2.0 * M * H * F

    def step(evs=None):
        for i, d in enumerate((up, dn)):
            mq.check(L.mq_quantize_act(d.wtype, ctypes.c_void_p(d.x.data_ptr()), d.k, d.m, d.k,
                                       ctypes.c_void_p(d.wsp), d.wsb, mq.PATH_GEMM, s))
            if evs is not None:
                evs[2 * i].record(stream)
            mq.check(L.mq_mul_mat_q(d.wtype, ctypes.c_void_p(d.wp), d.n, d.k, ctypes.c_void_p(d.wsp), d.m,
                                    ctypes.c_void_p(d.y.data_ptr()), d.n, mq.PATH_GEMM, s))
            if evs is not None:
                evs[2 * i + 1].record(stream)

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    # whole-step timing: no events between launches
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for _ in range(args.steps):
        step()
    e1.record(stream)
    torch.cuda.synchronize()
    ms_step = e0.elapsed_time(e1) / args.steps
    # per-GEMM timing on the same stream (events bracket only the GEMM launches)
    evs = [[torch.cuda.Event(enable_timing=True) for _ in range(4)] for _ in range(args.steps)]
    for i in range(args.steps):
        step(evs[i])
    torch.cuda.synchronize()
    t_up = sum(e[0].elapsed_time(e[1]) for e in evs) / args.steps
    t_dn = sum(e[2].elapsed_time(e[3]) for e in evs) / args.steps
    med = lambda v: sorted(v)[len(v) // 2]
    t_up_med = med([e[0].elapsed_time(e[1]) for e in evs])
    t_dn_med = med([e[2].elapsed_time(e[3]) for e in evs])

    def gemm_roofline(name, n, k, ops, t_ms, w_bytes):
        """One GEMM launch against its binding roofline: the larger of its MFMA time (int8 ops at
        5.0 POP/s) and its HBM time (algorithmic bytes: GGUF weight + quantized X + fp32 Y)."""
        xq_bytes = M * k + M * (k // 256) * 4  # Q8_K quants + scales
        nbytes = w_bytes + xq_bytes + M * n * 4
        t_mfma = ops / (PEAK_INT8_TOPS * 1e12)
        t_hbm = nbytes / (PEAK_HBM_GBS * 1e9)
        tops = ops / (t_ms * 1e-3) / 1e12
        gbs = nbytes / (t_ms * 1e-3) / 1e9
        hbm = t_hbm >= t_mfma
        return {
            "kernel": f"k_gemm<Q4_K> {name} (MFMA int8, 2 limbs), M {M} N {n} K {k}",
            "bound": "hbm" if hbm else "mfma",
            "achieved": gbs if hbm else tops,
            "peak": PEAK_HBM_GBS if hbm else PEAK_INT8_TOPS,
            "unit": "GB/s" if hbm else "TFLOP/s",
            "frac": (gbs / PEAK_HBM_GBS) if hbm else (tops / PEAK_INT8_TOPS),
            "us_per_launch": t_ms * 1e3,
            "algorithmic_ops_per_launch": ops,
            "algorithmic_bytes_per_launch": nbytes,
            "int8_tops": tops,
            "int8_mfma_frac": tops / PEAK_INT8_TOPS,
            "floor_us": {"mfma": t_mfma * 1e6, "hbm": t_hbm * 1e6},
        }

    up_rf = gemm_roofline("up", F, H, ops_up, t_up, q_up.size)
    dn_rf = gemm_roofline("down", H, F, ops_dn, t_dn, q_dn.size)
    up_rf["traffic"] = _measured_traffic("k_gemm<Q4_K>", "up")
    dn_rf["traffic"] = _measured_traffic("k_gemm<Q4_K>", "down")
    up_rf["us_per_launch_median"] = t_up_med * 1e3
    dn_rf["us_per_launch_median"] = t_dn_med * 1e3
    # the chip's sustained int8 MFMA rate, measured on it (the datasheet's 5.0 POP/s assumes a
    # clock the chip does not hold under MFMA load)
    peak = ctypes.c_double(0.0)
    mq.check(L.mq_measure_mfma_i8(4000, ctypes.byref(peak), s))
    for rf in (up_rf, dn_rf):
        rf["int8_mfma_frac_of_measured_peak"] = rf["int8_tops"] / peak.value
    measured_peak = {"int8_mfma_tops": peak.value,
                     "method": "mq_measure_mfma_i8: one wave per SIMD on every CU, 8 independent "
                               "v_mfma_i32_32x32x32_i8 chains each, no memory traffic, HIP events"}
    # the dominant kernel of the step is the up GEMM (the longer of the two launches)
    dom, other = (up_rf, dn_rf) if t_up >= t_dn else (dn_rf, up_rf)
    roof = dict(dom)
    roof.update({
        "peak_source": "MI355X datasheet: HBM3E 8 TB/s; dense int8 MFMA 5.0 POP/s (ops = 2*M*N*K)",
        "traffic_unit": "HBM bytes per launch of this kernel, rocprofv3 FETCH_SIZE + WRITE_SIZE (copy-calibrated)",
        "peak_measured": measured_peak,
        "second_kernel": other,
    })
    res = {
        "ms_per_step": ms_step,
        "value": (ops_up + ops_dn) / (ms_step * 1e-3) / 1e12,
        "gemm_up_us": t_up * 1e3,
        "gemm_down_us": t_dn * 1e3,
        "roofline": roof,
        "x": (x_up, x_dn, q_up, q_dn),
    }
    return res


def _upload_image(torch, L, mq, wtype, gguf, n, k):
    """Weight image in device memory (256-byte aligned) with its planes built."""
    size = L.mq_weight_image_bytes(wtype, n, k)
    buf = torch.zeros(size + 256, dtype=torch.uint8, device="cuda")
    wp = buf.data_ptr() + ((-buf.data_ptr()) % 256)
    off = wp - buf.data_ptr()
    buf[off:off + gguf.size] = torch.from_numpy(gguf.ravel()).cuda()
    s = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    mq.check(L.mq_weight_prepare(wtype, ctypes.c_void_p(wp), n, k, 0, n, s))
    return buf, wp


def _timed(torch, fn, reps):
    stream = torch.cuda.current_stream()
    fn()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for _ in range(reps):
        fn()
    e1.record(stream)
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / reps * 1e3  # us


def bench_q8_0_minilm(torch, L, mq, synth):
    """Q8_0 mul_mat at the MiniLM-L6 FFN-up shape: W[1536 x 384] x X[4096 x 384] (32 seq x 128)."""
    N, K, M = 1536, 384, 4096
    q = quantize_weights(L, mq.TYPE_Q8_0, synth.normal("minilm_ffn/W_up", (N, K), std=0.02))
    d = Dev(torch, L, mq, mq.TYPE_Q8_0, q, N, K, synth.normal("minilm_ffn/X", (M, K)), "minilm")
    s = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)

    def quant():
        mq.check(L.mq_quantize_act(d.wtype, ctypes.c_void_p(d.x.data_ptr()), K, M, K, ctypes.c_void_p(d.wsp), d.wsb,
                                   mq.PATH_GEMM, s))

    def gemm():
        mq.check(L.mq_mul_mat_q(d.wtype, ctypes.c_void_p(d.wp), N, K, ctypes.c_void_p(d.wsp), M,
                                ctypes.c_void_p(d.y.data_ptr()), N, mq.PATH_GEMM, s))

    quant()
    t_gemm = _timed(torch, gemm, 200)
    t_all = _timed(torch, lambda: (quant(), gemm()), 200)
    ops = 2.0 * M * N * K
    gemm_bytes = q.size + M * K + M * (K // 32) * 4 + M * N * 4  # W + X quants + X scales + Y
    return {
        "workload": "Q8_0 mul_mat, MiniLM-L6 FFN-up shape W[1536x384] x X[4096x384]",
        "mul_mat_us": round(t_all, 2), "gemm_us": round(t_gemm, 2),
        "tops": round(ops / (t_all * 1e-6) / 1e12, 1),
        "gemm_tops": round(ops / (t_gemm * 1e-6) / 1e12, 1),
        "gemm_hbm_gbs": round(gemm_bytes / (t_gemm * 1e-6) / 1e9, 1),
        "gemm_hbm_frac": round(gemm_bytes / (t_gemm * 1e-6) / 1e9 / PEAK_HBM_GBS, 3),
        "gemm_bytes": gemm_bytes,
    }


def bench_decode(torch, L, mq, synth):
    """M <= 8 GEMV at Qwen3-VL-2B text-decoder shapes: the Q6_K lm_head [151936 x 2048]
    and a sweep over 28 layers x 7 Q4_K matrices (792.7 MB of weights, beyond the 256 MB
    last-level cache), activation quantization included (shared by q/k/v and gate/up)."""
    import numpy as np
    s = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    out = {}
    # ---- lm_head: 4096 quantized rows tiled to 151936 (bandwidth does not depend on values) ----
    NV, H = 151936, 2048
    blk = quantize_weights(L, mq.TYPE_Q6_K, synth.normal("qwen3vl/lm_head_rows", (4096, H), std=0.02))
    rs = L.mq_row_size(mq.TYPE_Q6_K, H)
    g = np.tile(blk.reshape(4096, rs), (NV // 4096 + 1, 1))[:NV].copy()
    heads = [_upload_image(torch, L, mq, mq.TYPE_Q6_K, g, NV, H) for _ in range(2)]  # alternate: > cache
    del g
    for m in (1, 8):
        x = torch.from_numpy(synth.normal(f"qwen3vl/x_head_m{m}", (m, H))).cuda()
        y = torch.empty((m, NV), dtype=torch.float32, device="cuda")
        wsb = L.mq_workspace_bytes(mq.TYPE_Q6_K, m, H)
        ws = torch.empty(wsb + 256, dtype=torch.uint8, device="cuda")
        wsp = ws.data_ptr() + ((-ws.data_ptr()) % 256)
        mq.check(L.mq_quantize_act(mq.TYPE_Q6_K, ctypes.c_void_p(x.data_ptr()), H, m, H, ctypes.c_void_p(wsp), wsb,
                                   mq.PATH_GEMV, s))
        it = [0]

        def head():
            wp = heads[it[0] & 1][1]
            it[0] += 1
            mq.check(L.mq_mul_mat_q(mq.TYPE_Q6_K, ctypes.c_void_p(wp), NV, H, ctypes.c_void_p(wsp), m,
                                    ctypes.c_void_p(y.data_ptr()), NV, mq.PATH_GEMV, s))
        us = _timed(torch, head, 40)
        nbytes = blk.size // 4096 * NV + m * H + m * NV * 4
        out[f"lm_head_q6_K_m{m}"] = {"us": round(us, 2), "gbs": round(nbytes / (us * 1e-6) / 1e9, 1),
                                     "hbm_frac": round(nbytes / (us * 1e-6) / 1e9 / PEAK_HBM_GBS, 3)}
    del heads
    # ---- layer sweep ----
    H, F, KV = 2048, 6144, 1024
    mats = [("q", H, H), ("k", KV, H), ("v", KV, H), ("o", H, H), ("gate", F, H), ("up", F, H), ("down", H, F)]
    gguf = {nm: quantize_weights(L, mq.TYPE_Q4_K, synth.normal(f"qwen3vl/layer/{nm}", (n, k), std=0.02))
            for nm, n, k in mats}
    layers = [{nm: _upload_image(torch, L, mq, mq.TYPE_Q4_K, gguf[nm], n, k) for nm, n, k in mats} for _ in range(28)]
    wbytes = sum(gguf[nm].size for nm, _, _ in mats) * 28
    for m in (1, 8):
        xs = {kd: torch.from_numpy(synth.normal(f"qwen3vl/x_{kd}_m{m}", (m, kd))).cuda() for kd in (H, F)}
        ys = {nm: torch.empty((m, n), dtype=torch.float32, device="cuda") for nm, n, _ in mats}
        wss = {}
        for kd in (H, F):
            wsb = L.mq_workspace_bytes(mq.TYPE_Q4_K, m, kd)
            t = torch.empty(wsb + 256, dtype=torch.uint8, device="cuda")
            wss[kd] = (t, t.data_ptr() + ((-t.data_ptr()) % 256), wsb)

        def quant(kd):
            _, p, b = wss[kd]
            mq.check(L.mq_quantize_act(mq.TYPE_Q4_K, ctypes.c_void_p(xs[kd].data_ptr()), kd, m, kd, ctypes.c_void_p(p),
                                       b, mq.PATH_GEMV, s))

        VP, I64 = ctypes.c_void_p * 3, ctypes.c_int64 * 3
        dims = {nm: (n, k) for nm, n, k in mats}

        def sweep():
            # q/k/v and gate/up share their input: one quantization and one grouped GEMV each
            for lay in layers:
                for grp in (("q", "k", "v"), ("o",), ("gate", "up"), ("down",)):
                    k = dims[grp[0]][1]
                    quant(k)
                    if len(grp) == 1:
                        n = dims[grp[0]][0]
                        mq.check(L.mq_mul_mat_q(mq.TYPE_Q4_K, ctypes.c_void_p(lay[grp[0]][1]), n, k,
                                                ctypes.c_void_p(wss[k][1]), m, ctypes.c_void_p(ys[grp[0]].data_ptr()),
                                                n, mq.PATH_GEMV, s))
                        continue
                    g = len(grp)
                    mq.check(L.mq_mul_mat_q_group(
                        mq.TYPE_Q4_K, g, VP(*[lay[nm][1] for nm in grp]), I64(*[dims[nm][0] for nm in grp]), k,
                        ctypes.c_void_p(wss[k][1]), m, VP(*[ys[nm].data_ptr() for nm in grp]),
                        I64(*[dims[nm][0] for nm in grp]), None, mq.PATH_GEMV, s))
        us = _timed(torch, sweep, 5)
        out[f"layer_sweep_q4_K_m{m}_two_step"] = {"sweep_us": round(us, 1), "layer_us": round(us / 28, 2),
                                                  "weight_gbs": round(wbytes / (us * 1e-6) / 1e9, 1),
                                                  "kernels_per_layer": 8}
        # the decode step's chain with the quantization inside each GEMV (mq_mul_mat_gemv): q|k|v
        # on the layer input, o on q's output (standing in for the attention rows), gate|up on
        # the layer input, down on silu(gate) * up read from the gate|up output
        gu = torch.empty((m, 2 * F), dtype=torch.float32, device="cuda")
        q_out = ys["q"]

        st = [s]  # the launch stream (a capture stream while a HIP graph is recorded)

        def gemv(names, x, ldx, y_ptrs, ldys, x2=None, pre=0, lay=None):
            g = len(names)
            k = dims[names[0]][1]
            mq.check(L.mq_mul_mat_gemv(
                mq.TYPE_Q4_K, g, (ctypes.c_void_p * g)(*[lay[nm][1] for nm in names]),
                (ctypes.c_int64 * g)(*[dims[nm][0] for nm in names]), k, ctypes.c_void_p(x), ldx,
                ctypes.c_void_p(x2) if x2 else None, ldx, pre, m, (ctypes.c_void_p * g)(*y_ptrs),
                (ctypes.c_int64 * g)(*ldys), None, st[0]))

        def fused_sweep():
            for lay in layers:
                gemv(("q", "k", "v"), xs[H].data_ptr(), H, [ys[nm].data_ptr() for nm in ("q", "k", "v")],
                     [dims[nm][0] for nm in ("q", "k", "v")], lay=lay)
                gemv(("o",), q_out.data_ptr(), H, [ys["o"].data_ptr()], [H], lay=lay)
                gemv(("gate", "up"), xs[H].data_ptr(), H, [gu.data_ptr(), gu.data_ptr() + F * 4], [2 * F, 2 * F],
                     lay=lay)
                gemv(("down",), gu.data_ptr(), 2 * F, [ys["down"].data_ptr()], [H], x2=gu.data_ptr() + F * 4,
                     pre=mq.PRE_SILU_MUL, lay=lay)

        us_eager = _timed(torch, fused_sweep, 5)
        # the decode loop as a serving loop runs it: the 112 launches captured once into a HIP
        # graph and replayed, so the host's per-launch cost is out of the measured time
        cap = torch.cuda.Stream()
        with torch.cuda.stream(cap):
            st[0] = ctypes.c_void_p(cap.cuda_stream)
            fused_sweep()
            torch.cuda.synchronize()
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph, stream=cap):
                fused_sweep()
        st[0] = s
        us = _timed(torch, graph.replay, 5)
        out[f"layer_sweep_q4_K_m{m}"] = {"sweep_us": round(us, 1), "layer_us": round(us / 28, 2),
                                         "weight_gbs": round(wbytes / (us * 1e-6) / 1e9, 1),
                                         "hbm_frac": round(wbytes / (us * 1e-6) / 1e9 / PEAK_HBM_GBS, 3),
                                         "kernels_per_layer": 4, "launch": "HIP graph replay",
                                         "eager_layer_us": round(us_eager / 28, 2)}
        del graph
    out["workload"] = ("GEMV m in {1,8}: Qwen3-VL-2B lm_head Q6_K [151936x2048]; 28-layer sweep of Q4_K "
                       "q,k,v,o [2048|1024 x 2048], gate,up [6144x2048], down [2048x6144] (792.7 MB)")
    return out


def bench_minilm_e2e(torch, L, mq):
    """End-to-end MiniLM-L6-shaped encoder (6 layers, H 384, 12 heads, FFN 1536, vocab 30522,
    Q8_0 linears, random init), 32 sequences x 128 tokens, full attention mask, mean pool + L2:
    embeddings per second with every mul_mat on the quantized GPU path."""
    from crispembed_amd import bert, synth
    hp = dict(bert.MINILM_L6)
    B, T = 32, 128
    W = bert.synthetic_weights(hp, mq.TYPE_Q8_0, name="minilm")
    enc = bert.BertEncoder(hp, mq.TYPE_Q8_0, W)
    ids = torch.from_numpy(synth.integers(f"minilm/ids_{B}x{T}", (B * T,), 1000, 30521)).cuda()
    out = torch.empty((B, hp["n_embd"]), dtype=torch.float32, device="cuda")
    s = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    run = lambda: enc.encode(ids.data_ptr(), B, T, out.data_ptr(), s)  # noqa: E731
    for _ in range(3):
        run()
    us = _timed(torch, run, 20)
    H, F, nl, M = hp["n_embd"], hp["n_ff"], hp["n_layer"], B * T
    lin_ops = 2.0 * M * nl * (4 * H * H + 2 * H * F)
    return {"workload": "MiniLM-L6 shape, Q8_0 linears, 32 seq x 128 tokens, mean pool + L2",
            "batch_ms": round(us / 1e3, 3), "embeddings_per_s": round(B / (us * 1e-6), 1),
            "linear_tops": round(lin_ops / (us * 1e-6) / 1e12, 1)}


def bench_minilm_ggml_graph(torch, L, mq):
    """The same MiniLM-L6 workload through the ggml backend: CrispEmbed's encoder graph
    (build_encoder_graph's post-LN path, 182 nodes) built with ggml's graph API from a GGUF file
    and computed by ggml_backend_graph_compute on MI355X, as a CrispEmbed build using the
    backend runs it (tests/native/test_bert_graph_mi355.cpp, built by build_test_driver).
    Time per graph from the host's clock around ggml_backend_graph_compute (which
    synchronizes), inputs already uploaded."""
    import subprocess
    import tempfile

    import numpy as np
    from crispembed_amd import bert, gguf, synth
    exe = os.path.join(ROOT, "crispembed_amd", "bin", "test-bert-graph-mi355")
    if not os.path.exists(exe):
        return {"error": f"{exe} not built"}
    hp = dict(bert.MINILM_L6)
    B, T = 32, 128
    with tempfile.TemporaryDirectory() as d:
        W = bert.synthetic_weights(hp, mq.TYPE_Q8_0, name="minilm")
        gguf.write_bert_gguf(os.path.join(d, "m.gguf"), hp, mq.TYPE_Q8_0, W)
        synth.integers(f"minilm/ids_{B}x{T}", (B * T,), 1000, 30521).astype(np.int32).tofile(os.path.join(d, "ids"))
        np.zeros(B * T, np.int32).tofile(os.path.join(d, "types"))
        np.full(B, T, np.int32).tofile(os.path.join(d, "lens"))
        results = []
        for extra in ((), ("--packed",), ("--packed", "--pack-maxtok", str(B * T))):
            r = subprocess.run([exe, os.path.join(d, "m.gguf"), str(B), str(T), os.path.join(d, "ids"),
                                os.path.join(d, "types"), os.path.join(d, "lens"), os.path.join(d, "out"), "--iters",
                                "30", *extra], capture_output=True, text=True, timeout=300)
            try:
                res = json.loads(r.stdout.strip().splitlines()[-1])
            except (ValueError, IndexError):
                return {"error": (r.stderr or r.stdout)[-300:]}
            if not res.get("ok"):
                return {"error": res.get("error")}
            results.append(res)
    res, pk, pk1 = results
    ms = res["ms_per_graph"]
    return {"workload": "MiniLM-L6 shape, Q8_0, 32 seq x 128 tokens, CrispEmbed's ggml encoder graph on the "
                        "MI355X ggml backend (every node on the GPU): one 4-D batch graph (encode_tokens_group_4d's "
                        "shape, equal lengths: no mask), and the packed path the reference takes by default on a "
                        "GPU (encode_tokens_packed: 384-token groups with a block-diagonal mask)",
            "graph_nodes": res["nodes"], "nodes_not_on_gpu": res["unsupported"], "batch_ms": round(ms, 3),
            "embeddings_per_s": round(B / (ms * 1e-3), 1),
            "packed_groups": pk["groups"], "packed_nodes_not_on_gpu": pk["unsupported"],
            "packed_batch_ms": round(pk["ms_per_graph"], 3),
            "packed_embeddings_per_s": round(B / (pk["ms_per_graph"] * 1e-3), 1),
            "packed_one_group_ms": round(pk1["ms_per_graph"], 3),
            "packed_one_group_embeddings_per_s": round(B / (pk1["ms_per_graph"] * 1e-3), 1),
            "packed_one_group": "CRISPEMBED_ENCODER_PACK_MAXTOK=4096 (src/crispembed.cpp:2010-2022): the 32 items "
                                "as one 4096-token graph with a 4096 x 4096 block-diagonal mask"}


def bench_qwen3_ggml_graph(torch, L, mq):
    """CrispEmbed's Qwen3 decoder graphs on the MI355X ggml backend (tests/native/
    test_decoder_graph_mi355.cpp, built by build_test_driver), Qwen3-Embedding-0.6B shape, Q4_K,
    vocab 151643, from a CrispEmbed decoder GGUF: (1) decoder_encode_tokens_batch's graph for 16
    sequences x 512 tokens -- one 8192-token graph with the 8192 x 8192 F16 block-diagonal causal
    mask (src/decoder_embed.cpp:1322-1641), the drop-in path of the 16 x 512 workload -- and (2) one
    512-token sequence (decoder_encode_tokens' single-text path, 815 nodes) beside the runner
    (mq_decoder_encode) on the same model at B = 1.  Time per graph from the host's clock around
    ggml_backend_graph_compute (which synchronizes), inputs already uploaded."""
    import subprocess
    import tempfile

    import numpy as np
    from crispembed_amd import decoder, gguf, synth
    exe = os.path.join(ROOT, "crispembed_amd", "bin", "test-decoder-graph-mi355")
    if not os.path.exists(exe):
        return {"error": f"{exe} not built"}
    hp = dict(decoder.QWEN3_EMBED_0_6B)
    B, T = 16, 512
    one = decoder.synthetic_weights(dict(hp, n_layer=1, n_vocab=1), mq.TYPE_Q4_K, name="qwen3_graph")
    tok = np.random.default_rng(20260101).standard_normal((hp["n_vocab"], hp["n_embd"]), dtype=np.float32)
    tok *= 0.02
    W = {"tok": tok, "out_norm": one["out_norm"], "layers": one["layers"] * hp["n_layer"]}
    ids = synth.integers(f"qwen3/ids_{B}x{T}", (B, T), 0, hp["n_vocab"] - 1).astype(np.int32)

    def drive(d, ids_, extra, iters):
        ids_.tofile(os.path.join(d, "ids"))
        r = subprocess.run([exe, os.path.join(d, "m.gguf"), str(T), os.path.join(d, "ids"), os.path.join(d, "out"),
                            "--iters", str(iters), *extra], capture_output=True, text=True, timeout=600)
        try:
            res = json.loads(r.stdout.strip().splitlines()[-1])
        except (ValueError, IndexError):
            return {"ok": False, "error": (r.stderr or r.stdout)[-300:]}
        return res

    with tempfile.TemporaryDirectory() as d:
        gguf.write_decoder_gguf(os.path.join(d, "m.gguf"), hp, mq.TYPE_Q4_K, W)
        batched = drive(d, ids, ("--batch", str(B)), 5)
        single = drive(d, ids[0], (), 10)
    for res in (batched, single):
        if not res.get("ok"):
            return {"error": res.get("error")}
    dec = decoder.DecoderEmbedder(hp, mq.TYPE_Q4_K, W)
    del W, tok
    ids_d = torch.from_numpy(ids[0].copy()).cuda()
    out = torch.empty((1, hp["n_embd"]), dtype=torch.float32, device="cuda")
    stream = torch.cuda.current_stream()
    runner_ms = _timed(torch, lambda: dec.encode(ids_d.data_ptr(), 1, T, out.data_ptr(), stream.cuda_stream), 10) / 1e3
    del dec
    ms = batched["ms_per_graph"]
    return {"workload": "Qwen3-Embedding-0.6B shape, Q4_K, vocab 151643, CrispEmbed's decoder graphs on the "
                        "MI355X ggml backend: 16 seq x 512 tokens as decoder_encode_tokens_batch's one 8192-token "
                        "graph with its 8192 x 8192 F16 mask, and one 512-token sequence",
            "departures": "one random layer's Q4_K bytes in all 28 layers (28 separate device copies: the same "
                          "bytes move as with 28 distinct layers)",
            "batched_graph_nodes": batched["nodes"], "batched_nodes_not_on_gpu": batched["unsupported"],
            "batched_T_total": batched["T_total"], "batched_ms": round(ms, 3),
            "batched_embeddings_per_s": round(B / (ms * 1e-3), 1),
            "graph_nodes": single["nodes"], "nodes_not_on_gpu": single["unsupported"],
            "graph_ms": round(single["ms_per_graph"], 3), "runner_ms": round(runner_ms, 3)}


def bench_qwen3_e2e(torch, L, mq):
    """End-to-end Qwen3-Embedding-0.6B-shaped decoder embedder (28 layers, H 1024, 16 query /
    8 key-value heads of 128, SwiGLU FFN 3072, RMSNorm eps 1e-6, NEOX RoPE theta 1e6, causal,
    vocab 151643, Q4_K linears, random init), 16 sequences x 512 tokens, last-token pooling + L2.
    One random layer's Q4_K weights are uploaded into all 28 layers (separate device copies)."""
    import numpy as np
    from crispembed_amd import decoder, synth
    hp = dict(decoder.QWEN3_EMBED_0_6B)
    B, T = 16, 512
    one = decoder.synthetic_weights(dict(hp, n_layer=1, n_vocab=1), mq.TYPE_Q4_K, name="qwen3")
    tok = np.random.default_rng(20260101).standard_normal((hp["n_vocab"], hp["n_embd"]), dtype=np.float32)
    tok *= 0.02
    W = {"tok": tok, "out_norm": one["out_norm"], "layers": one["layers"] * hp["n_layer"]}
    dec = decoder.DecoderEmbedder(hp, mq.TYPE_Q4_K, W)
    del tok, W
    ids = torch.from_numpy(synth.integers(f"qwen3/ids_{B}x{T}", (B * T,), 0, hp["n_vocab"] - 1)).cuda()
    out = torch.empty((B, hp["n_embd"]), dtype=torch.float32, device="cuda")
    s = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    run = lambda: dec.encode(ids.data_ptr(), B, T, out.data_ptr(), s)  # noqa: E731
    run()
    us = _timed(torch, run, 5)
    H, F, nl, M = hp["n_embd"], hp["n_ff"], hp["n_layer"], B * T
    qd, kvd = hp["n_head"] * hp["head_dim"], hp["n_kv_head"] * hp["head_dim"]
    lin_ops = 2.0 * M * nl * (H * (qd + 2 * kvd) + qd * H + 3 * H * F)
    return {"workload": "Qwen3-Embedding-0.6B shape, Q4_K linears, 16 seq x 512 tokens, causal, last-token pool + L2",
            "batch_ms": round(us / 1e3, 3), "embeddings_per_s": round(B / (us * 1e-6), 1),
            "linear_tops": round(lin_ops / (us * 1e-6) / 1e12, 1)}


def cpu_baseline_q4k(args, x_up, x_dn, q_up, q_dn):
    """CPU baseline: the restated ggml-cpu mul_mat (Q8_K activation quantization, AVX2 integer
    block dots, fp32 scale accumulation, output tiles over threads) on a bounded sample of the
    workload's token rows, on the host cores."""
    sys.path.insert(0, os.path.join(ROOT, "tests"))
    import oracle_ffi as O
    orc = O.Oracle()
    nthreads, threads_src = cpu_threads()
    fast = orc.fast_supported(O.Q4_K)
    mm = (lambda w, x: orc.fast_mul_mat(O.Q4_K, w, x, nthreads=nthreads)) if fast else \
         (lambda w, x: orc.mul_mat(O.Q4_K, w, x, nthreads=nthreads))
    H, F = 1024, 4096
    # calibrate on 64 rows, then size the sample for about args.cpu_seconds
    t = time.perf_counter()
    mm(q_up, x_up[:64])
    mm(q_dn, x_dn[:64])
    per_row = (time.perf_counter() - t) / 64
    rows = int(max(64, min(x_up.shape[0], args.cpu_seconds / max(per_row, 1e-9))))
    mm(q_up, x_up[:rows])  # one full-size warm-up
    mm(q_dn, x_dn[:rows])
    reps, dt, times = 0, 0.0, []
    while reps < 10 and (reps < 3 or dt < 0.5 * args.cpu_seconds):
        t = time.perf_counter()
        mm(q_up, x_up[:rows])
        mm(q_dn, x_dn[:rows])
        times.append(time.perf_counter() - t)
        dt += times[-1]
        reps += 1
    ops_rep = 2.0 * rows * (F * H + H * F)
    ops = ops_rep * reps
    t_med = sorted(times)[len(times) // 2]
    isa = orc.fast_isa() if fast else "none"
    impl = {"avx512vnni": "AVX-512 VNNI integer dots", "avx2": "AVX2 integer dots"}.get(isa, "scalar C")
    model = cpu_model()
    return {
        "value": ops_rep / t_med / 1e12,
        "unit": "TOPS",
        "mean_value": ops / dt / 1e12,
        "cores": nthreads,
        "kind": "port",
        "cpu_model": model,
        "isa": isa,
        "host_cpus": len(os.sched_getaffinity(0)),
        "threads_from": threads_src,
        "sample": f"Q4_K up+down mul_mat incl. Q8_K activation quantization on the first {rows} of 8192 "
                  f"token rows, median of {reps} rep(s) after a warm-up ({dt:.1f} s); restated ggml-cpu "
                  f"algorithm ({impl}), "
                  f"{nthreads} threads ({threads_src}) on {model}",
    }


def cpu_threads():
    """Threads for the CPU baseline: the CPUs this process may run on (what nproc reports), or
    fewer when OMP_NUM_THREADS grants the job a smaller share of the host (BENCH_CPU_THREADS
    overrides).  Returns (threads, how they were chosen)."""
    if os.environ.get("BENCH_CPU_THREADS"):
        return int(os.environ["BENCH_CPU_THREADS"]), "BENCH_CPU_THREADS"
    n = len(os.sched_getaffinity(0))
    omp = os.environ.get("OMP_NUM_THREADS", "")
    if omp.isdigit() and 0 < int(omp) < n:
        return int(omp), f"the job's CPU share OMP_NUM_THREADS={omp} of nproc={n}"
    return n, f"nproc={n}"


def cpu_model():
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown CPU"


def main():
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--no-extras", action="store_true", help="skip the Q8_0 and GEMV side measurements")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--gemm-cfg", default=None, help="MQ_GEMM_CFG tile configuration (1 or 3)")
    ap.add_argument("--only", choices=["q8_0", "e2e", "graph", "qwen3", "qgraph", "decode"], default=None,
                    help="run one side measurement alone (for per-workload profiles) and print its JSON")
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="only run 10 device copies of 256 MiB (reference kernel for rocprof byte counters)")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU only: this build has no multi-GPU path (run with --gpus 1)",
              file=sys.stderr)
        sys.exit(2)

    if args.gemm_cfg:
        os.environ["MQ_GEMM_CFG"] = args.gemm_cfg
    import torch
    if args.calibrate_copy:
        src = torch.empty(64 << 20, dtype=torch.float32, device="cuda").fill_(1.0)
        dst = torch.empty_like(src)
        for _ in range(10):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_bytes_read": src.numel() * 4, "copy_bytes_written": dst.numel() * 4}))
        return
    from crispembed_amd import mq, synth
    L = mq.lib()
    mq.check(L.mq_init())
    if args.only:
        fn = {"q8_0": lambda: bench_q8_0_minilm(torch, L, mq, synth),
              "e2e": lambda: bench_minilm_e2e(torch, L, mq),
              "graph": lambda: bench_minilm_ggml_graph(torch, L, mq),
              "qwen3": lambda: bench_qwen3_e2e(torch, L, mq),
              "qgraph": lambda: bench_qwen3_ggml_graph(torch, L, mq),
              "decode": lambda: bench_decode(torch, L, mq, synth)}[args.only]
        print(json.dumps({"only": args.only, "result": fn()}), flush=True)
        return

    r = bench_q4k_ffn(args, torch, L, mq, synth)
    x_up, x_dn, q_up, q_dn = r.pop("x")
    extras = None
    if not args.no_extras:
        extras = {"q8_0_minilm_ffn_up": bench_q8_0_minilm(torch, L, mq, synth),
                  "minilm_l6_e2e": bench_minilm_e2e(torch, L, mq),
                  "minilm_l6_ggml_graph": bench_minilm_ggml_graph(torch, L, mq),
                  "qwen3_0_6b_e2e": bench_qwen3_e2e(torch, L, mq),
                  "qwen3_0_6b_ggml_graph": bench_qwen3_ggml_graph(torch, L, mq),
                  "decode_gemv": bench_decode(torch, L, mq, synth)}
    cpu = None
    if not args.no_cpu:
        cpu = cpu_baseline_q4k(args, x_up, x_dn, q_up, q_dn)
    out = {
        "metric": METRIC,
        "value": r["value"],
        "unit": "TOPS",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": r["ms_per_step"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8",
        "data": "synthetic",
        "config": {
            "workload": "Q4_K mul_mat, XLM-R-large/BGE-M3 FFN shape: up W[4096x1024] x X[8192x1024] + down "
                        "W[1024x4096] x GELU(X)[8192x4096], each with Q8_K activation quantization",
            "tokens": 8192,
            "weights": "fp32 N(0,0.02) -> Q4_K (ggml _ref quantizer)",
            "gemm_up_us": round(r["gemm_up_us"], 2),
            "gemm_down_us": round(r["gemm_down_us"], 2),
        },
        "roofline": r["roofline"],
        "cpu_baseline": cpu,
        "extras": extras,
    }
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
