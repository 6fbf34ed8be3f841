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
    # the same two products chained as the encoder FFN runs them: the up GEMM applies GELU-erf and
    # stores its output as the down GEMM's Q8_K activation (mq_mul_mat_q_requant), so the fp32
    # intermediate and its quantizer pass disappear
    chain = {}
    if L.mq_mul_mat_q_requant_supported(mq.TYPE_Q4_K, mq.TYPE_Q4_K, M, F):
        def step_chain(evs=None):
            mq.check(L.mq_quantize_act(up.wtype, ctypes.c_void_p(up.x.data_ptr()), H, M, H,
                                       ctypes.c_void_p(up.wsp), up.wsb, mq.PATH_GEMM, s))
            if evs is not None:
                evs[0].record(stream)
            mq.check(L.mq_mul_mat_q_requant(mq.TYPE_Q4_K, ctypes.c_void_p(up.wp), F, H, ctypes.c_void_p(up.wsp), M,
                                            None, mq.PRE_GELU_ERF, mq.TYPE_Q4_K, ctypes.c_void_p(dn.wsp), dn.wsb, s))
            if evs is not None:
                evs[1].record(stream)
            mq.check(L.mq_mul_mat_q(dn.wtype, ctypes.c_void_p(dn.wp), H, F, ctypes.c_void_p(dn.wsp), M,
                                    ctypes.c_void_p(dn.y.data_ptr()), H, mq.PATH_GEMM, s))
            if evs is not None:
                evs[2].record(stream)

        for _ in range(args.warmup):
            step_chain()
        torch.cuda.synchronize()
        e0.record(stream)
        for _ in range(args.steps):
            step_chain()
        e1.record(stream)
        torch.cuda.synchronize()
        ms_chain = e0.elapsed_time(e1) / args.steps
        evc = [[torch.cuda.Event(enable_timing=True) for _ in range(3)] for _ in range(args.steps)]
        for i in range(args.steps):
            step_chain(evc[i])
        torch.cuda.synchronize()
        chain = {"ms_per_step": ms_chain,
                 "tops": (ops_up + ops_dn) / (ms_chain * 1e-3) / 1e12,
                 "gemm_up_requant_us": sum(e[0].elapsed_time(e[1]) for e in evc) / args.steps * 1e3,
                 "gemm_down_us": sum(e[1].elapsed_time(e[2]) for e in evc) / args.steps * 1e3}

    def gemm_roofline(name, n, k, ops, t_ms, w_bytes):
        """One GEMM launch against its binding roofline: the larger of its MFMA time (int8 ops at
        5.0 POP/s) and its HBM time (algorithmic bytes: GGUF weight + quantized X + fp32 Y)."""
        # the Q8_K activation as ggml's block_q8_K counts it (292 bytes per 256 values: the scale,
        # the quants and the 16 sub-block sums), which the GEMM reads as quants, scales and the
        # min-term fragments of the same sums
        xq_bytes = M * (k // 256) * 292
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
        "chain": chain,
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
    out["departures"] = ("lm_head: 4096 distinct quantized rows tiled to 151936, in two device copies walked in "
                         "turn (510 MB, past the 256 MB last-level cache); layers: one random layer's matrices "
                         "in 28 device copies; o reads q's output and gate|up the layer input (stand-ins for "
                         "the attention rows and the normed residual)")
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
            "departures": "one random layer's Q4_K bytes in all 28 layers (28 separate device copies: the same "
                          "bytes move as with 28 distinct layers)",
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


def cpu_baselines_extras(args):
    """CPU baselines of the side workloads, on the restated ggml-cpu mul_mat (oracle/cpu_fast.c:
    the activation quantization, AVX-512 VNNI or AVX2 integer block dots, fp32 scales, output
    tiles over threads) at the same thread count as the headline's, each on a stated sample:
      q8_0_minilm_ffn_up  the whole W[1536x384] x X[4096x384] product (TOPS);
      minilm_l6_e2e       the 36 linear layers of one 32 x 128 batch (6 layers of q,k,v,o [384x384],
                          fc1 [1536x384], fc2 [384x1536] on 4096 rows; the layers differ only in their
                          values, so one layer is timed and counted six times): the CPU's
                          embeddings/s can be no higher than 32 / that time (LEARNINGS.md:3397-3402:
                          the linears are the CPU encoder's time);
      qwen3_0_6b_e2e      the 196 linear layers of a 16 x 512 batch, timed on one layer over 512 of the
                          8192 rows and scaled (x 28 layers x 16): the same bound;
      decode_gemv         the Qwen3-VL-2B layer sweep (28 distinct copies of one layer's 7 Q4_K
                          matrices, 792.7 MB, more than the host's caches) at m = 1 and 8, per-layer
                          time and weight GB/s; and the Q6_K lm_head [151936x2048] (4096 quantized rows
                          tiled) at m = 1."""
    sys.path.insert(0, os.path.join(ROOT, "tests"))
    import numpy as np
    import oracle_ffi as O
    from crispembed_amd import synth
    orc = O.Oracle()
    nth, src = cpu_threads()
    isa = orc.fast_isa()
    model = cpu_model()
    impl = {"avx512vnni": "AVX-512 VNNI integer dots", "avx2": "AVX2 integer dots"}.get(isa, "scalar C")
    budget = max(1.0, args.cpu_seconds / 4)

    def mm(wt, w, x):
        return orc.fast_mul_mat(wt, w, x, nthreads=nth)

    def timed(fn):
        fn()
        times, dt = [], 0.0
        while len(times) < 10 and (len(times) < 3 or dt < budget):
            t = time.perf_counter()
            fn()
            times.append(time.perf_counter() - t)
            dt += times[-1]
        return sorted(times)[len(times) // 2], len(times)

    def base(value, unit, sample):
        return {"value": value, "unit": unit, "cores": nth, "kind": "port", "cpu_model": model, "isa": isa,
                "threads_from": src, "sample": f"{sample}; restated ggml-cpu algorithm ({impl}), {nth} threads "
                                               f"({src}) on {model}, median of the timed reps"}

    def q(wt, name, n, k):
        return orc.quantize_chunk(wt, synth.normal(name, (n, k), std=0.02))

    out = {}
    # cfg1
    w1, x1 = q(O.Q8_0, "cpu/cfg1_w", 1536, 384), synth.normal("cpu/cfg1_x", (4096, 384))
    t, reps = timed(lambda: mm(O.Q8_0, w1, x1))
    out["q8_0_minilm_ffn_up"] = base(2.0 * 4096 * 1536 * 384 / t / 1e12, "TOPS",
                                     f"the full 4096 x 1536 x 384 Q8_0 product incl. Q8_0 activation quantization, "
                                     f"{reps} reps: {t * 1e3:.2f} ms")
    # cfg3: one MiniLM layer's six products on 4096 rows
    H, F, M = 384, 1536, 4096
    lay = [q(O.Q8_0, f"cpu/cfg3_{i}", n, k) for i, (n, k) in enumerate([(H, H)] * 4 + [(F, H), (H, F)])]
    xh, xf = synth.normal("cpu/cfg3_xh", (M, H)), synth.gelu_erf(synth.normal("cpu/cfg3_xf", (M, F)))
    t, reps = timed(lambda: [mm(O.Q8_0, w, xf if w.shape[1] == O.row_size(O.Q8_0, F) else xh) for w in lay])
    batch = 6 * t
    out["minilm_l6_e2e"] = base(32 / batch, "embeddings/s (upper bound: linear layers only)",
                                f"one layer's q, k, v, o, fc1, fc2 Q8_0 products on the batch's 4096 rows "
                                f"({reps} reps: {t * 1e3:.1f} ms) x 6 layers = {batch * 1e3:.1f} ms per 32-sequence "
                                f"batch")
    # cfg4: one Qwen3 layer's products (q|k|v, o, gate|up, down) on 512 of the 8192 rows
    H, F, QD, Ms = 1024, 3072, 2048, 512
    lay = [(q(O.Q4_K, "cpu/cfg4_qkv", QD + 2 * 512 * 2, H), H), (q(O.Q4_K, "cpu/cfg4_o", H, QD), QD),
           (q(O.Q4_K, "cpu/cfg4_gu", 2 * F, H), H), (q(O.Q4_K, "cpu/cfg4_down", H, F), F)]
    xs = {k: synth.normal(f"cpu/cfg4_x{k}", (Ms, k)) for k in (H, QD, F)}
    t, reps = timed(lambda: [mm(O.Q4_K, w, xs[k]) for w, k in lay])
    batch = t * 28 * (8192 / Ms)
    out["qwen3_0_6b_e2e"] = base(16 / batch, "embeddings/s (upper bound: linear layers only)",
                                 f"one layer's q|k|v, o, gate|up, down Q4_K products on 512 of the batch's 8192 "
                                 f"rows ({reps} reps: {t * 1e3:.1f} ms) x 28 layers x 16 = {batch:.2f} s per "
                                 f"16-sequence batch")
    # cfg5: layer sweep over 28 distinct copies, m = 1 and 8; lm_head m = 1
    H, FF = 2048, 6144
    shapes = [(H, H), (1024, H), (1024, H), (H, H), (FF, H), (FF, H), (H, FF)]
    one = [q(O.Q4_K, f"cpu/cfg5_{i}", n, k) for i, (n, k) in enumerate(shapes)]
    layers = [[w.copy() for w in one] for _ in range(28)]
    wbytes = 28 * sum(w.nbytes for w in one)
    dec = {}
    for m in (1, 8):
        xs = {k: synth.normal(f"cpu/cfg5_x{k}_{m}", (m, k)) for k in (H, FF)}
        t, reps = timed(lambda: [mm(O.Q4_K, w, xs[k]) for lay_ in layers for w, (n, k) in zip(lay_, shapes)])
        dec[f"layer_sweep_q4_K_m{m}"] = {"layer_us": round(t / 28 * 1e6, 1), "weight_gbs": round(wbytes / t / 1e9, 1),
                                         "sweep_ms": round(t * 1e3, 2), "reps": reps}
    rows = q(O.Q6_K, "cpu/cfg5_lm_head", 4096, H)
    head = np.tile(rows, (151936 // 4096 + 1, 1))[:151936]
    x = synth.normal("cpu/cfg5_xhead", (1, H))
    t, reps = timed(lambda: mm(O.Q6_K, head, x))
    dec["lm_head_q6_K_m1"] = {"us": round(t * 1e6, 1), "gbs": round(head.nbytes / t / 1e9, 1), "reps": reps}
    b = base(dec["layer_sweep_q4_K_m1"]["layer_us"], "us per layer (m = 1)",
             "28 distinct copies of one Qwen3-VL-2B layer's 7 Q4_K matrices (792.7 MB) swept at m = 1 and 8, and "
             "the Q6_K lm_head [151936 x 2048] (4096 quantized rows tiled) at m = 1, incl. activation quantization")
    b["detail"] = dec
    out["decode_gemv"] = b
    return out


def model_floor(kind):
    """The sum of per-op roofline floors of one batch of the end-to-end workloads (MI355X datasheet
    peaks: dense int8 5.0 POP/s, dense fp16 2.5 PFLOP/s, HBM 8 TB/s): each linear layer at
    max(2 M N K / int8 peak, (GGUF weight + quantized activation + fp32 output bytes) / HBM), the
    attention at max(its algorithmic flops / fp16 peak, q/k/v/out bytes / HBM), and each
    embedding / norm pass at its fp32 bytes / HBM.  Returns (floor in us, the formula's terms)."""
    P8, P16, BW = 5.0e15, 2.5e15, 8.0e12
    if kind == "minilm":
        B, T, H, F, nh, nl, wb, ab = 32, 128, 384, 1536, 12, 6, 34 / 32, 34 / 32
        lin = [(3 * H, H), (H, H), (F, H), (H, F)]
        att_flops = 4.0 * B * nh * T * T * (H // nh)  # full mask
        norm_bytes = nl * 2 * (12.0 * B * T * H) + 16.0 * B * T * H  # residual + LN per sublayer; embeddings
    else:
        B, T, H, F, nh, nl, wb, ab = 16, 512, 1024, 3072, 16, 28, 144 / 256, 292 / 256
        lin = [(4096, H), (H, 2048), (2 * F, H), (H, F)]
        att_flops = 2.0 * B * nh * T * T * 128  # causal: half of 4 T^2 hd
        norm_bytes = nl * 2 * (12.0 * B * T * H)
    M = B * T
    t_lin = nl * sum(max(2.0 * M * n * k / P8, (n * k * wb + M * k * ab + 4.0 * M * n) / BW) for n, k in lin)
    qd = (2048 if kind != "minilm" else H)
    att_bytes = 4.0 * M * (qd + 2 * (1024 if kind != "minilm" else H) + qd)
    t_att = nl * max(att_flops / P16, att_bytes / BW)
    t_norm = norm_bytes / BW
    return (t_lin + t_att + t_norm) * 1e6, {"linear_us": round(t_lin * 1e6, 1), "attention_us": round(t_att * 1e6, 1),
                                           "norm_us": round(t_norm * 1e6, 1)}


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
    """The host CPU: /proc/cpuinfo's model name, family / model / stepping, and the CPU count this
    process may use."""
    f = {}
    try:
        for line in open("/proc/cpuinfo"):
            k, _, v = line.partition(":")
            k = k.strip()
            if k in ("model name", "cpu family", "model", "stepping") and k not in f:
                f[k] = v.strip()
    except OSError:
        pass
    name = f.get("model name", "unknown CPU")
    return (f"{name} (family {f.get('cpu family', '?')} model {f.get('model', '?')} stepping "
            f"{f.get('stepping', '?')}, {len(os.sched_getaffinity(0))} CPUs visible)")


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
        if extras is not None:
            for name, b in cpu_baselines_extras(args).items():
                if isinstance(extras.get(name), dict):
                    extras[name]["cpu_baseline"] = b
    if extras is not None:
        for name, kind in (("minilm_l6_e2e", "minilm"), ("qwen3_0_6b_e2e", "qwen3")):
            e = extras.get(name)
            if isinstance(e, dict) and "batch_ms" in e:
                floor, terms = model_floor(kind)
                e["roofline"] = {"bound": "sum of per-op floors", "floor_us": round(floor, 1), "terms": terms,
                                 "achieved_us": round(e["batch_ms"] * 1e3, 1),
                                 "frac": round(floor / (e["batch_ms"] * 1e3), 4)}
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
            "ffn_chain": {k: round(v, 3) for k, v in r["chain"].items()},
        },
        "roofline": r["roofline"],
        "cpu_baseline": cpu,
        "extras": extras,
    }
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
