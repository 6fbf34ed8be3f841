"""The mixture-of-experts mat-mul (ggml_mul_mat_id, src/crispembed.cpp:1365,1371) with the routing
on the device (mq_op_mul_mat_id_device): no host copy of the ids, the rows sorted by expert in
whole row tiles on the GPU, one GEMM over every expert.  Every output row against the oracle's
integer-dot product of its expert (the mul_mat bar: 1e-4 of the row's largest value) and against
the host-routed mq_op_mul_mat_id; ids outside [0, n_exp) give NaN rows."""
import ctypes

import numpy as np
import pytest

import oracle_ffi as O
from gpu_util import dev, empty_u8, host, stream

pytestmark = pytest.mark.gpu

TOL = 1e-4


def _experts(oracle, wtype, n_exp, n, k, rng):
    """n_exp prepared weight images of n x k in one buffer (stride a multiple of 256 bytes), and
    the experts' GGUF rows for the oracle."""
    from crispembed_amd import mq
    L = mq.lib()
    size = L.mq_weight_image_bytes(wtype, n, k)
    stride = -(-size // 256) * 256
    buf, off = empty_u8(stride * n_exp)
    base = buf.data_ptr() + off
    ggufs = []
    for e in range(n_exp):
        w = (rng.standard_normal((n, k)) * 0.02).astype(np.float32)
        g = np.ascontiguousarray(oracle.quantize_chunk(wtype, w)).ravel()
        ggufs.append(g)
        buf[off + e * stride:off + e * stride + g.size] = dev(g)
        mq.check(L.mq_weight_prepare(wtype, ctypes.c_void_p(base + e * stride), n, k, 0, n, stream()))
    return buf, base, stride, ggufs


def _ref(oracle, wtype, g, rows):
    """The oracle's product of one expert's GGUF rows with fp32 activation rows (the threaded
    integer-dot restatement; F16 through the plain restatement)."""
    if wtype == O.F16:
        return oracle.mul_mat(wtype, g, rows)
    return oracle.fast_mul_mat(wtype, g, rows, nthreads=16)


def _run(entry, wtype, base, stride, n_exp, n, k, b, ids, n_used, T):
    import torch
    from crispembed_amd import mq
    L = mq.lib()
    dst = torch.full((T, n_used, n), 7.0, dtype=torch.float32, device="cuda")
    R = n_used * T
    if entry == "device":
        nb = L.mq_op_mul_mat_id_device_workspace_bytes(wtype, n_exp, n, k, R)
        fn = L.mq_op_mul_mat_id_device
    else:
        nb = L.mq_op_mul_mat_id_workspace_bytes(wtype, n, k, R)
        fn = L.mq_op_mul_mat_id
    assert nb > 0
    ws, off = empty_u8(nb)
    ws.fill_(0xAB)
    mq.check(fn(wtype, ctypes.c_void_p(base), stride, n_exp, n, k, mq.view(b), mq.view(ids), mq.view(dst),
                ctypes.c_void_p(ws.data_ptr() + off), nb, stream()))
    return host(dst)


@pytest.mark.parametrize("wtype,n_exp,n_used,T,k,n,b_slots,skew", [
    (O.Q8_0, 8, 2, 300, 384, 512, 1, None),      # b broadcast over the slots (ggml_mul_mat_id's nb1 = 1)
    (O.Q4_K, 8, 2, 4096, 512, 1024, 1, None),    # 8192 routed rows: 256-row tiles
    (O.Q6_K, 16, 4, 64, 256, 256, 4, None),      # a row of b per slot (the FFN-down's input)
    (O.F16, 4, 1, 33, 128, 96, 1, None),
    (O.Q4_K, 8, 2, 1, 256, 512, 1, None),        # one token (decode)
    (O.Q8_0, 8, 2, 500, 256, 384, 2, 3),         # every slot on one expert
    (O.Q8_0, 8, 2, 700, 256, 384, 2, "bad"),     # ids outside [0, n_exp): NaN rows
])
def test_mul_mat_id_device_routing(oracle, wtype, n_exp, n_used, T, k, n, b_slots, skew):
    import torch
    rng = np.random.default_rng(n_exp * 1000 + T + wtype)
    buf, base, stride, ggufs = _experts(oracle, wtype, n_exp, n, k, rng)
    x = rng.standard_normal((T, b_slots, k)).astype(np.float32)
    ids = np.stack([rng.permutation(n_exp)[:n_used] for _ in range(T)]).astype(np.int32)  # distinct per token
    if skew == 3:
        ids[:] = 3
    bad = np.zeros_like(ids, dtype=bool)
    if skew == "bad":
        bad = rng.random(ids.shape) < 0.05
        ids[bad] = np.where(rng.random(int(bad.sum())) < 0.5, -1, n_exp)
    b = dev(x)
    ids_d = dev(ids)
    got = _run("device", wtype, base, stride, n_exp, n, k, b, ids_d, n_used, T)
    # the oracle: each expert's rows through its integer-dot product
    want = np.full((T, n_used, n), np.nan, np.float32)
    for e in range(n_exp):
        sel = np.argwhere(ids == e)
        if sel.size == 0:
            continue
        rows = x[sel[:, 0], sel[:, 1] % b_slots]
        want[sel[:, 0], sel[:, 1]] = _ref(oracle, wtype, ggufs[e], rows)
    assert np.isnan(got[bad]).all()
    g, w = got[~bad], want[~bad]
    assert np.isfinite(g).all()
    row_err = np.abs(g.astype(np.float64) - w).max(1) / np.abs(w).max(1)
    assert row_err.max() <= TOL, (int(row_err.argmax()), row_err.max())
    if skew != "bad":  # the host-routed op fails on such ids
        ref = _run("host", wtype, base, stride, n_exp, n, k, b, ids_d, n_used, T)
        assert np.abs(got - ref).max() <= 1e-5 * np.abs(ref).max()
    del buf


def test_mul_mat_id_device_no_sync_between_calls(oracle):
    """Two device-routed calls enqueued back to back on one stream with different routings, the
    ids of the second written by a kernel enqueued after the first call: both results right (the
    routing reads the ids when the stream reaches it, not when the call is made)."""
    import torch
    from crispembed_amd import mq
    L = mq.lib()
    wtype, n_exp, n_used, T, k, n = O.Q8_0, 8, 2, 200, 256, 256
    rng = np.random.default_rng(5)
    buf, base, stride, ggufs = _experts(oracle, wtype, n_exp, n, k, rng)
    x = rng.standard_normal((T, 1, k)).astype(np.float32)
    b = dev(x)
    ids = [np.stack([rng.permutation(n_exp)[:n_used] for _ in range(T)]).astype(np.int32) for _ in range(2)]
    ids_d = dev(ids[0])
    R = n_used * T
    nb = L.mq_op_mul_mat_id_device_workspace_bytes(wtype, n_exp, n, k, R)
    outs = []
    keep = []
    for j in range(2):
        if j == 1:
            ids_d.copy_(dev(ids[1]), non_blocking=True)  # same stream: after the first call's routing
        dst = torch.empty((T, n_used, n), dtype=torch.float32, device="cuda")
        ws, off = empty_u8(nb)
        keep.append(ws)
        mq.check(L.mq_op_mul_mat_id_device(wtype, ctypes.c_void_p(base), stride, n_exp, n, k, mq.view(b),
                                           mq.view(ids_d), mq.view(dst), ctypes.c_void_p(ws.data_ptr() + off), nb,
                                           stream()))
        outs.append(dst)
    for j in range(2):
        got = host(outs[j])
        want = np.empty_like(got)
        for e in range(n_exp):
            sel = np.argwhere(ids[j] == e)
            if sel.size:
                want[sel[:, 0], sel[:, 1]] = _ref(oracle, wtype, ggufs[e], x[sel[:, 0], 0])
        err = np.abs(got.astype(np.float64) - want).max(2) / np.abs(want).max(2)
        assert err.max() <= TOL, (j, err.max())
    del buf
