"""The graph ops of mq_ops.h on the GPU against numpy restatements of ggml's CPU semantics, on
strided views as ggml hands them over (permuted, sliced, broadcast).

Bars: get_rows is bit-exact against the oracle's dequantize_row (ggml's arithmetic); binary ops
and copies are single IEEE operations per element, so bit-exact against numpy float32; norms,
GELU/SiLU and attention are compared with float64 evaluations of their formulas at the stated
tolerances (fp32 rounding of a row reduction, libm-vs-device transcendental ulps, and the
split-fp16 products of the attention kernel)."""
import ctypes

import numpy as np
import pytest

import oracle_ffi as O
from crispembed_amd import mq
from gpu_util import host, stream

pytestmark = pytest.mark.gpu


def _t():
    import torch
    return torch


_KEEP = []  # an mq_view holds only the address: the tensors behind views live until the test ends


@pytest.fixture(autouse=True)
def _release_tensors():
    yield
    _KEEP.clear()


def _cuda(a):
    t = _t().from_numpy(np.ascontiguousarray(a)).cuda()
    _KEEP.append(t)
    return t


def _rng(seed):
    return np.random.default_rng(seed)


def _call(fn, *args):
    mq.check(fn(*args))
    _t().cuda.synchronize()


# ------------------------------------------------------------------ get_rows ----
@pytest.mark.parametrize("ttype", [O.F32, O.F16, O.Q8_0, O.Q4_K, O.Q6_K])
def test_get_rows_bit_exact(oracle, ttype):
    L = mq.lib()
    H, V, n = 512, 97, 40
    tbl = _rng(1).standard_normal((V, H)).astype(np.float32)
    if ttype == O.F32:
        raw, ref_tbl = tbl.view(np.uint8).reshape(V, -1), tbl
    elif ttype == O.F16:
        raw = tbl.astype(np.float16).view(np.uint8).reshape(V, -1)
        ref_tbl = tbl.astype(np.float16).astype(np.float32)
    else:
        raw = np.ascontiguousarray(oracle.quantize_chunk(ttype, tbl)).reshape(V, -1)
        ref_tbl = oracle.dequantize(ttype, raw, H)
    ids = _rng(2).integers(0, V, n).astype(np.int32)
    ids[3] = V + 5  # out of range: zero row
    ids[7] = -1
    d_raw, d_ids = _cuda(raw), _cuda(ids)
    out = _t().full((n, H), np.nan, dtype=_t().float32, device="cuda")
    rs = raw.shape[1]
    nb0 = {O.F32: 4, O.F16: 2, O.Q8_0: 34, O.Q4_K: 144, O.Q6_K: 210}[ttype]
    src = mq.view(d_raw, type=ttype, ne=[H, V, 1, 1], nb=[nb0, rs, rs * V, rs * V])
    _call(L.mq_op_get_rows, src, mq.view(d_ids), mq.view(out), stream())
    ref = ref_tbl[np.clip(ids, 0, V - 1)].copy()
    ref[[3, 7]] = 0
    assert np.array_equal(host(out), ref)


def test_get_rows_planes_and_strided_dst():
    """ids [n, 3] pick rows of table plane i11; dst written through a strided view."""
    L = mq.lib()
    H, V, P, n = 64, 11, 3, 5
    tbl = _rng(3).standard_normal((P, V, H)).astype(np.float32)
    ids = _rng(4).integers(0, V, (P, n)).astype(np.int32)
    big = _t().zeros((P, n, 2 * H), dtype=_t().float32, device="cuda")
    dst = big[:, :, H:]
    _call(L.mq_op_get_rows, mq.view(_cuda(tbl)), mq.view(_cuda(ids)), mq.view(dst), stream())
    ref = np.stack([tbl[p][ids[p]] for p in range(P)])
    got = host(big)
    assert np.array_equal(got[:, :, H:], ref) and not got[:, :, :H].any()


# -------------------------------------------------------------------- binary ----
@pytest.mark.parametrize("op,f", [(mq.BIN_ADD, np.add), (mq.BIN_SUB, np.subtract), (mq.BIN_MUL, np.multiply),
                                  (mq.BIN_DIV, np.divide)])
@pytest.mark.parametrize("bshape", ["row", "full", "col", "plane"])
def test_binary_broadcast_bit_exact(op, f, bshape):
    L = mq.lib()
    B, T, H = 3, 17, 384
    a = _rng(5).standard_normal((B, T, H)).astype(np.float32)
    b = {"row": (1, 1, H), "full": (B, T, H), "col": (B, T, 1), "plane": (1, T, H)}[bshape]
    bv = (_rng(6).standard_normal(b) + (3.0 if op == mq.BIN_DIV else 0.0)).astype(np.float32)
    da, db = _cuda(a), _cuda(bv)
    out = _t().empty_like(da)
    _call(L.mq_op_binary, op, mq.view(da), mq.view(db), mq.view(out), stream())
    assert np.array_equal(host(out), f(a, bv))


def test_binary_on_permuted_views():
    """src0 a permuted (non-contiguous) view, dst a column slice: the scalar path."""
    L = mq.lib()
    a = _rng(7).standard_normal((4, 6, 32)).astype(np.float32)
    da = _cuda(a).permute(1, 0, 2)  # torch (6, 4, 32)
    b = _rng(8).standard_normal((1, 1, 32)).astype(np.float32)
    big = _t().zeros((6, 4, 40), dtype=_t().float32, device="cuda")
    dst = big[:, :, 3:35]
    _call(L.mq_op_binary, mq.BIN_ADD, mq.view(da), mq.view(_cuda(b)), mq.view(dst), stream())
    assert np.array_equal(host(big)[:, :, 3:35], a.transpose(1, 0, 2) + b)


# --------------------------------------------------------------------- unary ----
def _gelu_erf64(x):
    from scipy.special import erf
    return 0.5 * x * (1.0 + erf(x / np.sqrt(2.0)))


UNARY = [
    (mq.UNARY_GELU_ERF, _gelu_erf64, 1e-6),
    (mq.UNARY_GELU, lambda x: 0.5 * x * (1 + np.tanh(np.sqrt(2 / np.pi) * (x + 0.044715 * x ** 3))), 1e-6),
    (mq.UNARY_SILU, lambda x: x / (1 + np.exp(-x)), 1e-6),
    (mq.UNARY_RELU, lambda x: np.maximum(x, 0), 0.0),
]


@pytest.mark.parametrize("op,f,tol", UNARY)
def test_unary(op, f, tol):
    L = mq.lib()
    x = (_rng(9).standard_normal((33, 1536)) * 3).astype(np.float32)
    x[0, :8] = [0.0, -0.0, 1e-30, -1e-30, 20.0, -20.0, 8.0, -8.0]
    dx = _cuda(x)
    out = _t().empty_like(dx)
    _call(L.mq_op_unary, op, mq.view(dx), mq.view(out), stream())
    ref = f(x.astype(np.float64))
    got = host(out).astype(np.float64)
    # relative to max(|f(x)|, 1): the 1 + erf / 1 + tanh forms cancel for negative x in fp32
    # (as in ggml's CPU kernels), which leaves an absolute error of a few 1e-8 |x| there
    err = np.abs(got - ref) / np.maximum(np.abs(ref), 1.0)
    assert err.max() <= tol, err.max()
    # strided view (every other row)
    sub = dx[::2]
    out2 = _t().empty_like(sub)
    _call(L.mq_op_unary, op, mq.view(sub), mq.view(out2), stream())
    assert np.array_equal(host(out2), host(out)[::2])


# ---------------------------------------------------------------------- norm ----
@pytest.mark.parametrize("n", [100, 384, 768, 1024, 2560])
@pytest.mark.parametrize("kind", [mq.NORM_LAYER, mq.NORM_RMS])
def test_norm(kind, n):
    L = mq.lib()
    rows = 37
    x = (_rng(10).standard_normal((rows, n)) * 2 + 0.5).astype(np.float32)
    w = _rng(11).standard_normal(n).astype(np.float32)
    b = _rng(12).standard_normal(n).astype(np.float32)
    eps = 1e-12 if kind == mq.NORM_LAYER else 1e-6
    x64 = x.astype(np.float64)
    if kind == mq.NORM_LAYER:
        y = (x64 - x64.mean(-1, keepdims=True)) / np.sqrt(x64.var(-1, keepdims=True) + eps)
    else:
        y = x64 / np.sqrt((x64 ** 2).mean(-1, keepdims=True) + eps)
    dx = _cuda(x)
    out = _t().empty_like(dx)
    _call(L.mq_op_norm, kind, mq.view(dx), None, mq.view(out), eps, None, None, stream())
    assert np.abs(host(out) - y).max() <= 5e-6 * np.abs(y).max()
    dw, db = _cuda(w), _cuda(b)
    _call(L.mq_op_norm, kind, mq.view(dx), None, mq.view(out), eps, ctypes.c_void_p(dw.data_ptr()),
          ctypes.c_void_p(db.data_ptr()), stream())
    ref = y * w + b
    assert np.abs(host(out) - ref).max() <= 5e-6 * np.abs(ref).max()
    # with the residual: norm(x + r) * w + b, the sum rounded to fp32 first as the ADD node does;
    # also written in place over x
    r = _rng(13).standard_normal((rows, n)).astype(np.float32)
    s64 = (x + r).astype(np.float64)
    if kind == mq.NORM_LAYER:
        y2 = (s64 - s64.mean(-1, keepdims=True)) / np.sqrt(s64.var(-1, keepdims=True) + eps)
    else:
        y2 = s64 / np.sqrt((s64 ** 2).mean(-1, keepdims=True) + eps)
    ref2 = y2 * w + b
    _call(L.mq_op_norm, kind, mq.view(dx), mq.view(_cuda(r)), mq.view(dx), eps, ctypes.c_void_p(dw.data_ptr()),
          ctypes.c_void_p(db.data_ptr()), stream())
    assert np.abs(host(dx) - ref2).max() <= 5e-6 * np.abs(ref2).max()


@pytest.mark.parametrize("kind", [0, 1])
@pytest.mark.parametrize("n,rows", [(128, 37), (384, 4096), (768, 300), (1024, 70)])
def test_norm_q8_0(kind, n, rows):
    """mq_op_norm_q8_0: the residual + norm + scale + shift of mq_op_norm, its fp32 result within
    the norm bar of the fp64 reference, and the quantized activation it leaves bit-identical to
    the activation quantizer run on that result (GEMM layout, every live row)."""
    from gpu_util import empty_u8, live_q8_0_planes
    L = mq.lib()
    kind = mq.NORM_LAYER if kind == 0 else mq.NORM_RMS
    x = (_rng(20 + n).standard_normal((rows, n)) * 2 + 0.5).astype(np.float32)
    r = _rng(21 + n).standard_normal((rows, n)).astype(np.float32)
    w = _rng(22).standard_normal(n).astype(np.float32)
    b = _rng(23).standard_normal(n).astype(np.float32)
    eps = 1e-12 if kind == mq.NORM_LAYER else 1e-6
    s64 = (x + r).astype(np.float64)
    if kind == mq.NORM_LAYER:
        y = (s64 - s64.mean(-1, keepdims=True)) / np.sqrt(s64.var(-1, keepdims=True) + eps)
    else:
        y = s64 / np.sqrt((s64 ** 2).mean(-1, keepdims=True) + eps)
    ref = y * w + b
    dx, dr, dw, db = _cuda(x), _cuda(r), _cuda(w), _cuda(b)
    out = _t().empty_like(dx)
    nb = L.mq_workspace_bytes(mq.TYPE_Q8_0, rows, n)
    ws, off = empty_u8(nb)
    ws.fill_(0xAB)
    _call(L.mq_op_norm_q8_0, kind, mq.view(dx), mq.view(dr), mq.view(out), eps, ctypes.c_void_p(dw.data_ptr()),
          ctypes.c_void_p(db.data_ptr()), ctypes.c_void_p(ws.data_ptr() + off), nb, stream())
    got = host(out)
    assert np.abs(got - ref).max() <= 5e-6 * np.abs(ref).max()
    ws2, off2 = empty_u8(nb)
    mq.check(L.mq_quantize_act_ex(mq.TYPE_Q8_0, ctypes.c_void_p(out.data_ptr()), n, rows, n, None, 0,
                                  ctypes.c_void_p(ws2.data_ptr() + off2), nb, mq.PATH_GEMM, stream()))
    qa, da = live_q8_0_planes(host(ws2)[off2:off2 + nb], rows, n)
    qb, db_ = live_q8_0_planes(host(ws)[off:off + nb], rows, n)
    assert np.array_equal(qa, qb)
    assert np.array_equal(da.view(np.uint32), db_.view(np.uint32))
    # in place over x, no w / b: the same as mq_op_norm's result within the bar
    _call(L.mq_op_norm_q8_0, kind, mq.view(dx), None, mq.view(dx), eps, None, None,
          ctypes.c_void_p(ws.data_ptr() + off), nb, stream())
    x64 = x.astype(np.float64)
    if kind == mq.NORM_LAYER:
        y0 = (x64 - x64.mean(-1, keepdims=True)) / np.sqrt(x64.var(-1, keepdims=True) + eps)
    else:
        y0 = x64 / np.sqrt((x64 ** 2).mean(-1, keepdims=True) + eps)
    assert np.abs(host(dx) - y0).max() <= 5e-6 * np.abs(y0).max()


def test_norm_q8_0_refusals():
    L = mq.lib()
    x = _cuda(np.zeros((4, 200), np.float32))
    ws = _t().empty(1 << 20, dtype=_t().uint8, device="cuda")
    rc = L.mq_op_norm_q8_0(mq.NORM_LAYER, mq.view(x), None, mq.view(x), 1e-5, None, None,
                           ctypes.c_void_p(ws.data_ptr()), 1 << 20, stream())
    assert rc == -2 and b"multiple of 128" in L.mq_last_error()


@pytest.mark.parametrize("ntab,ne0", [(3, 384), (2, 384), (3, 30)])
def test_get_rows_sum(ntab, ne0):
    """mq_op_get_rows_sum: the token + position (+ type) embedding sum, bit-identical to the
    GET_ROWS and ADD nodes in float32 (added in table order), ids outside a table adding zeros."""
    L = mq.lib()
    rows = 300
    rng = _rng(ne0 + ntab)
    tabs = [rng.standard_normal((n, ne0)).astype(np.float32) for n in (1000, 512, 2)[:ntab]]
    ids = [rng.integers(0, t.shape[0], rows).astype(np.int32) for t in tabs]
    ids[0][5] = -3
    ids[1][7] = 10 ** 6
    ref = np.zeros((rows, ne0), np.float32)
    for t, i in zip(tabs, ids):
        g = np.where(((i >= 0) & (i < t.shape[0]))[:, None], t[np.clip(i, 0, t.shape[0] - 1)], np.float32(0))
        ref = (ref + g).astype(np.float32) if t is not tabs[0] else g.astype(np.float32)
    dts = [_cuda(t) for t in tabs]
    dis = [_cuda(i) for i in ids]
    out = _t().full((rows, ne0), np.nan, dtype=_t().float32, device="cuda")
    tv = [mq.view(t) for t in dts]
    iv = [mq.view(i) for i in dis]
    PV = ctypes.POINTER(mq.View) * ntab
    _call(L.mq_op_get_rows_sum, ntab, PV(*[ctypes.pointer(v) for v in tv]), PV(*[ctypes.pointer(v) for v in iv]),
          mq.view(out), stream())
    assert np.array_equal(host(out), ref)


# ----------------------------------------------------------------------- cpy ----
def test_cpy_cont_of_permute_and_qkv_slices():
    L = mq.lib()
    # ggml_cont(ggml_permute(x, 0, 2, 1, 3)) of x [hd, nh, T, B]
    x = _rng(13).standard_normal((2, 9, 6, 32)).astype(np.float32)  # torch (B, T, nh, hd)
    src = _cuda(x).permute(0, 2, 1, 3)  # (B, nh, T, hd)
    out = _t().empty(src.shape, dtype=_t().float32, device="cuda")
    _call(L.mq_op_cpy, mq.view(src), mq.view(out), stream())
    assert np.array_equal(host(out), x.transpose(0, 2, 1, 3))
    # ggml_cont(ggml_view_2d(qkv, H, TB, 3H*4, H*4)): the K third of fused q|k|v rows
    qkv = _rng(14).standard_normal((50, 3 * 384)).astype(np.float32)
    dq = _cuda(qkv)
    k = dq[:, 384:768]
    out = _t().empty((50, 384), dtype=_t().float32, device="cuda")
    _call(L.mq_op_cpy, mq.view(k), mq.view(out), stream())
    assert np.array_equal(host(out), qkv[:, 384:768])


def test_cpy_types_and_reshape_order():
    L = mq.lib()
    x = (_rng(15).standard_normal((8, 6, 10)) * 100).astype(np.float32)
    dx = _cuda(x)
    h = _t().empty((8, 6, 10), dtype=_t().float16, device="cuda")
    _call(L.mq_op_cpy, mq.view(dx), mq.view(h), stream())
    assert np.array_equal(host(h).view(np.uint16), x.astype(np.float16).view(np.uint16))
    back = _t().empty((8, 6, 10), dtype=_t().float32, device="cuda")
    _call(L.mq_op_cpy, mq.view(h), mq.view(back), stream())
    assert np.array_equal(host(back), x.astype(np.float16).astype(np.float32))
    # different shapes: element order is row-major over both views (a transposed source)
    src = dx.permute(2, 1, 0)  # (10, 6, 8) non-contiguous
    dst = _t().empty((4, 120), dtype=_t().float32, device="cuda")
    _call(L.mq_op_cpy, mq.view(src), mq.view(dst), stream())
    assert np.array_equal(host(dst).ravel(), x.transpose(2, 1, 0).ravel())


# ----------------------------------------------------------------- attention ----
def _attn64(q, k, v, mask, scale):
    """q [B, nh, Tq, hd], k/v [B, nkv, Tk, hd], mask [B|1, nh|1, Tq, Tk] or None -> [B, Tq, nh, hd]"""
    B, nh, Tq, hd = q.shape
    g = nh // k.shape[1]
    kk = np.repeat(k, g, axis=1).astype(np.float64)
    vv = np.repeat(v, g, axis=1).astype(np.float64)
    s = np.einsum("bhqd,bhkd->bhqk", q.astype(np.float64), kk) * scale
    if mask is not None:
        s = s + mask.astype(np.float64)
    mx = s.max(-1, keepdims=True)
    mx = np.where(np.isfinite(mx), mx, 0.0)
    p = np.exp(s - mx)
    den = p.sum(-1, keepdims=True)
    o = np.einsum("bhqk,bhkd->bhqd", p, vv) / np.where(den > 0, den, np.inf)
    return o.transpose(0, 2, 1, 3)


def _flash(q_t, k_t, v_t, mask_t, scale, out_t):
    L = mq.lib()
    kv = mq.view(k_t)
    ws_bytes = L.mq_op_flash_attn_workspace_bytes(kv)
    ws = _t().empty(ws_bytes + 256, dtype=_t().uint8, device="cuda")
    wp = ws.data_ptr() + (-ws.data_ptr()) % 256
    mv = mq.view(mask_t) if mask_t is not None else None
    _call(L.mq_op_flash_attn, mq.view(q_t), kv, mq.view(v_t), mv, mq.view(out_t), scale, ctypes.c_void_p(wp),
          ws_bytes, stream())


@pytest.fixture(params=["auto", "split", "nosplit"])
def attn_form(request, monkeypatch):
    """Both attention forms: the 8-wave kernel and the split-key kernel (chosen by grid size,
    or forced through MQ_ATTN_SPLIT, read at each launch)."""
    if request.param != "auto":
        monkeypatch.setenv("MQ_ATTN_SPLIT", "1" if request.param == "split" else "0")
    return request.param


@pytest.mark.parametrize("hd,nh,nkv,B,T", [(32, 12, 12, 3, 77), (64, 12, 12, 2, 128), (128, 8, 2, 2, 45),
                                           (32, 4, 4, 1, 300), (128, 16, 8, 1, 200), (128, 5, 5, 1, 200),
                                           (128, 3, 1, 2, 64)])
def test_flash_attn_permuted_views(attn_form, hd, nh, nkv, B, T):
    """q/k/v as ggml_permute(reshape(x, hd, nh, T, B), 0, 2, 1, 3) of contiguous projections.  Odd
    head counts at head_dim 128: the 8-wave kernel's key/value ring then has workgroups whose
    second head does not exist (its waves stay in the loop for the barriers and compute nothing),
    and grouped heads (3 query heads on one key/value head) straddle workgroups."""
    rng = _rng(hd + T)
    qx = rng.standard_normal((B, T, nh, hd)).astype(np.float32)
    kx = rng.standard_normal((B, T, nkv, hd)).astype(np.float32)
    vx = rng.standard_normal((B, T, nkv, hd)).astype(np.float32)
    q = _cuda(qx).permute(0, 2, 1, 3)  # torch (B, nh, T, hd) = ggml [hd, T, nh, B]
    k = _cuda(kx).permute(0, 2, 1, 3)
    v = _cuda(vx).permute(0, 2, 1, 3)
    out = _t().full((B, T, nh, hd), np.nan, dtype=_t().float32, device="cuda")  # ggml [hd, nh, T, B]
    scale = 1.0 / np.sqrt(hd)
    _flash(q, k, v, None, scale, out)
    ref = _attn64(qx.transpose(0, 2, 1, 3), kx.transpose(0, 2, 1, 3), vx.transpose(0, 2, 1, 3), None, scale)
    err = np.abs(host(out) - ref).max() / np.abs(ref).max()
    assert err <= 2e-5, err


@pytest.mark.parametrize("hd,nh,B,T,masked", [(32, 12, 3, 77, False), (32, 12, 32, 128, False), (64, 12, 2, 128, True),
                                              (64, 2, 5, 40, False), (128, 8, 2, 45, False)])
def test_flash_attn_q8_0(attn_form, hd, nh, B, T, masked):
    """mq_op_flash_attn_q8_0: dst as mq_op_flash_attn writes it (bit for bit), and the rows left
    quantized for the output projection bit-identical to the activation quantizer run on dst --
    from the attention kernel's own store (head_dim 32 / 64, 8-wave form) or the quantizer after
    it (split-key form, head_dim 128)."""
    from gpu_util import empty_u8, live_q8_0_planes
    L = mq.lib()
    rng = _rng(hd + T + B)
    qx, kx, vx = (rng.standard_normal((B, T, nh, hd)).astype(np.float32) for _ in range(3))
    q, k, v = (_cuda(x).permute(0, 2, 1, 3) for x in (qx, kx, vx))
    mask_t = None
    if masked:
        mask = np.zeros((B, 1, T, T), dtype=np.float16)
        for b in range(B):
            mask[b, 0, :, T - 7 * b:] = -np.inf if b else 0
        mask_t = _cuda(mask)
    scale = 1.0 / np.sqrt(hd)
    ref = _t().empty((B, T, nh, hd), dtype=_t().float32, device="cuda")
    _flash(q, k, v, mask_t, scale, ref)
    out = _t().full((B, T, nh, hd), np.nan, dtype=_t().float32, device="cuda")
    kv = mq.view(k)
    ws_bytes = L.mq_op_flash_attn_workspace_bytes(kv)
    ws, wo = empty_u8(ws_bytes)
    K, M = nh * hd, B * T
    nb = L.mq_workspace_bytes(mq.TYPE_Q8_0, M, K)
    act, ao = empty_u8(nb)
    act.fill_(0xAB)
    mv = mq.view(mask_t) if mask_t is not None else None
    _call(L.mq_op_flash_attn_q8_0, mq.view(q), kv, mq.view(v), mv, mq.view(out), scale,
          ctypes.c_void_p(ws.data_ptr() + wo), ws_bytes, ctypes.c_void_p(act.data_ptr() + ao), nb, stream())
    a, b_ = host(ref), host(out)
    assert np.array_equal(a.view(np.uint32), b_.view(np.uint32))
    want, wo2 = empty_u8(nb)
    mq.check(L.mq_quantize_act_ex(mq.TYPE_Q8_0, ctypes.c_void_p(out.data_ptr()), K, M, K, None, 0,
                                  ctypes.c_void_p(want.data_ptr() + wo2), nb, mq.PATH_GEMM, stream()))
    qa, da = live_q8_0_planes(host(want)[wo2:wo2 + nb], M, K)
    qb, db = live_q8_0_planes(host(act)[ao:ao + nb], M, K)
    assert np.array_equal(qa, qb)
    assert np.array_equal(da.view(np.uint32), db.view(np.uint32))


def test_flash_attn_pad_mask(attn_form):
    """The rectangular batch of encode_tokens_group_4d: F16 mask [T, T, 1, B], 0 for real keys,
    -inf for padding; padded query rows still attend to the real keys."""
    hd, nh, B, T = 32, 6, 4, 50
    lens = [50, 31, 1, 17]
    rng = _rng(21)
    qx, kx, vx = (rng.standard_normal((B, T, nh, hd)).astype(np.float32) for _ in range(3))
    mask = np.zeros((B, 1, T, T), dtype=np.float16)
    for b, n in enumerate(lens):
        mask[b, 0, :, n:] = -np.inf
    q, k, v = (_cuda(x).permute(0, 2, 1, 3) for x in (qx, kx, vx))
    out = _t().empty((B, T, nh, hd), dtype=_t().float32, device="cuda")
    _flash(q, k, v, _cuda(mask), 1.0 / np.sqrt(hd), out)
    ref = _attn64(qx.transpose(0, 2, 1, 3), kx.transpose(0, 2, 1, 3), vx.transpose(0, 2, 1, 3), mask,
                  1.0 / np.sqrt(hd))
    assert np.abs(host(out) - ref).max() / np.abs(ref).max() <= 2e-5


def test_flash_attn_general_mask_and_empty_rows(attn_form):
    """A finite additive mask per head (relative-position bias style), Tq != Tk, and query rows
    whose keys are all masked (zero output)."""
    hd, nh, B, Tq, Tk = 64, 4, 2, 20, 170
    rng = _rng(22)
    qx = rng.standard_normal((B, Tq, nh, hd)).astype(np.float32)
    kx, vx = (rng.standard_normal((B, Tk, nh, hd)).astype(np.float32) for _ in range(2))
    mask = (rng.standard_normal((B, nh, Tq, Tk)) * 2).astype(np.float16)
    mask[:, :, 5, :] = -np.inf
    mask[1, 2, 7, :] = -np.inf
    mask[0, 1, 9, 40:] = -np.inf
    q, k, v = (_cuda(x).permute(0, 2, 1, 3) for x in (qx, kx, vx))
    out = _t().empty((B, Tq, nh, hd), dtype=_t().float32, device="cuda")
    _flash(q, k, v, _cuda(mask), 0.125, out)
    ref = _attn64(qx.transpose(0, 2, 1, 3), kx.transpose(0, 2, 1, 3), vx.transpose(0, 2, 1, 3), mask, 0.125)
    got = host(out)
    assert np.isfinite(got).all()
    assert not got[:, 5].any() and not got[1, 7, 2].any()
    assert np.abs(got - ref).max() / np.abs(ref).max() <= 2e-5


@pytest.mark.parametrize("rows", ["aligned", "unaligned"])
@pytest.mark.parametrize("waves", ["4", "8"])
@pytest.mark.parametrize("hd,nh,nkv,Tq,Tk", [(128, 4, 2, 300, 300), (128, 2, 1, 40, 16500), (64, 4, 4, 100, 2100)])
def test_flash_attn_mask_block_classes(monkeypatch, rows, waves, hd, nh, nkv, Tq, Tk):
    """The split-key kernel's mask block classes: 32 x 32 blocks fully masked (skipped), all zero
    (run unmasked) and mixed (a causal band, finite values, a partly masked band), at 4 and 8
    waves per workgroup, with key blocks past the 64 each wave classifies up front (Tk 16500:
    516 blocks, 129 per wave at 4 waves, 65 at 8); mask rows 16-byte aligned (vector reads) or
    not (2-byte reads)."""
    monkeypatch.setenv("MQ_ATTN_SPLIT", "1")
    monkeypatch.setenv("MQ_ATTN_SPLIT_WAVES", waves)
    rng = _rng(hd + Tq + Tk)
    qx = rng.standard_normal((1, Tq, nh, hd)).astype(np.float32)
    kx, vx = (rng.standard_normal((1, Tk, nkv, hd)).astype(np.float32) for _ in range(2))
    qpos = np.arange(Tq)[:, None] + (Tk - Tq)
    mask = np.where(np.arange(Tk)[None, :] > qpos, -np.inf, 0.0)  # causal, query i at key Tk - Tq + i
    mask[:, 64:100] += rng.standard_normal((Tq, 36)) * 2  # finite values: mixed blocks
    mask[:, Tk // 2:Tk // 2 + 70] = -np.inf  # fully masked blocks (and two partly masked)
    mask[::3, Tk - 40:Tk - 20] = -np.inf
    if Tk > 16384:
        mask[:, 16400:16420] += rng.standard_normal((Tq, 20))  # finite values past block 512
    mask = mask.astype(np.float16)[None, None]
    stride = (Tk + 7) // 8 * 8 + (rows == "unaligned")
    padded = np.full((1, 1, Tq, stride), np.nan, np.float16)
    padded[..., :Tk] = mask
    q, k, v = (_cuda(x).permute(0, 2, 1, 3) for x in (qx, kx, vx))
    out = _t().empty((1, Tq, nh, hd), dtype=_t().float32, device="cuda")
    scale = 1.0 / np.sqrt(hd)
    _flash(q, k, v, _cuda(padded)[..., :Tk], scale, out)
    ref = _attn64(qx.transpose(0, 2, 1, 3), kx.transpose(0, 2, 1, 3), vx.transpose(0, 2, 1, 3), mask, scale)
    got = host(out)
    assert np.isfinite(got).all()
    assert np.abs(got - ref).max() / np.abs(ref).max() <= 2e-5


def _batch_mask(lens, slot, prefix=0):
    """The T_total x T_total mask decoder_encode_tokens_batch builds (src/decoder_embed.cpp:
    1406-1443), restated: items of lens[b] tokens in slots of `slot` positions after a shared
    prefix of `prefix` tokens (lens include the prefix); causal within an item and to the prefix,
    a padding position sees only itself."""
    B = len(lens)
    T = prefix + slot * B
    m = np.full((T, T), -np.inf, np.float32)
    for t in range(prefix):
        m[t, :t + 1] = 0
    for b, n in enumerate(lens):
        base, sl = prefix + b * slot, n - prefix
        for s in range(sl):
            m[base + s, :prefix] = 0
            m[base + s, base:base + s + 1] = 0
        for s in range(sl, slot):
            m[base + s, base + s] = 0
    return m.astype(np.float16)


def _block_lists(mask, Tq, Tk):
    """The block lists mq_op_mask_blocks must write for mask [Bm, >= Tq, >= Tk] (f16): per mask
    plane and tile of 32 query rows (rows past Tq repeat row Tq - 1), the 32-key blocks with a
    finite value, each flagged when a value is not zero (+-0 are zero; keys past Tk ignored)."""
    out = []
    for bm in range(mask.shape[0]):
        for qt in range((Tq + 31) // 32):
            rows = np.minimum(qt * 32 + np.arange(32), Tq - 1)
            blk = mask[bm, rows, :Tk].astype(np.float32)
            lst = []
            for kb in range((Tk + 31) // 32):
                v = blk[:, kb * 32:min(kb * 32 + 32, Tk)]
                if (v != -np.inf).any():
                    lst.append((kb, bool((v != 0).any())))
            out.append(lst)
    return out


@pytest.mark.parametrize("case", ["batch_ragged", "prefix", "planes", "unaligned", "tq_ne_tk"])
def test_mask_block_lists(case):
    """mq_op_mask_blocks against the lists restated in numpy (every entry, in order), and
    mq_op_flash_attn_blocks with those lists against fp64 softmax attention and against the same
    call without lists: the batched decoder's block-diagonal causal mask with ragged items and
    padding positions, its prefix-sharing layout, per-batch mask planes, mask rows that are not
    16-byte aligned (2-byte reads), and Tq != Tk with a finite bias band."""
    L = mq.lib()
    rng = _rng(len(case))
    hd, nh, nkv, B = 128, 4, 2, 1
    if case == "batch_ragged":
        mask = _batch_mask([100, 37, 64, 1], 100)[None]
    elif case == "prefix":
        mask = _batch_mask([70, 47, 90], 50, prefix=40)[None]
    elif case == "planes":
        B = 2
        mask = np.stack([_batch_mask([60, 5, 33], 60), _batch_mask([17, 60, 60], 60)])
    elif case == "unaligned":
        mask = _batch_mask([45, 45, 10], 45)[None]
    else:
        Tq, Tk = 70, 333
        m = np.where(np.arange(Tk)[None, :] > np.arange(Tq)[:, None] + (Tk - Tq), -np.inf, 0.0)
        m[:, 100:140] += rng.standard_normal((Tq, 40))
        m[:, 200:290] = -np.inf
        mask = m.astype(np.float16)[None]
    Tq, Tk = mask.shape[1], mask.shape[2]
    stride = (Tk + 7) // 8 * 8 + (case == "unaligned")
    padded = np.full((mask.shape[0], 1, Tq, stride), np.nan, np.float16)
    padded[:, 0, :, :Tk] = mask
    mask_d = _cuda(padded)[..., :Tk]
    qx = rng.standard_normal((B, Tq, nh, hd)).astype(np.float32)
    kx, vx = (rng.standard_normal((B, Tk, nkv, hd)).astype(np.float32) for _ in range(2))
    q, k, v = (_cuda(x).permute(0, 2, 1, 3) for x in (qx, kx, vx))
    qv, kv, vv, mv = mq.view(q), mq.view(k), mq.view(v), mq.view(mask_d)
    nbytes = L.mq_op_mask_blocks_bytes(qv, kv, mv)
    nqt, nkb = (Tq + 31) // 32, (Tk + 31) // 32
    assert nbytes == mask.shape[0] * nqt * (nkb + 1) * 4
    blocks = _t().full((nbytes // 4,), 0x7777, dtype=_t().int32, device="cuda")
    _call(L.mq_op_mask_blocks, qv, kv, mv, ctypes.c_void_p(blocks.data_ptr()), nbytes, stream())
    got = host(blocks).view(np.uint32).reshape(mask.shape[0] * nqt, nkb + 1)
    want = _block_lists(mask, Tq, Tk)
    for i, lst in enumerate(want):
        n = int(got[i, 0])
        assert n == len(lst), (i, n, len(lst))
        assert [(int(e & 0x7FFFFFFF), bool(e >> 31)) for e in got[i, 1:1 + n]] == lst, i
    ws_bytes = L.mq_op_flash_attn_workspace_bytes(kv)
    ws = _t().empty(ws_bytes + 256, dtype=_t().uint8, device="cuda")
    wp = ctypes.c_void_p(ws.data_ptr() + (-ws.data_ptr()) % 256)
    scale = 1.0 / np.sqrt(hd)
    ref = _attn64(qx.transpose(0, 2, 1, 3), kx.transpose(0, 2, 1, 3), vx.transpose(0, 2, 1, 3), mask[:, None], scale)
    outs = []
    for bl in (ctypes.c_void_p(blocks.data_ptr()), None):
        out = _t().full((B, Tq, nh, hd), np.nan, dtype=_t().float32, device="cuda")
        _call(L.mq_op_flash_attn_blocks, qv, kv, vv, mv, mq.view(out), scale, None, None, 0.0, None, bl, 0, wp,
              ws_bytes, None, 0, 0, 0, stream())
        outs.append(host(out))
        assert np.isfinite(outs[-1]).all()
        assert np.abs(outs[-1] - ref).max() / np.abs(ref).max() <= 2e-5
    assert np.abs(outs[0] - outs[1]).max() / np.abs(ref).max() <= 1e-6


@pytest.mark.parametrize("case,want", [("zeros", 1), ("neg_zero", 1), ("pad_rows", 1), ("last", 0), ("plane1", 0),
                                       ("half", 0)])
def test_mask_is_zero(case, want):
    """mq_op_mask_is_zero: 1 exactly when every value of the Tq x Tk region the attention reads, in
    every plane, is +-0 (an equal-length batch's padding mask): -0.0 counts as zero, values past
    the region (the mask's padded query rows) are not read; one -inf in the region's last row and
    column, a nonzero in the second plane, a 0.5 anywhere make it 0."""
    L = mq.lib()
    B, T, Tp = 3, 96, 128  # mask [T keys (+ stride pad), Tp >= T query rows, 1, B]
    m = np.zeros((B, 1, Tp, T + 8), np.float16)
    if case == "neg_zero":
        m[1, 0, 5, 7] = np.float16(-0.0)
    elif case == "pad_rows":
        m[:, 0, T:, :] = np.float16(-np.inf)  # query rows past Tq
        m[:, 0, :, T:] = np.float16(3.0)      # the row stride's unused tail
    elif case == "last":
        m[2, 0, T - 1, T - 1] = np.float16(-np.inf)
    elif case == "plane1":
        m[1, 0, 40, 3] = np.float16(-np.inf)
    elif case == "half":
        m[0, 0, 0, 50] = np.float16(0.5)
    mask_d = _cuda(m)[..., :T]
    hd, nh = 64, 2
    q = _cuda(np.zeros((B, nh, T, hd), np.float32))
    k = _cuda(np.zeros((B, nh, T, hd), np.float32))
    scratch = _t().zeros(64, dtype=_t().int32, device="cuda")
    z = ctypes.c_int(-1)
    _call(L.mq_op_mask_is_zero, mq.view(q), mq.view(k), mq.view(mask_d), ctypes.c_void_p(scratch.data_ptr()), 256,
          ctypes.byref(z), stream())
    assert z.value == want, case


@pytest.mark.parametrize("case,want", [("uniform", 128), ("single", 320), ("unaligned", 64), ("ragged", 0),
                                       ("prefix", 0), ("finite", 0), ("bidirectional", 0), ("odd", 96)])
def test_mask_segments(case, want):
    """mq_op_mask_segments finds the segment length exactly when the mask is block-diagonal causal
    over uniform segments (the batched decoder's mask with full-length items; one causal sequence;
    rows not 16-byte aligned), and 0 for every near miss: ragged items (padding rows see only
    themselves), a shared prefix, one finite nonzero value, bidirectional blocks.  With a segment a
    multiple of 32 the attention then runs per causal segment: equal to the mask's attention (fp64)
    and to the block-list form, with the q / k norm and rotation (positions restarting per segment)
    and with the o projection's Q8_K activation stored as the quantizer would write it."""
    L = mq.lib()
    rng = _rng(len(case) + want)
    if case in ("uniform", "unaligned", "finite"):
        S = 128 if case != "unaligned" else 64
        mask = _batch_mask([S] * 4, S)
        if case == "finite":
            mask[300, 260] = np.float16(-0.5)
    elif case == "single":
        mask = _batch_mask([320], 320)
    elif case == "odd":
        mask = _batch_mask([96] * 3, 96)
    elif case == "ragged":
        mask = _batch_mask([128, 100, 128, 128], 128)
    elif case == "prefix":
        mask = _batch_mask([70, 47, 90], 50, prefix=40)
    else:
        mask = np.full((384, 384), -np.inf, np.float16)
        for b in range(3):
            mask[128 * b:128 * (b + 1), 128 * b:128 * (b + 1)] = 0
    T = mask.shape[0]
    stride = T + 8 + (case == "unaligned")
    padded = np.full((1, 1, T, stride), np.nan, np.float16)
    padded[0, 0, :, :T] = mask
    mask_d = _cuda(padded)[..., :T]
    hd, nh, nkv = 128, 4, 2
    qx = rng.standard_normal((1, T, nh, hd)).astype(np.float32)
    kx, vx = (rng.standard_normal((1, T, nkv, hd)).astype(np.float32) for _ in range(2))
    q, k, v = (_cuda(x).permute(0, 2, 1, 3) for x in (qx, kx, vx))
    qv, kv, vv, mv = mq.view(q), mq.view(k), mq.view(v), mq.view(mask_d)
    nbytes = L.mq_op_mask_segments_bytes(qv, kv, mv)
    assert nbytes == T * 4
    scratch = _t().empty(T, dtype=_t().int32, device="cuda")
    seg = ctypes.c_int64(-1)
    _call(L.mq_op_mask_segments, qv, kv, mv, ctypes.c_void_p(scratch.data_ptr()), nbytes, ctypes.byref(seg), stream())
    assert seg.value == want, (case, seg.value)
    if want == 0 or want % 32:
        return
    ws_bytes = L.mq_op_flash_attn_workspace_bytes(kv)
    ws = _t().empty(ws_bytes + 256, dtype=_t().uint8, device="cuda")
    wp = ctypes.c_void_p(ws.data_ptr() + (-ws.data_ptr()) % 256)
    scale = 1.0 / np.sqrt(hd)
    ref = _attn64(qx.transpose(0, 2, 1, 3), kx.transpose(0, 2, 1, 3), vx.transpose(0, 2, 1, 3), mask[None, None],
                  scale)
    nb = L.mq_op_mask_blocks_bytes(qv, kv, mv)
    blocks = _t().empty(nb // 4, dtype=_t().int32, device="cuda")
    _call(L.mq_op_mask_blocks, qv, kv, mv, ctypes.c_void_p(blocks.data_ptr()), nb, stream())
    # q / k norm weights and the angles of positions restarting per segment
    qw, kw = (_cuda((1.0 + 0.1 * rng.standard_normal(hd)).astype(np.float32)) for _ in range(2))
    pos = _cuda((np.arange(T) % want).astype(np.int32))
    cs = _t().empty((T, hd), dtype=_t().float32, device="cuda")
    _call(L.mq_op_rope_cache, mq.view(pos), None, hd, 0, 1e6, 1.0, 0.0, 1.0, 0.0, 0.0,
          ctypes.c_void_p(cs.data_ptr()), stream())
    K, M = nh * hd, T
    act_bytes = L.mq_workspace_bytes(mq.TYPE_Q4_K, M, K)
    outs = {}
    for name, s_, bl, norm in (("seg", want, None, False), ("lists", 0, blocks, False), ("seg_qk", want, None, True),
                               ("lists_qk", 0, blocks, True)):
        out = _t().full((1, T, nh, hd), np.nan, dtype=_t().float32, device="cuda")
        act = _t().full((act_bytes + 256,), 0xAB, dtype=_t().uint8, device="cuda")
        ap = act.data_ptr() + (-act.data_ptr()) % 256
        nw = (ctypes.c_void_p(qw.data_ptr()), ctypes.c_void_p(kw.data_ptr()), 1e-6,
              ctypes.c_void_p(cs.data_ptr())) if norm else (None, None, 0.0, None)
        _call(L.mq_op_flash_attn_blocks, qv, kv, vv, mv, mq.view(out), scale, *nw,
              None if bl is None else ctypes.c_void_p(bl.data_ptr()), s_, wp, ws_bytes, ctypes.c_void_p(ap),
              act_bytes, mq.TYPE_Q4_K, 0, stream())
        want_act = _t().empty((act_bytes + 256,), dtype=_t().uint8, device="cuda")
        wq = want_act.data_ptr() + (-want_act.data_ptr()) % 256
        mq.check(L.mq_quantize_act_ex(mq.TYPE_Q4_K, ctypes.c_void_p(out.data_ptr()), K, M, K, None, 0,
                                      ctypes.c_void_p(wq), act_bytes, mq.PATH_GEMM, stream()))
        _t().cuda.synchronize()
        import act_layout as AL
        o1, o2 = (ap - act.data_ptr()), (wq - want_act.data_ptr())
        diff = AL.live_difference(host(act)[o1:o1 + act_bytes], host(want_act)[o2:o2 + act_bytes], mq.TYPE_Q4_K, M, K)
        assert diff is None, (name, diff)
        outs[name] = host(out)
        assert np.isfinite(outs[name]).all()
    assert np.abs(outs["seg"] - ref).max() / np.abs(ref).max() <= 2e-5
    for a, b in (("seg", "lists"), ("seg_qk", "lists_qk")):
        assert np.abs(outs[a] - outs[b]).max() / np.abs(outs[b]).max() <= 1e-6, (a, b)


def test_mask_block_lists_not_taken():
    """Operands whose attention reads no block lists get 0 bytes (and mq_op_mask_blocks refuses
    them): a mask that differs per head and no mask; a mask shared by the heads takes them at
    every length (here a 4-D padding mask at head_dim 64, on a grid the 8-wave kernel would fill)."""
    L = mq.lib()
    q = _cuda(np.zeros((1, 4, 64, 128), np.float32))
    k = _cuda(np.zeros((1, 2, 64, 128), np.float32))
    per_head = _cuda(np.zeros((1, 4, 64, 64), np.float16))
    assert L.mq_op_mask_blocks_bytes(mq.view(q), mq.view(k), mq.view(per_head)) == 0
    assert L.mq_op_mask_blocks_bytes(mq.view(q), mq.view(k), None) == 0
    assert L.mq_op_mask_blocks(mq.view(q), mq.view(k), mq.view(per_head), None, 0, stream()) < 0
    q64 = _cuda(np.zeros((32, 12, 128, 64), np.float32))
    k64 = _cuda(np.zeros((32, 12, 128, 64), np.float32))
    m64 = _cuda(np.zeros((32, 1, 128, 128), np.float16))
    assert L.mq_op_mask_blocks_bytes(mq.view(q64), mq.view(k64), mq.view(m64)) == 32 * 4 * 5 * 4


@pytest.mark.parametrize("case", ["plain", "yarn", "freq_factors"])
def test_rope_cache_matches_rope(case):
    """mq_op_rope_cache against mq_op_rope: rotating the pair (1, 0) gives (cos, sin) x mscale
    of the pair's angle, bit for bit."""
    L = mq.lib()
    T, n_dims = 45, 128
    rng = _rng(40)
    pos = (np.arange(T) * 7 + 3).astype(np.int32)
    kw = dict(n_ctx_orig=0, base=1e6, freq_scale=1.0, ext_factor=0.0, attn_factor=1.0, beta_fast=0.0, beta_slow=0.0)
    if case == "yarn":
        kw.update(n_ctx_orig=4096, freq_scale=0.25, ext_factor=1.0, attn_factor=0.9, beta_fast=32.0, beta_slow=1.0)
    ff = (1.0 + rng.random(n_dims // 2) * 3).astype(np.float32) if case == "freq_factors" else None
    fv = mq.view(_cuda(ff)) if ff is not None else None
    dp = _cuda(pos)
    args = (kw["n_ctx_orig"], kw["base"], kw["freq_scale"], kw["ext_factor"], kw["attn_factor"], kw["beta_fast"],
            kw["beta_slow"])
    cs = _t().empty((T, n_dims), dtype=_t().float32, device="cuda")
    _call(L.mq_op_rope_cache, mq.view(dp), fv, n_dims, *args, ctypes.c_void_p(cs.data_ptr()), stream())
    x = np.zeros((1, T, 1, n_dims), np.float32)
    x[..., :n_dims // 2] = 1.0  # NEOX pairs (i, i + n_dims / 2) = (1, 0)
    dx = _cuda(x)
    out = _t().empty_like(dx)
    _call(L.mq_op_rope, mq.view(dx), mq.view(dp), fv, mq.view(out), n_dims, mq.ROPE_NEOX, *args, stream())
    r = host(out).reshape(T, n_dims)
    want = np.stack([r[:, :n_dims // 2], r[:, n_dims // 2:]], -1).reshape(T, n_dims)
    assert np.array_equal(host(cs).view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("hd,nh,nkv,B,T,masked", [(128, 4, 2, 1, 300, True), (128, 8, 4, 2, 64, False),
                                                  (64, 4, 4, 2, 100, True), (32, 6, 2, 1, 77, False),
                                                  (128, 5, 5, 1, 200, False), (128, 3, 1, 2, 64, False)])
def test_flash_attn_qk_norm_rope(attn_form, hd, nh, nkv, B, T, masked):
    """mq_op_flash_attn_qk_norm_rope (q and k normed and rotated as the attention reads them)
    against mq_op_norm + mq_op_rope of q and k followed by mq_op_flash_attn: equal up to the RMS
    norm's summation order."""
    L = mq.lib()
    rng = _rng(hd + nh + T)
    qx = rng.standard_normal((B, T, nh, hd)).astype(np.float32) * 3
    kx, vx = (rng.standard_normal((B, T, nkv, hd)).astype(np.float32) for _ in range(2))
    qw, kw = (rng.standard_normal(hd).astype(np.float32) for _ in range(2))
    pos = np.arange(T, dtype=np.int32)
    eps, base = 1e-6, 1e6
    dq, dk, dv, dp, dqw, dkw = (_cuda(a) for a in (qx, kx, vx, pos, qw, kw))
    mask_t = None
    if masked:
        mask = np.where(np.arange(T)[None, :] > np.arange(T)[:, None], -np.inf, 0.0).astype(np.float16)
        mask_t = _cuda(mask[None, None])
    # the separate ops: norm x w, rope, attention
    rot = []
    for x, w in ((dq, dqw), (dk, dkw)):
        t = _t().empty_like(x)
        _call(L.mq_op_norm, mq.NORM_RMS, mq.view(x), None, mq.view(t), eps, ctypes.c_void_p(w.data_ptr()), None,
              stream())
        _call(L.mq_op_rope, mq.view(t), mq.view(dp), None, mq.view(t), hd, mq.ROPE_NEOX, 0, base, 1.0, 0.0, 1.0, 0.0,
              0.0, stream())
        rot.append(t)
    scale = 1.0 / np.sqrt(hd)
    want = _t().empty((B, T, nh, hd), dtype=_t().float32, device="cuda")
    mv = mq.view(mask_t) if mask_t is not None else None
    _flash(rot[0].permute(0, 2, 1, 3), rot[1].permute(0, 2, 1, 3), dv.permute(0, 2, 1, 3), mask_t, scale, want)
    # fused
    cs = _t().empty((T, hd), dtype=_t().float32, device="cuda")
    _call(L.mq_op_rope_cache, mq.view(dp), None, hd, 0, base, 1.0, 0.0, 1.0, 0.0, 0.0, ctypes.c_void_p(cs.data_ptr()),
          stream())
    kv = mq.view(dk.permute(0, 2, 1, 3))
    ws_bytes = L.mq_op_flash_attn_workspace_bytes(kv)
    ws = _t().empty(ws_bytes + 256, dtype=_t().uint8, device="cuda")
    wp = ws.data_ptr() + (-ws.data_ptr()) % 256
    got = _t().full((B, T, nh, hd), np.nan, dtype=_t().float32, device="cuda")
    _call(L.mq_op_flash_attn_qk_norm_rope, mq.view(dq.permute(0, 2, 1, 3)), kv, mq.view(dv.permute(0, 2, 1, 3)), mv,
          mq.view(got), scale, ctypes.c_void_p(dqw.data_ptr()), ctypes.c_void_p(dkw.data_ptr()), eps,
          ctypes.c_void_p(cs.data_ptr()), ctypes.c_void_p(wp), ws_bytes, None, 0, stream())
    a, b = host(want), host(got)
    assert np.isfinite(b).all()
    assert np.abs(a - b).max() / np.abs(a).max() <= 2e-5
    # with the output projection's Q8_0 activation: dst bit for bit as without it, the rows
    # bit-identical to the quantizer run on dst (the 8-wave kernel's own store at head_dim <= 64)
    from gpu_util import empty_u8, live_q8_0_planes
    K, M = nh * hd, B * T
    if K % 128 == 0:
        nb = L.mq_workspace_bytes(mq.TYPE_Q8_0, M, K)
        act, ao = empty_u8(nb)
        got2 = _t().full((B, T, nh, hd), np.nan, dtype=_t().float32, device="cuda")
        _call(L.mq_op_flash_attn_qk_norm_rope, mq.view(dq.permute(0, 2, 1, 3)), kv, mq.view(dv.permute(0, 2, 1, 3)),
              mv, mq.view(got2), scale, ctypes.c_void_p(dqw.data_ptr()), ctypes.c_void_p(dkw.data_ptr()), eps,
              ctypes.c_void_p(cs.data_ptr()), ctypes.c_void_p(wp), ws_bytes, ctypes.c_void_p(act.data_ptr() + ao), nb,
              stream())
        assert np.array_equal(host(got2).view(np.uint32), b.view(np.uint32))
        ref_act, ro = empty_u8(nb)
        mq.check(L.mq_quantize_act_ex(mq.TYPE_Q8_0, ctypes.c_void_p(got2.data_ptr()), K, M, K, None, 0,
                                      ctypes.c_void_p(ref_act.data_ptr() + ro), nb, mq.PATH_GEMM, stream()))
        qa, da = live_q8_0_planes(host(ref_act)[ro:ro + nb], M, K)
        qb, db = live_q8_0_planes(host(act)[ao:ao + nb], M, K)
        assert np.array_equal(qa, qb) and np.array_equal(da.view(np.uint32), db.view(np.uint32))
    # q and k must share positions; K/V fragments from elsewhere are refused
    short = mq.view(dk[:, :T - 1].permute(0, 2, 1, 3))
    assert L.mq_op_flash_attn_qk_norm_rope(mq.view(dq.permute(0, 2, 1, 3)), short, short, None, mq.view(got), scale,
                                           ctypes.c_void_p(dqw.data_ptr()), ctypes.c_void_p(dkw.data_ptr()), eps,
                                           ctypes.c_void_p(cs.data_ptr()), ctypes.c_void_p(wp), ws_bytes, None, 0,
                                           stream()) != 0


def test_op_rejections_name_the_problem():
    L = mq.lib()
    x = _t().zeros((4, 48), dtype=_t().float32, device="cuda")
    v = mq.view(x.view(1, 4, 1, 48))
    assert L.mq_op_flash_attn(v, v, v, None, v, 1.0, None, 0, stream()) == -2
    assert b"head_dim" in L.mq_last_error()
    assert L.mq_op_supported(mq.OP_FLASH_ATTN, 0, v, v, v, None, v) == 0
    a, b = mq.view(x), mq.view(_t().zeros((3, 48), dtype=_t().float32, device="cuda"))
    assert L.mq_op_binary(mq.BIN_ADD, a, b, a, stream()) == -2
    assert b"broadcast" in L.mq_last_error()
    assert L.mq_op_supported(mq.OP_BINARY, mq.BIN_ADD, a, a, None, None, a) == 1


# ---------------------------------------------------------------------- rope ----
def _rope_ref(x, pos, n_dims, mode, base, freq_scale=1.0, ext_factor=0.0, attn_factor=1.0, n_ctx_orig=0,
              beta_fast=32.0, beta_slow=1.0, ff=None):
    """x torch-order [B, T, nh, ne0] float32.  Angles by the rope cache's fp32 product chain
    theta_i = p * s * ... * s (i products), YaRN as ggml's rope_yarn; rotation in fp64."""
    half = n_dims // 2
    s = np.float32(np.float32(base) ** np.float32(-2.0 / n_dims))
    th = np.zeros((len(pos), half), np.float32)
    for t, p in enumerate(pos):
        v = np.float32(p)
        for i in range(half):
            th[t, i] = v
            v = np.float32(v * s)
    extrap = th.astype(np.float64) / (1.0 if ff is None else ff[None, :half].astype(np.float64))
    theta = freq_scale * extrap
    msc = attn_factor
    if ext_factor != 0.0:
        def corr(nr):
            return n_dims * np.log(n_ctx_orig / (nr * 2 * np.pi)) / (2 * np.log(base))
        lo, hi = max(0.0, np.floor(corr(beta_fast))), min(n_dims - 1.0, np.ceil(corr(beta_slow)))
        y = (np.arange(half) - lo) / max(0.001, hi - lo)
        mix = (1 - np.clip(y, 0, 1)) * ext_factor
        theta = theta * (1 - mix) + extrap * mix
        msc = attn_factor * (1 + 0.1 * np.log(1.0 / freq_scale))
    c, sn = np.cos(theta) * msc, np.sin(theta) * msc  # [T, half]
    c, sn = c[None, :, None, :], sn[None, :, None, :]
    out = x.astype(np.float64).copy()
    if mode == mq.ROPE_NEOX:
        a, b = x[..., :half].astype(np.float64), x[..., half:n_dims].astype(np.float64)
        out[..., :half], out[..., half:n_dims] = a * c - b * sn, a * sn + b * c
    else:
        a, b = x[..., 0:n_dims:2].astype(np.float64), x[..., 1:n_dims:2].astype(np.float64)
        out[..., 0:n_dims:2], out[..., 1:n_dims:2] = a * c - b * sn, a * sn + b * c
    return out


@pytest.mark.parametrize("mode", [mq.ROPE_NEOX, mq.ROPE_NORMAL])
@pytest.mark.parametrize("case", ["plain", "partial", "yarn", "freq_factors", "offset_pos"])
def test_rope(mode, case):
    L = mq.lib()
    B, T, nh, ne0 = 2, 37, 5, 128
    rng = _rng(30 + mode)
    x = rng.standard_normal((B, T, nh, ne0)).astype(np.float32)
    pos = np.arange(T, dtype=np.int32) + (1000 if case == "offset_pos" else 0)
    n_dims = 64 if case == "partial" else ne0
    kw = dict(base=1e6)
    ff = None
    if case == "yarn":
        kw.update(freq_scale=0.25, ext_factor=1.0, attn_factor=1.0 / (1 + 0.1 * np.log(4.0)), n_ctx_orig=4096,
                  beta_fast=32.0, beta_slow=1.0)
    if case == "freq_factors":
        ff = (1.0 + rng.random(n_dims // 2) * 3).astype(np.float32)
    ref = _rope_ref(x, pos, n_dims, mode, ff=ff, **kw)
    dx, dp = _cuda(x), _cuda(pos)
    out = _t().empty_like(dx)
    fv = mq.view(_cuda(ff)) if ff is not None else None
    _call(L.mq_op_rope, mq.view(dx), mq.view(dp), fv, mq.view(out), n_dims, mode, kw.get("n_ctx_orig", 0),
          kw["base"], kw.get("freq_scale", 1.0), kw.get("ext_factor", 0.0), kw.get("attn_factor", 1.0),
          kw.get("beta_fast", 0.0), kw.get("beta_slow", 0.0), stream())
    got = host(out)
    # device cosf / sinf against fp64 of the same fp32 angles: a few 1e-7
    assert np.abs(got - ref).max() <= 2e-6 * max(1.0, np.abs(ref).max()), np.abs(got - ref).max()
    assert np.array_equal(got[..., n_dims:], x[..., n_dims:])  # dimensions past n_dims copied
    if case == "plain":
        assert np.array_equal(got[:, 0], x[:, 0])  # position 0: cos 1, sin 0
        # in place over x
        _call(L.mq_op_rope, mq.view(dx), mq.view(dp), None, mq.view(dx), n_dims, mode, 0, 1e6, 1.0, 0.0, 1.0, 0.0,
              0.0, stream())
        assert np.array_equal(host(dx), got)


@pytest.mark.parametrize("hd", [64, 128])
def test_flash_attn_causal_mask_one_sequence(attn_form, hd):
    """The decoder graph's attention: one sequence, grouped-query heads, the causal F16 mask
    [T, T] (0 on and below the diagonal, -inf above), whose upper blocks are skipped."""
    nh, nkv, T = 16, 8, 333
    rng = _rng(hd + 5)
    qx = rng.standard_normal((1, T, nh, hd)).astype(np.float32)
    kx, vx = (rng.standard_normal((1, T, nkv, hd)).astype(np.float32) for _ in range(2))
    mask = np.where(np.tril(np.ones((T, T), bool)), 0.0, -np.inf).astype(np.float16)[None, None]
    q, k, v = (_cuda(x).permute(0, 2, 1, 3) for x in (qx, kx, vx))
    out = _t().empty((1, T, nh, hd), dtype=_t().float32, device="cuda")
    scale = 1.0 / np.sqrt(hd)
    _flash(q, k, v, _cuda(mask), scale, out)
    ref = _attn64(qx.transpose(0, 2, 1, 3), kx.transpose(0, 2, 1, 3), vx.transpose(0, 2, 1, 3), mask, scale)
    got = host(out)
    assert np.abs(got - ref).max() / np.abs(ref).max() <= 2e-5
    # closed form: the first query sees only its own key, so it returns that value row
    assert np.allclose(got[0, 0], np.repeat(vx[0, 0], nh // nkv, axis=0), atol=1e-6)


# ------------------------------------------------------- the MoE block's ops ----
@pytest.mark.parametrize("mask", [None, "f16", "f32"])
def test_soft_max(mask):
    L = mq.lib()
    rng = _rng(40)
    x = (rng.standard_normal((3, 17, 70)) * 3).astype(np.float32)
    m = None
    ref_in = x.astype(np.float64) * 0.5
    if mask:
        mv = (rng.standard_normal((1, 20, 70)) * 2).astype(np.float32)
        mv[0, 4, :] = -np.inf  # a fully masked row -> zeros
        mv[0, 6, 10:] = -np.inf
        m = mv.astype(np.float16 if mask == "f16" else np.float32)
        ref_in = ref_in + m[:, :17].astype(np.float64)
    mx = ref_in.max(-1, keepdims=True)
    e = np.exp(ref_in - np.where(np.isfinite(mx), mx, 0))
    den = e.sum(-1, keepdims=True)
    ref = np.where(den > 0, e / np.where(den > 0, den, 1), 0)
    dx = _cuda(x)
    out = _t().empty_like(dx)
    _call(L.mq_op_soft_max, mq.view(dx), mq.view(_cuda(m)) if m is not None else None, mq.view(out), 0.5, stream())
    got = host(out)
    assert np.isfinite(got).all() and np.abs(got - ref).max() <= 1e-6
    if mask:
        assert not got[:, 4].any()


@pytest.mark.parametrize("order", [mq.SORT_DESC, mq.SORT_ASC])
def test_argsort_stable(order):
    L = mq.lib()
    rng = _rng(41)
    x = rng.standard_normal((40, 37)).astype(np.float32)
    x[3, 5:9] = 0.25  # ties keep index order
    x[7] = 1.0
    dx = _cuda(x)
    out = _t().empty((40, 37), dtype=_t().int32, device="cuda")
    _call(L.mq_op_argsort, mq.view(dx), mq.view(out), order, stream())
    key = -x if order == mq.SORT_DESC else x
    ref = np.argsort(key, axis=-1, kind="stable").astype(np.int32)
    assert np.array_equal(host(out), ref)


def test_repeat_and_mul_mat_f32():
    L = mq.lib()
    rng = _rng(42)
    a = rng.standard_normal((5, 1, 64)).astype(np.float32)  # ggml [64, 1, 5]
    out = _t().empty((5, 3, 64), dtype=_t().float32, device="cuda")
    _call(L.mq_op_repeat, mq.view(_cuda(a)), mq.view(out), stream())
    assert np.array_equal(host(out), np.repeat(a, 3, axis=1))
    # the expert mix: [K, 1, T] weights times [K, H, T] expert outputs -> [1, H, T]
    K, H, T = 2, 96, 11
    w = rng.standard_normal((T, 1, K)).astype(np.float32)
    d = rng.standard_normal((T, H, K)).astype(np.float32)
    y = _t().empty((T, H, 1), dtype=_t().float32, device="cuda")
    _call(L.mq_op_mul_mat_f32, mq.view(_cuda(w)), mq.view(_cuda(d)), mq.view(y), stream())
    ref = np.einsum("tik,tjk->tji", w.astype(np.float64), d.astype(np.float64))
    assert np.abs(host(y) - ref).max() <= 1e-5
    # a's batches broadcast over b's (router [H, E] on [H, T] is the 2-D case)
    a2 = rng.standard_normal((2, 8, 33)).astype(np.float32)
    b2 = rng.standard_normal((6, 10, 33)).astype(np.float32)
    y2 = _t().empty((6, 10, 8), dtype=_t().float32, device="cuda")
    _call(L.mq_op_mul_mat_f32, mq.view(_cuda(a2)), mq.view(_cuda(b2)), mq.view(y2), stream())
    ref2 = np.einsum("bik,bjk->bji", np.repeat(a2, 3, axis=0).astype(np.float64), b2.astype(np.float64))
    assert np.abs(host(y2) - ref2).max() <= 1e-5


@pytest.mark.parametrize("case", ["plain", "yarn", "freq_factors"])
def test_rms_norm_rope_equals_separate(case):
    """mq_op_rms_norm_rope (the backend's fusion of a head's RMS_NORM, MUL by the norm weight and
    ROPE, src/decoder_embed.cpp:737-759) against mq_op_norm then mq_op_rope: bit for bit."""
    L = mq.lib()
    B, T, nh, ne0 = 2, 37, 5, 128
    rng = _rng(77)
    x = (rng.standard_normal((B, T, nh, ne0)) * 3.0).astype(np.float32)
    w = (1.0 + 0.1 * rng.standard_normal(ne0)).astype(np.float32)
    pos = (np.arange(T, dtype=np.int32) * 3 + 5).astype(np.int32)
    kw = dict(n_ctx_orig=0, base=1e6, freq_scale=1.0, ext_factor=0.0, attn_factor=1.0, beta_fast=0.0, beta_slow=0.0)
    ff = None
    if case == "yarn":
        kw.update(freq_scale=0.25, ext_factor=1.0, attn_factor=1.0 / (1 + 0.1 * np.log(4.0)), n_ctx_orig=4096,
                  beta_fast=32.0, beta_slow=1.0)
    if case == "freq_factors":
        ff = (1.0 + rng.random(ne0 // 2) * 3).astype(np.float32)
    dx, dp, dw = _cuda(x), _cuda(pos), _cuda(w)
    fv = mq.view(_cuda(ff)) if ff is not None else None
    args = (128, mq.ROPE_NEOX, kw["n_ctx_orig"], kw["base"], kw["freq_scale"], kw["ext_factor"], kw["attn_factor"],
            kw["beta_fast"], kw["beta_slow"])
    tmp, want, got = _t().empty_like(dx), _t().empty_like(dx), _t().empty_like(dx)
    _call(L.mq_op_norm, mq.NORM_RMS, mq.view(dx), None, mq.view(tmp), 1e-6, ctypes.c_void_p(dw.data_ptr()), None,
          stream())
    _call(L.mq_op_rope, mq.view(tmp), mq.view(dp), fv, mq.view(want), *args, stream())
    _call(L.mq_op_rms_norm_rope, mq.view(dx), 1e-6, ctypes.c_void_p(dw.data_ptr()), mq.view(dp), fv, mq.view(got),
          *args, stream())
    assert np.array_equal(host(got).view(np.uint32), host(want).view(np.uint32))
