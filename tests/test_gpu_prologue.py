"""Fused activation prologue (mq_quantize_act_ex): the bias ADD and GELU_ERF nodes that feed
the FFN-down MUL_MAT (src/crispembed.cpp:1410-1416) applied inside the activation quantizer.

Bias only: the quantized workspace is byte-identical to quantizing x + bias (one fp32 add
per element, the rounding numpy does), so bit-exactness carries over from the plain
quantizer.  GELU-erf: the device erff may differ from a correctly rounded erf by an ulp,
which can move a quant by one step near a rounding boundary, so the check is the mul_mat
bar (max|dY| / max|Y_ref| <= 1e-4) against the oracle fed gelu(x + bias) computed in fp64
and rounded to fp32, plus >= 99% identical workspace bytes.
"""
import ctypes

import numpy as np
import pytest
from scipy.special import erf

import oracle_ffi as O
from ggml_numpy import rel_err
from gpu_util import dev, empty_u8, host, live_q8_0_planes, stream, weight_image

pytestmark = pytest.mark.gpu

TOL = 1e-4
TYPES = [O.Q8_0, O.Q4_K, O.Q6_K, O.F16]


def _quant(wtype, x_dev, m, k, path, bias_dev=None, op=0):
    from crispembed_amd import mq
    L = mq.lib()
    nb = L.mq_workspace_bytes(wtype, m, k)
    buf, off = empty_u8(nb)
    buf.zero_()
    ptr = buf.data_ptr() + off
    bias = ctypes.c_void_p(bias_dev.data_ptr()) if bias_dev is not None else None
    mq.check(L.mq_quantize_act_ex(wtype, ctypes.c_void_p(x_dev.data_ptr()), x_dev.stride(0), m, k, bias, op,
                                  ctypes.c_void_p(ptr), nb, path, stream()))
    return buf, ptr, host(buf)[off:off + nb]


def _gelu_ref(t32):
    t = t32.astype(np.float64)
    return (0.5 * t * (1.0 + erf(t / np.sqrt(2.0)))).astype(np.float32)


def _inputs(m, k, ld, seed):
    rng = np.random.default_rng(seed)
    x = (rng.standard_normal((m, k)) * 2.0).astype(np.float32)
    b = rng.standard_normal(k).astype(np.float32)
    full = np.zeros((m, ld), np.float32)
    full[:, :k] = x
    return x, b, dev(full)[:, :k]


@pytest.mark.parametrize("wtype", TYPES)
@pytest.mark.parametrize("m,k,ld,path", [(5, 1536, 1536, 1), (8, 512, 520, 1), (37, 1536, 1536, 2),
                                         (300, 512, 516, 2)])
def test_bias_prologue_bit_exact(wtype, m, k, ld, path):
    x, b, xd = _inputs(m, k, ld, 11 * m + k)
    _, _, got = _quant(wtype, xd, m, k, path, dev(b), 0)
    _, _, want = _quant(wtype, dev((x + b).astype(np.float32)), m, k, path)
    assert np.array_equal(got, want)


@pytest.mark.parametrize("wtype", TYPES)
@pytest.mark.parametrize("m,n,k,ld,path", [(3, 70, 1536, 1536, 1), (8, 33, 512, 520, 1), (64, 96, 1536, 1536, 2),
                                           (129, 70, 512, 516, 2)])
def test_gelu_prologue_mul_mat(oracle, wtype, m, n, k, ld, path):
    from crispembed_amd import mq
    import torch
    x, b, xd = _inputs(m, k, ld, 7 * m + n + k)
    xg = _gelu_ref((x + b).astype(np.float32))
    keep, ws, got = _quant(wtype, xd, m, k, path, dev(b), 1)  # keep: the workspace read by mq_mul_mat_q
    _, _, want = _quant(wtype, dev(xg), m, k, path)
    same = np.mean(got == want)
    assert same >= 0.99, same
    wf = (np.random.default_rng(n).standard_normal((n, k)) * 0.02).astype(np.float32)
    w = oracle.quantize_chunk(wtype, wf)
    _, wp = weight_image(wtype, w, n, k)
    y = torch.empty((m, n), dtype=torch.float32, device="cuda")
    mq.check(mq.lib().mq_mul_mat_q(wtype, ctypes.c_void_p(wp), n, k, ctypes.c_void_p(ws), m,
                                   ctypes.c_void_p(y.data_ptr()), n, path, stream()))
    y = host(y)
    xq = oracle.quantize_act(wtype, xg)
    e1 = rel_err(y, oracle.mul_mat_exact(wtype, w, xq, k))
    e2 = rel_err(y, oracle.mul_mat_q(wtype, w, xq, k))
    assert e1 <= TOL and e2 <= TOL, (e1, e2, same)



@pytest.mark.parametrize("wtype", TYPES)
@pytest.mark.parametrize("m,n,k,path", [(1, 300, 512, 1), (6, 70, 1536, 1), (19, 70, 1536, 1), (77, 96, 512, 2),
                                        (300, 200, 1536, 2)])
def test_mul_mat_q_ex_bias_in_store(wtype, m, n, k, path):
    """mq_mul_mat_q_ex adds the bias as the GEMM / GEMV stores each row: bit-identical to the
    plain mat-mul followed by one fp32 add per element (the graph's ADD node)."""
    import torch
    from crispembed_amd import mq
    L = mq.lib()
    rng = np.random.default_rng(m * 7 + n + k + wtype)
    w = rng.standard_normal((n, k)).astype(np.float32)
    wq = np.ascontiguousarray(mq_quantized(wtype, w))
    _, wptr = img = weight_image(wtype, wq, n, k)
    x = dev(rng.standard_normal((m, k)).astype(np.float32))
    bias = rng.standard_normal(n).astype(np.float32)
    _, ptr, _ = ws = _quant(wtype, x, m, k, path)
    y0 = torch.full((m, n + 3), np.nan, dtype=torch.float32, device="cuda")
    y1 = torch.full((m, n + 3), np.nan, dtype=torch.float32, device="cuda")
    mq.check(L.mq_mul_mat_q(wtype, ctypes.c_void_p(wptr), n, k, ctypes.c_void_p(ptr), m, ctypes.c_void_p(y0.data_ptr()),
                            n + 3, path, stream()))
    bd = dev(bias)
    mq.check(L.mq_mul_mat_q_ex(wtype, ctypes.c_void_p(wptr), n, k, ctypes.c_void_p(ptr), m,
                               ctypes.c_void_p(y1.data_ptr()), n + 3, ctypes.c_void_p(bd.data_ptr()), path, stream()))
    a, b = host(y0), host(y1)
    assert np.array_equal(b[:, :n], a[:, :n] + bias)
    assert np.isnan(b[:, n:]).all()
    del img, ws


def mq_quantized(wtype, w):
    from crispembed_amd import mq
    L = mq.lib()
    n, k = w.shape
    out = np.zeros(L.mq_gguf_bytes(wtype, n, k), dtype=np.uint8)
    L.mq_quantize_chunk(wtype, w.ctypes.data, out.ctypes.data, n, k)
    return out


@pytest.mark.parametrize("wtype", TYPES)
@pytest.mark.parametrize("m,k,path", [(5, 512, 1), (21, 512, 1), (300, 512, 2), (4096, 256, 2)])
def test_mul_mat_q_group_equals_separate(wtype, m, k, path):
    """mq_mul_mat_q_group (one launch over the feature tiles of every weight) against one
    mq_mul_mat_q_ex per weight: bit-identical, with ragged n, per-group biases (one absent)
    and output strides."""
    import torch
    from crispembed_amd import mq
    L = mq.lib()
    rng = np.random.default_rng(m + k + wtype)
    ns = [384, 100, 37]
    imgs, wps = [], []
    for n in ns:
        w = rng.standard_normal((n, k)).astype(np.float32)
        img = weight_image(wtype, np.ascontiguousarray(mq_quantized(wtype, w)), n, k)
        imgs.append(img)
        wps.append(img[1])
    x = dev(rng.standard_normal((m, k)).astype(np.float32))
    _, ptr, _ = ws = _quant(wtype, x, m, k, path)
    biases = [dev(rng.standard_normal(n).astype(np.float32)) for n in ns]
    bptr = [biases[0].data_ptr(), None, biases[2].data_ptr()]
    lds = [n + 5 for n in ns]
    ref = [torch.full((m, ld), np.nan, dtype=torch.float32, device="cuda") for ld in lds]
    got = [torch.full((m, ld), np.nan, dtype=torch.float32, device="cuda") for ld in lds]
    for g, n in enumerate(ns):
        mq.check(L.mq_mul_mat_q_ex(wtype, ctypes.c_void_p(wps[g]), n, k, ctypes.c_void_p(ptr), m,
                                   ctypes.c_void_p(ref[g].data_ptr()), lds[g], bptr[g], path, stream()))
    VP = ctypes.c_void_p * 3
    I64 = ctypes.c_int64 * 3
    mq.check(L.mq_mul_mat_q_group(wtype, 3, VP(*wps), I64(*ns), k, ctypes.c_void_p(ptr), m,
                                  VP(*[t.data_ptr() for t in got]), I64(*lds), VP(*bptr), path, stream()))
    for g, n in enumerate(ns):
        a, b = host(ref[g]), host(got[g])
        assert np.array_equal(a[:, :n], b[:, :n]), g
        assert np.isnan(b[:, n:]).all()
    del imgs, ws


@pytest.mark.parametrize("wtype", TYPES)
@pytest.mark.parametrize("m,k,n,op,with_bias", [(37, 512, 384, 1, True), (300, 384, 1536, 1, True),
                                                (1000, 512, 512, 0, False), (4096, 384, 1536, 1, True),
                                                (520, 256, 256, 0, True)])
def test_mul_mat_q_requant_equals_separate(wtype, m, k, n, op, with_bias):
    """mq_mul_mat_q_requant (the GEMM quantizing its own output for the next mat-mul) against the
    GEMM's fp32 output quantized by mq_quantize_act_ex with the same bias and op: the quants and
    scales of every row are bit-identical, and so is the next Q8_0 mat-mul read from either."""
    import torch
    from crispembed_amd import mq
    L = mq.lib()
    if wtype in (O.Q4_K, O.Q6_K) and k % 256:
        k = 512  # K-quant rows are whole 256-value superblocks
    rng = np.random.default_rng(7 * m + n + wtype)
    w = rng.standard_normal((n, k)).astype(np.float32)
    img = weight_image(wtype, np.ascontiguousarray(mq_quantized(wtype, w)), n, k)
    n2 = 200
    w2 = rng.standard_normal((n2, n)).astype(np.float32)
    img2 = weight_image(O.Q8_0, np.ascontiguousarray(mq_quantized(O.Q8_0, w2)), n2, n)
    x = dev(rng.standard_normal((m, k)).astype(np.float32))
    _, ptr, _ = ws = _quant(wtype, x, m, k, 2)
    bias = dev(rng.standard_normal(n).astype(np.float32)) if with_bias else None
    bptr = ctypes.c_void_p(bias.data_ptr()) if with_bias else None
    # separate: fp32 GEMM output, then the quantizer with the bias and op
    y = torch.empty((m, n), dtype=torch.float32, device="cuda")
    mq.check(L.mq_mul_mat_q_ex(wtype, ctypes.c_void_p(img[1]), n, k, ctypes.c_void_p(ptr), m,
                               ctypes.c_void_p(y.data_ptr()), n, None, 2, stream()))
    ref_buf, ref_ptr, ref_raw = _quant(O.Q8_0, y, m, n, 2, bias, op)
    # fused, into a workspace filled with garbage
    nb = L.mq_workspace_bytes(O.Q8_0, m, n)
    out, off = empty_u8(nb)
    out.fill_(0xAB)
    optr = out.data_ptr() + off
    mq.check(L.mq_mul_mat_q_requant(wtype, ctypes.c_void_p(img[1]), n, k, ctypes.c_void_p(ptr), m, bptr, op,
                                    O.Q8_0, ctypes.c_void_p(optr), nb, stream()))
    got_raw = host(out)[off:off + nb]
    qa, da = live_q8_0_planes(ref_raw, m, n)
    qb, db = live_q8_0_planes(got_raw, m, n)
    assert np.array_equal(qa, qb)
    assert np.array_equal(da.view(np.uint32), db.view(np.uint32))
    # the next mat-mul reads either workspace to the same result
    z = [torch.full((m, n2), np.nan, dtype=torch.float32, device="cuda") for _ in range(2)]
    for t, p in zip(z, (ref_ptr, optr)):
        mq.check(L.mq_mul_mat_q_ex(O.Q8_0, ctypes.c_void_p(img2[1]), n2, n, ctypes.c_void_p(p), m,
                                   ctypes.c_void_p(t.data_ptr()), n2, None, 2, stream()))
    assert np.array_equal(host(z[0]), host(z[1]))
    del img, img2, ws, ref_buf


@pytest.mark.parametrize("variant", [1, 2])
def test_mul_mat_q_requant_variants(variant):
    """The NEON and reference rounding variants of the Q8_0 quantizer carry over to the GEMM's
    quantized output (bit-identical planes)."""
    import torch
    from crispembed_amd import mq
    L = mq.lib()
    old = L.mq_q8_0_variant()
    L.mq_set_q8_0_variant(variant)
    try:
        m, k, n, wtype = 700, 512, 768, O.Q8_0
        rng = np.random.default_rng(variant)
        w = rng.standard_normal((n, k)).astype(np.float32)
        img = weight_image(wtype, np.ascontiguousarray(mq_quantized(wtype, w)), n, k)
        x = dev(rng.standard_normal((m, k)).astype(np.float32))
        _, ptr, _ = ws = _quant(wtype, x, m, k, 2)
        bias = dev(rng.standard_normal(n).astype(np.float32))
        y = torch.empty((m, n), dtype=torch.float32, device="cuda")
        mq.check(L.mq_mul_mat_q_ex(wtype, ctypes.c_void_p(img[1]), n, k, ctypes.c_void_p(ptr), m,
                                   ctypes.c_void_p(y.data_ptr()), n, None, 2, stream()))
        _, _, ref_raw = _quant(O.Q8_0, y, m, n, 2, bias, 1)
        nb = L.mq_workspace_bytes(O.Q8_0, m, n)
        out, off = empty_u8(nb)
        out.fill_(0xAB)
        mq.check(L.mq_mul_mat_q_requant(wtype, ctypes.c_void_p(img[1]), n, k, ctypes.c_void_p(ptr), m,
                                        ctypes.c_void_p(bias.data_ptr()), 1, O.Q8_0,
                                        ctypes.c_void_p(out.data_ptr() + off), nb, stream()))
        got_raw = host(out)[off:off + nb]
        qa, da = live_q8_0_planes(ref_raw, m, n)
        qb, db = live_q8_0_planes(got_raw, m, n)
        assert np.array_equal(qa, qb)
        assert np.array_equal(da.view(np.uint32), db.view(np.uint32))
        del img, ws
    finally:
        L.mq_set_q8_0_variant(old)


@pytest.mark.parametrize("wtype", [O.Q8_0, O.Q4_K])
@pytest.mark.parametrize("hd,nh,B,T", [(32, 12, 4, 64), (64, 4, 3, 96), (128, 2, 2, 32)])
def test_qkv_fragments_equal_kv_pass(wtype, hd, nh, B, T):
    """mq_mul_mat_q_qkv (k and v stored by the GEMM as attention fragments) + mq_op_flash_attn_ex
    with MQ_ATTN_KV_READY against mq_mul_mat_q_group + mq_op_flash_attn (the K/V pass): q and the
    attention output bit-identical."""
    import torch
    from crispembed_amd import mq
    L = mq.lib()
    H = nh * hd
    k = 512  # whole K-quant superblocks
    m = B * T
    rng = np.random.default_rng(hd + T + wtype)
    imgs, wps = [], []
    for _ in range(3):
        w = (rng.standard_normal((H, k)) * 0.05).astype(np.float32)
        img = weight_image(wtype, np.ascontiguousarray(mq_quantized(wtype, w)), H, k)
        imgs.append(img)
        wps.append(img[1])
    x = dev(rng.standard_normal((m, k)).astype(np.float32))
    _, ptr, _ = ws = _quant(wtype, x, m, k, 2)
    biases = [dev(rng.standard_normal(H).astype(np.float32)) for _ in range(3)]
    VP, I64 = ctypes.c_void_p * 3, ctypes.c_int64 * 3
    ys = [torch.empty((m, H), dtype=torch.float32, device="cuda") for _ in range(3)]
    mq.check(L.mq_mul_mat_q_group(wtype, 3, VP(*wps), I64(H, H, H), k, ctypes.c_void_p(ptr), m,
                                  VP(*[t.data_ptr() for t in ys]), I64(H, H, H), VP(*[b.data_ptr() for b in biases]),
                                  2, stream()))

    def views(t):  # ggml [hd, T, nh, B] over rows of H floats
        return t.view(B, T, nh, hd).permute(0, 2, 1, 3)
    qv, kv, vv = (mq.view(views(t)) for t in ys)
    fb = L.mq_op_flash_attn_workspace_bytes(kv)
    f1, o1 = empty_u8(fb)
    out1 = torch.empty((B, T, nh, hd), dtype=torch.float32, device="cuda")
    mq.check(L.mq_op_flash_attn(qv, kv, vv, None, mq.view(out1), 1.0 / np.sqrt(hd),
                                ctypes.c_void_p(f1.data_ptr() + o1), fb, stream()))
    yq = torch.full((m, H), np.nan, dtype=torch.float32, device="cuda")
    f2, o2 = empty_u8(fb)
    mq.check(L.mq_mul_mat_q_qkv(wtype, VP(*wps), I64(H, H, H), k, ctypes.c_void_p(ptr), m,
                                ctypes.c_void_p(yq.data_ptr()), H, VP(*[b.data_ptr() for b in biases]), T, hd, nh,
                                ctypes.c_void_p(f2.data_ptr() + o2), fb, stream()))
    assert np.array_equal(host(yq), host(ys[0]))
    assert np.array_equal(host(f2)[o2:o2 + fb], host(f1)[o1:o1 + fb])
    out2 = torch.full((B, T, nh, hd), np.nan, dtype=torch.float32, device="cuda")
    mq.check(L.mq_op_flash_attn_ex(mq.view(views(yq)), kv, vv, None, mq.view(out2), 1.0 / np.sqrt(hd),
                                   ctypes.c_void_p(f2.data_ptr() + o2), fb, None, 0, mq.ATTN_KV_READY, stream()))
    assert np.array_equal(host(out2), host(out1))
    del imgs, ws


def _silu_mul(g, u):
    g = g.astype(np.float32)
    return ((g / (np.float32(1.0) + np.exp(-g))) * u).astype(np.float32)


@pytest.mark.parametrize("wtype", TYPES)
@pytest.mark.parametrize("m,n_ff,k,cfg", [(4096, 1024, 512, ""), (4000, 1536, 256, ""), (2048, 2048, 512, "3")])
def test_mul_mat_q_swiglu_equals_two_step(oracle, wtype, m, n_ff, k, cfg, monkeypatch):
    """mq_mul_mat_q_swiglu (silu(gate) * up formed in the gate|up GEMM's store) against the
    two-step form of the decoder FFN (src/decoder_embed.cpp:793-802): the gate|up product by
    mq_mul_mat_q_ex, then the quantizer's MQ_PRE_SILU_MUL prologue.  The down projection's
    quantized activation is byte-identical whichever form made it; the fp32 product equals
    silu(g) * u of the GEMM's own gate and up to the last bits (device expf), with the columns
    past n_ff untouched; sampled rows match the oracle's gate and up products at the mul_mat
    bar.  cfg "3" forces the 128x128 workgroups (the other large-grid configuration)."""
    import torch
    from crispembed_amd import mq
    L = mq.lib()
    if k % 256 and wtype in (O.Q4_K, O.Q6_K):
        pytest.skip("K-quant rows are whole superblocks")
    if cfg:
        monkeypatch.setenv("MQ_GEMM_CFG", cfg)
    rng = np.random.default_rng(m + n_ff + k + wtype)
    wf = (rng.standard_normal((2 * n_ff, k)) * 0.05).astype(np.float32)  # gate rows, then up rows
    w = oracle.quantize_chunk(wtype, wf)
    _, wp = img = weight_image(wtype, w, 2 * n_ff, k)
    x = rng.standard_normal((m, k)).astype(np.float32)
    keep, ptr, _ = _quant(wtype, dev(x), m, k, 2)
    # two-step
    gu = torch.empty((m, 2 * n_ff), dtype=torch.float32, device="cuda")
    mq.check(L.mq_mul_mat_q_ex(wtype, ctypes.c_void_p(wp), 2 * n_ff, k, ctypes.c_void_p(ptr), m,
                               ctypes.c_void_p(gu.data_ptr()), 2 * n_ff, None, 2, stream()))
    _, _, want = _quant(wtype, gu, m, n_ff, 2, None, mq.PRE_SILU_MUL)
    # fused, into an output with padding columns
    y = torch.full((m, n_ff + 8), np.nan, dtype=torch.float32, device="cuda")
    mq.check(L.mq_mul_mat_q_swiglu(wtype, ctypes.c_void_p(wp), n_ff, k, ctypes.c_void_p(ptr), m,
                                   ctypes.c_void_p(y.data_ptr()), n_ff + 8, stream()))
    _, _, got = _quant(wtype, y[:, :n_ff], m, n_ff, 2)
    assert np.array_equal(got, want)
    yh, guh = host(y), host(gu)
    assert np.isnan(yh[:, n_ff:]).all()
    ref = _silu_mul(guh[:, :n_ff], guh[:, n_ff:])
    np.testing.assert_allclose(yh[:, :n_ff], ref, rtol=2e-6, atol=1e-30)
    rows = np.unique(np.concatenate([np.arange(0, m, 61), [m - 1]]))
    xq = oracle.quantize_act(wtype, np.ascontiguousarray(x[rows]))
    yo = oracle.mul_mat_q(wtype, w, xq, k)
    assert rel_err(yh[rows, :n_ff], _silu_mul(yo[:, :n_ff], yo[:, n_ff:])) <= TOL
    del img, keep


@pytest.mark.parametrize("m,n_ff", [(1000, 1024), (4096, 1000), (8, 3072)])
def test_mul_mat_q_swiglu_unsupported_shapes(m, n_ff):
    """Shapes the fused form does not take (fewer than 512 tiles of 128x128, n_ff not a multiple
    of 64) are refused with MQ_EUNSUPPORTED before anything is launched."""
    import torch
    from crispembed_amd import mq
    L = mq.lib()
    k = 256
    w = np.zeros(L.mq_gguf_bytes(O.Q8_0, 2 * n_ff, k), dtype=np.uint8)
    _, wp = img = weight_image(O.Q8_0, w, 2 * n_ff, k)
    keep, ptr, _ = _quant(O.Q8_0, dev(np.ones((m, k), np.float32)), m, k, 2)
    y = torch.full((m, n_ff), np.nan, dtype=torch.float32, device="cuda")
    rc = L.mq_mul_mat_q_swiglu(O.Q8_0, ctypes.c_void_p(wp), n_ff, k, ctypes.c_void_p(ptr), m,
                               ctypes.c_void_p(y.data_ptr()), n_ff, stream())
    assert rc == -2, rc
    assert np.isnan(host(y)).all()
    del img, keep


@pytest.mark.parametrize("wtype", TYPES)
@pytest.mark.parametrize("m,k,ld,gap,path", [(5, 1536, 1536, 0, 1), (8, 512, 516, 3, 1), (300, 512, 512, 0, 2),
                                             (37, 1536, 1540, 1, 2)])
def test_silu_mul_separate_tensors_bit_exact(wtype, m, k, ld, gap, path):
    """mq_quantize_act_silu_mul (gate and up in two tensors of one row stride, the backend's
    fusion of the SILU and MUL nodes into the down MUL_MAT's quantizer) writes the bytes that
    mq_quantize_act_ex(MQ_PRE_SILU_MUL) writes for the same values side by side; gap (floats
    between the two tensors) makes their distance unaligned to 16 bytes (the scalar-load form)."""
    import torch
    from crispembed_amd import mq
    L = mq.lib()
    rng = np.random.default_rng(m + k + ld + gap + wtype)
    g = (rng.standard_normal((m, k)) * 2.0).astype(np.float32)
    u = rng.standard_normal((m, k)).astype(np.float32)
    side = dev(np.concatenate([g, u], axis=1))
    _, _, want = _quant(wtype, side, m, k, path, None, mq.PRE_SILU_MUL)
    buf = torch.full((2 * m * ld + gap + 64,), np.nan, dtype=torch.float32, device="cuda")
    gv = buf[:m * ld].view(m, ld)
    uv = buf[m * ld + gap:m * ld + gap + m * ld].view(m, ld)
    gv[:, :k] = torch.from_numpy(g).cuda()
    uv[:, :k] = torch.from_numpy(u).cuda()
    nb = L.mq_workspace_bytes(wtype, m, k)
    ws, off = empty_u8(nb)
    ws.zero_()
    mq.check(L.mq_quantize_act_silu_mul(wtype, ctypes.c_void_p(gv.data_ptr()), ctypes.c_void_p(uv.data_ptr()), ld, m,
                                        k, ctypes.c_void_p(ws.data_ptr() + off), nb, path, stream()))
    got = host(ws)[off:off + nb]
    assert np.array_equal(got, want)
