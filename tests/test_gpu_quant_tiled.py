"""The activation quantization the GEMM actually reads, byte for byte against the oracle.

The batched mul_mat does not read ggml's block_q8_0 / block_q8_K rows: the GEMM-path
quantizer (k_quantize_tiled) and every producer that quantizes its own output for the next
mat-mul (the residual + norm kernels, the attention's Q8_0 store, the FFN-up GEMM's requantizing
epilogue) write the tiled layout of tests/act_layout.py.  Each test here builds the whole
expected workspace from `oracle.quantize_act` -- ggml's quantize_row_q8_0 (three rounding
variants) / quantize_row_q8_K restated -- applied to the fp32 rows the kernel quantized, and
requires every byte of every plane (quants, scales, Q8_K min-term operands, pad rows and pad
K bytes) to be identical.  One flipped quant moves a mul_mat result by ~1e-5 of its range,
below the 1e-4 mul_mat bar, so only this comparison pins the requantization of
LEARNINGS.md:4826-4830 (every MUL_MAT requantizes its F32 src1 to the weight's vec_dot_type).
"""
import ctypes

import numpy as np
import pytest

import act_layout as AL
import oracle_ffi as O
from gpu_util import dev, empty_u8, host, stream, weight_image

pytestmark = pytest.mark.gpu


def _mq():
    from crispembed_amd import mq
    return mq


def _crafted(k):
    """Rows that separate rounding rules and tie-breaks: zeros, exact .5 ties at the scale, the
    largest magnitude first negative then positive, fp16-subnormal scales, a ramp."""
    rows = [np.zeros(k, np.float32)]
    r = np.zeros(k, np.float32)
    r[:32] = np.array([127.0] + [i + 0.5 for i in range(-15, 16)])
    rows += [r, -r]
    r = np.full(k, 1e-6, np.float32)
    r[0] = -2e-6
    rows.append(r)
    rows.append(np.full(k, 3e-8, np.float32))
    r = np.random.default_rng(1).standard_normal(k).astype(np.float32)
    r[17], r[min(200, k - 1)] = -9.0, 9.0  # equal magnitudes: ggml takes the first
    rows.append(r)
    rows.append((np.arange(k) % 256 - 127.0).astype(np.float32))
    rows.append(np.full(k, 1e-30, np.float32))
    return np.stack(rows)


def _rows(m, k, seed):
    x = np.random.default_rng(seed).standard_normal((m, k)).astype(np.float32)
    return np.concatenate([x, _crafted(k)])


def _gemm_ws(wtype, xd, m, k):
    """mq_quantize_act on the GEMM path into a buffer filled with 0xAB: the workspace bytes."""
    mq = _mq()
    L = mq.lib()
    total = AL.planes(wtype, m, k)["total"]
    nb = L.mq_workspace_bytes(wtype, m, k)
    assert nb >= total
    buf, off = empty_u8(nb)
    buf.fill_(0xAB)
    mq.check(L.mq_quantize_act(wtype, ctypes.c_void_p(xd.data_ptr()), xd.stride(0), m, k,
                               ctypes.c_void_p(buf.data_ptr() + off), nb, mq.PATH_GEMM, stream()))
    return host(buf)[off:off + total]


def _assert_image(got, want, wtype, m, k):
    """The quantizer's whole workspace, pad rows and pad K bytes included."""
    diff = AL.first_difference(got, want, wtype, m, k)
    assert diff is None, diff


def _assert_live(got, want, wtype, m, k):
    """What the GEMM reads for the m live rows (producers leave row tiles past them alone)."""
    diff = AL.live_difference(got, want, wtype, m, k)
    assert diff is None, diff


@pytest.fixture
def q8_0_variant():
    """Sets the library's Q8_0 rounding variant for one test and restores it."""
    L = _mq().lib()
    old = L.mq_q8_0_variant()
    yield lambda v: _mq().check(L.mq_set_q8_0_variant(v))
    L.mq_set_q8_0_variant(old)


@pytest.mark.parametrize("variant", [O.Q8_0_X86, O.Q8_0_NEON, O.Q8_0_REF])
@pytest.mark.parametrize("m,k", [(4096, 384), (4096, 1536), (300, 1024), (37, 96), (5, 160)])
def test_q8_0_gemm_layout(oracle, q8_0_variant, variant, m, k):
    """k_quantize_tiled<Q8_0>: cfg1's X [4096 x 384], the MiniLM FFN-down input width, ragged row
    counts and K not a multiple of the 128-byte stage (pad bytes zero)."""
    q8_0_variant(variant)
    x = _rows(m, k, 1000 + k)
    rows = x.shape[0]
    got = _gemm_ws(O.Q8_0, dev(x), rows, k)
    _assert_image(got, AL.oracle_image(oracle, O.Q8_0, x, variant), O.Q8_0, rows, k)


@pytest.mark.parametrize("m,k", [(4096, 384), (300, 1024), (37, 96), (5, 160)])
def test_f16_gemm_layout(oracle, m, k):
    """k_quantize_tiled<F16> (the F16 weights' activation, ggml's F16 vec_dot_type: fp32 -> fp16
    round to nearest even): every byte against the oracle's fp16 rows, with rows of exact fp16
    rounding ties (1 + (2j + 1) 2^-11, halfway between fp16 neighbours, both directions of the
    even rule), fp16 subnormals, values that overflow to inf, and -0."""
    x = _rows(m, k, 3000 + k)
    ties = np.zeros((4, k), np.float32)
    j = np.arange(k) % 64
    ties[0] = 1.0 + (2 * j + 1) * 2.0 ** -11
    ties[1] = -(1.0 + (2 * j + 1) * 2.0 ** -11)
    ties[2] = (j + 0.5) * 2.0 ** -24  # subnormal ties
    ties[3, ::2], ties[3, 1::2] = 70000.0, -0.0
    x = np.concatenate([x, ties])
    rows = x.shape[0]
    got = _gemm_ws(O.F16, dev(x), rows, k)
    _assert_image(got, AL.oracle_image(oracle, O.F16, x), O.F16, rows, k)


@pytest.mark.parametrize("m,k", [(8192, 1024), (8192, 4096), (8192, 3072), (300, 512), (37, 2048)])
def test_q8_K_gemm_layout(oracle, m, k):
    """k_quantize_tiled<Q8_K>: the cfg2a / cfg2b activations X [8192 x 1024] and [8192 x 4096],
    the Qwen3 FFN-down width 3072, ragged rows: quants, d, and the min-term fragments built
    from ggml's bsums."""
    x = _rows(m, k, 2000 + k)
    rows = x.shape[0]
    got = _gemm_ws(O.Q4_K, dev(x), rows, k)
    _assert_image(got, AL.oracle_image(oracle, O.Q4_K, x), O.Q4_K, rows, k)


def test_q8_K_gemm_layout_strided(oracle):
    """A row stride that is not the row length (a view of wider rows), unaligned for float4."""
    m, k, ld = 77, 768, 771
    x = _rows(m, k, 31)
    full = np.zeros((x.shape[0], ld), np.float32)
    full[:, :k] = x
    xd = dev(full)[:, :k]
    got = _gemm_ws(O.Q4_K, xd, x.shape[0], k)
    _assert_image(got, AL.oracle_image(oracle, O.Q4_K, x), O.Q4_K, x.shape[0], k)


@pytest.mark.parametrize("wtype", [O.Q8_0, O.Q4_K])
def test_bias_prologue_gemm_layout(oracle, wtype):
    """The bias prologue of mq_quantize_act_ex: the bytes of x + bias (one fp32 add per value)
    quantized by the oracle."""
    mq = _mq()
    L = mq.lib()
    m, k = 300, 1536
    x = _rows(m, k, 5)
    rows = x.shape[0]
    b = np.random.default_rng(6).standard_normal(k).astype(np.float32)
    nb = L.mq_workspace_bytes(wtype, rows, k)
    buf, off = empty_u8(nb)
    buf.fill_(0xAB)
    xd, bd = dev(x), dev(b)
    mq.check(L.mq_quantize_act_ex(wtype, ctypes.c_void_p(xd.data_ptr()), k, rows, k, ctypes.c_void_p(bd.data_ptr()),
                                  mq.PRE_NONE, ctypes.c_void_p(buf.data_ptr() + off), nb, mq.PATH_GEMM, stream()))
    total = AL.planes(wtype, rows, k)["total"]
    _assert_image(host(buf)[off:off + total], AL.oracle_image(oracle, wtype, (x + b).astype(np.float32)), wtype,
                  rows, k)


@pytest.mark.parametrize("H", [256, 1024, 2048])
@pytest.mark.parametrize("rows", [37, 300, 4101])
def test_norm_q8_K(oracle, H, rows):
    """mq_op_norm_q8_K (k_add_rmsnorm_q8_K, the decoder's residual + RMS norm whose result leaves
    as the Q8_K activation of the q/k/v and gate/up GEMMs): the residual sum bit-exact (one fp32
    add), the normed rows within 5e-6 of an fp64 RMS norm, and the workspace byte-identical to
    the oracle's quantization of those normed rows -- for H = 256, 1024 (Qwen3-0.6B) and 2048
    (Qwen3-VL-2B), i.e. 1, 4 and 8 superblocks per row, with the last row tile partly empty."""
    import torch
    mq = _mq()
    L = mq.lib()
    rng = np.random.default_rng(H + rows)
    x = (rng.standard_normal((rows, H)) * 2).astype(np.float32)
    r = rng.standard_normal((rows, H)).astype(np.float32)
    w = (1 + 0.1 * rng.standard_normal(H)).astype(np.float32)
    eps = 1e-6
    dx, dr, dw = dev(x), dev(r), dev(w)
    dsum = torch.empty_like(dx)
    dnorm = torch.empty_like(dx)
    nb = L.mq_workspace_bytes(O.Q4_K, rows, H)
    ws, off = empty_u8(nb)
    ws.fill_(0xAB)
    mq.check(L.mq_op_norm_q8_K(mq.NORM_RMS, mq.view(dx), mq.view(dr), mq.view(dsum), mq.view(dnorm), eps,
                               ctypes.c_void_p(dw.data_ptr()), ctypes.c_void_p(ws.data_ptr() + off), nb, stream()))
    s = host(dsum)
    assert np.array_equal(s, x + r)
    h = host(dnorm)
    s64 = s.astype(np.float64)
    ref = s64 / np.sqrt((s64 ** 2).mean(-1, keepdims=True) + eps) * w
    assert np.abs(h - ref).max() <= 5e-6 * np.abs(ref).max()
    total = AL.planes(O.Q4_K, rows, H)["total"]
    got = host(ws)[off:off + total]
    _assert_live(got, AL.oracle_image(oracle, O.Q4_K, h), O.Q4_K, rows, H)
    # without the fp32 outputs (the runner's form inside the layer stack): the same bytes
    ws.fill_(0xCD)
    mq.check(L.mq_op_norm_q8_K(mq.NORM_RMS, mq.view(dx), mq.view(dr), None, None, eps,
                               ctypes.c_void_p(dw.data_ptr()), ctypes.c_void_p(ws.data_ptr() + off), nb, stream()))
    _assert_live(host(ws)[off:off + total], got, O.Q4_K, rows, H)


def test_norm_q8_K_refusals():
    mq = _mq()
    L = mq.lib()
    import torch
    x = torch.zeros((4, 384), dtype=torch.float32, device="cuda")
    w = torch.ones(384, dtype=torch.float32, device="cuda")
    ws, off = empty_u8(1 << 20)
    args = (ctypes.c_void_p(w.data_ptr()), ctypes.c_void_p(ws.data_ptr() + off), 1 << 20, stream())
    assert L.mq_op_norm_q8_K(mq.NORM_RMS, mq.view(x), None, None, mq.view(x), 1e-6, *args) == -2  # 384 % 256
    x = torch.zeros((4, 512), dtype=torch.float32, device="cuda")
    assert L.mq_op_norm_q8_K(mq.NORM_LAYER, mq.view(x), None, None, mq.view(x), 1e-6, *args) == -2
    assert L.mq_op_norm_q8_K(mq.NORM_RMS, mq.view(x), None, None, mq.view(x), 1e-6,
                             ctypes.c_void_p(w.data_ptr()), ctypes.c_void_p(ws.data_ptr() + off), 1024, stream()) == -2
    assert b"workspace" in L.mq_last_error()


@pytest.mark.parametrize("variant", [O.Q8_0_X86, O.Q8_0_REF])
@pytest.mark.parametrize("kind,n,rows", [(0, 384, 4096), (0, 1024, 77), (1, 768, 300)])
def test_norm_q8_0_against_oracle(oracle, q8_0_variant, variant, kind, n, rows):
    """mq_op_norm_q8_0 (the encoder's residual + LayerNorm leaving the q/k/v or FFN-up GEMM's
    Q8_0 activation): the workspace equals the oracle's quantization of the norm's own fp32
    result, MiniLM width 384 at 32 x 128 tokens included."""
    import torch
    mq = _mq()
    L = mq.lib()
    q8_0_variant(variant)
    rng = np.random.default_rng(n + rows)
    x = (rng.standard_normal((rows, n)) * 2 + 0.5).astype(np.float32)
    r = rng.standard_normal((rows, n)).astype(np.float32)
    w = rng.standard_normal(n).astype(np.float32)
    b = rng.standard_normal(n).astype(np.float32)
    dx, dr, dw, db = dev(x), dev(r), dev(w), dev(b)
    out = torch.empty_like(dx)
    nb = L.mq_workspace_bytes(O.Q8_0, rows, n)
    ws, off = empty_u8(nb)
    ws.fill_(0xAB)
    mq.check(L.mq_op_norm_q8_0(kind, mq.view(dx), mq.view(dr), mq.view(out), 1e-12 if kind == 0 else 1e-6,
                               ctypes.c_void_p(dw.data_ptr()), ctypes.c_void_p(db.data_ptr()),
                               ctypes.c_void_p(ws.data_ptr() + off), nb, stream()))
    total = AL.planes(O.Q8_0, rows, n)["total"]
    _assert_live(host(ws)[off:off + total], AL.oracle_image(oracle, O.Q8_0, host(out), variant), O.Q8_0, rows, n)


@pytest.mark.parametrize("hd,nh,B,T,masked", [(32, 12, 32, 128, False), (64, 6, 3, 96, True), (128, 2, 2, 64, False)])
def test_flash_attn_q8_0_against_oracle(oracle, hd, nh, B, T, masked):
    """mq_op_flash_attn_q8_0 (the attention storing its rows as the o projection's Q8_0
    activation): the workspace equals the oracle's quantization of the attention's own fp32
    output rows (MiniLM's 12 heads of 32 at 32 x 128 included)."""
    import torch
    mq = _mq()
    L = mq.lib()
    rng = np.random.default_rng(hd + T)
    q, k, v = (torch.from_numpy(rng.standard_normal((B, T, nh, hd)).astype(np.float32)).cuda() for _ in range(3))
    mv = None
    if masked:
        mk = np.zeros((B, 1, T, T), np.float16)
        for b in range(B):
            mk[b, :, :, T - 7 * b:] = -np.inf  # padded keys of shorter items
        mdev = torch.from_numpy(mk).cuda()
        mv = mq.view(mdev)
    perm = lambda t: t.permute(0, 2, 1, 3)  # noqa: E731  ggml [hd, T, nh, B]
    out = torch.empty((B, T, nh, hd), dtype=torch.float32, device="cuda")  # ggml [hd, nh, T, B]
    fb = L.mq_op_flash_attn_workspace_bytes(mq.view(perm(k)))
    fbuf, foff = empty_u8(fb)
    K = nh * hd
    nb = L.mq_workspace_bytes(O.Q8_0, B * T, K)
    ws, off = empty_u8(nb)
    ws.fill_(0xAB)
    mq.check(L.mq_op_flash_attn_q8_0(mq.view(perm(q)), mq.view(perm(k)), mq.view(perm(v)), mv, mq.view(out),
                                     1.0 / np.sqrt(hd), ctypes.c_void_p(fbuf.data_ptr() + foff), fb,
                                     ctypes.c_void_p(ws.data_ptr() + off), nb, stream()))
    rows = host(out).reshape(B * T, K)
    total = AL.planes(O.Q8_0, B * T, K)["total"]
    _assert_live(host(ws)[off:off + total], AL.oracle_image(oracle, O.Q8_0, rows), O.Q8_0, B * T, K)


@pytest.mark.parametrize("wtype", [O.Q8_0, O.Q4_K])
@pytest.mark.parametrize("op", [0, 1])
@pytest.mark.parametrize("m,k,n", [(4096, 384, 1536), (300, 512, 768)])
def test_requant_against_oracle(oracle, wtype, op, m, k, n):
    """mq_mul_mat_q_requant (the FFN-up GEMM storing gelu_erf(y + bias) as the FFN-down GEMM's
    Q8_0 activation, y never written): the workspace equals the oracle's quantization of
    op(y + bias) computed from the plain GEMM's fp32 output y (the bias ADD as one fp32 add;
    GELU-erf as the backend's own GELU_ERF node computes it), at cfg1's FFN-up shape."""
    import torch
    mq = _mq()
    L = mq.lib()
    if wtype == O.Q4_K:
        k = 512
    rng = np.random.default_rng(m + n + op)
    w = (rng.standard_normal((n, k)) * 0.02).astype(np.float32)
    wq = oracle.quantize_chunk(wtype, w)
    img = weight_image(wtype, wq, n, k)
    x = dev(rng.standard_normal((m, k)).astype(np.float32))
    nb1 = L.mq_workspace_bytes(wtype, m, k)
    ws1, o1 = empty_u8(nb1)
    p1 = ctypes.c_void_p(ws1.data_ptr() + o1)
    mq.check(L.mq_quantize_act(wtype, ctypes.c_void_p(x.data_ptr()), k, m, k, p1, nb1, mq.PATH_GEMM, stream()))
    bias = rng.standard_normal(n).astype(np.float32)
    bd = dev(bias)
    y = torch.empty((m, n), dtype=torch.float32, device="cuda")
    mq.check(L.mq_mul_mat_q_ex(wtype, ctypes.c_void_p(img[1]), n, k, p1, m, ctypes.c_void_p(y.data_ptr()), n,
                               ctypes.c_void_p(bd.data_ptr()), mq.PATH_GEMM, stream()))
    v = y
    if op == 1:
        v = torch.empty_like(y)
        mq.check(L.mq_op_unary(mq.UNARY_GELU_ERF, mq.view(y), mq.view(v), stream()))
    nb = L.mq_workspace_bytes(O.Q8_0, m, n)
    ws, off = empty_u8(nb)
    ws.fill_(0xAB)
    mq.check(L.mq_mul_mat_q_requant(wtype, ctypes.c_void_p(img[1]), n, k, p1, m, ctypes.c_void_p(bd.data_ptr()), op,
                                    O.Q8_0, ctypes.c_void_p(ws.data_ptr() + off), nb, stream()))
    total = AL.planes(O.Q8_0, m, n)["total"]
    _assert_live(host(ws)[off:off + total], AL.oracle_image(oracle, O.Q8_0, host(v)), O.Q8_0, m, n)
    del img


@pytest.mark.parametrize("wtype,out_type,op,m,k,n", [
    (O.Q4_K, O.Q4_K, 1, 8192, 1024, 4096),  # the XLM-R-large / BGE-M3 FFN-up at 8192 tokens
    (O.Q4_K, O.Q4_K, 0, 2048, 1024, 4096),
    (O.Q6_K, O.Q6_K, 1, 2048, 512, 4096),
    (O.Q4_K, O.Q6_K, 1, 1060, 512, 8192),   # ragged rows: a last 128-row tile past m_pad
    (O.Q6_K, O.Q4_K, 0, 1060, 256, 8192),
])
def test_requant_q8_k_against_oracle(oracle, wtype, out_type, op, m, k, n):
    """mq_mul_mat_q_requant with a K-quant next product (the FFN-up GEMM storing gelu_erf(y + bias)
    as the FFN-down GEMM's Q8_K activation from its 128 x 256 workgroups, y never written): the
    quants, scales and min-term fragments of every live row equal the oracle's quantize_row_q8_K
    of op(y + bias), y the plain GEMM's fp32 output; and the FFN-down product reads the same
    result from it as from the separate quantizer's workspace."""
    import torch
    mq = _mq()
    L = mq.lib()
    assert L.mq_mul_mat_q_requant_supported(wtype, out_type, m, n) == 1
    rng = np.random.default_rng(m + n + op + 10 * wtype)
    w = (rng.standard_normal((n, k)) * 0.02).astype(np.float32)
    img = weight_image(wtype, oracle.quantize_chunk(wtype, w), n, k)
    x = dev(rng.standard_normal((m, k)).astype(np.float32))
    nb1 = L.mq_workspace_bytes(wtype, m, k)
    ws1, o1 = empty_u8(nb1)
    p1 = ctypes.c_void_p(ws1.data_ptr() + o1)
    mq.check(L.mq_quantize_act(wtype, ctypes.c_void_p(x.data_ptr()), k, m, k, p1, nb1, mq.PATH_GEMM, stream()))
    bias = rng.standard_normal(n).astype(np.float32)
    bd = dev(bias)
    y = torch.empty((m, n), dtype=torch.float32, device="cuda")
    mq.check(L.mq_mul_mat_q_ex(wtype, ctypes.c_void_p(img[1]), n, k, p1, m, ctypes.c_void_p(y.data_ptr()), n,
                               ctypes.c_void_p(bd.data_ptr()), mq.PATH_GEMM, stream()))
    v = y
    if op == 1:
        v = torch.empty_like(y)
        mq.check(L.mq_op_unary(mq.UNARY_GELU_ERF, mq.view(y), mq.view(v), stream()))
    nb = L.mq_workspace_bytes(out_type, m, n)
    ws, off = empty_u8(nb)
    ws.fill_(0xAB)
    pw = ctypes.c_void_p(ws.data_ptr() + off)
    mq.check(L.mq_mul_mat_q_requant(wtype, ctypes.c_void_p(img[1]), n, k, p1, m, ctypes.c_void_p(bd.data_ptr()), op,
                                    out_type, pw, nb, stream()))
    total = AL.planes(out_type, m, n)["total"]
    vh = host(v)
    del y, v
    _assert_live(host(ws)[off:off + total], AL.oracle_image(oracle, out_type, vh), out_type, m, n)
    # the next product (n2 = 256 features) from the fused and from the separate quantizer's workspace
    n2 = 256
    w2 = (rng.standard_normal((n2, n)) * 0.02).astype(np.float32)
    img2 = weight_image(out_type, oracle.quantize_chunk(out_type, w2), n2, n)
    ws3, o3 = empty_u8(nb)
    p3 = ctypes.c_void_p(ws3.data_ptr() + o3)
    vd = dev(vh)
    mq.check(L.mq_quantize_act(out_type, ctypes.c_void_p(vd.data_ptr()), n, m, n, p3, nb, mq.PATH_GEMM, stream()))
    z = [torch.full((m, n2), np.nan, dtype=torch.float32, device="cuda") for _ in range(2)]
    for t, p in zip(z, (pw, p3)):
        mq.check(L.mq_mul_mat_q_ex(out_type, ctypes.c_void_p(img2[1]), n2, n, p, m, ctypes.c_void_p(t.data_ptr()), n2,
                                   None, mq.PATH_GEMM, stream()))
    assert np.array_equal(host(z[0]), host(z[1]))
    del img, img2
