"""The M <= 8 GEMV at the Qwen3-VL-2B text-decoder shapes of the decode step
(src/qwen2vl_ocr.cpp:2368-2452: q/k/v, o, gate/up, down and the lm_head for one to eight
activation rows), against the oracle's exact product of the quantized operands.

The K-quant GEMV is a persistent kernel: each workgroup walks 16-row tiles t, t + grid, ...
with the weight loads of the next tiles in flight.  At these shapes a workgroup owns many
tiles (the lm_head's 9496 tiles on 512 workgroups, ~18.5 each), and a grouped launch walks the
concatenated tiles of several weights, so a tile of one weight can follow a tile of another
inside one workgroup.  Each test states the tiles per workgroup it exercises (the launch
policy: min(tiles, CUs x 2) workgroups at one cached superblock per wave, i.e. K <= 2048,
CUs x 1 beyond; MQ_GEMV_WGS=1 caps it at one workgroup per CU) and checks that it is > 1.

Weights are random GGUF blocks (every nibble, 6-bit scale and sign pattern occurs; d and dmin
are bounded so the outputs stay finite) rather than quantized rows tiled, so a tile read from
the wrong place cannot match by repetition.
"""
import ctypes

import numpy as np
import pytest

import oracle_ffi as O
from ggml_numpy import rel_err
from gpu_util import dev, empty_u8, host, stream, weight_image

pytestmark = pytest.mark.gpu

TOL = 1e-4


def random_blocks(wtype, n, k, seed):
    """n rows of k values as random, valid GGUF blocks of wtype."""
    rng = np.random.default_rng(seed)
    nb = n * (k // 256)
    if wtype == O.Q4_K:
        b = rng.integers(0, 256, size=(nb, 144), dtype=np.uint8)
        d = (rng.uniform(0.5, 1.5, nb) * 2e-5).astype(np.float16)
        dmin = (rng.uniform(0.0, 1.0, nb) * 2e-5).astype(np.float16)
        b[:, 0:2] = d.view(np.uint8).reshape(nb, 2)
        b[:, 2:4] = dmin.view(np.uint8).reshape(nb, 2)
    else:
        b = rng.integers(0, 256, size=(nb, 210), dtype=np.uint8)
        d = (rng.choice([-1.0, 1.0], nb) * rng.uniform(0.5, 1.5, nb) * 2e-5).astype(np.float16)
        b[:, 208:210] = d.view(np.uint8).reshape(nb, 2)
    return b.reshape(n, -1)


def _cus():
    import torch
    return torch.cuda.get_device_properties(0).multi_processor_count


def tiles_per_wg(n_total, k, wgs_per_cu=None):
    ntiles = -(-n_total // 16)
    per_cu = wgs_per_cu or (2 if k <= 2048 else 1)
    return ntiles / min(ntiles, _cus() * per_cu)


def _quant(wtype, x, m, k):
    from crispembed_amd import mq
    L = mq.lib()
    nb = L.mq_workspace_bytes(wtype, m, k)
    buf, off = empty_u8(nb)
    mq.check(L.mq_quantize_act(wtype, ctypes.c_void_p(x.data_ptr()), k, m, k, ctypes.c_void_p(buf.data_ptr() + off),
                               nb, mq.PATH_GEMV, stream()))
    return buf, buf.data_ptr() + off


@pytest.fixture(scope="module")
def lm_head(oracle):
    n, k = 151936, 2048
    w = random_blocks(O.Q6_K, n, k, 151936)
    img = weight_image(O.Q6_K, w, n, k)
    yield w, img, n, k
    del img


@pytest.mark.parametrize("m", [1, 2, 4, 8])
def test_lm_head_q6_K(oracle, lm_head, m):
    """The Q6_K lm_head [151936 x 2048] (src/qwen2vl_ocr.cpp:2452) at m = 1, 2, 4, 8."""
    import torch
    from crispembed_amd import mq
    w, img, n, k = lm_head
    assert tiles_per_wg(n, k) > 18
    x = np.random.default_rng(m).standard_normal((m, k)).astype(np.float32)
    xd = dev(x)
    keep, ws = _quant(O.Q6_K, xd, m, k)
    y = torch.full((m, n + 1), np.nan, dtype=torch.float32, device="cuda")
    mq.check(mq.lib().mq_mul_mat_q(O.Q6_K, ctypes.c_void_p(img[1]), n, k, ctypes.c_void_p(ws), m,
                                   ctypes.c_void_p(y.data_ptr()), n + 1, mq.PATH_GEMV, stream()))
    got = host(y)
    assert np.isnan(got[:, n]).all()
    got = got[:, :n]
    xq = oracle.quantize_act(O.Q6_K, x)
    assert rel_err(got, oracle.mul_mat_exact(O.Q6_K, w, xq, k)) <= TOL
    # every row tile: the largest error of any 16-row tile against its own scale
    ref = oracle.mul_mat_exact(O.Q6_K, w, xq, k)
    per_tile = np.abs(got - ref).reshape(m, -1, 16).max(-1) / np.abs(ref).max()
    assert per_tile.max() <= TOL


def _group_check(oracle, monkeypatch, wtype, ns, k, m, wgs):
    import torch
    from crispembed_amd import mq
    L = mq.lib()
    if wgs:
        monkeypatch.setenv("MQ_GEMV_WGS", str(wgs))
    else:
        monkeypatch.delenv("MQ_GEMV_WGS", raising=False)
    ws_ = [random_blocks(wtype, n, k, 17 * n + g + k) for g, n in enumerate(ns)]
    imgs = [weight_image(wtype, w, n, k) for w, n in zip(ws_, ns)]
    x = np.random.default_rng(m + k).standard_normal((m, k)).astype(np.float32)
    keep, ws = _quant(wtype, dev(x), m, k)
    g = len(ns)
    bias = [dev(np.random.default_rng(n).standard_normal(n).astype(np.float32)) for n in ns]
    sep = [torch.full((m, n), np.nan, dtype=torch.float32, device="cuda") for n in ns]
    grp = [torch.full((m, n), np.nan, dtype=torch.float32, device="cuda") for n in ns]
    for i, n in enumerate(ns):
        mq.check(L.mq_mul_mat_q_ex(wtype, ctypes.c_void_p(imgs[i][1]), n, k, ctypes.c_void_p(ws), m,
                                   ctypes.c_void_p(sep[i].data_ptr()), n, ctypes.c_void_p(bias[i].data_ptr()),
                                   mq.PATH_GEMV, stream()))
    VP, I64 = ctypes.c_void_p * g, ctypes.c_int64 * g
    mq.check(L.mq_mul_mat_q_group(wtype, g, VP(*[im[1] for im in imgs]), I64(*ns), k, ctypes.c_void_p(ws), m,
                                  VP(*[t.data_ptr() for t in grp]), I64(*ns), VP(*[b.data_ptr() for b in bias]),
                                  mq.PATH_GEMV, stream()))
    xq = oracle.quantize_act(wtype, x)
    for i, n in enumerate(ns):
        a, b = host(sep[i]), host(grp[i])
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), i
        ref = oracle.mul_mat_exact(wtype, ws_[i], xq, k) + host(bias[i]).astype(np.float64)
        assert rel_err(b, ref) <= TOL, i
    del imgs, keep


@pytest.mark.parametrize("wtype", [O.Q4_K, O.Q6_K])
@pytest.mark.parametrize("m", [1, 8])
@pytest.mark.parametrize("wgs", [None, 1])
def test_group_ring_steady_state(oracle, monkeypatch, wtype, m, wgs):
    """Three weights [4096, 4096, 1024] x 2048 as one grouped launch, with the default grid and
    with one workgroup per CU: bit-identical to one launch per weight, and within the bar of
    the oracle's exact product (with each weight's bias)."""
    ns = [4096, 4096, 1024]
    assert tiles_per_wg(sum(ns), 2048, wgs) > 1
    _group_check(oracle, monkeypatch, wtype, ns, 2048, m, wgs)


@pytest.mark.parametrize("m", [1, 2, 4, 8])
def test_qwen3vl_gate_up(oracle, monkeypatch, m):
    """gate | up, 2 x [6144 x 2048] Q4_K (src/qwen2vl_ocr.cpp:2437-2438): 768 tiles."""
    assert tiles_per_wg(2 * 6144, 2048) > 1
    _group_check(oracle, monkeypatch, O.Q4_K, [6144, 6144], 2048, m, None)


@pytest.mark.parametrize("m", [1, 8])
def test_qwen3vl_qkv(oracle, monkeypatch, m):
    """q | k | v, [2048, 1024, 1024] x 2048 Q4_K (src/qwen2vl_ocr.cpp:2368-2372)."""
    _group_check(oracle, monkeypatch, O.Q4_K, [2048, 1024, 1024], 2048, m, 1)


@pytest.mark.parametrize("m", [1, 3, 8])
def test_qwen3vl_down(oracle, monkeypatch, m):
    """down [2048 x 6144] Q4_K (src/qwen2vl_ocr.cpp:2439): K = 6144, three cached superblocks per
    wave, one workgroup per CU; and o [2048 x 2048]."""
    _group_check(oracle, monkeypatch, O.Q4_K, [2048], 6144, m, None)
    _group_check(oracle, monkeypatch, O.Q4_K, [2048], 2048, m, 1)


def _fused(wtype, imgs, ns, k, x, m, bias=None, x2=None, ldx=None, pre=0):
    import torch
    from crispembed_amd import mq
    g = len(ns)
    ys = [torch.full((m, n), np.nan, dtype=torch.float32, device="cuda") for n in ns]
    VP, I64 = ctypes.c_void_p * g, ctypes.c_int64 * g
    ld = ldx or x.stride(0)
    mq.check(mq.lib().mq_mul_mat_gemv(wtype, g, VP(*[im[1] for im in imgs]), I64(*ns), k, ctypes.c_void_p(x.data_ptr()),
                                      ld, ctypes.c_void_p(x2) if x2 else None, ld, pre, m,
                                      VP(*[t.data_ptr() for t in ys]), I64(*ns),
                                      VP(*[b.data_ptr() for b in bias]) if bias else None, stream()))
    return [host(t) for t in ys]


@pytest.fixture(params=["fused", "auto"])
def gemv_form(request, monkeypatch):
    """mq_mul_mat_gemv with the activation always quantized inside the GEMV (MQ_GEMV_FUSED=1),
    and with its own choice (large activations quantized once, then the GEMV)."""
    if request.param == "fused":
        monkeypatch.setenv("MQ_GEMV_FUSED", "1")
    else:
        monkeypatch.delenv("MQ_GEMV_FUSED", raising=False)
    return request.param


@pytest.mark.parametrize("wtype", [O.Q4_K, O.Q6_K])
@pytest.mark.parametrize("m", [1, 2, 3, 5, 8])
@pytest.mark.parametrize("ns,k", [([2048, 1024, 1024], 2048), ([2048], 6144), ([300, 77], 4096)])
def test_fused_gemv_equals_two_step(oracle, gemv_form, wtype, m, ns, k):
    """mq_mul_mat_gemv (the activation quantized inside the GEMV) against mq_quantize_act +
    mq_mul_mat_q_group on the GEMV path: bit-identical, and within the bar of the oracle."""
    import torch
    from crispembed_amd import mq
    L = mq.lib()
    ws_ = [random_blocks(wtype, n, k, 31 * n + k + g) for g, n in enumerate(ns)]
    imgs = [weight_image(wtype, w, n, k) for w, n in zip(ws_, ns)]
    x = np.random.default_rng(m * k).standard_normal((m, k)).astype(np.float32)
    x[0, 5] = 0.0
    xd = dev(x)
    bias = [dev(np.random.default_rng(n + 1).standard_normal(n).astype(np.float32)) for n in ns]
    got = _fused(wtype, imgs, ns, k, xd, m, bias)
    keep, wsp = _quant(wtype, xd, m, k)
    g = len(ns)
    ref = [torch.full((m, n), np.nan, dtype=torch.float32, device="cuda") for n in ns]
    VP, I64 = ctypes.c_void_p * g, ctypes.c_int64 * g
    mq.check(L.mq_mul_mat_q_group(wtype, g, VP(*[im[1] for im in imgs]), I64(*ns), k, ctypes.c_void_p(wsp), m,
                                  VP(*[t.data_ptr() for t in ref]), I64(*ns), VP(*[b.data_ptr() for b in bias]),
                                  mq.PATH_GEMV, stream()))
    xq = oracle.quantize_act(wtype, x)
    for i, n in enumerate(ns):
        assert np.array_equal(got[i].view(np.uint32), host(ref[i]).view(np.uint32)), i
        assert rel_err(got[i], oracle.mul_mat_exact(wtype, ws_[i], xq, k) + host(bias[i])) <= TOL
    del imgs, keep


@pytest.mark.parametrize("wtype", [O.Q4_K, O.Q6_K])
@pytest.mark.parametrize("m", [1, 4, 8])
def test_fused_gemv_silu_mul(gemv_form, wtype, m):
    """The down projection of the decode step on silu(gate) * up formed inside the GEMV, the
    gate and up rows read from one [gate | up] buffer: bit-identical to the quantizer's
    MQ_PRE_SILU_MUL prologue followed by the GEMV."""
    import torch
    from crispembed_amd import mq
    L = mq.lib()
    n, F = 2048, 6144
    w = random_blocks(wtype, n, F, 7 + m)
    img = weight_image(wtype, w, n, F)
    gu = dev((np.random.default_rng(m).standard_normal((m, 2 * F)) * 3).astype(np.float32))
    got = _fused(wtype, [img], [n], F, gu, m, x2=gu.data_ptr() + F * 4, ldx=2 * F, pre=mq.PRE_SILU_MUL)[0]
    nb = L.mq_workspace_bytes(wtype, m, F)
    buf, off = empty_u8(nb)
    mq.check(L.mq_quantize_act_ex(wtype, ctypes.c_void_p(gu.data_ptr()), 2 * F, m, F, None, mq.PRE_SILU_MUL,
                                  ctypes.c_void_p(buf.data_ptr() + off), nb, mq.PATH_GEMV, stream()))
    ref = torch.full((m, n), np.nan, dtype=torch.float32, device="cuda")
    mq.check(L.mq_mul_mat_q(wtype, ctypes.c_void_p(img[1]), n, F, ctypes.c_void_p(buf.data_ptr() + off), m,
                            ctypes.c_void_p(ref.data_ptr()), n, mq.PATH_GEMV, stream()))
    assert np.array_equal(got.view(np.uint32), host(ref).view(np.uint32))
    del img


def test_fused_gemv_lm_head(oracle, gemv_form, lm_head):
    """The Q6_K lm_head with the activation quantized inside the kernel, m = 1 and 8."""
    import torch
    from crispembed_amd import mq
    w, img, n, k = lm_head
    for m in (1, 8):
        x = np.random.default_rng(100 + m).standard_normal((m, k)).astype(np.float32)
        got = _fused(O.Q6_K, [img], [n], k, dev(x), m)[0]
        assert rel_err(got, oracle.mul_mat_exact(O.Q6_K, w, oracle.quantize_act(O.Q6_K, x), k)) <= TOL


def test_fused_gemv_refusals():
    from crispembed_amd import mq
    L = mq.lib()
    VP, I64 = ctypes.c_void_p * 1, ctypes.c_int64 * 1
    args = lambda wt, k, m: (wt, 1, VP(256), I64(64), k, ctypes.c_void_p(256), k, None, 0, 0, m, VP(256),  # noqa: E731
                             I64(64), None, stream())
    assert L.mq_mul_mat_gemv(*args(mq.TYPE_Q8_0, 512, 1)) == -2  # not a K-quant
    assert L.mq_mul_mat_gemv(*args(mq.TYPE_Q4_K, 8192, 1)) == -2  # k > 6144
    assert L.mq_mul_mat_gemv(*args(mq.TYPE_Q4_K, 512, 9)) == -2  # m > 8
