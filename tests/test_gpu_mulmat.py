"""GPU mul_mat (GEMM and GEMV paths) against the oracle.

Bar: max|dY| / max|Y_ref| <= 1e-4, where Y_ref is (a) the fp64 integer-exact
product of the quantized operands and (b) the oracle's ggml-order fp32 result.
"""
import numpy as np
import pytest

import oracle_ffi as O
from ggml_numpy import rel_err
from gpu_util import dev, host, mul_mat, weight_image

pytestmark = pytest.mark.gpu

TOL = 1e-4
TYPES = [O.Q8_0, O.Q4_K, O.Q6_K, O.F16]


def _mk(oracle, wtype, m, n, k, seed, act_fn=None):
    rng = np.random.default_rng(seed)
    wf = (rng.standard_normal((n, k)) * 0.02).astype(np.float32)
    x = rng.standard_normal((m, k)).astype(np.float32)
    if act_fn is not None:
        x = act_fn(x)
    w = oracle.quantize_chunk(wtype, wf)
    return w, x


def _check(oracle, wtype, w, x, y, k):
    xq = oracle.quantize_act(wtype, x)
    ex = oracle.mul_mat_exact(wtype, w, xq, k)
    ref = oracle.mul_mat_q(wtype, w, xq, k)
    e1, e2 = rel_err(y, ex), rel_err(y, ref)
    assert e1 <= TOL and e2 <= TOL, (e1, e2)
    return e1


@pytest.mark.parametrize("cfg", ["1", "3", "4", "5", "6", "7", "8", "9", "11", "12", "15"])
@pytest.mark.parametrize("wtype", TYPES)
@pytest.mark.parametrize("m,n,k", [(37, 70, 512), (128, 128, 256), (300, 260, 768), (129, 257, 1024), (9, 33, 256),
                                   (520, 390, 1536), (200, 140, 384)])
def test_gemm(oracle, wtype, m, n, k, cfg, monkeypatch):
    """Every tile configuration (MQ_GEMM_CFG) on ragged and multi-tile shapes."""
    from crispembed_amd import mq
    if wtype in (O.Q4_K, O.Q6_K) and k % 256:
        pytest.skip("K-quant rows are whole 256-value superblocks")
    if cfg == "15" and wtype != O.Q8_0:
        pytest.skip("the K-group configuration is a Q8_0 form")
    monkeypatch.setenv("MQ_GEMM_CFG", cfg)
    w, x = _mk(oracle, wtype, m, n, k, m * 7 + n + k)
    _, wp = weight_image(wtype, w, n, k)
    y = host(mul_mat(wtype, wp, n, k, dev(x), path=mq.PATH_GEMM))
    _check(oracle, wtype, w, x, y, k)


@pytest.mark.parametrize("wtype", TYPES)
@pytest.mark.parametrize("m", [1, 2, 3, 4, 5, 8, 9, 16, 27, 32])
@pytest.mark.parametrize("n,k", [(67, 256), (130, 2048), (20, 6144)])
def test_gemv(oracle, wtype, m, n, k):
    """m <= 8 in one launch; 9..32 in 8-row launches over the chunked activation layout."""
    from crispembed_amd import mq
    w, x = _mk(oracle, wtype, m, n, k, 1000 + m * 13 + n + k)
    _, wp = weight_image(wtype, w, n, k)
    y = host(mul_mat(wtype, wp, n, k, dev(x), path=mq.PATH_GEMV))
    _check(oracle, wtype, w, x, y, k)


def test_q8_0_k_tail_and_strides(oracle):
    """k not a multiple of the 128-byte stage; row strides ldx > k and ldy > n."""
    from crispembed_amd import mq
    import torch
    m, n, k = 70, 90, 96
    w, x = _mk(oracle, O.Q8_0, m, n, k, 77)
    _, wp = weight_image(O.Q8_0, w, n, k)
    xpad = np.zeros((m, k + 40), np.float32)
    xpad[:, :k] = x
    ybuf = torch.full((m, n + 5), 7.0, device="cuda")
    for path in (mq.PATH_GEMM,):
        mul_mat(O.Q8_0, wp, n, k, dev(xpad)[:, :k], path=path, y_dev=ybuf, ldy=n + 5)
        yy = host(ybuf)
        _check(oracle, O.Q8_0, w, x, yy[:, :n], k)
        assert np.all(yy[:, n:] == 7.0)  # columns past n untouched


def test_library_workspace_and_auto_path(oracle):
    from crispembed_amd import mq
    m, n, k = 8, 64, 512
    w, x = _mk(oracle, O.Q4_K, m, n, k, 78)
    _, wp = weight_image(O.Q4_K, w, n, k)
    y1 = host(mul_mat(O.Q4_K, wp, n, k, dev(x), path=mq.PATH_AUTO, workspace=False))
    y2 = host(mul_mat(O.Q4_K, wp, n, k, dev(x), path=mq.PATH_GEMM, workspace=False))
    _check(oracle, O.Q4_K, w, x, y1, k)
    _check(oracle, O.Q4_K, w, x, y2, k)


def _full_check(oracle, wtype, w, x, y, k):
    """Every output element against the oracle's threaded integer-dot product (or_fast_mul_mat:
    the same activation quantization, integer block dots, fp32 scales; pinned against the exact
    product by tests/test_oracle_mulmat.py), within 1e-4 of max|Y|, and no row off by more than
    1e-4 of its own largest value."""
    import os
    ref = oracle.fast_mul_mat(wtype, w, x, nthreads=min(16, os.cpu_count() or 8))
    assert y.shape == ref.shape and np.isfinite(y).all()
    err = np.abs(y.astype(np.float64) - ref)
    assert err.max() / np.abs(ref).max() <= TOL, err.max() / np.abs(ref).max()
    row = err.max(1) / np.abs(ref).max(1)
    assert row.max() <= TOL, (int(row.argmax()), row.max())
    return err.max() / np.abs(ref).max()


@pytest.mark.parametrize("wtype,n,k,m,act", [
    (O.Q8_0, 1536, 384, 4096, None),          # MiniLM-L6 FFN-up
    (O.Q8_0, 384, 1536, 4096, "gelu"),        # MiniLM-L6 FFN-down
    (O.Q4_K, 4096, 1024, 8192, None),         # XLM-R-large FFN-up
    (O.Q4_K, 1024, 4096, 8192, "gelu"),       # XLM-R-large FFN-down on GELU(N(0,1))
])
def test_full_size(oracle, wtype, n, k, m, act):
    """Full-size GEMM: every output element against the oracle's integer-dot product, sampled
    rows against the fp64 exact product, and the GEMV on 8 of them."""
    from crispembed_amd import mq, synth
    rng = np.random.default_rng(n + k)
    wf = (rng.standard_normal((n, k)) * 0.02).astype(np.float32)
    from crispembed_amd.mq import lib
    import ctypes
    w = np.empty((n, O.row_size(wtype, k)), np.uint8)
    lib().mq_quantize_chunk(wtype, wf.ctypes.data_as(ctypes.c_void_p), w.ctypes.data_as(ctypes.c_void_p), n, k)
    x = rng.standard_normal((m, k)).astype(np.float32)
    if act == "gelu":
        x = synth.gelu_erf(x)
    _, wp = weight_image(wtype, w, n, k)
    xd = dev(x)
    y = host(mul_mat(wtype, wp, n, k, xd, path=mq.PATH_GEMM))
    print("full-output relative error", _full_check(oracle, wtype, w, x, y, k))
    rows = np.unique(np.concatenate([[0, m - 1], rng.integers(0, m, 38)]))
    _check(oracle, wtype, w, x[rows], y[rows], k)
    yv = host(mul_mat(wtype, wp, n, k, dev(x[rows[:8]]), path=mq.PATH_GEMV))
    assert rel_err(yv, y[rows[:8]]) <= TOL


@pytest.mark.parametrize("wtype", [O.Q4_K, O.Q6_K])
@pytest.mark.parametrize("m,n,k,pad", [(2048, 4608, 512, 0), (2048, 16384, 768, 64), (4096, 4096, 2048, 0)])
def test_gemm_many_tiles(oracle, wtype, m, n, k, pad, monkeypatch):
    """256x128 tiles (MQ_GEMM_CFG=1) on grids of 288-1024 tiles, more than the chip holds at once,
    with K from 2 to 8 superblocks: every output against the oracle's integer-dot product, sampled
    rows (first and last of a tile row among them) against the exact product, columns past n
    untouched (ldy = n + pad)."""
    from crispembed_amd import mq
    import torch
    monkeypatch.setenv("MQ_GEMM_CFG", "1")
    w, x = _mk(oracle, wtype, m, n, k, m + n + k + pad)
    _, wp = weight_image(wtype, w, n, k)
    ybuf = torch.full((m, n + pad), 7.0, device="cuda")
    mul_mat(wtype, wp, n, k, dev(x), path=mq.PATH_GEMM, y_dev=ybuf)
    y = host(ybuf)
    assert np.all(y[:, n:] == 7.0)
    _full_check(oracle, wtype, w, x, np.ascontiguousarray(y[:, :n]), k)
    rng = np.random.default_rng(k)
    rows = np.unique(np.concatenate([[0, 255, 256, m - 1], rng.integers(0, m, 36)]))
    _check(oracle, wtype, w, x[rows], y[rows, :n], k)
