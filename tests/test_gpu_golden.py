"""The HIP kernels against the frozen golden fixtures (tests/golden/*.npz):
quantization and dequantization bit-exact, mul_mat on both paths within
max|d|/max|ref| <= 1e-4 of the fp64 product of the quantized operands."""
import ctypes

import numpy as np
import pytest

import oracle_ffi as O
from ggml_numpy import rel_err
from gpu_util import dev, empty_u8, host, mul_mat, stream, weight_image
from test_golden import TYPES, load

pytestmark = pytest.mark.gpu

MUL_MAT_TOL = 1e-4


def _mq():
    from crispembed_amd import mq
    return mq


@pytest.mark.parametrize("variant", ["x86", "neon", "ref"])
def test_act_q8_0(variant):
    mq = _mq()
    g = load("act_q8_0.npz")
    x, y = g["x"], g[f"y_{variant}"]
    buf, off = empty_u8(y.size)
    xd = dev(x)
    mq.check(mq.lib().mq_quantize_q8_0(ctypes.c_void_p(xd.data_ptr()), x.shape[1],
                                       ctypes.c_void_p(buf.data_ptr() + off), x.shape[0], x.shape[1],
                                       ["x86", "neon", "ref"].index(variant), stream()))
    assert np.array_equal(host(buf)[off:off + y.size].reshape(y.shape), y)


def test_act_q8_K():
    mq = _mq()
    g = load("act_q8_K.npz")
    x, y = g["x"], g["y"]
    buf, off = empty_u8(y.size)
    xd = dev(x)
    mq.check(mq.lib().mq_quantize_q8_K(ctypes.c_void_p(xd.data_ptr()), x.shape[1],
                                       ctypes.c_void_p(buf.data_ptr() + off), x.shape[0], x.shape[1], stream()))
    assert np.array_equal(host(buf)[off:off + y.size].reshape(y.shape), y)


@pytest.mark.parametrize("name,fused", [("q8_0", 0), ("q4_K", 0), ("q4_K", 1), ("q6_K", 0)])
def test_dequant(name, fused):
    mq = _mq()
    import torch
    g = load(f"dequant_{name}.npz")
    w, k = g["w"], int(g["k"])
    want = g["y_fused"] if fused else g["y"]
    wd = dev(w)
    y = torch.empty(want.shape, dtype=torch.float32, device="cuda")
    mq.check(mq.lib().mq_dequantize(TYPES[name], ctypes.c_void_p(wd.data_ptr()), ctypes.c_void_p(y.data_ptr()),
                                    w.shape[0], k, fused, stream()))
    assert np.array_equal(host(y), want)


@pytest.mark.parametrize("path", ["gemm", "gemv"])
@pytest.mark.parametrize("name", list(TYPES))
def test_mulmat(name, path):
    mq = _mq()
    t = TYPES[name]
    g = load(f"mulmat_{name}.npz")
    w, x = g["w"], g["x"]
    n, k = w.shape[0], x.shape[1]
    _, wp = weight_image(t, w, n, k)
    if path == "gemm":
        y = host(mul_mat(t, wp, n, k, dev(x), path=mq.PATH_GEMM))
        assert rel_err(y, g["y_exact"]) <= MUL_MAT_TOL
        assert rel_err(y, g["y"]) <= MUL_MAT_TOL
    else:
        for m0 in range(0, x.shape[0], 8):       # the GEMV takes at most 8 rows
            xs = x[m0:m0 + 8]
            y = host(mul_mat(t, wp, n, k, dev(xs), path=mq.PATH_GEMV))
            assert rel_err(y, g["y_exact"][m0:m0 + 8]) <= MUL_MAT_TOL
            assert rel_err(y, g["y"][m0:m0 + 8]) <= MUL_MAT_TOL
