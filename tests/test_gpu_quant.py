"""GPU activation quantization and dequantization: bit-exact against the oracle."""
import ctypes

import numpy as np
import pytest

import oracle_ffi as O
from gpu_util import dev, empty_u8, host, stream

pytestmark = pytest.mark.gpu


def _lib():
    from crispembed_amd import mq
    return mq


def _crafted_rows(k):
    rows = [np.zeros(k, np.float32)]
    r = np.zeros(k, np.float32); r[: 32] = np.array([127.0] + [i + 0.5 for i in range(-15, 16)]); rows.append(r)
    rows.append(-r)
    r = np.full(k, 1e-6, np.float32); r[0] = -2e-6; rows.append(r)
    r = np.full(k, 3e-8, np.float32); rows.append(r)
    r = np.random.default_rng(1).standard_normal(k).astype(np.float32); r[17] = -9.0; r[200 % k] = 9.0; rows.append(r)
    r = np.arange(k, dtype=np.float32) % 256 - 127.0; rows.append(r)
    r = np.full(k, 1e-30, np.float32); rows.append(r)
    return np.stack(rows)


def _acts(m, k, seed, ld=None):
    x = np.random.default_rng(seed).standard_normal((m, k)).astype(np.float32)
    x = np.concatenate([x, _crafted_rows(k)])
    if ld is None:
        return x, dev(x)
    full = np.zeros((x.shape[0], ld), np.float32)
    full[:, :k] = x
    return x, dev(full)[:, :k]


@pytest.mark.parametrize("variant", [0, 1, 2])
@pytest.mark.parametrize("m,k,ld", [(4096, 384, None), (64, 1536, None), (33, 256, 264), (19, 96, 99)])
def test_quantize_q8_0_bit_exact(oracle, variant, m, k, ld):
    mq = _lib()
    x, xd = _acts(m, k, 100 + k, ld)
    rows = x.shape[0]
    nbytes = rows * O.row_size(O.Q8_0, k)
    buf, off = empty_u8(nbytes)
    mq.check(mq.lib().mq_quantize_q8_0(ctypes.c_void_p(xd.data_ptr()), xd.stride(0),
                                       ctypes.c_void_p(buf.data_ptr() + off), rows, k, variant, stream()))
    got = host(buf)[off:off + nbytes].reshape(rows, -1)
    assert np.array_equal(got, oracle.quantize_act(O.Q8_0, x, variant))


@pytest.mark.parametrize("m,k,ld", [(2048, 1024, None), (64, 4096, None), (9, 256, 260), (5, 512, 515)])
def test_quantize_q8_K_bit_exact(oracle, m, k, ld):
    mq = _lib()
    x, xd = _acts(m, k, 200 + k, ld)
    rows = x.shape[0]
    nbytes = rows * O.row_size(O.Q8_K, k)
    buf, off = empty_u8(nbytes)
    mq.check(mq.lib().mq_quantize_q8_K(ctypes.c_void_p(xd.data_ptr()), xd.stride(0),
                                       ctypes.c_void_p(buf.data_ptr() + off), rows, k, stream()))
    got = host(buf)[off:off + nbytes].reshape(rows, -1)
    assert np.array_equal(got, oracle.quantize_act(O.Q4_K, x))


def test_quantize_f16_bit_exact(oracle):
    mq = _lib()
    x, xd = _acts(100, 512, 3)
    rows = x.shape[0]
    buf, off = empty_u8(rows * 512 * 2)
    mq.check(mq.lib().mq_quantize_f16(ctypes.c_void_p(xd.data_ptr()), 512, ctypes.c_void_p(buf.data_ptr() + off),
                                      rows, 512, stream()))
    got = host(buf)[off:off + rows * 1024].view(np.uint16).reshape(rows, 512)
    assert np.array_equal(got, x.astype(np.float16).view(np.uint16))


@pytest.mark.parametrize("wtype,fused", [(O.Q8_0, 0), (O.Q4_K, 0), (O.Q4_K, 1), (O.Q6_K, 0), (O.F16, 0)])
def test_dequantize_bit_exact(oracle, wtype, fused):
    mq = _lib()
    n, k = 37, 1024
    w = oracle.quantize_chunk(wtype, (np.random.default_rng(4).standard_normal((n, k)) * 0.02).astype(np.float32))
    wd = dev(w.ravel())
    y = dev(np.zeros((n, k), np.float32))
    mq.check(mq.lib().mq_dequantize(wtype, ctypes.c_void_p(wd.data_ptr()), ctypes.c_void_p(y.data_ptr()), n, k,
                                    fused, stream()))
    got = host(y)
    ref = oracle.dequantize(wtype, w, k, fused)
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))


def test_dequantize_q8_K_bit_exact(oracle):
    mq = _lib()
    x = np.random.default_rng(5).standard_normal((7, 512)).astype(np.float32)
    q = oracle.quantize_act(O.Q4_K, x)
    qd = dev(q.ravel())
    y = dev(np.zeros((7, 512), np.float32))
    mq.check(mq.lib().mq_dequantize(O.Q8_K, ctypes.c_void_p(qd.data_ptr()), ctypes.c_void_p(y.data_ptr()), 7, 512,
                                    0, stream()))
    assert np.array_equal(host(y).view(np.uint32), oracle.dequantize(O.Q8_K, q, 512).view(np.uint32))
