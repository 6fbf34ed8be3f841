"""mq_mul_mat_noalloc (include/mq.h) against mq_mul_mat_ex with the library's own workspace.

The no-allocation entry point quantizes the activations into a fixed device array instead of
a caller or hipMalloc'd workspace; its results must equal mq_mul_mat_ex's bit for bit.  Two
calls in a row, the second on a smaller input, show that the array's leftover contents from
the first call do not leak into the second (every byte the kernels read is rewritten).
"""
import ctypes

import numpy as np
import pytest

import oracle_ffi as O
from ggml_numpy import rel_err
from gpu_util import dev, host, stream, weight_image

pytestmark = pytest.mark.gpu


def _both(L, mq, wtype, wp, n, k, x, path):
    import torch
    m = x.shape[0]
    ya = torch.full((m, n), np.nan, dtype=torch.float32, device="cuda")
    yb = torch.full((m, n), np.nan, dtype=torch.float32, device="cuda")
    mq.check(L.mq_mul_mat_ex(wtype, ctypes.c_void_p(wp), n, k, ctypes.c_void_p(x.data_ptr()), x.stride(0), m,
                             ctypes.c_void_p(ya.data_ptr()), n, None, 0, path, stream()))
    mq.check(L.mq_mul_mat_noalloc(wtype, ctypes.c_void_p(wp), n, k, ctypes.c_void_p(x.data_ptr()), x.stride(0), m,
                                  ctypes.c_void_p(yb.data_ptr()), n, path, stream()))
    return host(ya), host(yb)


@pytest.mark.parametrize("wtype", [O.Q8_0, O.Q4_K, O.Q6_K, O.F16])
@pytest.mark.parametrize("path,m1,m2", [(2, 1000, 300), (1, 8, 3), (0, 4096, 5)])
def test_noalloc_equals_mul_mat_ex(oracle, wtype, path, m1, m2):
    from crispembed_amd import mq
    L = mq.lib()
    n, k = 768, 1024
    rng = np.random.default_rng(wtype * 31 + m1)
    w = oracle.quantize_chunk(wtype, (rng.standard_normal((n, k)) * 0.02).astype(np.float32))
    img = weight_image(wtype, w, n, k)
    for m in (m1, m2):  # the second call on a smaller input
        xh = rng.standard_normal((m, k)).astype(np.float32)
        a, b = _both(L, mq, wtype, img[1], n, k, dev(xh), path)
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), (m, path)
        if m <= 300:  # and against the oracle (quantized operands, exact product)
            assert rel_err(b, oracle.mul_mat_exact(wtype, w, oracle.quantize_act(wtype, xh), k)) <= 1e-4
    del img


def test_noalloc_refuses_beyond_the_array():
    from crispembed_amd import mq
    L = mq.lib()
    k = 4096
    m = 16384  # Q8_K activations of 16384 x 4096 need more than 64 MiB
    assert L.mq_workspace_bytes(mq.TYPE_Q4_K, 8192, k) <= 64 << 20 < L.mq_workspace_bytes(mq.TYPE_Q4_K, m, k)
    # refused on the host, before any device access (the pointers are never dereferenced)
    rc = L.mq_mul_mat_noalloc(mq.TYPE_Q4_K, ctypes.c_void_p(256), 1024, k, ctypes.c_void_p(256), k, m,
                              ctypes.c_void_p(256), 1024, mq.PATH_GEMM, stream())
    assert rc == -1
    assert b"scratch array" in L.mq_last_error()
