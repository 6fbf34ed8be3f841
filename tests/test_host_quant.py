"""The product's host weight quantizer (mq_quantize_chunk, the producer of GGUF
bytes) writes exactly the oracle's bytes."""
import ctypes

import numpy as np
import pytest

import oracle_ffi as O


@pytest.mark.parametrize("wtype", [O.Q8_0, O.Q4_K, O.Q6_K, O.Q8_K, O.F16])
def test_quantize_chunk_bytes_match_oracle(oracle, wtype):
    from crispembed_amd import mq
    L = mq.lib()
    rng = np.random.default_rng(20 + wtype)
    x = (rng.standard_normal((24, 512)) * 0.02).astype(np.float32)
    x[3] = 0.0                                  # zero rows / blocks
    x[5, :256] = 1e-30                          # tiny values
    x[7, :32] = np.array([127.0] + [k + 0.5 for k in range(-15, 16)], np.float32) * 1e-3
    out = np.zeros(24 * O.row_size(wtype, 512), np.uint8)
    n = L.mq_quantize_chunk(wtype, x.ctypes.data_as(ctypes.c_void_p), out.ctypes.data_as(ctypes.c_void_p), 24, 512)
    assert n == out.size
    assert np.array_equal(out.reshape(24, -1), oracle.quantize_chunk(wtype, x))
