"""Pins the oracle's block dots and mul_mat: the fp64 integer-exact product of the
quantized operands computed by an independent numpy implementation is the judge.
"""
import numpy as np
import pytest

import oracle_ffi as O
from ggml_numpy import mul_mat_exact, rel_err

TYPES = [O.Q8_0, O.Q4_K, O.Q6_K, O.F16]


def _case(wtype, m, n, k, seed):
    rng = np.random.default_rng(seed)
    w = (rng.standard_normal((n, k)) * 0.02).astype(np.float32)
    x = rng.standard_normal((m, k)).astype(np.float32)
    return w, x


@pytest.mark.parametrize("wtype", TYPES)
@pytest.mark.parametrize("m,n,k", [(1, 1, 256), (3, 5, 512), (9, 7, 256), (16, 33, 768)])
def test_mul_mat_matches_exact_product(oracle, wtype, m, n, k):
    wf, x = _case(wtype, m, n, k, 100 + m + n + k + wtype)
    w = oracle.quantize_chunk(wtype, wf)
    xq = oracle.quantize_act(wtype, x)
    ex_np = mul_mat_exact(wtype, w, xq, k)
    ex_or = oracle.mul_mat_exact(wtype, w, xq, k)
    assert rel_err(ex_or, ex_np) < 1e-12
    y = oracle.mul_mat(wtype, w, x)
    assert rel_err(y, ex_np) < 1e-5
    y2 = oracle.mul_mat_q(wtype, w, xq, k, nthreads=3)
    assert np.array_equal(y, y2)


def test_mul_mat_transposed_operand_is_caught(oracle):
    """The exact-product check separates W from W^T (a plausible indexing slip)."""
    k = 256
    wf, x = _case(O.Q8_0, 256, 256, k, 5)
    w = oracle.quantize_chunk(O.Q8_0, wf)
    xq = oracle.quantize_act(O.Q8_0, x)
    y = oracle.mul_mat_q(O.Q8_0, w, xq, k)
    assert rel_err(y.T, mul_mat_exact(O.Q8_0, w, xq, k)) > 0.1


def test_q4_K_min_term_matters(oracle):
    """Dropping the dmin * sum(m_j * bsum) term would be far outside tolerance."""
    k = 512
    wf, x = _case(O.Q4_K, 4, 8, k, 6)
    w = oracle.quantize_chunk(O.Q4_K, wf)
    xq = oracle.quantize_act(O.Q4_K, x)
    w_nomin = w.copy().reshape(-1, 144)
    w_nomin[:, 2:4] = 0  # dmin = 0
    a = oracle.mul_mat_q(O.Q4_K, w, xq, k)
    b = oracle.mul_mat_q(O.Q4_K, w_nomin.ravel(), xq, k)
    assert rel_err(b, a) > 1e-2


@pytest.mark.parametrize("isa", ["host", "avx2"])
@pytest.mark.parametrize("wtype", [O.Q8_0, O.Q4_K, O.Q6_K])
@pytest.mark.parametrize("m,n,k", [(1, 3, 256), (17, 33, 512), (40, 20, 1536), (5, 9, 2304)])
def test_cpu_baseline_matches_exact_product(oracle, monkeypatch, isa, wtype, m, n, k):
    """The SIMD + threads CPU baseline computes the same mul_mat (block dots in another order),
    in its AVX-512 VNNI form where the host has it and in its AVX2 form."""
    if not oracle.fast_supported(wtype):
        pytest.skip("host without AVX2/FMA/F16C")
    if isa == "avx2":
        monkeypatch.setenv("OR_FAST_ISA", "avx2")
        assert oracle.fast_isa() == "avx2"
    wf, x = _case(wtype, m, n, k, 300 + m + n + k + wtype)
    w = oracle.quantize_chunk(wtype, wf)
    xq = oracle.quantize_act(wtype, x)
    y = oracle.fast_mul_mat(wtype, w, x, nthreads=3)
    assert rel_err(y, mul_mat_exact(wtype, w, xq, k)) < 1e-5
    assert rel_err(y, oracle.mul_mat(wtype, w, x)) < 1e-5


@pytest.mark.parametrize("k", [96, 288])
def test_cpu_baseline_q8_0_odd_block_count(oracle, k):
    """An odd number of Q8_0 blocks per row: the VNNI form's pairs plus its one-block tail."""
    if not oracle.fast_supported(O.Q8_0):
        pytest.skip("host without AVX2/FMA/F16C")
    wf, x = _case(O.Q8_0, 7, 5, k, k)
    w = oracle.quantize_chunk(O.Q8_0, wf)
    y = oracle.fast_mul_mat(O.Q8_0, w, x, nthreads=2)
    assert rel_err(y, mul_mat_exact(O.Q8_0, w, oracle.quantize_act(O.Q8_0, x), k)) < 1e-5
