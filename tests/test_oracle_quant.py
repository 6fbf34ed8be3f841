"""Pins the oracle's quantizers and dequantizers.

Q8_0 / Q8_K activation quantizers: closed-form invariants per block plus crafted
blocks (exact .5 ties that separate round-half-even from round-half-away, zero
blocks, negative maxima, repeated maxima of opposite sign, fp16-subnormal scales).
Dequantizers: an independent numpy decoder of the block layout.
Q4_K / Q6_K weight quantizers: invariants only (their exact bytes are not pinned).
"""
import numpy as np
import pytest

import oracle_ffi as O
from ggml_numpy import (q4_K_dequant, q4_K_fields, q6_K_dequant, q6_K_fields, q8_0_dequant, q8_0_fields,
                        q8_K_fields)


def _rand(shape, seed, scale=1.0):
    return (np.random.default_rng(seed).standard_normal(shape) * scale).astype(np.float32)


def _crafted_q8_0():
    blocks = []
    z = np.zeros(32, np.float32)
    blocks.append(z)                                   # all zero
    b = np.zeros(32, np.float32); b[5] = -3.0; blocks.append(b)  # single negative max
    b = np.linspace(-1, 1, 32).astype(np.float32); blocks.append(b)
    # ties: amax = 127 makes id = 1, so x = k + 0.5 lands exactly on .5
    b = np.array([127.0] + [k + 0.5 for k in range(-15, 16)], np.float32); blocks.append(b)
    b = -b; blocks.append(b)
    b = np.full(32, 1e-6, np.float32); b[0] = -2e-6; blocks.append(b)  # fp16-subnormal d
    b = np.full(32, 3e-8, np.float32); blocks.append(b)                 # d underflows toward 0
    b = np.array([5.0, -5.0] * 16, np.float32); blocks.append(b)
    return np.concatenate(blocks)[None, :]


@pytest.mark.parametrize("variant", [O.Q8_0_X86, O.Q8_0_NEON, O.Q8_0_REF])
def test_q8_0_activation_invariants(oracle, variant):
    x = np.concatenate([_rand((64, 256), 3), np.pad(_crafted_q8_0(), ((0, 63), (0, 0)))[:, :256]])
    q = oracle.quantize_act(O.Q8_0, x, variant)
    d, qi = q8_0_fields(q, 256)
    xb = x.reshape(x.shape[0], -1, 32).astype(np.float32)
    amax = np.abs(xb).max(-1)
    d_ref = (amax / np.float32(127)).astype(np.float32).astype(np.float16).astype(np.float32)
    assert np.array_equal(d, d_ref)
    if variant == O.Q8_0_X86:
        idv = np.where(amax != 0, np.float32(127) / np.where(amax != 0, amax, 1), 0).astype(np.float32)
    else:
        dd = (amax / np.float32(127)).astype(np.float32)
        idv = np.where(dd != 0, np.float32(1) / np.where(dd != 0, dd, 1), 0).astype(np.float32)
    t = (xb * idv[..., None]).astype(np.float32).astype(np.float64)
    if variant == O.Q8_0_REF:
        ref = np.sign(t) * np.floor(np.abs(t) + 0.5)    # half away from zero
    else:
        ref = np.rint(t)                                # half to even
    assert np.array_equal(qi.reshape(ref.shape), ref.astype(np.int64))
    # invariants: |q| <= 127 and the largest-magnitude value maps to +-127
    nz = amax > 0
    qb = qi.reshape(ref.shape)
    assert np.abs(qb).max() <= 127
    top = np.abs(qb)[nz].max(-1)
    assert np.all(top == 127)


def test_q8_0_tie_rounding_differs_between_variants(oracle):
    x = np.zeros((1, 32), np.float32)
    x[0, 0] = 127.0
    x[0, 1:] = np.array([k + 0.5 for k in range(-15, 16)], np.float32)
    qx = q8_0_fields(oracle.quantize_act(O.Q8_0, x, O.Q8_0_X86), 32)[1][0]
    qr = q8_0_fields(oracle.quantize_act(O.Q8_0, x, O.Q8_0_REF), 32)[1][0]
    ties = x[0, 1:]
    assert np.array_equal(qx[1:], np.rint(ties).astype(np.int64))           # 2.5 -> 2
    assert np.array_equal(qr[1:], (np.sign(ties) * np.floor(np.abs(ties) + 0.5)).astype(np.int64))  # 2.5 -> 3
    assert not np.array_equal(qx, qr)


def _crafted_q8_K():
    rows = []
    rows.append(np.zeros(256, np.float32))
    r = _rand(256, 5); r[17] = -9.0; r[200] = 9.0; rows.append(r)       # tie in |x|: first (negative) wins
    r = _rand(256, 6); r[3] = 9.0; r[100] = -9.0; rows.append(r)        # tie: first (positive) wins
    r = np.zeros(256, np.float32); r[255] = 1e-30; rows.append(r)       # tiny, fp32 only
    r = np.arange(256, dtype=np.float32) - 127.0; rows.append(r)        # integers, max -127
    return np.stack(rows)


def test_q8_K_invariants(oracle):
    x = np.concatenate([_rand((32, 1024), 7).reshape(-1, 256), _crafted_q8_K()])
    q = oracle.quantize_act(O.Q4_K, x)
    d, qi, bs = q8_K_fields(q, 256)
    d = d[:, 0]
    for r in range(x.shape[0]):
        xr = x[r]
        amax = np.abs(xr).max()
        if amax == 0:
            assert d[r] == 0 and not qi[r].any() and not bs[r].any()
            continue
        i0 = int(np.argmax(np.abs(xr)))                 # numpy argmax: first occurrence
        vmax = xr[i0]
        iscale = np.float32(-127.0) / np.float32(vmax)
        assert d[r] == np.float32(1.0) / iscale
        assert qi[r, i0] == -127
        t = (np.float32(iscale) * xr).astype(np.float32).astype(np.float64)
        assert np.array_equal(qi[r], np.minimum(127, np.rint(t)).astype(np.int64))
        assert np.array_equal(bs[r], qi[r].reshape(16, 16).sum(-1))


@pytest.mark.parametrize("k", [256, 768])
def test_dequant_q8_0_q4_K_q6_K_against_numpy_decoders(oracle, k):
    x = _rand((9, k), 11, 0.02)
    w8 = oracle.quantize_chunk(O.Q8_0, x)
    assert np.array_equal(oracle.dequantize(O.Q8_0, w8, k), q8_0_dequant(w8, k))
    w4 = oracle.quantize_chunk(O.Q4_K, x)
    assert np.array_equal(oracle.dequantize(O.Q4_K, w4, k).view(np.uint32), q4_K_dequant(w4, k).view(np.uint32))
    w6 = oracle.quantize_chunk(O.Q6_K, x)
    assert np.array_equal(oracle.dequantize(O.Q6_K, w6, k).view(np.uint32), q6_K_dequant(w6, k).view(np.uint32))


def test_dequant_random_bytes(oracle):
    """Arbitrary block bytes (every scale/nibble pattern class) decode identically."""
    rng = np.random.default_rng(12)
    for t, bsz, dec in [(O.Q4_K, 144, q4_K_dequant), (O.Q6_K, 210, q6_K_dequant)]:
        b = rng.integers(0, 256, (64, bsz), dtype=np.uint8)
        if t == O.Q4_K:
            b[:, 0:4] = np.frombuffer(np.float16(rng.uniform(-1, 1, 128)).tobytes(), np.uint8).reshape(64, 4)
        else:
            b[:, 208:210] = np.frombuffer(np.float16(rng.uniform(-1, 1, 64)).tobytes(), np.uint8).reshape(64, 2)
        got = oracle.dequantize(t, b.ravel(), 256 * 64)
        assert np.array_equal(got.view(np.uint32), dec(b.ravel(), 256 * 64).view(np.uint32))


def test_q4_K_weight_quantizer_invariants(oracle):
    x = _rand((16, 1024), 13, 0.02)
    w = oracle.quantize_chunk(O.Q4_K, x)
    d, dmin, sc, mn, q = q4_K_fields(w, 1024)
    assert q.min() >= 0 and q.max() <= 15 and sc.max() <= 63 and mn.max() <= 63
    assert np.all(d >= 0) and np.all(dmin >= 0)
    # the sub-block of largest scale uses the full 6-bit range
    assert np.all(sc.max(-1) == 63)
    y = oracle.dequantize(O.Q4_K, w, 1024)
    rel_rmse = np.sqrt(np.mean((y - x) ** 2)) / np.sqrt(np.mean(x ** 2))
    assert rel_rmse < 0.12
    # all-zero rows quantize to all-zero values
    z = oracle.quantize_chunk(O.Q4_K, np.zeros((1, 256), np.float32))
    assert not oracle.dequantize(O.Q4_K, z, 256).any()


def test_q6_K_weight_quantizer_invariants(oracle):
    x = _rand((16, 1024), 14, 0.02)
    w = oracle.quantize_chunk(O.Q6_K, x)
    d, sc, q = q6_K_fields(w, 1024)
    assert q.min() >= -32 and q.max() <= 31
    assert np.all(np.abs(sc).max(-1) >= 127)
    y = oracle.dequantize(O.Q6_K, w, 1024)
    rel_rmse = np.sqrt(np.mean((y - x) ** 2)) / np.sqrt(np.mean(x ** 2))
    assert rel_rmse < 0.03
    z = oracle.quantize_chunk(O.Q6_K, np.zeros((1, 256), np.float32))
    assert not z.any()


def test_q8_0_weight_quantizer_is_ref_variant(oracle):
    x = _rand((8, 256), 15, 0.02)
    w = oracle.quantize_chunk(O.Q8_0, x)
    a = oracle.quantize_act(O.Q8_0, x, O.Q8_0_REF)
    assert np.array_equal(w, a)
