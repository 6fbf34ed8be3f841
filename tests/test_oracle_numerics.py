"""Pins the oracle's scalar building blocks against independent implementations:
numpy's IEEE binary16 conversion and numpy.rint (round half to even)."""
import numpy as np
import pytest


def test_fp16_to_fp32_exhaustive(oracle):
    bits = np.arange(65536, dtype=np.uint32)
    ref = bits.astype(np.uint16).view(np.float16).astype(np.float32)
    got = np.array([oracle.L.or_fp16_to_fp32(int(b)) for b in bits], dtype=np.float32)
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), ref[~nan].view(np.uint32))


def test_fp32_to_fp16_matches_numpy(oracle):
    rng = np.random.default_rng(1)
    # every fp16 value, every midpoint between neighbours (ties), neighbours of the
    # midpoints, random magnitudes from fp32 subnormals to overflow
    h = np.arange(0, 0x7c00, dtype=np.uint16).view(np.float16).astype(np.float32)
    mids = ((h[:-1].astype(np.float64) + h[1:].astype(np.float64)) / 2).astype(np.float32)
    near = np.concatenate([np.nextafter(mids, np.float32(0)), np.nextafter(mids, np.float32(np.inf))])
    rnd = (rng.standard_normal(200000) * np.exp2(rng.uniform(-40, 20, 200000))).astype(np.float32)
    edge = np.array([0.0, -0.0, 65504, 65519.99, 65520, 65536, 1e-8, 2.0**-25, 2.0**-24, 3 * 2.0**-26,
                     np.inf, -np.inf, 1e-45], dtype=np.float32)
    x = np.concatenate([h, -h, mids, -mids, near, -near, rnd, edge]).astype(np.float32)
    got = oracle.fp32_to_fp16(x)
    ref = x.astype(np.float16).view(np.uint16)
    assert np.array_equal(got, ref)


def test_nearest_int_is_round_half_even(oracle):
    rng = np.random.default_rng(2)
    vals = np.concatenate([
        rng.uniform(-4e6, 4e6, 20000),
        np.arange(-300, 300) + 0.5,             # exact ties
        rng.uniform(-200, 200, 20000),
    ]).astype(np.float32)
    got = np.array([oracle.nearest_int(v) for v in vals])
    assert np.array_equal(got, np.rint(vals.astype(np.float64)).astype(np.int64))


def test_get_scale_min_k4_exhaustive(oracle):
    """Pack every (sc, m) pair with an independent packer, unpack with the oracle."""
    import ctypes
    from ggml_numpy import pack_q4_K_scales
    vals = np.arange(64)
    for j in range(8):
        sc = np.zeros((64 * 64, 8), np.int64)
        mn = np.zeros((64 * 64, 8), np.int64)
        sc[:, j] = np.repeat(vals, 64)
        mn[:, j] = np.tile(vals, 64)
        # fill the other slots with a different pattern so cross-talk shows up
        others = [i for i in range(8) if i != j]
        sc[:, others] = (np.arange(64 * 64)[:, None] * 7 + np.arange(7)[None]) % 64
        mn[:, others] = (np.arange(64 * 64)[:, None] * 11 + 3 * np.arange(7)[None]) % 64
        packed = pack_q4_K_scales(sc, mn)
        a, b = ctypes.c_uint8(), ctypes.c_uint8()
        for r in range(0, 64 * 64, 37):  # sample rows for speed; every j and value class covered
            buf = (ctypes.c_uint8 * 12)(*packed[r].tolist())
            oracle.L.or_get_scale_min_k4(j, buf, ctypes.byref(a), ctypes.byref(b))
            assert (a.value, b.value) == (sc[r, j], mn[r, j])
