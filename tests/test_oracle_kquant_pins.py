"""Pins of the oracle's K-quant weight quantizers (quantize_row_q4_K_ref / quantize_row_q6_K_ref,
the bytes ggml_quantize_chunk writes for tools/quantize.cpp:804-805), from what the published
algorithm fixes rather than from a second copy of it:

* the sub-block search reaches the error its definition implies (Q4_K, make_qkx2_quants: the
  weighted squared error of the returned (scale, min, levels) equals that of the best of the
  initial guess and the nstep + 1 least-squares refits, walked in order in float64 here) or is
  an argmax (Q6_K, make_qx_quants with weights x^2: (sum w x l)^2 / sum w l^2 is the largest
  over the levels at inverse scales -(nmax + 0.1 i) / max, i = -9..9, each candidate computed
  here in float64 over the levels fp32 rounding gives);
* idempotence on exactly representable blocks: a block whose every sub-block spans levels 0 and
  15 (Q4_K; scale and min at 63 somewhere in the superblock) or holds a level -32 at its largest
  magnitude (Q6_K; one sub-block scale at -128) dequantizes to values the quantizer must map
  back to the same bytes;
* the whole Q4_K row (quantize_row_q4_K_ref's call site included: the weights av_x + |x|, rmin -1,
  rdelta 0.1, nstep 20, the 6-bit codes and the recomputed levels) against its definition
  restated in float64 over that search: byte-identical superblocks but for rounding ties;
* planted mistakes (the oracle's or_set_mutation, CPU only): no search, a wrong search step,
  swapped packing bits, a wrong scale divisor, and at the wrapper's call of the search nstep 0,
  unit weights, rmin -0.5 -- each makes at least one pin above fail.
"""
import numpy as np
import pytest

import oracle_ffi as O
from ggml_numpy import pack_q4_K_scales, q4_K_dequant, q6_K_dequant

F32 = np.float32


def _rint(v):
    """ggml's nearest_int on fp32 values: round half to even."""
    return np.rint(v.astype(F32)).astype(np.int64)


# ------------------------------------------------------------------ Q4_K ----
def qkx2_search_full(x, w, nmax=15, rmin=-1.0, rdelta=0.1, nstep=20):
    """make_qkx2_quants as its definition reads, in float64 for the least-squares refits and the
    errors (levels rounded in fp32): start from the levels of the full range [min(x, 0), max],
    then for i = 0..nstep refit (scale, min) by weighted least squares to the levels at inverse
    scale (rmin + rdelta i + nmax) / (max - min) -- min being the best refit's so far -- clamp a
    positive min to 0, keep the refit whenever its error is lower.  Returns the best error and
    its (scale, min, levels)."""
    x = x.astype(F32)
    mn, mx = min(F32(x.min()), F32(0)), F32(x.max())
    w64, x64 = w.astype(np.float64), x.astype(np.float64)
    iscale = F32(nmax) / (mx - mn)
    L = np.clip(_rint(iscale * (x - mn)), 0, nmax)
    best_scale, best_min, best_L = 1.0 / float(iscale), float(mn), L.copy()
    best = float((w64 * (best_scale * L + float(mn) - x64) ** 2).sum())
    cur_min = float(mn)
    for i in range(nstep + 1):
        iscale = (F32(rmin) + F32(rdelta) * F32(i) + F32(nmax)) / (mx - F32(cur_min))
        Li = np.clip(_rint(F32(iscale) * (x - F32(cur_min))), 0, nmax)
        L = Li.astype(np.float64)
        sw, sl, sl2, sxl, sx = w64.sum(), (w64 * L).sum(), (w64 * L * L).sum(), (w64 * L * x64).sum(), (w64 * x64).sum()
        D = sw * sl2 - sl * sl
        if D <= 0:
            continue
        scale, minv = (sw * sxl - sx * sl) / D, (sl2 * sx - sl * sxl) / D
        if minv > 0:
            minv, scale = 0.0, sxl / sl2
        err = float((w64 * (scale * L + minv - x64) ** 2).sum())
        if err < best:
            best, cur_min = err, minv
            best_scale, best_min, best_L = scale, minv, Li.copy()
    return best, best_scale, best_min, best_L


def qkx2_search(x, w, **kw):
    return qkx2_search_full(x, w, **kw)[0]


def q4_K_row_from_definition(xs):
    """quantize_row_q4_K_ref as ggml publishes it, restated in float64 on top of the search
    above: per 32-value sub-block the weights av_x + |x| (av_x the rms of the sub-block) and
    make_qkx2_quants(32, 15, ..., rmin -1, rdelta 0.1, nstep 20); the sub-block scales and mins
    (minus the search's min) as 6-bit codes nearest_int(63 / max * v) clamped to 63, d and dmin =
    fp16(max / 63); then each level recomputed from the codes, nearest_int((x + dmin m) / (d sc))
    clamped to [0, 15] (a sub-block whose scale code is 0 keeps the search's levels); nibbles
    packed low half / high half of each 64 values.  xs [nsb, 256] -> the [nsb, 144] blocks."""
    nsb = xs.shape[0]
    out = np.zeros((nsb, 144), np.uint8)
    for b in range(nsb):
        x = xs[b].astype(F32)
        scales, mins, L = np.zeros(8), np.zeros(8), np.zeros(256, np.int64)
        for j in range(8):
            xj = x[32 * j:32 * j + 32]
            s2 = F32(0)
            for v in xj:  # the definition's fp32 running sum
                s2 = F32(s2 + v * v)
            w = (np.sqrt(s2 / F32(32)).astype(F32) + np.abs(xj)).astype(F32)
            _, scales[j], mn, L[32 * j:32 * j + 32] = qkx2_search_full(xj, w)
            mins[j] = -mn
        ms, mm = scales.max(), mins.max()
        sc = np.minimum(_rint(np.float64(63.0 / ms if ms > 0 else 0.0) * scales), 63)
        mn_ = np.minimum(_rint(np.float64(63.0 / mm if mm > 0 else 0.0) * mins), 63)
        d, dmin = np.float16(ms / 63.0), np.float16(mm / 63.0)
        for j in range(8):
            d1 = F32(d) * F32(sc[j])
            if d1 == 0:
                continue
            dm = F32(dmin) * F32(mn_[j])
            L[32 * j:32 * j + 32] = np.clip(_rint((x[32 * j:32 * j + 32] + dm) / d1), 0, 15)
        out[b, 0:2] = np.frombuffer(d.tobytes(), np.uint8)
        out[b, 2:4] = np.frombuffer(dmin.tobytes(), np.uint8)
        out[b, 4:16] = pack_q4_K_scales(sc, mn_)
        q = L.reshape(4, 2, 32)
        out[b, 16:] = (q[:, 0] | (q[:, 1] << 4)).reshape(128).astype(np.uint8)
    return out


def q4_wrapper_mismatch(oracle, seed=5, nsb=160):
    """Fraction of superblocks whose oracle bytes differ from the restatement from the definition
    (random N(0, 0.02) rows, a quarter of them shifted positive so mins clamp to 0)."""
    rng = np.random.default_rng(seed)
    xs = (rng.standard_normal((nsb, 256)) * 0.02).astype(F32)
    xs[: nsb // 4] += F32(0.015)
    got = oracle.quantize_chunk(O.Q4_K, xs.reshape(1, -1)).reshape(nsb, 144)
    return float((got != q4_K_row_from_definition(xs)).any(-1).mean())


def test_q4_K_row_bytes_from_the_definition(oracle):
    """The whole wrapper -- weights, search parameters, 6-bit codes, level recomputation, packing
    -- against its definition restated with float64 refits: the bytes agree except where fp32 and
    float64 rounding fall on different sides of a tie (a 6-bit code's .5, or two refits at nearly
    equal error: then d moves and the superblock's levels with it).  Measured: 3 of 160 superblocks
    (1.9 %), each such a tie; the planted call-site mistakes (nstep 0, unit weights, rmin -0.5) and
    the search mistakes change 76-100 % of them, so the bar sits at 5 %."""
    assert q4_wrapper_mismatch(oracle) <= 0.05


def _q4_subblocks(seed, n=400):
    rng = np.random.default_rng(seed)
    xs = (rng.standard_normal((n, 32)) * 0.02).astype(F32)
    xs[: n // 4] += F32(0.01)  # some all-positive-leaning sub-blocks (min clamped to 0)
    return xs


def q4_search_gap(oracle, seed=1):
    """Largest relative distance between the returned error and the best candidate's."""
    gap = 0.0
    for x in _q4_subblocks(seed):
        w = (np.sqrt((x.astype(F32) ** 2).sum(dtype=F32) / F32(32)) + np.abs(x)).astype(F32)
        scale, the_min, L = oracle.make_qkx2_quants(x, w)
        got = float((w.astype(np.float64) * (float(scale) * L - float(the_min) - x.astype(np.float64)) ** 2).sum())
        best = qkx2_search(x, w)
        gap = max(gap, abs(got - best) / max(best, 1e-30))
    return gap


def test_q4_K_search_is_the_argmin(oracle):
    assert q4_search_gap(oracle) <= 1e-4


def representable_q4_K(seed, nsb=8):
    """GGUF Q4_K superblocks that are exactly representable by the quantizer's own search:
    every sub-block holds levels 0 and 15, and scale and min 63 occur in every superblock."""
    rng = np.random.default_rng(seed)
    b = np.zeros((nsb, 144), np.uint8)
    d = (rng.uniform(0.5, 2.0, nsb) * 1e-4).astype(np.float16)
    dmin = (rng.uniform(0.5, 2.0, nsb) * 1e-4).astype(np.float16)
    sc = rng.integers(1, 64, (nsb, 8))
    mn = rng.integers(0, 64, (nsb, 8))
    sc[np.arange(nsb), rng.integers(0, 8, nsb)] = 63
    mn[np.arange(nsb), rng.integers(0, 8, nsb)] = 63
    q = rng.integers(0, 16, (nsb, 8, 32))
    q[:, :, 0], q[:, :, 1] = 0, 15
    q = np.take_along_axis(q, rng.permuted(np.tile(np.arange(32), (nsb, 8, 1)), axis=-1), -1).reshape(nsb, 256)
    b[:, 0:2] = d.view(np.uint8).reshape(nsb, 2)
    b[:, 2:4] = dmin.view(np.uint8).reshape(nsb, 2)
    b[:, 4:16] = pack_q4_K_scales(sc, mn)
    qq = q.reshape(nsb, 4, 2, 32)
    b[:, 16:] = (qq[:, :, 0] | (qq[:, :, 1] << 4)).reshape(nsb, 128).astype(np.uint8)
    return b


def q4_roundtrip_mismatch(oracle, seed=2, nsb=64):
    b = representable_q4_K(seed, nsb)
    y = q4_K_dequant(b.ravel(), 256 * nsb).reshape(1, -1)
    again = oracle.quantize_chunk(O.Q4_K, y)
    return int((again.reshape(nsb, 144) != b).any(-1).sum())


def test_q4_K_idempotent_on_representable_blocks(oracle):
    assert q4_roundtrip_mismatch(oracle) == 0


# ------------------------------------------------------------------ Q6_K ----
def qx_objectives(x, nmax=32):
    """(sum w x l)^2 / sum w l^2 (w = x^2) of every candidate level set make_qx_quants weighs."""
    x = x.astype(F32)
    mx = x[np.argmax(np.abs(x))]
    out = []
    w = x.astype(np.float64) ** 2
    for i in range(-9, 10):
        iscale = -(F32(nmax) + F32(0.1) * F32(i)) / mx if i else -F32(nmax) / mx
        L = np.clip(_rint(F32(iscale) * x), -nmax, nmax - 1).astype(np.float64)
        sl2 = (w * L * L).sum()
        if sl2 > 0:
            out.append((w * x * L).sum() ** 2 / sl2)
    return out


def q6_search_gap(oracle, seed=3, n=400):
    rng = np.random.default_rng(seed)
    gap = 0.0
    for x in (rng.standard_normal((n, 16)) * 0.02).astype(F32):
        scale, L = oracle.make_qx_quants(x)
        lv = L.astype(np.float64) - 32
        w = x.astype(np.float64) ** 2
        got = (w * x * lv).sum() ** 2 / (w * lv * lv).sum()
        best = max(qx_objectives(x))
        gap = max(gap, abs(got - best) / best)
        # the returned scale is the least-squares one for the returned levels
        assert abs(float(scale) - (w * x * lv).sum() / (w * lv * lv).sum()) <= 1e-5 * abs(float(scale))
    return gap


def test_q6_K_search_is_the_argmax(oracle):
    assert q6_search_gap(oracle) <= 1e-6


def representable_q6_K(seed, nsb=8):
    """GGUF Q6_K superblocks the quantizer maps back to themselves: each 16-value sub-block has
    its single largest magnitude at level -32, and one sub-block per superblock has scale -128."""
    rng = np.random.default_rng(seed)
    d = (rng.choice([-1.0, 1.0], nsb) * rng.uniform(0.5, 2.0, nsb) * 1e-4).astype(np.float16)
    sc = rng.integers(-127, 128, (nsb, 16))
    sc[sc == 0] = 1
    sc[np.arange(nsb), rng.integers(0, 16, nsb)] = -128
    lv = rng.integers(-31, 32, (nsb, 16, 16))
    lv[np.arange(nsb)[:, None], np.arange(16)[None, :], rng.integers(0, 16, (nsb, 16))] = -32
    L = (lv + 32).reshape(nsb, 2, 4, 32)  # [superblock][half][quarter][l]: value 128 h + 32 c + l
    b = np.zeros((nsb, 210), np.uint8)
    ql = np.zeros((nsb, 2, 64), np.int64)
    ql[:, :, 0:32] = (L[:, :, 0] & 15) | ((L[:, :, 2] & 15) << 4)
    ql[:, :, 32:64] = (L[:, :, 1] & 15) | ((L[:, :, 3] & 15) << 4)
    qh = (L[:, :, 0] >> 4) | ((L[:, :, 1] >> 4) << 2) | ((L[:, :, 2] >> 4) << 4) | ((L[:, :, 3] >> 4) << 6)
    b[:, 0:128] = ql.reshape(nsb, 128)
    b[:, 128:192] = qh.reshape(nsb, 64)
    b[:, 192:208] = sc.astype(np.int8).view(np.uint8)
    b[:, 208:210] = d.view(np.uint8).reshape(nsb, 2)
    return b


def q6_roundtrip_mismatch(oracle, seed=4, nsb=64):
    b = representable_q6_K(seed, nsb)
    y = q6_K_dequant(b.ravel(), 256 * nsb).reshape(1, -1)
    again = oracle.quantize_chunk(O.Q6_K, y)
    return int((again.reshape(nsb, 210) != b).any(-1).sum())


def test_q6_K_idempotent_on_representable_blocks(oracle):
    assert q6_roundtrip_mismatch(oracle) == 0


# ------------------------------------------------------- planted mistakes ----
PINS = {
    "q4_search": lambda o: q4_search_gap(o) <= 1e-4,
    "q4_wrapper": lambda o: q4_wrapper_mismatch(o) <= 0.05,
    "q4_roundtrip": lambda o: q4_roundtrip_mismatch(o) == 0,
    "q6_search": lambda o: q6_search_gap(o) <= 1e-6,
    "q6_roundtrip": lambda o: q6_roundtrip_mismatch(o) == 0,
}


@pytest.mark.parametrize("mutation,caught_by", [
    (O.MUT_Q4K_NO_SEARCH, "q4_search"), (O.MUT_Q4K_RDELTA, "q4_search"), (O.MUT_Q4K_PACK, "q4_roundtrip"),
    (O.MUT_Q4K_CALL_NSTEP0, "q4_wrapper"), (O.MUT_Q4K_CALL_UNIT_WEIGHTS, "q4_wrapper"),
    (O.MUT_Q4K_CALL_RMIN, "q4_wrapper"),
    (O.MUT_Q6K_NO_SEARCH, "q6_search"), (O.MUT_Q6K_STEP, "q6_search"), (O.MUT_Q6K_ISCALE, "q6_roundtrip")])
def test_planted_mistake_is_caught(oracle, mutation, caught_by):
    oracle.set_mutation(mutation)
    try:
        assert not PINS[caught_by](oracle)
    finally:
        oracle.set_mutation(O.MUT_NONE)
    assert all(pin(oracle) for pin in PINS.values())  # and all pass again without it
