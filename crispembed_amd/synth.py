"""Deterministic synthetic inputs: splitmix64 counter stream -> fp64 uniforms ->
Box-Muller normals in fp64 -> fp32.  The same bytes feed every consumer.

Seeds are FNV-1a 64 of "<config>/<tensor>" so each tensor of each workload has
its own stream, independent of generation order.
"""
import numpy as np

_GOLDEN = np.uint64(0x9E3779B97F4A7C15)
_M1 = np.uint64(0xBF58476D1CE4E5B9)
_M2 = np.uint64(0x94D049BB133111EB)


def seed_of(name: str) -> int:
    h = 0xCBF29CE484222325
    for b in name.encode():
        h ^= b
        h = (h * 0x100000001B3) & 0xFFFFFFFFFFFFFFFF
    return h


def splitmix64(seed: int, n: int, offset: int = 0) -> np.ndarray:
    """n outputs of splitmix64 started at `seed`, skipping `offset` outputs."""
    with np.errstate(over="ignore"):
        z = np.uint64(seed) + (np.arange(offset + 1, offset + n + 1, dtype=np.uint64) * _GOLDEN)
        z = (z ^ (z >> np.uint64(30))) * _M1
        z = (z ^ (z >> np.uint64(27))) * _M2
        return z ^ (z >> np.uint64(31))


def uniform01(seed: int, n: int, offset: int = 0) -> np.ndarray:
    """fp64 uniforms in (0, 1]."""
    z = splitmix64(seed, n, offset)
    return ((z >> np.uint64(11)).astype(np.float64) + 1.0) * (1.0 / 9007199254740992.0)


def normal(name: str, shape, mean=0.0, std=1.0, chunk=1 << 22) -> np.ndarray:
    """fp32 N(mean, std^2) array, generated in chunks to bound memory."""
    n = int(np.prod(shape))
    seed = seed_of(name)
    out = np.empty(n, dtype=np.float32)
    npairs = (n + 1) // 2
    for p0 in range(0, npairs, chunk):
        p1 = min(npairs, p0 + chunk)
        u = uniform01(seed, 2 * (p1 - p0), 2 * p0)
        u1, u2 = u[0::2], u[1::2]
        r = np.sqrt(-2.0 * np.log(u1))
        t = 2.0 * np.pi * u2
        z = np.empty(2 * (p1 - p0), dtype=np.float64)
        z[0::2] = r * np.cos(t)
        z[1::2] = r * np.sin(t)
        z = mean + std * z
        lo = 2 * p0
        hi = min(n, 2 * p1)
        out[lo:hi] = z[: hi - lo].astype(np.float32)
    return out.reshape(shape)


def integers(name: str, shape, lo: int, hi: int) -> np.ndarray:
    """Uniform integers in [lo, hi] (inclusive), int32."""
    n = int(np.prod(shape))
    z = splitmix64(seed_of(name), n)
    span = np.uint64(hi - lo + 1)
    return (lo + (z % span).astype(np.int64)).astype(np.int32).reshape(shape)


def gelu_erf(x: np.ndarray) -> np.ndarray:
    """0.5*x*(1+erf(x/sqrt2)) in fp64, rounded to fp32 (ggml_gelu_erf, src/crispembed.cpp:1415)."""
    from math import erf
    xv = x.astype(np.float64)
    try:
        from scipy.special import erf as verf
        e = verf(xv / np.sqrt(2.0))
    except ImportError:  # pragma: no cover
        e = np.vectorize(erf)(xv / np.sqrt(2.0))
    return (0.5 * xv * (1.0 + e)).astype(np.float32)
