"""The decoder runner's non-MUL_MAT kernels on identical inputs against fp64 references
(no quantization in the loop, so these bars are the kernels' own fp32 error):
  mq_qk_norm_rope: per-head RMS norm + NEOX RoPE, max|d| <= 1e-4 max|ref| (the angle is built
                   like ggml's rope cache, pos * theta_scale^i by repeated fp32 products, so
                   it differs from the exact fp64 angle by a few fp32 ulps of pos)
  mq_attention:    causal / full, grouped-query attention, max|d| <= 1e-5 max|ref|."""
import ctypes

import numpy as np
import pytest

import decoder_oracle as D
from gpu_util import dev, host, stream

pytestmark = pytest.mark.gpu


def _qkv(B, T, nq, nkv, hd, seed, pad=4):
    rng = np.random.default_rng(seed)
    ld = (nq + 2 * nkv) * hd + pad
    x = np.zeros((B * T, ld), np.float32)
    x[:, : ld - pad] = rng.standard_normal((B * T, ld - pad)).astype(np.float32)
    return x, ld


@pytest.mark.parametrize("hd,nq,nkv", [(64, 4, 2), (128, 2, 1), (128, 4, 4)])
@pytest.mark.parametrize("norm", [True, False])
def test_qk_norm_rope(hd, nq, nkv, norm):
    from crispembed_amd import mq
    B, T, theta, eps = 2, 37, 1e6, 1e-6
    x, ld = _qkv(B, T, nq, nkv, hd, 11 * hd + nq)
    rng = np.random.default_rng(5)
    qn = (1 + 0.1 * rng.standard_normal(hd)).astype(np.float32)
    kn = (1 + 0.1 * rng.standard_normal(hd)).astype(np.float32)
    xd, qd, kd = dev(x), dev(qn), dev(kn)
    mq.check(mq.lib().mq_qk_norm_rope(ctypes.c_void_p(xd.data_ptr()), ld,
                                      ctypes.c_void_p(qd.data_ptr()) if norm else None,
                                      ctypes.c_void_p(kd.data_ptr()) if norm else None, eps, nq, nkv, hd, T, theta,
                                      B * T, stream()))
    got = host(xd)
    ref = x.copy()
    pos = np.arange(B * T) % T
    for h in range(nq + nkv):
        blk = x[:, h * hd:(h + 1) * hd]
        if norm:
            blk = D.rms_norm(blk, qn if h < nq else kn, eps)
        for r in range(B * T):
            ref[r, h * hd:(h + 1) * hd] = D.rope_neox(blk[r:r + 1], np.array([pos[r]]), theta)[0]
    n = (nq + nkv) * hd
    assert np.abs(got[:, :n] - ref[:, :n]).max() <= 1e-4 * np.abs(ref[:, :n]).max()
    assert np.array_equal(got[:, n:], x[:, n:])  # value heads and padding untouched


def _attn_ref(x, B, T, nq, nkv, hd, scale, causal):
    q = x[:, : nq * hd].reshape(B, T, nq, hd).transpose(0, 2, 1, 3).astype(np.float64)
    k = x[:, nq * hd:(nq + nkv) * hd].reshape(B, T, nkv, hd).transpose(0, 2, 1, 3).astype(np.float64)
    v = x[:, (nq + nkv) * hd:(nq + 2 * nkv) * hd].reshape(B, T, nkv, hd).transpose(0, 2, 1, 3).astype(np.float64)
    k, v = np.repeat(k, nq // nkv, axis=1), np.repeat(v, nq // nkv, axis=1)
    s = np.einsum("bhid,bhjd->bhij", q, k) * scale
    if causal:
        s = np.where(np.tril(np.ones((T, T), bool)), s, -np.inf)
    p = np.exp(s - s.max(-1, keepdims=True))
    p /= p.sum(-1, keepdims=True)
    return np.einsum("bhij,bhjd->bihd", p, v).reshape(B * T, nq * hd)


@pytest.mark.parametrize("form", ["auto", "frag"])
@pytest.mark.parametrize("causal", [1, 0])
@pytest.mark.parametrize("hd,nq,nkv", [(64, 4, 2), (128, 2, 1), (128, 16, 8), (64, 3, 3), (128, 6, 2)])
@pytest.mark.parametrize("B,T", [(1, 1), (2, 37), (2, 200), (1, 300)])
def test_attention(causal, hd, nq, nkv, B, T, form, monkeypatch):
    """The runner's attention against an fp64 reference.  form "frag" forces the 8-wave kernel
    (its key/value blocks shared through LDS by both heads of a workgroup: an odd nq leaves a
    workgroup's second head empty, nq / nkv = 3 gives workgroups whose two heads read different
    key/value heads, and ragged T leaves query tiles empty); "auto" lets small grids take the
    split-key kernel."""
    from crispembed_amd import mq
    import torch
    if form == "frag":
        monkeypatch.setenv("MQ_ATTN_SPLIT", "0")
    x, ld = _qkv(B, T, nq, nkv, hd, 7 * T + hd + nq + causal)
    x *= 2.0  # sharper softmax
    scale = 1.0 / np.sqrt(hd)
    xd = dev(x)
    out = torch.full((B * T, nq * hd), float("nan"), dtype=torch.float32, device="cuda")
    nws = mq.lib().mq_attention_workspace_bytes(B, T, nkv, hd)
    assert nws == B * nkv * ((T + 31) // 32) * (hd // 4) * 1024
    ws = torch.full((nws // 4,), float("nan"), dtype=torch.float32, device="cuda")  # stale contents must not leak
    mq.check(mq.lib().mq_attention(ctypes.c_void_p(xd.data_ptr()), ld, ctypes.c_void_p(out.data_ptr()), nq * hd, B, T,
                                   nq, nkv, hd, scale, causal, ctypes.c_void_p(ws.data_ptr()), nws, stream()))
    got = host(out)
    ref = _attn_ref(x, B, T, nq, nkv, hd, scale, causal)
    assert np.isfinite(got).all()
    assert np.abs(got - ref).max() <= 1e-5 * np.abs(ref).max()
    if causal:  # the first query of each sequence attends to its own value only
        vcol = (nq + nkv) * hd
        for b in range(B):
            for h in range(nq):
                kv = h // (nq // nkv)
                assert np.allclose(got[b * T, h * hd:(h + 1) * hd], x[b * T, vcol + kv * hd:vcol + (kv + 1) * hd],
                                   atol=1e-6)
