"""End to end: the decoder-embedder runner (Qwen3-style graph, every mul_mat on the
quantized GPU path, the other ops as fp32 kernels) against the CPU reference decoder on the
same weight bytes and token ids.  Gates: the pooled embeddings at cosine >= 0.9999 and, for
one-layer models, the median row of the last hidden state within 1e-5 of the reference (the
kernels are exact up to fp32 rounding).

Why 0.9999 and not the encoder's 0.99999: each mul_mat requantizes its fp32 input, so an
activation that the GPU and the fp64 reference round to fp32 an ulp apart can land on
different quants (about 1e-5 of the elements quantized, a few per layer at these sizes).
Such a flip moves its row by one quant step (~1e-3 relative) and, through causal attention,
the later rows of the next layer.  Mean pooling (the encoder) averages it away; last-token
pooling does not, so a flip reaching the last row costs ~1e-5 of cosine whichever fp32
evaluation order is used -- changing only the attention's rounding moved a Q8_0 case from
1.0 to 0.999989.  A flip in an early row of the first layer also reaches most rows of the
second through its key and value, so the row-error gate applies to one-layer models only.  The kernels themselves are checked without quantization in the loop by
tests/test_gpu_decoder_ops.py (attention to 1e-5 of its output).  F16 activations round every
element to fp16 (a 2^-11 step), so its median bound is that step instead.
"""
import numpy as np
import pytest

import decoder_oracle
import oracle_ffi as O
from gpu_util import host, stream

pytestmark = pytest.mark.gpu

COSINE_MIN = 0.9999
SMALL = dict(n_layer=2, n_embd=256, n_head=4, n_kv_head=2, head_dim=64, n_ff=512, n_vocab=1000, rms_norm_eps=1e-6,
             rope_theta=1e6, causal=1, pooling=2)


def _check(hp, wtype, B, T, name, oracle, cos_min=COSINE_MIN):
    """Runs both sides; returns nothing, asserts the gates (row gate for one-layer models)."""
    import torch
    from crispembed_amd import decoder, synth
    W = decoder.synthetic_weights(hp, wtype, name=name)
    ids = synth.integers(f"{name}/ids_{B}x{T}", (B, T), 0, hp["n_vocab"] - 1)
    dec = decoder.DecoderEmbedder(hp, wtype, W)
    ids_d = torch.from_numpy(ids.ravel().copy()).cuda()
    out = torch.empty((B, hp["n_embd"]), dtype=torch.float32, device="cuda")
    hid = torch.empty((B * T, hp["n_embd"]), dtype=torch.float32, device="cuda")
    dec.encode(ids_d.data_ptr(), B, T, out.data_ptr(), stream(), hidden_dev=hid.data_ptr())
    pooled, hidden = host(out), host(hid)
    ref_pooled, ref_hidden = decoder_oracle.encode(oracle, hp, wtype, W, ids)
    cos = (pooled * ref_pooled).sum(-1) / (np.linalg.norm(pooled, axis=-1) * np.linalg.norm(ref_pooled, axis=-1))
    row_err = np.abs(hidden - ref_hidden).max(-1) / np.abs(ref_hidden).max()
    print(f"{name}: min cosine {cos.min():.8f}, hidden row error max {row_err.max():.2e} "
          f"median {np.median(row_err):.2e}")
    assert np.isfinite(pooled).all()
    assert np.allclose(np.linalg.norm(pooled, axis=-1), 1.0, atol=1e-5)
    assert cos.min() >= cos_min
    if hp["n_layer"] == 1:
        assert np.median(row_err) <= (5e-4 if wtype == O.F16 else 1e-5)


@pytest.mark.parametrize("wtype", [O.Q8_0, O.Q4_K, O.Q6_K, O.F16])
def test_small_decoder(oracle, wtype):
    _check(dict(SMALL), wtype, 2, 40, f"dec_small_{wtype}", oracle)


@pytest.mark.parametrize("wtype", [O.Q8_0, O.Q4_K, O.Q6_K, O.F16])
def test_one_layer_rows(oracle, wtype):
    _check(dict(SMALL, n_layer=1), wtype, 2, 40, f"dec_l1_{wtype}", oracle)


def test_head_dim_128_multi_block(oracle):
    """head_dim 128, one key/value head for two query heads, T spanning two query workgroups."""
    hp = dict(SMALL, n_layer=1, n_head=2, n_kv_head=1, head_dim=128)
    _check(hp, O.Q4_K, 2, 200, "dec_hd128", oracle)


@pytest.mark.parametrize("wtype", [O.Q8_0, O.Q6_K])
def test_long_sequence_causal(oracle, wtype):
    """T = 200: seven key blocks, the last one partly past the sequence end."""
    _check(dict(SMALL, n_layer=1), wtype, 2, 200, f"dec_long_{wtype}", oracle)


def test_gemv_rows(oracle):
    """B*T <= 8: every mul_mat takes the GEMV path."""
    _check(dict(SMALL), O.Q4_K, 2, 3, "dec_gemv", oracle)


def test_bidirectional_mean_pooling(oracle):
    _check(dict(SMALL, causal=0, pooling=1), O.Q8_0, 3, 33, "dec_mean", oracle)


def test_bidirectional_long(oracle):
    _check(dict(SMALL, n_layer=1, causal=0, pooling=1), O.Q4_K, 2, 150, "dec_mean_long", oracle)


def _encode(hp, wtype, B, T, name):
    import torch
    from crispembed_amd import decoder, synth
    W = decoder.synthetic_weights(hp, wtype, name=name)
    ids = synth.integers(f"{name}/ids_{B}x{T}", (B, T), 0, hp["n_vocab"] - 1)
    dec = decoder.DecoderEmbedder(hp, wtype, W)
    ids_d = torch.from_numpy(ids.ravel().copy()).cuda()
    out = torch.empty((B, hp["n_embd"]), dtype=torch.float32, device="cuda")
    hid = torch.empty((B * T, hp["n_embd"]), dtype=torch.float32, device="cuda")
    dec.encode(ids_d.data_ptr(), B, T, out.data_ptr(), stream(), hidden_dev=hid.data_ptr())
    return host(out), host(hid)


@pytest.mark.parametrize("wtype", [O.Q4_K, O.Q6_K])
def test_norm_q8_K_matches_separate_quantizer(monkeypatch, wtype):
    """The residual + RMS norm that also leaves its result as the Q8_K activation of the qkv and
    gate|up products, against the norm followed by the activation quantizer
    (MQ_DECODER_NORM_PASS=1).  The quantization code is shared; only the norm's sum order
    differs, so the embeddings agree to a cosine of 0.99999 and the hidden states closely."""
    hp = dict(SMALL)
    a_pool, a_hid = _encode(hp, wtype, 2, 64, f"dec_nq_{wtype}")
    monkeypatch.setenv("MQ_DECODER_NORM_PASS", "1")
    b_pool, b_hid = _encode(hp, wtype, 2, 64, f"dec_nq_{wtype}")
    cos = (a_pool * b_pool).sum(-1) / (np.linalg.norm(a_pool, axis=-1) * np.linalg.norm(b_pool, axis=-1))
    assert cos.min() >= 0.99999
    assert np.median(np.abs(a_hid - b_hid)) <= 1e-4 * np.abs(b_hid).max()
