"""End to end: the BERT-encoder runner (all mul_mats on the quantized GPU path, the
other ops as fp32 kernels) against the CPU reference encoder on the same weight bytes
and token ids.  Gate: cosine of the pooled embeddings >= 0.99999."""
import ctypes

import numpy as np
import pytest

import bert_oracle
import oracle_ffi as O
from gpu_util import host, stream

pytestmark = pytest.mark.gpu

COSINE_MIN = 0.99999
SMALL = dict(n_layer=2, n_embd=128, n_head=4, n_ff=512, n_vocab=1000, n_max_pos=64, n_type=2, layer_norm_eps=1e-12)


def _run(hp, wtype, B, T, name):
    import torch
    from crispembed_amd import bert, synth
    W = bert.synthetic_weights(hp, wtype, name=name)
    ids = synth.integers(f"{name}/ids_{B}x{T}", (B, T), min(1000, hp["n_vocab"] // 2), hp["n_vocab"] - 1)
    enc = bert.BertEncoder(hp, wtype, W)
    ids_d = torch.from_numpy(ids.ravel().copy()).cuda()
    out = torch.empty((B, hp["n_embd"]), dtype=torch.float32, device="cuda")
    hid = torch.empty((B * T, hp["n_embd"]), dtype=torch.float32, device="cuda")
    enc.encode(ids_d.data_ptr(), B, T, out.data_ptr(), stream(), hidden_dev=hid.data_ptr())
    return W, ids, host(out), host(hid)


def _check(hp, wtype, B, T, name, oracle):
    W, ids, pooled, hidden = _run(hp, wtype, B, T, name)
    ref_pooled, ref_hidden = bert_oracle.encode(oracle, hp, wtype, W, ids)
    cos = (pooled * ref_pooled).sum(-1) / (np.linalg.norm(pooled, axis=-1) * np.linalg.norm(ref_pooled, axis=-1))
    rel = np.abs(hidden - ref_hidden).max() / np.abs(ref_hidden).max()
    print(f"{name}: min cosine {cos.min():.8f}, hidden max rel err {rel:.2e}")
    assert np.isfinite(pooled).all()
    assert np.allclose(np.linalg.norm(pooled, axis=-1), 1.0, atol=1e-5)
    assert cos.min() >= COSINE_MIN
    return cos.min(), rel


@pytest.mark.parametrize("wtype", [O.Q8_0, O.Q4_K, O.Q6_K, O.F16])
def test_small_encoder(oracle, wtype):
    hp = dict(SMALL)
    if wtype in (O.Q4_K, O.Q6_K):
        hp.update(n_embd=256, n_head=4, n_ff=512)  # K-quants need k % 256 == 0
    _check(hp, wtype, 3, 16, f"small_{wtype}", oracle)


def test_small_encoder_gemv_rows(oracle):
    """B*T <= 8: every mul_mat takes the GEMV path."""
    _check(dict(SMALL), O.Q8_0, 2, 4, "small_gemv", oracle)


def test_minilm_l6_full_batch(oracle):
    """MiniLM-L6 shape, Q8_0, 32 sequences x 128 tokens (the embeddings/sec workload)."""
    from crispembed_amd import bert
    _check(dict(bert.MINILM_L6), O.Q8_0, 32, 128, "minilm", oracle)


@pytest.mark.parametrize("n_head", [8, 4, 2])
def test_q8_0_fused_path_head_dims(oracle, n_head):
    """The runner's Q8_0 path with every producer quantizing for its GEMM (norm, attention, FFN-up)
    and K / V written by the qkv GEMM as attention fragments, at head_dim 32, 64 and 128 (128:
    the attention's rows quantized after it)."""
    hp = dict(SMALL)
    hp.update(n_embd=256, n_head=n_head, n_ff=512, n_max_pos=128)
    _check(hp, O.Q8_0, 8, 64, f"fused_hd{256 // n_head}", oracle)


def test_kv_direct_equals_kv_pass(monkeypatch):
    """K / V fragments stored by the qkv GEMM are the bytes the attention's K / V pass writes:
    embeddings and hidden states bit-identical with MQ_BERT_KV_PASS=1 (the separate pass)."""
    hp = dict(SMALL)
    hp.update(n_embd=256, n_head=4, n_ff=512, n_max_pos=128)
    a = _run(hp, O.Q8_0, 8, 64, "kvd")
    monkeypatch.setenv("MQ_BERT_KV_PASS", "1")
    b = _run(hp, O.Q8_0, 8, 64, "kvd")
    assert np.array_equal(a[2], b[2]) and np.array_equal(a[3], b[3])
