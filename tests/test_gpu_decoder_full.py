"""The Qwen3-Embedding-0.6B-shaped decoder embedder at its real workload: 28 layers, H 1024,
16 query / 8 key-value heads of 128, SwiGLU FFN 3072, RMS norm eps 1e-6, NEOX RoPE theta 1e6,
causal, Q4_K linears, 16 sequences x 512 tokens, last-token pooling (src/decoder_embed.cpp:
565-830, pooling :1044-1100).

The CPU decoder cannot run 16 x 512 tokens x 28 layers in seconds, and sequences are
independent (each attends causally to its own tokens), so the checks are:

* the whole batch: finite, unit-norm, pairwise-distinct embeddings, and two sampled sequences'
  embeddings in the batch of 16 against the same sequences encoded as a batch of 2 (a different
  GEMM tile grid);
* every layer of the 16 x 512 batch through the runner's observer (the scheduler eval callback
  contract): (1) each quantized activation a mat-mul reads (the q/k/v, o and gate/up inputs, all
  8192 rows) is byte-identical to the oracle's quantize_row_q8_K of the GPU's own fp32 input,
  and the down projection's input (silu(gate) * up, formed inside the quantizer with the device
  expf) to at least 99.9 % of its quants on the sampled rows; (2) teacher forcing on the two
  sampled sequences: every fp32 tensor of the layer (attention rows, normed FFN input, gate/up,
  the residual stream) equals the CPU decoder's layer computed from the GPU's own quantized
  activations, within 1e-5 of each tensor's scale;
* the two sequences end to end against the free-running CPU decoder: pooled cosine >= 0.9999.

Together: the GPU's quantization has no error of its own, every op between the quantizations
matches the CPU decoder to fp32 rounding, so what separates the free-running runs is an
activation the two sides round an ulp apart landing on a different quant (a flip), amplified
over 28 layers.  The free-running cosine is printed.

Weights: four random layers, each uploaded to seven of the 28 layers (separate device copies;
quantizing 28 distinct layers on the host takes about a minute), token table N(0, 0.02).
"""
import ctypes

import numpy as np
import pytest

import act_layout as AL
import decoder_oracle
import oracle_ffi as O
from bert_oracle import _w_deq
from gpu_util import fetch, host, stream

pytestmark = pytest.mark.gpu

B, T = 16, 512
SAMPLED = (0, 9)


@pytest.fixture(scope="module")
def qwen3(oracle):
    """The model, the 16 x 512 batch encoded once with the observer set; keeps the pooled
    embeddings, the sampled sequences' rows of every observed fp32 tensor, their quantized
    activations (decoded), and the byte checks of every row's quantization (run in the
    observer, on all 8192 rows, for the q/k/v, o and gate/up inputs)."""
    import torch
    from crispembed_amd import decoder, mq, synth
    hp = dict(decoder.QWEN3_EMBED_0_6B)
    sets = [decoder.synthetic_weights(dict(hp, n_layer=1, n_vocab=1), O.Q4_K, name=f"qwen3_full{j}")["layers"][0]
            for j in range(4)]
    tok = np.random.default_rng(20261202).standard_normal((hp["n_vocab"], hp["n_embd"]), dtype=np.float32) * 0.02
    out_norm = (1.0 + 0.02 * np.random.default_rng(7).standard_normal(hp["n_embd"])).astype(np.float32)
    W = {"tok": tok, "out_norm": out_norm, "layers": [sets[il % 4] for il in range(hp["n_layer"])]}
    dec = decoder.DecoderEmbedder(hp, O.Q4_K, W)
    ids = synth.integers(f"qwen3/ids_{B}x{T}", (B, T), 0, hp["n_vocab"] - 1).astype(np.int32)
    rows = np.concatenate([np.arange(b * T, (b + 1) * T) for b in SAMPLED])
    F = hp["n_ff"]
    seen, byte_checks, silu_same = {}, [], []

    def cb(name, layer, x, r, c, xq, xq_bytes, user):
        try:
            name = name.decode()
            k = F if name == "ffn_gate_up" else c
            q = AL.decode_image(O.Q4_K, fetch(xq, AL.planes(O.Q4_K, r, k)["total"]), r, k) if xq else None
            if name in ("attn_norm", "attn_out", "ffn_norm"):  # every row: the oracle's bytes
                xa = fetch(x, r * c * 4).view(np.float32).reshape(r, c)
                qo, do_, _ = AL.decode_q8_K_blocks(oracle.quantize_act(O.Q4_K, xa), k)
                byte_checks.append((name, layer, bool(np.array_equal(q[0], qo)),
                                    bool(np.array_equal(q[1].view(np.uint32), do_.view(np.uint32)))))
                xs = xa[rows].copy()
            else:
                xs = np.concatenate([fetch(x + int(b * T * c * 4), T * c * 4).view(np.float32).reshape(T, c)
                                     for b in SAMPLED])
            if name == "ffn_gate_up":  # silu(gate) * up is formed with the device expf
                qo, _, _ = AL.decode_q8_K_blocks(oracle.quantize_act(O.Q4_K, decoder_oracle.silu_mul(xs)), F)
                silu_same.append(float(np.mean(q[0][rows] == qo)))
            seen[(name, layer)] = (xs, None if q is None else (q[0][rows].copy(), q[1][rows].copy()))
        except Exception as e:  # an exception cannot cross the C callback: record it
            byte_checks.append((f"observer error: {e!r}", layer, False, False))

    fn = mq.DECODER_OBSERVER(cb)
    mq.check(mq.lib().mq_decoder_set_observer(dec.h, fn, None))
    ids_d = torch.from_numpy(ids.ravel().copy()).cuda()
    out = torch.empty((B, hp["n_embd"]), dtype=torch.float32, device="cuda")
    try:
        dec.encode(ids_d.data_ptr(), B, T, out.data_ptr(), stream())
        pooled = host(out)
    finally:
        mq.check(mq.lib().mq_decoder_set_observer(dec.h, None, None))
    yield dict(hp=hp, W=W, dec=dec, ids=ids, pooled=pooled, seen=seen, byte_checks=byte_checks, silu_same=silu_same)
    del dec


def test_full_batch_properties(qwen3):
    pooled = qwen3["pooled"]
    assert np.isfinite(pooled).all()
    assert np.allclose(np.linalg.norm(pooled, axis=-1), 1.0, atol=1e-5)
    cos = pooled @ pooled.T
    assert (cos[~np.eye(B, dtype=bool)] < 0.9999).all()  # 16 distinct sequences, 16 distinct embeddings
    assert len(qwen3["seen"]) == 5 * qwen3["hp"]["n_layer"]


def test_unobserved_batch_bit_identical(qwen3, monkeypatch):
    """The 16 x 512 batch without the observer: the gate|up GEMM then forms silu(gate) * up in
    its store (mq_mul_mat_q_swiglu) instead of writing gate and up for the quantizer's prologue,
    and the normed rows stay in quantized form only.  Every quantized byte is the same, so the
    pooled embeddings equal the observed run's bit for bit; so do those of the two-step form
    (MQ_DECODER_NO_GLU=1) without the observer."""
    import torch
    hp, dec, ids = qwen3["hp"], qwen3["dec"], qwen3["ids"]
    ids_d = torch.from_numpy(ids.ravel().copy()).cuda()
    for no_glu in (False, True):
        if no_glu:
            monkeypatch.setenv("MQ_DECODER_NO_GLU", "1")
        out = torch.empty((B, hp["n_embd"]), dtype=torch.float32, device="cuda")
        dec.encode(ids_d.data_ptr(), B, T, out.data_ptr(), stream())
        assert np.array_equal(host(out).view(np.uint32), qwen3["pooled"].view(np.uint32)), no_glu


def test_sampled_batch_independent(qwen3):
    """A sequence's embedding in a batch of 2 against the batch of 16 (another GEMM tile grid):
    the same computation up to fp32 rounding, so at the end-to-end bar."""
    import torch
    hp, dec, ids = qwen3["hp"], qwen3["dec"], qwen3["ids"]
    ids2 = ids[list(SAMPLED)]
    ids_d = torch.from_numpy(ids2.ravel().copy()).cuda()
    out = torch.empty((len(SAMPLED), hp["n_embd"]), dtype=torch.float32, device="cuda")
    dec.encode(ids_d.data_ptr(), len(SAMPLED), T, out.data_ptr(), stream())
    p2 = host(out)
    cos = [float(p2[i] @ qwen3["pooled"][b]) for i, b in enumerate(SAMPLED)]
    print("batch of 2 against batch of 16, pooled cosine:", cos)
    assert min(cos) >= 0.9999


def test_quantized_activations_are_the_oracles(qwen3):
    """(1): every quantized activation equals the oracle's quantization of the GPU's own input."""
    bad = [c for c in qwen3["byte_checks"] if not (c[2] and c[3])]
    assert len(qwen3["byte_checks"]) == 3 * qwen3["hp"]["n_layer"]
    assert not bad, bad[:5]
    worst = min(qwen3["silu_same"])
    print(f"silu(gate) * up quants identical to the oracle's: worst layer {worst:.6f}")
    assert worst >= 0.999


def test_teacher_forced_layers(qwen3):
    """(2): each layer from the GPU's own quantized activations, every fp32 tensor within 1e-5,
    on the sampled sequences' rows of the 16 x 512 batch."""
    hp, W, ids, seen = qwen3["hp"], qwen3["W"], qwen3["ids"], qwen3["seen"]
    ids2 = ids[list(SAMPLED)]
    Bs = ids2.shape[0]
    H, F, eps = hp["n_embd"], hp["n_ff"], hp["rms_norm_eps"]
    qd = hp["n_head"] * hp["head_dim"]
    deq = {}
    x = W["tok"][ids2.ravel()].astype(np.float32)
    worst = {}
    for il, lay in enumerate(W["layers"]):
        key = id(lay)
        if key not in deq:
            deq[key] = {"qkv": np.concatenate([_w_deq(O.Q4_K, lay[w], H) for w in ("wq", "wk", "wv")]),
                        "o": _w_deq(O.Q4_K, lay["wo"], qd),
                        "gu": np.concatenate([_w_deq(O.Q4_K, lay[w], H) for w in ("wgate", "wup")]),
                        "down": _w_deq(O.Q4_K, lay["wdown"], F)}
        acts = {}
        for n in ("attn_norm", "attn_out", "ffn_norm", "ffn_gate_up"):
            q, d = seen[(n, il)][1]
            acts[n] = (q.reshape(q.shape[0], -1, 256).astype(np.float64) *
                       d[:, :, None].astype(np.float64)).reshape(q.shape[0], -1)
        ref = decoder_oracle.layer_from_quants(hp, lay, deq[key], x, acts, Bs, T)
        ref["attn_norm"] = decoder_oracle.rms_norm(x, lay["attn_norm"], eps)
        for name in ("attn_norm", "attn_out", "ffn_norm", "ffn_gate_up", "l_out"):
            g, r = seen[(name, il)][0], ref[name]
            err = float(np.abs(g.astype(np.float64) - r).max() / np.abs(r).max())
            worst[name] = max(worst.get(name, 0.0), err)
            assert err <= 1e-5, (name, il, err)
        x = seen[("l_out", il)][0]
    print("teacher-forced worst relative error per tensor:", worst)


def test_sampled_sequences_end_to_end(oracle, qwen3):
    """The sampled sequences of the 16 x 512 batch against the free-running CPU decoder, and
    where the decoder's end-to-end bar sits: the same decoder run on the CPU as an fp32 pipeline
    (ggml-CPU-like order, decoder_oracle.encode_f32) lands as far from the fp64 one as the GPU
    does -- measured 0.999956 / 0.999965 -- so 0.99999 is out of reach for any fp32 pipeline that
    requantizes every mat-mul's input over 28 layers; the GPU's spread must be of that order (no
    more than 3 times the fp32 CPU pipeline's distance), and the GPU and the fp32 CPU pipeline
    are as close to each other."""
    import os
    hp, W, ids = qwen3["hp"], qwen3["W"], qwen3["ids"]
    ids2 = ids[list(SAMPLED)]
    ref, _ = decoder_oracle.encode(oracle, hp, O.Q4_K, W, ids2)
    got = qwen3["pooled"][list(SAMPLED)]
    cos = (got * ref).sum(-1)
    cpu32 = decoder_oracle.encode_f32(oracle, hp, O.Q4_K, W, ids2, nthreads=min(16, os.cpu_count() or 8))
    cos32 = (cpu32.astype(np.float64) * ref).sum(-1)
    cos_gc = (cpu32.astype(np.float64) * got).sum(-1)
    print("free-running pooled cosine per sequence: GPU vs fp64", cos, "fp32 CPU vs fp64", cos32,
          "GPU vs fp32 CPU", cos_gc)
    assert cos.min() >= 0.9999
    assert cos32.max() < 0.99999  # an fp32 CPU pipeline does not reach the north star's bar either
    assert (1 - cos).max() <= 3 * (1 - cos32).max() and (1 - cos_gc).max() <= 3 * (1 - cos32).max()
