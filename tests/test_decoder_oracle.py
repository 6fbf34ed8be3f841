"""Pins the CPU reference decoder's building blocks with closed forms (no GPU)."""
import numpy as np

import decoder_oracle as D


def test_rope_neox_is_a_complex_rotation():
    rng = np.random.default_rng(0)
    d, T, base = 64, 9, 1e6
    x = rng.standard_normal((T, d)).astype(np.float32)
    y = D.rope_neox(x, np.arange(T), base)
    z = (x[:, : d // 2] + 1j * x[:, d // 2:]).astype(np.complex128)
    ang = np.arange(T)[:, None] * base ** (-np.arange(d // 2) / (d // 2))
    w = z * np.exp(1j * ang)
    assert np.allclose(y[:, : d // 2], w.real, atol=2e-6) and np.allclose(y[:, d // 2:], w.imag, atol=2e-6)
    # position 0 is the identity; rotation preserves each pair's norm
    assert np.array_equal(y[0], x[0])
    assert np.allclose(np.abs(w), np.abs(z))


def test_rms_norm_closed_form():
    x = np.array([[3.0, -4.0, 0.0, 0.0]], np.float32)
    w = np.array([1.0, 2.0, 3.0, 4.0], np.float32)
    y = D.rms_norm(x, w, 0.0)
    assert np.allclose(y, [[3 / 2.5, -8 / 2.5, 0, 0]])


def test_rms_norm_catches_mean_subtraction():
    """A LayerNorm-style mean subtraction would change a constant row; RMS norm keeps it."""
    x = np.full((1, 8), 2.0, np.float32)
    assert np.allclose(D.rms_norm(x, np.ones(8, np.float32), 0.0), 1.0)


def test_fp32_pipeline_is_the_same_decoder(oracle):
    """decoder_oracle.encode_f32 (the fp32, ggml-CPU-like pipeline that measures how far an fp32
    run lands from the fp64 one) computes the same model as encode: a 2-layer decoder's pooled
    embeddings agree at the decoder bar, and its rope cache's angles are pos * base^(-2i/d) to fp32
    precision."""
    from crispembed_amd import decoder
    import oracle_ffi as O
    hp = dict(n_layer=2, n_embd=256, n_head=4, n_kv_head=2, head_dim=128, n_ff=512, n_vocab=300, rms_norm_eps=1e-6,
              rope_theta=1e6, causal=1, pooling=2)
    W = decoder.synthetic_weights(hp, O.Q4_K, name="fp32pipe")
    ids = np.random.default_rng(3).integers(0, hp["n_vocab"], (2, 40)).astype(np.int32)
    ref, _ = D.encode(oracle, hp, O.Q4_K, W, ids)
    got = D.encode_f32(oracle, hp, O.Q4_K, W, ids, nthreads=4)
    assert ((got.astype(np.float64) * ref).sum(-1) >= 0.9999).all()
    c, s = D.rope_cache_f32(40, 128, 1e6)
    ang = np.arange(40)[:, None] * 1e6 ** (-2.0 * np.arange(64) / 128)
    assert np.abs(c - np.cos(ang)).max() < 1e-4 and np.abs(s - np.sin(ang)).max() < 1e-4
