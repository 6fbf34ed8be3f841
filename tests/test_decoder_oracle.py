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
