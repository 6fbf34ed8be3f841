"""CPU checks of tests/act_layout.py, the expected GEMM-path workspace built from oracle blocks.

The builder scatters with an index formula; these tests read its output back with an
independent reshape/transpose decoder (gpu_util.live_q8_0_planes, the fragment order written
as array axes) and recompute the Q8_K min-term operands from the quants themselves rather
than from ggml's bsums, so an index slip in either would show.
"""
import numpy as np
import pytest

import act_layout as AL
import oracle_ffi as O
from gpu_util import live_q8_0_planes


def _x(m, k, seed):
    return np.random.default_rng(seed).standard_normal((m, k)).astype(np.float32)


@pytest.mark.parametrize("m,k", [(37, 384), (300, 1536), (5, 128)])
def test_q8_0_image_reads_back(oracle, m, k):
    x = _x(m, k, m + k)
    blocks = oracle.quantize_act(O.Q8_0, x)
    img = AL.expected_image(O.Q8_0, blocks, m, k)
    q, d = live_q8_0_planes(img, m, k)
    q0, d0 = AL.decode_q8_0_blocks(blocks, k)
    assert np.array_equal(q.view(np.int8), q0)
    assert np.array_equal(d.T, d0)
    p = AL.planes(O.Q8_0, m, k)
    o, n = p["xq"]
    assert np.count_nonzero(img[o:o + n]) == np.count_nonzero(q0)  # pad rows are zero


def test_q8_0_image_k_padding(oracle):
    """K = 96 is padded to a 128-byte stage: the last 32 bytes of every row and their scale
    row are zero."""
    m, k = 40, 96
    x = _x(m, k, 3)
    img = AL.expected_image(O.Q8_0, oracle.quantize_act(O.Q8_0, x), m, k)
    p = AL.planes(O.Q8_0, m, k)
    assert p["kb_pad"] == 128
    m_pad = p["m_pad"]
    o, n = p["xq"]
    frag = img[o:o + n].reshape(m_pad // 32, 4, 2, 32, 16)  # [tile][chunk][half][row][byte]
    assert not frag[:, 3].any()
    o, n = p["xd"]
    d = img[o:o + n].view(np.float32).reshape(4, m_pad)
    assert not d[3].any() and d[:3, :m].all()


@pytest.mark.parametrize("m,k", [(37, 512), (70, 1024)])
def test_q8_K_image_reads_back(oracle, m, k):
    x = _x(m, k, 7 * m + k)
    blocks = oracle.quantize_act(O.Q4_K, x)
    img = AL.expected_image(O.Q4_K, blocks, m, k)
    p = AL.planes(O.Q4_K, m, k)
    m_pad, nsb = p["m_pad"], k // 256
    q0, d0, _ = AL.decode_q8_K_blocks(blocks, k)
    # quants: the same fragment order as Q8_0's (read back by the reshape decoder)
    o, n = p["xq"]
    q = img[o:o + n].view(np.int8).reshape(m_pad // 32, k // 32, 2, 32, 16).transpose(0, 3, 1, 2, 4)
    assert np.array_equal(q.reshape(m_pad, k)[:m], q0)
    o, n = p["xd"]
    assert np.array_equal(img[o:o + n].view(np.float32).reshape(nsb, m_pad)[:, :m].T, d0)
    # min-term fragments: lanes 0-31 B & 63, lanes 32-63 64 (B >> 6), B from the quants
    o, n = p["xmin"]
    f = img[o:o + n].view(np.float16).reshape(m_pad // 32, nsb, 64, 8).astype(np.int64)
    B = q0.astype(np.int64).reshape(m, nsb, 8, 32).sum(-1)
    r = np.arange(m)
    assert np.array_equal(f[r // 32, :, r % 32, :] + f[r // 32, :, 32 + r % 32, :], B)
    assert (f[r // 32, :, r % 32, :] >= 0).all() and (f[r // 32, :, r % 32, :] < 64).all()
    live = np.zeros(m_pad // 32 * 32, bool)
    live[:m] = True
    pad = ~live.reshape(-1, 32)
    assert not f.transpose(0, 2, 1, 3)[:, :32][pad].any()
