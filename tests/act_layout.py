"""The GEMM-path activation workspace, built on the host from the oracle's GGUF blocks.

The MFMA GEMM reads X quantized in a tiled ("fragment-major") layout, not in ggml's block
layout: quants in 1 KB fragments (lane L of fragment (row tile rt, 32-byte K chunk kc) holds
row 32 rt + L % 32, bytes 32 kc + 16 (L // 32) .. + 16), the per-block scales as float
planes [block][m_pad], and for Q8_K the min-term operand of the Q4_K GEMM (B_j = the sum of
the 32 quants of sub-block j, as B_j & 63 and 64 (B_j >> 6) in fp16).  Rows past m and K
bytes past the row are zero.  This module restates that layout from its definition so a test
can build the bytes the GPU must write from `oracle.quantize_act` output and compare the whole
buffer: a quantizer whose quants, scales or sums differ from ggml's in any block fails.
"""
import numpy as np

import oracle_ffi as O


def _pad(x, a):
    return -(-x // a) * a


def _align256(x):
    return _pad(x, 256)


def planes(wtype, m, k):
    """Byte offsets and sizes of the tiled layout: dict(xq, xd, xmin, total, m_pad, kb_pad)."""
    m_pad = _pad(m, 256)
    kb_pad = _pad(2 * k if wtype == O.F16 else k, 128)
    off = 0
    p = {"m_pad": m_pad, "kb_pad": kb_pad}

    def take(name, nbytes):
        nonlocal off
        p[name] = (off, nbytes)
        off = _align256(off + nbytes)

    take("xq", m_pad * kb_pad)
    if wtype == O.Q8_0:
        take("xd", kb_pad // 32 * m_pad * 4)
    elif wtype in (O.Q4_K, O.Q6_K):
        take("xd", k // 256 * m_pad * 4)
        take("xmin", m_pad // 32 * (k // 256) * 1024)
    p["total"] = off
    return p


def tiled_index(m_pad, kb_pad):
    """idx[r, b] = byte offset of row r, K byte b in the fragment-major plane."""
    r = np.arange(m_pad)[:, None]
    b = np.arange(kb_pad)[None, :]
    rt, lr, kc, w = r // 32, r % 32, b // 32, b % 32
    return (((rt * (kb_pad // 32) + kc) * 64 + (w // 16) * 32 + lr) * 16 + (w % 16)).astype(np.int64)


def decode_q8_0_blocks(blocks, k):
    """GGUF block_q8_0 rows -> (int8 quants [m][k], fp16 d as float32 [m][k/32])."""
    b = np.ascontiguousarray(blocks).reshape(blocks.shape[0], k // 32, 34)
    d = b[:, :, :2].copy().view(np.float16)[:, :, 0].astype(np.float32)
    q = b[:, :, 2:].copy().view(np.int8).reshape(blocks.shape[0], k)
    return q, d


def decode_q8_K_blocks(blocks, k):
    """GGUF block_q8_K rows -> (int8 quants [m][k], float32 d [m][k/256], int16 bsums [m][k/16])."""
    b = np.ascontiguousarray(blocks).reshape(blocks.shape[0], k // 256, 292)
    d = b[:, :, :4].copy().view(np.float32)[:, :, 0]
    q = b[:, :, 4:260].copy().view(np.int8).reshape(blocks.shape[0], k)
    bs = b[:, :, 260:292].copy().view(np.int16).reshape(blocks.shape[0], k // 16)
    return q, d, bs


def expected_image(wtype, blocks, m, k):
    """The tiled workspace bytes (length planes()['total']) for the oracle's blocks of m rows
    (GGUF layout: block_q8_0 rows for Q8_0, block_q8_K rows for Q4_K / Q6_K, fp16 rows for F16)."""
    p = planes(wtype, m, k)
    m_pad, kb_pad = p["m_pad"], p["kb_pad"]
    img = np.zeros(p["total"], np.uint8)
    if wtype == O.F16:  # fp16 activations (ggml's F16 vec_dot_type): the row's fp16 bytes, tiled
        bfull = np.zeros((m_pad, kb_pad), np.uint8)
        bfull[:m, :2 * k] = np.ascontiguousarray(blocks).reshape(m, 2 * k)
        o, n = p["xq"]
        img[o:o + n][tiled_index(m_pad, kb_pad).ravel()] = bfull.ravel()
        return img
    qfull = np.zeros((m_pad, kb_pad), np.int8)
    if wtype == O.Q8_0:
        q, d = decode_q8_0_blocks(blocks, k)
    else:
        q, d, bs = decode_q8_K_blocks(blocks, k)
    qfull[:m, :k] = q
    o, n = p["xq"]
    img[o:o + n][tiled_index(m_pad, kb_pad).ravel()] = qfull.view(np.uint8).ravel()
    o, n = p["xd"]
    dfull = np.zeros((n // 4 // m_pad, m_pad), np.float32)
    dfull[:d.shape[1], :m] = d.T
    img[o:o + n] = dfull.view(np.uint8).ravel()
    if wtype != O.Q8_0:
        nsb = k // 256
        B = bs.reshape(m, nsb, 8, 2).astype(np.int32).sum(-1)  # the 32-quant sub-block sums
        lo, hi = B & 63, (B >> 6) * 64
        frag = np.zeros((m_pad // 32, nsb, 64, 8), np.float16)
        r = np.arange(m)
        frag[r // 32, :, r % 32, :] = lo.astype(np.float16)
        frag[r // 32, :, 32 + r % 32, :] = hi.astype(np.float16)
        o, n = p["xmin"]
        img[o:o + n] = frag.view(np.uint8).ravel()
    return img


def oracle_image(oracle, wtype, x, variant=O.Q8_0_X86):
    """expected_image of oracle.quantize_act(wtype, x): what the GEMM-path quantizer must write."""
    m, k = x.shape
    return expected_image(wtype, oracle.quantize_act(wtype, x, variant), m, k)


def first_difference(got, want, wtype, m, k):
    """A readable description of where two workspace images differ (None if equal)."""
    if np.array_equal(got, want):
        return None
    p = planes(wtype, m, k)
    bad = np.flatnonzero(got != want)
    for name in ("xq", "xd", "xmin"):
        if name in p:
            o, n = p[name]
            inside = bad[(bad >= o) & (bad < o + n)]
            if inside.size:
                return f"{name}: {inside.size} bytes differ, first at +{inside[0] - o}"
    return f"{bad.size} bytes differ outside the planes, first at {bad[0]}"


def decode_image(wtype, img, m, k):
    """A tiled workspace (as the GPU wrote it) -> (int8 quants [m][k], float32 scales [m][nblocks]),
    nblocks = k / 32 (Q8_0) or k / 256 (Q8_K): the activation the GEMM multiplies."""
    p = planes(wtype, m, k)
    m_pad, kb_pad = p["m_pad"], p["kb_pad"]
    o, n = p["xq"]
    q = np.asarray(img[o:o + n]).view(np.int8).reshape(m_pad // 32, kb_pad // 32, 2, 32, 16)
    q = q.transpose(0, 3, 1, 2, 4).reshape(m_pad, kb_pad)[:m, :k]
    o, n = p["xd"]
    d = np.asarray(img[o:o + n]).view(np.float32).reshape(-1, m_pad)[:, :m].T
    nblk = k // (32 if wtype == O.Q8_0 else 256)
    return q, np.ascontiguousarray(d[:, :nblk])


def dequant_image(wtype, img, m, k):
    """decode_image as float64 values q * d (exact)."""
    q, d = decode_image(wtype, img, m, k)
    bs = 32 if wtype == O.Q8_0 else 256
    return (q.reshape(m, -1, bs).astype(np.float64) * d[:, :, None].astype(np.float64)).reshape(m, k)


def live_difference(got, want, wtype, m, k):
    """first_difference restricted to what a GEMM reads for its m live rows: the quants and
    scales of rows < m (and for Q8_K their min-term operands).  The producers that quantize their
    own output (norms, attention, the requantizing GEMM) write whole 32-row tiles of live rows;
    row tiles past them are never read for a stored output and are left as they were."""
    qg, dg = decode_image(wtype, got, m, k)
    qw, dw = decode_image(wtype, want, m, k)
    if not np.array_equal(qg, qw):
        r, c = np.argwhere(qg != qw)[0]
        return f"quants: {int((qg != qw).sum())} differ, first at row {r} col {c}"
    if not np.array_equal(dg.view(np.uint32), dw.view(np.uint32)):
        r, c = np.argwhere(dg.view(np.uint32) != dw.view(np.uint32))[0]
        return f"scales: first difference at row {r} block {c}"
    if wtype != O.Q8_0:
        p = planes(wtype, m, k)
        o, n = p["xmin"]
        fg = np.asarray(got[o:o + n]).view(np.uint16).reshape(p["m_pad"] // 32, k // 256, 64, 8)
        fw = np.asarray(want[o:o + n]).view(np.uint16).reshape(p["m_pad"] // 32, k // 256, 64, 8)
        r = np.arange(m)
        for half in (0, 32):
            if not np.array_equal(fg[r // 32, :, half + r % 32], fw[r // 32, :, half + r % 32]):
                return "min-term operands differ"
    return None
