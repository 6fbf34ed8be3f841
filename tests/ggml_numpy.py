"""Independent numpy decoders of the GGUF block formats, written from the format
description (field offsets, nibble order, 6-bit scale packing), plus an exact
integer mul_mat built on them.  They share no code with the C oracle or the HIP
kernels, so agreement pins indexing and packing in both.
"""
import numpy as np

QK8_0, QK_K = 32, 256


def f16(b2):
    """uint8 [..., 2] little-endian -> float32."""
    return np.ascontiguousarray(b2).view(np.float16)[..., 0].astype(np.float32)


# ---------------------------------------------------------------- Q8_0 ----
def q8_0_fields(rows, k):
    b = np.asarray(rows, dtype=np.uint8).reshape(-1, 34)
    d = f16(b[:, 0:2])
    q = b[:, 2:34].view(np.int8).astype(np.int64)
    nr = b.shape[0] // (k // QK8_0)
    return d.reshape(nr, k // QK8_0), q.reshape(nr, k)


def q8_0_dequant(rows, k):
    d, q = q8_0_fields(rows, k)
    return (q.reshape(q.shape[0], -1, QK8_0).astype(np.float32) * d[:, :, None]).reshape(q.shape[0], k)


# ---------------------------------------------------------------- Q4_K ----
def q4_K_fields(rows, k):
    """-> d, dmin [nr, nsb] f32; sc, mn [nr, nsb, 8] int; q [nr, k] int (0..15)."""
    b = np.asarray(rows, dtype=np.uint8).reshape(-1, 144)
    nb = b.shape[0]
    d, dmin = f16(b[:, 0:2]), f16(b[:, 2:4])
    s = b[:, 4:16].astype(np.int64)
    sc = np.empty((nb, 8), np.int64)
    mn = np.empty((nb, 8), np.int64)
    sc[:, :4] = s[:, 0:4] & 63
    mn[:, :4] = s[:, 4:8] & 63
    sc[:, 4:] = (s[:, 8:12] & 0xF) | ((s[:, 0:4] >> 6) << 4)
    mn[:, 4:] = (s[:, 8:12] >> 4) | ((s[:, 4:8] >> 6) << 4)
    qs = b[:, 16:144].reshape(nb, 4, 32).astype(np.int64)
    q = np.stack([qs & 0xF, qs >> 4], axis=2).reshape(nb, 256)  # [chunk][lo/hi][32]
    nr = nb // (k // QK_K)
    nsb = k // QK_K
    return (d.reshape(nr, nsb), dmin.reshape(nr, nsb), sc.reshape(nr, nsb, 8), mn.reshape(nr, nsb, 8),
            q.reshape(nr, k))


def q4_K_dequant(rows, k, fused=False):
    d, dmin, sc, mn, q = q4_K_fields(rows, k)
    nr, nsb = d.shape
    d1 = (d[:, :, None] * sc.astype(np.float32)).astype(np.float32)
    m1 = (dmin[:, :, None] * mn.astype(np.float32)).astype(np.float32)
    qf = q.reshape(nr, nsb, 8, 32).astype(np.float32)
    if fused:
        y = (d1[..., None].astype(np.float64) * qf - m1[..., None].astype(np.float64)).astype(np.float32)
    else:
        y = (d1[..., None] * qf).astype(np.float32) - m1[..., None]
    return y.astype(np.float32).reshape(nr, k)


def pack_q4_K_scales(sc, mn):
    """Inverse of the 6-bit unpacking: sc, mn int [..., 8] in [0,63] -> bytes [..., 12]."""
    sc = np.asarray(sc, np.int64)
    mn = np.asarray(mn, np.int64)
    out = np.zeros(sc.shape[:-1] + (12,), np.int64)
    out[..., 0:4] = (sc[..., 0:4] & 63) | ((sc[..., 4:8] >> 4) << 6)
    out[..., 4:8] = (mn[..., 0:4] & 63) | ((mn[..., 4:8] >> 4) << 6)
    out[..., 8:12] = (sc[..., 4:8] & 0xF) | ((mn[..., 4:8] & 0xF) << 4)
    return out.astype(np.uint8)


# ---------------------------------------------------------------- Q6_K ----
def q6_K_fields(rows, k):
    """-> d [nr, nsb] f32; sc [nr, nsb, 16] int; q [nr, k] int in [-32, 31]."""
    b = np.asarray(rows, dtype=np.uint8).reshape(-1, 210)
    nb = b.shape[0]
    ql = b[:, 0:128].reshape(nb, 2, 64).astype(np.int64)
    qh = b[:, 128:192].reshape(nb, 2, 32).astype(np.int64)
    sc = b[:, 192:208].view(np.int8).astype(np.int64)
    d = f16(b[:, 208:210])
    q = np.empty((nb, 2, 4, 32), np.int64)
    q[:, :, 0] = (ql[:, :, 0:32] & 0xF) | (((qh >> 0) & 3) << 4)
    q[:, :, 1] = (ql[:, :, 32:64] & 0xF) | (((qh >> 2) & 3) << 4)
    q[:, :, 2] = (ql[:, :, 0:32] >> 4) | (((qh >> 4) & 3) << 4)
    q[:, :, 3] = (ql[:, :, 32:64] >> 4) | (((qh >> 6) & 3) << 4)
    nr = nb // (k // QK_K)
    nsb = k // QK_K
    return d.reshape(nr, nsb), sc.reshape(nr, nsb, 16), (q - 32).reshape(nr, k)


def q6_K_dequant(rows, k):
    d, sc, q = q6_K_fields(rows, k)
    nr, nsb = d.shape
    ds = (d[:, :, None] * sc.astype(np.float32)).astype(np.float32)  # d * sc first
    y = (ds[..., None] * q.reshape(nr, nsb, 16, 16).astype(np.float32)).astype(np.float32)
    return y.reshape(nr, k)


# ---------------------------------------------------------------- Q8_K ----
def q8_K_fields(rows, k):
    b = np.asarray(rows, dtype=np.uint8).reshape(-1, 292)
    nb = b.shape[0]
    d = np.ascontiguousarray(b[:, 0:4]).view(np.float32)[:, 0]
    q = b[:, 4:260].view(np.int8).astype(np.int64)
    bs = np.ascontiguousarray(b[:, 260:292]).view(np.int16).astype(np.int64)
    nr = nb // (k // QK_K)
    return d.reshape(nr, -1), q.reshape(nr, k), bs.reshape(nr, -1)


# ------------------------------------------------------- exact mul_mat ----
def mul_mat_exact(wtype, w, xq, k):
    """fp64 Y[m, n] from quantized operands with integer block sums (ggml type ids)."""
    if wtype == 8:
        dw, qw = q8_0_fields(w, k)
        dx, qx = q8_0_fields(xq, k)
        nb = k // QK8_0
        isum = np.einsum("mbk,nbk->mnb", qx.reshape(-1, nb, 32), qw.reshape(-1, nb, 32))
        return np.einsum("mnb,mb,nb->mn", isum.astype(np.float64), dx.astype(np.float64), dw.astype(np.float64))
    if wtype == 12:
        d, dmin, sc, mn, q = q4_K_fields(w, k)
        dx, qx, bs = q8_K_fields(xq, k)
        nr, nsb = d.shape
        v = (q.reshape(nr, nsb, 8, 32) * sc[..., None]).reshape(nr, nsb, 256)
        main = np.einsum("msk,nsk->mns", qx.reshape(-1, nsb, 256), v)
        b32 = bs.reshape(-1, nsb, 8, 2).sum(-1)
        mins = np.einsum("msj,nsj->mns", b32, mn)
        return np.einsum("ms,mns->mn", dx.astype(np.float64),
                         d[None].astype(np.float64) * main - dmin[None].astype(np.float64) * mins)
    if wtype == 14:
        d, sc, q = q6_K_fields(w, k)
        dx, qx, _ = q8_K_fields(xq, k)
        nr, nsb = d.shape
        v = (q.reshape(nr, nsb, 16, 16) * sc[..., None]).reshape(nr, nsb, 256)
        main = np.einsum("msk,nsk->mns", qx.reshape(-1, nsb, 256), v)
        return np.einsum("ms,mns->mn", dx.astype(np.float64), d[None].astype(np.float64) * main)
    if wtype == 1:
        wf = np.ascontiguousarray(w).view(np.float16).reshape(-1, k).astype(np.float64)
        xf = np.ascontiguousarray(xq).view(np.float16).reshape(-1, k).astype(np.float64)
        return xf @ wf.T
    raise ValueError(wtype)


def rel_err(got, ref):
    """max|got - ref| / max|ref| (the mul_mat acceptance metric)."""
    ref = np.asarray(ref, np.float64)
    den = np.max(np.abs(ref))
    return float(np.max(np.abs(np.asarray(got, np.float64) - ref)) / (den if den > 0 else 1.0))
