"""Device plumbing for the GPU tests: torch owns the memory, libmq does the work."""
import ctypes

import numpy as np

from crispembed_amd import mq


def torch():
    import torch as _t
    return _t


def stream():
    return ctypes.c_void_p(torch().cuda.current_stream().cuda_stream)


def dev(a):
    return torch().from_numpy(np.ascontiguousarray(a)).cuda()


def host(t):
    torch().cuda.synchronize()
    return t.cpu().numpy()


def empty_u8(nbytes):
    t = torch().empty(max(1, nbytes) + 256, dtype=torch().uint8, device="cuda")
    off = (-t.data_ptr()) % 256
    return t, off  # keep t alive; use t.data_ptr() + off


def weight_image(wtype, w_gguf, n, k):
    """Upload GGUF rows into a 256-aligned weight image and build its planes."""
    L = mq.lib()
    size = L.mq_weight_image_bytes(wtype, n, k)
    assert size > 0
    buf, off = empty_u8(size)
    g = np.ascontiguousarray(w_gguf, dtype=np.uint8).ravel()
    assert g.size == L.mq_gguf_bytes(wtype, n, k)
    buf[off:off + g.size] = dev(g)
    ptr = buf.data_ptr() + off
    mq.check(L.mq_weight_prepare(wtype, ctypes.c_void_p(ptr), n, k, 0, n, stream()))
    return buf, ptr


def mul_mat(wtype, wptr, n, k, x_dev, path=mq.PATH_AUTO, y_dev=None, ldy=None, workspace=True):
    """x_dev: torch float32 [m, ldx>=k] (row stride from the tensor)."""
    L = mq.lib()
    m = x_dev.shape[0]
    ldx = x_dev.stride(0)
    if y_dev is None:
        y_dev = torch().empty((m, n), dtype=torch().float32, device="cuda")
    ldy = y_dev.stride(0) if ldy is None else ldy
    ws_ptr, ws_bytes, keep = None, 0, None
    if workspace:
        ws_bytes = L.mq_workspace_bytes(wtype, m, k)
        keep, off = empty_u8(ws_bytes)
        ws_ptr = ctypes.c_void_p(keep.data_ptr() + off)
    mq.check(L.mq_mul_mat_ex(wtype, ctypes.c_void_p(wptr), n, k, ctypes.c_void_p(x_dev.data_ptr()), ldx, m,
                             ctypes.c_void_p(y_dev.data_ptr()), ldy, ws_ptr, ws_bytes, path, stream()))
    torch().cuda.synchronize()
    return y_dev


def live_q8_0_planes(raw, m, k):
    """The Q8_0 GEMM-layout activation planes (quants in 1 KB fragments per 32-row tile and
    32-value chunk, scales [k / 32][m_pad]) of rows < m, as a row-major int8 [m][k] and a
    float32 [k / 32][m]; k a multiple of 128, m_pad = m rounded up to 256."""
    m_pad = -(-m // 256) * 256
    kch = k // 32
    q = raw[:m_pad * k].reshape(m_pad // 32, kch, 2, 32, 16)   # [row tile][chunk][half][row][byte]
    q = q.transpose(0, 3, 1, 2, 4).reshape(m_pad, k)[:m]
    off = -(-(m_pad * k) // 256) * 256
    d = raw[off:off + kch * m_pad * 4].view(np.float32).reshape(kch, m_pad)[:, :m]
    return q, d


def fetch(ptr, nbytes):
    """nbytes (a multiple of 4) of device memory at ptr, copied into a new host uint8 array by a
    device-to-device copy (mq_op_cpy) into torch memory."""
    t = torch()
    n = nbytes // 4
    dst = t.empty(max(n, 1), dtype=t.float32, device="cuda")
    src = mq.View()
    src.data, src.type = ptr, mq.TYPE_F32
    for i, (ne, nb) in enumerate(((n, 4), (1, 4 * n), (1, 4 * n), (1, 4 * n))):
        src.ne[i], src.nb[i] = ne, nb
    mq.check(mq.lib().mq_op_cpy(ctypes.byref(src), ctypes.byref(mq.view(dst)), stream()))
    return host(dst)[:n].view(np.uint8)
