"""The C-ABI libraries load without a GPU and export every declared symbol."""
import ctypes
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _declared(header):
    text = open(os.path.join(ROOT, "include", header)).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(mq_\w+|\w*mi355\w*|ggml_backend_init|ggml_backend_score)\s*\(", text)))


def test_libmq_exports_all_declared_symbols():
    from crispembed_amd import mq
    L = mq.lib()
    names = (_declared("mq.h") + _declared("mq_bert.h") + _declared("mq_decoder.h") + _declared("mq_gguf.h") +
             _declared("mq_ops.h"))
    assert len(names) >= 30
    missing = [n for n in names if not hasattr(L, n)]
    assert not missing, missing


def test_host_only_entry_points_without_gpu():
    from crispembed_amd import mq
    L = mq.lib()
    assert L.mq_blck_size(mq.TYPE_Q4_K) == 256
    assert L.mq_type_size(mq.TYPE_Q6_K) == 210
    assert L.mq_row_size(mq.TYPE_Q8_0, 384) == 12 * 34
    assert L.mq_vec_dot_type(mq.TYPE_Q4_K) == mq.TYPE_Q8_K
    assert L.mq_supports(mq.TYPE_Q4_K, 384) == 0 and L.mq_supports(mq.TYPE_Q8_0, 384) == 1
    # the weight image starts with the untouched GGUF bytes
    assert L.mq_gguf_bytes(mq.TYPE_Q4_K, 4096, 1024) == 4096 * 4 * 144
    assert L.mq_weight_image_bytes(mq.TYPE_Q4_K, 4096, 1024) > L.mq_gguf_bytes_aligned(mq.TYPE_Q4_K, 4096, 1024)
    assert L.mq_weight_image_bytes(mq.TYPE_F16, 8, 64) >= L.mq_gguf_bytes_aligned(mq.TYPE_F16, 8, 64) + 256 * 128
    # the auto path: GEMV for m <= 8, and up to 32 rows on narrow layers (few GEMM tiles)
    assert L.mq_mul_mat_path(mq.TYPE_Q8_0, 384, 384, 4) == mq.PATH_GEMV
    assert L.mq_mul_mat_path(mq.TYPE_Q8_0, 384, 384, 16) == mq.PATH_GEMV
    assert L.mq_mul_mat_path(mq.TYPE_Q8_0, 384, 384, 33) == mq.PATH_GEMM
    assert L.mq_mul_mat_path(mq.TYPE_Q6_K, 151936, 2048, 16) == mq.PATH_GEMM
    # argument errors come back as codes with a message, before any HIP call
    rc = L.mq_mul_mat(mq.TYPE_Q4_K, None, 8, 300, None, 300, 1, None, 8, None, 0, None)
    assert rc == -2 and b"multiple" in L.mq_last_error()
    rc = L.mq_quantize_act_ex(mq.TYPE_Q8_0, 256, 256, 2, 256, None, 7, 4096, 1 << 20, mq.PATH_AUTO, None)
    assert rc == -1 and b"prologue" in L.mq_last_error()
    # the quantized-output GEMM: Q8_0 output only, n a multiple of 128, GELU-erf or no op
    rq = L.mq_mul_mat_q_requant
    assert rq(mq.TYPE_Q8_0, 256, 1536, 384, 256, 4096, None, 1, mq.TYPE_Q4_K, 256, 1 << 30, None) == -2
    assert rq(mq.TYPE_Q8_0, 256, 1500, 384, 256, 4096, None, 1, mq.TYPE_Q8_0, 256, 1 << 30, None) == -1
    assert b"multiple of 128" in L.mq_last_error()
    assert rq(mq.TYPE_Q8_0, 256, 1536, 384, 256, 4096, None, 2, mq.TYPE_Q8_0, 256, 1 << 30, None) == -1
    assert rq(mq.TYPE_Q8_0, 256, 1536, 384, 256, 4096, None, 1, mq.TYPE_Q8_0, 256, 1024, None) == -1
    assert b"output workspace" in L.mq_last_error()
    # Q8_K output (a K-quant next product): K-quant weights, n a multiple of 256, >= 256 workgroups
    # of 128 x 256 -- else unsupported, with the same answer from the query
    sup = L.mq_mul_mat_q_requant_supported
    assert sup(mq.TYPE_Q4_K, mq.TYPE_Q4_K, 8192, 4096) == 1 and sup(mq.TYPE_Q6_K, mq.TYPE_Q4_K, 2048, 4096) == 1
    assert sup(mq.TYPE_Q8_0, mq.TYPE_Q8_0, 4096, 1536) == 1
    assert sup(mq.TYPE_Q8_0, mq.TYPE_Q4_K, 8192, 4096) == 0  # Q8_0 weights: Q8_0 output only
    assert sup(mq.TYPE_Q4_K, mq.TYPE_Q4_K, 512, 4096) == 0   # 64 workgroups
    assert sup(mq.TYPE_Q4_K, mq.TYPE_Q4_K, 8192, 4224) == 0  # not whole superblocks
    assert rq(mq.TYPE_Q4_K, 256, 4096, 1024, 256, 512, None, 1, mq.TYPE_Q4_K, 256, 1 << 30, None) == -2
    assert b"Q8_K output" in L.mq_last_error()


def test_op_support_checks_without_gpu():
    """mq_op_supported and the argument checks of the graph ops are host code."""
    from crispembed_amd import mq
    L = mq.lib()
    V = mq.View

    def view(ne, type=mq.TYPE_F32, esize=4, data=None):
        nb = [esize]
        for i in range(3):
            nb.append(nb[-1] * ne[i])
        return mq.view(None, type=type, ne=ne, nb=nb)

    q = view([64, 40, 12, 2])
    out = view([64, 12, 40, 2])
    assert L.mq_op_supported(mq.OP_FLASH_ATTN, 0, q, q, q, None, out) == 1
    assert L.mq_op_supported(mq.OP_FLASH_ATTN, 0, view([48, 40, 12, 2]), view([48, 40, 12, 2]),
                             view([48, 40, 12, 2]), None, view([48, 12, 40, 2])) == 0  # head_dim 48
    kv = view([64, 40, 5, 2])
    assert L.mq_op_supported(mq.OP_FLASH_ATTN, 0, q, kv, kv, None, out) == 0  # 12 heads over 5 kv heads
    mask = view([40, 40, 1, 2], mq.TYPE_F16, 2)
    assert L.mq_op_supported(mq.OP_FLASH_ATTN, 0, q, q, q, mask, out) == 1
    assert L.mq_op_supported(mq.OP_FLASH_ATTN, 0, q, q, q, view([30, 40, 1, 2], mq.TYPE_F16, 2), out) == 0
    x = view([384, 128, 1, 1])
    assert L.mq_op_supported(mq.OP_BINARY, mq.BIN_ADD, x, view([384, 1, 1, 1]), None, None, x) == 1
    assert L.mq_op_supported(mq.OP_BINARY, mq.BIN_ADD, x, view([100, 1, 1, 1]), None, None, x) == 0
    assert L.mq_op_supported(mq.OP_NORM, mq.NORM_LAYER, x, None, None, None, x) == 1
    assert L.mq_op_supported(mq.OP_UNARY, 9, x, None, None, None, x) == 0
    ids = view([128, 1, 1, 1], mq.TYPE_I32)
    tbl = mq.view(None, type=mq.TYPE_Q8_0, ne=[384, 1000, 1, 1], nb=[34, 408, 408000, 408000])
    assert L.mq_op_supported(mq.OP_GET_ROWS, 0, tbl, ids, None, None, x) == 1
    assert L.mq_op_supported(mq.OP_GET_ROWS, 0, tbl, ids, None, None, view([384, 127, 1, 1])) == 0
    # the entry points reject before launching anything
    assert L.mq_op_binary(mq.BIN_ADD, x, view([100, 1, 1, 1]), x, None) == -2
    assert b"broadcast" in L.mq_last_error()
    assert L.mq_op_norm(mq.NORM_LAYER, x, None, x, 1e-5, None, None, None) == -1  # no data
    assert L.mq_op_supported(mq.OP_NORM, mq.NORM_LAYER, x, view([384, 64, 1, 1]), None, None, x) == 0
    assert V is not None


def test_ggml_backend_library_exports():
    import ctypes
    from crispembed_amd import mq
    mq.lib()
    here = mq.LIB_DIR
    ctypes.CDLL(os.path.join(here, "libggml-compat.so"), mode=ctypes.RTLD_GLOBAL)
    L = ctypes.CDLL(os.path.join(here, "libggml-mi355.so"))
    names = _declared("ggml-mi355.h")
    assert set(names) >= {"ggml_backend_mi355_reg", "ggml_backend_mi355_init", "ggml_backend_is_mi355",
                          "ggml_backend_mi355_buffer_type", "ggml_backend_mi355_get_device_count",
                          "ggml_backend_init", "ggml_backend_score"}
    missing = [n for n in names if not hasattr(L, n)]
    assert not missing, missing


def test_backend_driver_without_gpu_reports_no_device():
    """On a machine without a gfx950 device the registry is empty and the driver
    exits cleanly with device_available false (no crash, no fallback)."""
    import json
    import subprocess
    import torch
    if torch.cuda.is_available():
        pytest.skip("a GPU is present; the GPU test covers the driver")
    exe = os.path.join(ROOT, "crispembed_amd", "bin", "test-backend-mi355")
    r = subprocess.run([exe, "--json"], capture_output=True, text=True, timeout=120)
    assert r.returncode == 1
    out = json.loads(r.stdout.strip().splitlines()[-1])
    assert out["device_available"] is False
    assert out["dl_score"] == 0  # ggml_backend_init / ggml_backend_score resolve; no gfx950 device here
