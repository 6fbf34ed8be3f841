"""The C-ABI libraries load without a GPU and export every declared symbol."""
import ctypes
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _declared(header):
    text = open(os.path.join(ROOT, "include", header)).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b((?:mq|ggml_backend_mi355)\w*)\s*\(", text)))


def test_libmq_exports_all_declared_symbols():
    from crispembed_amd import mq
    L = mq.lib()
    names = _declared("mq.h")
    assert len(names) >= 20
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
    # argument errors come back as codes with a message, before any HIP call
    rc = L.mq_mul_mat(mq.TYPE_Q4_K, None, 8, 300, None, 300, 1, None, 8, None, 0, None)
    assert rc == -2 and b"multiple" in L.mq_last_error()
