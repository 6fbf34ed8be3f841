"""ctypes binding of the CPU oracle (oracle/liboracle.so) for the tests.

The oracle is the checker; only tests/, the smoke check and bench.py's
cpu_baseline leg load it.
"""
import ctypes
import os
import subprocess

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
ORACLE_DIR = os.path.join(ROOT, "oracle")
# MQ_ORACLE_SO: another build of the oracle (the sanitized one, oracle/_asan/liboracle.so)
ORACLE_SO = os.environ.get("MQ_ORACLE_SO") or os.path.join(ORACLE_DIR, "liboracle.so")

F32, F16, Q8_0, Q4_K, Q6_K, Q8_K = 0, 1, 8, 12, 14, 15
# planted mistakes of the oracle (ggml_oracle.h OR_MUT_*)
MUT_NONE, MUT_Q4K_NO_SEARCH, MUT_Q4K_RDELTA, MUT_Q4K_PACK, MUT_Q6K_NO_SEARCH, MUT_Q6K_STEP, MUT_Q6K_ISCALE = range(7)
MUT_Q4K_CALL_NSTEP0, MUT_Q4K_CALL_UNIT_WEIGHTS, MUT_Q4K_CALL_RMIN = 7, 8, 9  # at quantize_row_q4_K_ref's call
Q8_0_X86, Q8_0_NEON, Q8_0_REF = 0, 1, 2
BLCK = {F32: 1, F16: 1, Q8_0: 32, Q4_K: 256, Q6_K: 256, Q8_K: 256}
TSIZE = {F32: 4, F16: 2, Q8_0: 34, Q4_K: 144, Q6_K: 210, Q8_K: 292}
VEC_DOT = {Q8_0: Q8_0, Q4_K: Q8_K, Q6_K: Q8_K, F16: F16}


def row_size(t, k):
    return (k // BLCK[t]) * TSIZE[t]


def _ptr(a):
    return a.ctypes.data_as(ctypes.c_void_p)


class Oracle:
    def __init__(self):
        if not os.path.exists(ORACLE_SO) and not os.environ.get("MQ_ORACLE_SO"):
            subprocess.run(["make", "-C", ORACLE_DIR], check=True, capture_output=True)
        L = ctypes.CDLL(ORACLE_SO)
        i64, vp, ci, sz = ctypes.c_int64, ctypes.c_void_p, ctypes.c_int, ctypes.c_size_t
        sig = {
            "or_fp32_to_fp16": (ctypes.c_uint16, [ctypes.c_float]),
            "or_fp16_to_fp32": (ctypes.c_float, [ctypes.c_uint16]),
            "or_nearest_int": (ci, [ctypes.c_float]),
            "or_get_scale_min_k4": (None, [ci, vp, vp, vp]),
            "or_quantize_row_q8_0_act": (None, [vp, vp, i64, ci]),
            "or_quantize_row_q8_K": (None, [vp, vp, i64]),
            "or_quantize_row_f16": (None, [vp, vp, i64]),
            "or_quantize_chunk": (sz, [ci, vp, vp, i64, i64]),
            "or_dequantize_row": (None, [ci, vp, vp, i64, ci]),
            "or_quantize_act_rows": (None, [ci, vp, i64, vp, i64, i64, ci]),
            "or_vec_dot": (ctypes.c_float, [ci, i64, vp, vp]),
            "or_mul_mat": (None, [ci, vp, i64, i64, vp, i64, i64, vp, i64, ci, ci]),
            "or_mul_mat_q": (None, [ci, vp, i64, i64, vp, i64, vp, i64, ci]),
            "or_mul_mat_exact": (None, [ci, vp, i64, i64, vp, i64, vp]),
            "or_fast_supported": (ci, [ci]),
            "or_fast_mul_mat": (ci, [ci, vp, i64, i64, vp, i64, i64, vp, i64, ci]),
            "or_make_qkx2_quants": (ctypes.c_float, [ci, ci, vp, vp, vp, vp, ctypes.c_float, ctypes.c_float, ci]),
            "or_make_qx_quants": (ctypes.c_float, [ci, ci, vp, vp]),
            "or_set_mutation": (None, [ci]),
            "or_fast_isa": (ctypes.c_char_p, []),
        }
        for name, (res, args) in sig.items():
            f = getattr(L, name)
            f.restype = res
            f.argtypes = args
        self.L = L

    # ---- elementwise helpers ----
    def fp32_to_fp16(self, x):
        x = np.ascontiguousarray(x, dtype=np.float32).ravel()
        out = np.empty(x.size, dtype=np.uint16)
        self.L.or_quantize_row_f16(_ptr(x), _ptr(out), x.size)
        return out

    def nearest_int(self, v):
        return self.L.or_nearest_int(float(v))

    # ---- quantization ----
    def quantize_chunk(self, t, x):
        x = np.ascontiguousarray(x, dtype=np.float32)
        n, k = x.shape
        out = np.zeros(n * row_size(t, k), dtype=np.uint8)
        self.L.or_quantize_chunk(t, _ptr(x), _ptr(out), n, k)
        return out.reshape(n, row_size(t, k))

    def quantize_act(self, wtype, x, variant=Q8_0_X86):
        """Rows of x -> vec_dot_type(wtype) blocks (GGUF layout)."""
        x = np.ascontiguousarray(x, dtype=np.float32)
        m, k = x.shape
        vt = VEC_DOT[wtype]
        out = np.zeros(m * row_size(vt, k), dtype=np.uint8)
        self.L.or_quantize_act_rows(wtype, _ptr(x), k, _ptr(out), m, k, variant)
        return out.reshape(m, row_size(vt, k))

    def make_qkx2_quants(self, x, weights, nmax=15, rmin=-1.0, rdelta=0.1, nstep=20):
        """-> (scale, the_min, levels uint8) of one sub-block (Q4_K's search)."""
        x = np.ascontiguousarray(x, dtype=np.float32)
        w = np.ascontiguousarray(weights, dtype=np.float32)
        L = np.zeros(x.size, np.uint8)
        mn = ctypes.c_float()
        s = self.L.or_make_qkx2_quants(x.size, nmax, _ptr(x), _ptr(w), _ptr(L), ctypes.byref(mn), rmin, rdelta, nstep)
        return np.float32(s), np.float32(mn.value), L

    def make_qx_quants(self, x, nmax=32):
        """-> (scale, levels int8 = level + nmax) of one sub-block (Q6_K's search)."""
        x = np.ascontiguousarray(x, dtype=np.float32)
        L = np.zeros(x.size, np.int8)
        s = self.L.or_make_qx_quants(x.size, nmax, _ptr(x), _ptr(L))
        return np.float32(s), L

    def set_mutation(self, m):
        self.L.or_set_mutation(m)

    def dequantize(self, t, w, k, fused=0):
        w = np.ascontiguousarray(w, dtype=np.uint8)
        n = w.size // row_size(t, k)
        out = np.empty((n, k), dtype=np.float32)
        for r in range(n):
            self.L.or_dequantize_row(t, _ptr(w[r * row_size(t, k):]) if w.ndim == 1 else _ptr(w[r]),
                                     _ptr(out[r]), k, fused)
        return out

    # ---- mul_mat ----
    def mul_mat(self, wtype, w, x, nthreads=8, variant=Q8_0_X86):
        x = np.ascontiguousarray(x, dtype=np.float32)
        w = np.ascontiguousarray(w, dtype=np.uint8)
        m, k = x.shape
        n = w.size // row_size(wtype, k)
        y = np.empty((m, n), dtype=np.float32)
        self.L.or_mul_mat(wtype, _ptr(w), n, k, _ptr(x), k, m, _ptr(y), n, nthreads, variant)
        return y

    def mul_mat_q(self, wtype, w, xq, k, nthreads=8):
        w = np.ascontiguousarray(w, dtype=np.uint8)
        xq = np.ascontiguousarray(xq, dtype=np.uint8)
        n = w.size // row_size(wtype, k)
        m = xq.size // row_size(VEC_DOT[wtype], k)
        y = np.empty((m, n), dtype=np.float32)
        self.L.or_mul_mat_q(wtype, _ptr(w), n, k, _ptr(xq), m, _ptr(y), n, nthreads)
        return y

    def fast_supported(self, wtype):
        return bool(self.L.or_fast_supported(wtype))

    def fast_isa(self):
        """The SIMD form the CPU baseline uses on this host: "avx512vnni", "avx2" or "none"."""
        return self.L.or_fast_isa().decode()

    def fast_mul_mat(self, wtype, w, x, nthreads=8):
        """The CPU baseline (AVX2 integer dots, threads); same semantics as mul_mat."""
        x = np.ascontiguousarray(x, dtype=np.float32)
        w = np.ascontiguousarray(w, dtype=np.uint8)
        m, k = x.shape
        n = w.size // row_size(wtype, k)
        y = np.empty((m, n), dtype=np.float32)
        rc = self.L.or_fast_mul_mat(wtype, _ptr(w), n, k, _ptr(x), k, m, _ptr(y), n, nthreads)
        if rc != 0:
            raise RuntimeError(f"or_fast_mul_mat: type {wtype} unsupported on this host")
        return y

    def mul_mat_exact(self, wtype, w, xq, k):
        w = np.ascontiguousarray(w, dtype=np.uint8)
        xq = np.ascontiguousarray(xq, dtype=np.uint8)
        n = w.size // row_size(wtype, k)
        m = xq.size // row_size(VEC_DOT[wtype], k)
        y = np.empty((m, n), dtype=np.float64)
        self.L.or_mul_mat_exact(wtype, _ptr(w), n, k, _ptr(xq), m, _ptr(y))
        return y
