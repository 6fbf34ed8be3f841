"""CPU reference of the post-LN BERT encoder (src/crispembed.cpp:1043-1468) for the
end-to-end check of the GPU runner.

Every mul_mat follows ggml's CPU semantics: the fp32 activation is requantized to the
weight's vec_dot_type by the oracle (bit-exact ggml rounding), and the product of the
two quantized operands is taken exactly (fp64 over exactly dequantized values), then
rounded to fp32 -- the value ggml's integer block dots approximate to ~1e-7.  The other
ops run in fp64 and round to fp32 where the graph materialises a tensor.
"""
import numpy as np

import oracle_ffi as O
from ggml_numpy import q4_K_dequant, q6_K_dequant, q8_0_dequant, q8_K_fields

_DEQ = {O.Q8_0: q8_0_dequant, O.Q4_K: q4_K_dequant, O.Q6_K: q6_K_dequant}


def _act_deq(orc, wtype, x):
    xq = orc.quantize_act(wtype, x)
    k = x.shape[1]
    if wtype == O.Q8_0:
        return q8_0_dequant(xq, k).astype(np.float64)
    if wtype in (O.Q4_K, O.Q6_K):
        d, q, _ = q8_K_fields(xq, k)
        return (q.reshape(q.shape[0], -1, 256) * d[:, :, None].astype(np.float64)).reshape(q.shape[0], k)
    if wtype == O.F16:
        return np.ascontiguousarray(xq).view(np.float16).reshape(-1, k).astype(np.float64)
    raise ValueError(wtype)


def _w_deq(wtype, w, k):
    if wtype == O.F16:
        return np.ascontiguousarray(w).view(np.float16).reshape(-1, k).astype(np.float64)
    return _DEQ[wtype](w, k).astype(np.float64)


def linear(orc, wtype, x32, w, bias):
    k = x32.shape[1]
    y = (_act_deq(orc, wtype, x32) @ _w_deq(wtype, w, k).T).astype(np.float32)
    return (y + bias).astype(np.float32)


def layernorm(x, w, b, eps):
    x = x.astype(np.float64)
    mean = x.mean(-1, keepdims=True)
    var = ((x - mean) ** 2).mean(-1, keepdims=True)
    return ((x - mean) / np.sqrt(var + eps) * w + b).astype(np.float32)


def gelu_erf(x):
    from scipy.special import erf
    x = x.astype(np.float64)
    return (0.5 * x * (1.0 + erf(x / np.sqrt(2.0)))).astype(np.float32)


def encode(orc, hp, wtype, W, ids, types=None):
    """ids (and token types, default 0) int32 [B, T] -> (pooled fp32 [B, H], last hidden fp32 [B*T, H])."""
    B, T = ids.shape
    H, nh = hp["n_embd"], hp["n_head"]
    hd = H // nh
    eps = hp["layer_norm_eps"]
    x = (W["tok"][ids.ravel()] + np.tile(W["pos"][:T], (B, 1))).astype(np.float32)
    x = (x + (W["type"][0] if types is None else W["type"][np.asarray(types).ravel()])).astype(np.float32)
    x = layernorm(x, W["ln_w"], W["ln_b"], eps)
    for lay in W["layers"]:
        q = linear(orc, wtype, x, lay["wq"], lay["bq"]).astype(np.float64).reshape(B, T, nh, hd)
        k = linear(orc, wtype, x, lay["wk"], lay["bk"]).astype(np.float64).reshape(B, T, nh, hd)
        v = linear(orc, wtype, x, lay["wv"], lay["bv"]).astype(np.float64).reshape(B, T, nh, hd)
        s = np.einsum("bihd,bjhd->bhij", q, k) / np.sqrt(hd)
        s = np.exp(s - s.max(-1, keepdims=True))
        p = s / s.sum(-1, keepdims=True)
        a = np.einsum("bhij,bjhd->bihd", p, v).reshape(B * T, H).astype(np.float32)
        o = linear(orc, wtype, a, lay["wo"], lay["bo"])
        x = layernorm(x.astype(np.float64) + o, lay["ln1_w"], lay["ln1_b"], eps)
        h = gelu_erf(linear(orc, wtype, x, lay["wfc1"], lay["bfc1"]))
        f = linear(orc, wtype, h, lay["wfc2"], lay["bfc2"])
        x = layernorm(x.astype(np.float64) + f, lay["ln2_w"], lay["ln2_b"], eps)
    pooled = x.astype(np.float64).reshape(B, T, H).mean(1)
    norm = np.sqrt(np.maximum((pooled ** 2).sum(-1, keepdims=True), 1e-12))
    return (pooled / norm).astype(np.float32), x
