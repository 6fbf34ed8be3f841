"""CPU reference of CrispEmbed's decoder embedding graph for the Qwen3 family
(src/decoder_embed.cpp:565-830, pooling :1044-1100), for the end-to-end check of the GPU runner.

Every mul_mat follows ggml's CPU semantics as in bert_oracle: the fp32 activation is
requantized to the weight's vec_dot_type by the oracle and the product of the quantized
operands is taken exactly (fp64), then rounded to fp32.  RMS norms, RoPE (angle
pos * base^(-2i/d), NEOX pairs (i, i + d/2)), causal attention and SiLU run in fp64 and round to
fp32 where the graph materialises a tensor.
"""
import numpy as np

from bert_oracle import linear


def rms_norm(x, w, eps):
    x = x.astype(np.float64)
    return (x / np.sqrt((x * x).mean(-1, keepdims=True) + eps) * w).astype(np.float32)


def rope_neox(x, pos, base):
    """x [..., T, d] fp32 with positions pos [T]; pairs (i, i + d/2) rotated by pos * base^(-2i/d)."""
    d = x.shape[-1]
    half = d // 2
    inv = base ** (-2.0 * np.arange(half) / d)
    ang = pos[:, None].astype(np.float64) * inv[None, :]
    c, s = np.cos(ang), np.sin(ang)
    a, b = x[..., :half].astype(np.float64), x[..., half:].astype(np.float64)
    return np.concatenate([a * c - b * s, a * s + b * c], -1).astype(np.float32)


def attention(hp, lay, q, k, v, B, T):
    """The projections q [B*T, nq*hd], k, v [B*T, nkv*hd] (fp32) -> attention rows fp32
    [B*T, nq*hd]: per-head RMS norms of q and k, NEOX RoPE, causal (or full) softmax attention of
    each query head over its key/value head, per sequence."""
    nq, nkv, hd = hp["n_head"], hp["n_kv_head"], hp["head_dim"]
    eps, base = hp["rms_norm_eps"], hp["rope_theta"]
    pos = np.arange(T)
    q = q.reshape(B, T, nq, hd)
    k = k.reshape(B, T, nkv, hd)
    v = v.reshape(B, T, nkv, hd).astype(np.float64)
    if lay.get("q_norm") is not None:
        q = rms_norm(q, lay["q_norm"], eps)
    if lay.get("k_norm") is not None:
        k = rms_norm(k, lay["k_norm"], eps)
    q = rope_neox(q.transpose(0, 2, 1, 3), pos, base).astype(np.float64)  # [B, nq, T, hd]
    k = rope_neox(k.transpose(0, 2, 1, 3), pos, base).astype(np.float64)  # [B, nkv, T, hd]
    v = v.transpose(0, 2, 1, 3)
    grp = nq // nkv
    kk, vv = np.repeat(k, grp, axis=1), np.repeat(v, grp, axis=1)
    s = np.einsum("bhid,bhjd->bhij", q, kk) / np.sqrt(hd)
    if hp["causal"]:
        s = np.where(np.tril(np.ones((T, T), bool)), s, -np.inf)
    s = np.exp(s - s.max(-1, keepdims=True))
    p = s / s.sum(-1, keepdims=True)
    return np.einsum("bhij,bhjd->bihd", p, vv).reshape(B * T, nq * hd).astype(np.float32)


def silu_mul(gu):
    """[g | u] rows (fp32) -> silu(g) * u in fp64, rounded to fp32."""
    F = gu.shape[1] // 2
    g, u = gu[:, :F].astype(np.float64), gu[:, F:].astype(np.float64)
    return (g / (1.0 + np.exp(-g)) * u).astype(np.float32)


def encode(orc, hp, wtype, W, ids):
    """ids int32 [B, T] -> (pooled fp32 [B, H], last residual stream fp32 [B*T, H])."""
    B, T = ids.shape
    H, nq, nkv, hd, F = hp["n_embd"], hp["n_head"], hp["n_kv_head"], hp["head_dim"], hp["n_ff"]
    eps = hp["rms_norm_eps"]
    zq, zkv, zh, zf = (np.zeros(n, np.float32) for n in (nq * hd, nkv * hd, H, F))
    x = W["tok"][ids.ravel()].astype(np.float32)
    for lay in W["layers"]:
        h = rms_norm(x, lay["attn_norm"], eps)
        q = linear(orc, wtype, h, lay["wq"], zq)
        k = linear(orc, wtype, h, lay["wk"], zkv)
        v = linear(orc, wtype, h, lay["wv"], zkv)
        a = attention(hp, lay, q, k, v, B, T)
        x = (x + linear(orc, wtype, a, lay["wo"], zh)).astype(np.float32)
        h = rms_norm(x, lay["ffn_norm"], eps)
        g = linear(orc, wtype, h, lay["wgate"], zf)
        u = linear(orc, wtype, h, lay["wup"], zf)
        f = silu_mul(np.concatenate([g, u], 1))
        x = (x + linear(orc, wtype, f, lay["wdown"], zh)).astype(np.float32)
    if hp["pooling"] == 1:
        pooled = rms_norm(x, W["out_norm"], eps).astype(np.float64).reshape(B, T, H).mean(1)
    else:
        pooled = rms_norm(x.reshape(B, T, H)[:, -1], W["out_norm"], eps).astype(np.float64)
    norm = np.sqrt(np.maximum((pooled ** 2).sum(-1, keepdims=True), 1e-12))
    return (pooled / norm).astype(np.float32), x


def layer_from_quants(hp, lay, wdeq, x, acts, B, T):
    """One layer recomputed from the GPU's own quantized activations (teacher forcing): every
    mat-mul multiplies the activation exactly as the GPU quantized it (acts: name -> the
    dequantized values, fp64 [rows, k], for "attn_norm", "attn_out", "ffn_norm", "ffn_gate_up")
    by the dequantized weights (wdeq: "qkv", "o", "gu", "down" -> fp64 [n, k]), so no quant can
    land differently on the two sides; x is the GPU's input residual stream.  Returns the fp32
    tensors the runner exposes under the same names: attn_out, ffn_norm, ffn_gate_up, l_out
    (and x1, the residual after the attention)."""
    H, nq, nkv, hd = hp["n_embd"], hp["n_head"], hp["n_kv_head"], hp["head_dim"]
    eps = hp["rms_norm_eps"]
    qkv = (acts["attn_norm"] @ wdeq["qkv"].T).astype(np.float32)
    qd, kvd = nq * hd, nkv * hd
    a = attention(hp, lay, qkv[:, :qd], qkv[:, qd:qd + kvd], qkv[:, qd + kvd:], B, T)
    x1 = (x + (acts["attn_out"] @ wdeq["o"].T).astype(np.float32)).astype(np.float32)
    h = rms_norm(x1, lay["ffn_norm"], eps)
    gu = (acts["ffn_norm"] @ wdeq["gu"].T).astype(np.float32)
    x2 = (x1 + (acts["ffn_gate_up"] @ wdeq["down"].T).astype(np.float32)).astype(np.float32)
    return {"attn_out": a, "x1": x1, "ffn_norm": h, "ffn_gate_up": gu, "l_out": x2}
