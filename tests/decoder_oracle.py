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


# ---------------------------------------------------------------- fp32 pipeline ----
# The same decoder with every step in fp32 as ggml's CPU backend runs it (rms_norm: fp32 squares
# summed in double, fp32 scale; the rope cache's fp32 angles; fp32 attention scores, softmax and
# P V; fp32 SiLU; mul_mat on the oracle's integer-dot product with fp32 accumulation) -- another
# fp32 pipeline with the same requantization points, to measure how far any fp32 pipeline lands
# from the fp64 one above.
F32 = np.float32


def rms_norm_f32(x, w, eps):
    x = x.astype(F32)
    ss = (x * x).astype(np.float64).sum(-1, keepdims=True)
    scale = (F32(1.0) / np.sqrt((ss / x.shape[-1]).astype(F32) + F32(eps))).astype(F32)
    return ((x * scale).astype(F32) * w.astype(F32)).astype(F32)


def rope_cache_f32(T, d, base):
    """cos / sin [T, d/2] of ggml's rope cache: theta_i = p * s^i by repeated fp32 products."""
    half = d // 2
    s = F32(base) ** F32(-2.0 / d)
    th = np.zeros((T, half), F32)
    th[:, 0] = np.arange(T, dtype=F32)
    for i in range(1, half):
        th[:, i] = (th[:, i - 1] * s).astype(F32)
    return np.cos(th).astype(F32), np.sin(th).astype(F32)


def attention_f32(hp, lay, q, k, v, B, T, cs):
    nq, nkv, hd, eps = hp["n_head"], hp["n_kv_head"], hp["head_dim"], hp["rms_norm_eps"]
    q = rms_norm_f32(q.reshape(B, T, nq, hd), lay["q_norm"], eps)
    k = rms_norm_f32(k.reshape(B, T, nkv, hd), lay["k_norm"], eps)
    c, s = cs[0][None, :, None, :], cs[1][None, :, None, :]
    half = hd // 2

    def rot(x):
        a, b = x[..., :half], x[..., half:]
        return np.concatenate([(a * c - b * s).astype(F32), (a * s + b * c).astype(F32)], -1)

    q, k = rot(q).transpose(0, 2, 1, 3), rot(k).transpose(0, 2, 1, 3)
    v = v.reshape(B, T, nkv, hd).transpose(0, 2, 1, 3).astype(F32)
    g = nq // nkv
    kk, vv = np.repeat(k, g, 1), np.repeat(v, g, 1)
    sc = (np.matmul(q, np.ascontiguousarray(kk.transpose(0, 1, 3, 2))) * F32(1.0 / np.sqrt(hd))).astype(F32)
    if hp["causal"]:
        sc = np.where(np.tril(np.ones((T, T), bool)), sc, F32(-np.inf))
    e = np.exp((sc - sc.max(-1, keepdims=True)).astype(F32)).astype(F32)
    p = (e / e.sum(-1, keepdims=True, dtype=F32)).astype(F32)
    return np.matmul(p, vv).astype(F32).transpose(0, 2, 1, 3).reshape(B * T, nq * hd)


def encode_f32(orc, hp, wtype, W, ids, nthreads=8):
    """encode() as an fp32 pipeline (last-token pooling): the pooled, L2-normalised rows."""
    B, T = ids.shape
    eps = hp["rms_norm_eps"]
    cs = rope_cache_f32(T, hp["head_dim"], hp["rope_theta"])

    def mm(x, w):
        return orc.fast_mul_mat(wtype, w, x, nthreads=nthreads)

    x = W["tok"][ids.ravel()].astype(F32)
    for lay in W["layers"]:
        h = rms_norm_f32(x, lay["attn_norm"], eps)
        a = attention_f32(hp, lay, mm(h, lay["wq"]), mm(h, lay["wk"]), mm(h, lay["wv"]), B, T, cs)
        x = (x + mm(a, lay["wo"])).astype(F32)
        h = rms_norm_f32(x, lay["ffn_norm"], eps)
        g, u = mm(h, lay["wgate"]), mm(h, lay["wup"])
        x = (x + mm(((g / (F32(1) + np.exp(-g).astype(F32))).astype(F32) * u).astype(F32), lay["wdown"])).astype(F32)
    pooled = rms_norm_f32(x.reshape(B, T, -1)[:, -1], W["out_norm"], eps).astype(np.float64)
    return (pooled / np.linalg.norm(pooled, axis=-1, keepdims=True)).astype(F32)
