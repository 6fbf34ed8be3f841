"""Runners built from GGUF files (mq_bert_load, mq_decoder_load) against the same weights
uploaded from memory: the loaded model must be the uploaded model, so the pooled embeddings are
bit-identical.  Variants: CrispEmbed names (enc.N / dec.N) and llama.cpp names (blk.N), a fused
q|k|v tensor, F16 and quantized embedding tables (compared with the model built from the
dequantized table, which is what ggml's get_rows feeds the graph)."""
import numpy as np
import pytest

import oracle_ffi as O
from crispembed_amd import bert, decoder, gguf, mq
from gpu_util import dev, host, stream

pytestmark = pytest.mark.gpu

BERT_HP = dict(n_layer=2, n_embd=128, n_head=4, n_ff=256, n_vocab=300, n_max_pos=64, n_type=2, layer_norm_eps=1e-12)
DEC_HP = dict(n_layer=2, n_embd=256, n_head=4, n_kv_head=2, head_dim=128, n_ff=512, n_vocab=300, rms_norm_eps=1e-6,
              rope_theta=1e6, causal=1, pooling=2)


def _ids(B, T, V, seed):
    return np.random.default_rng(seed).integers(0, V, B * T).astype(np.int32)


def _bert_out(model, ids, B, T):
    import torch
    out = torch.empty((B, model.hp["n_embd"]), dtype=torch.float32, device="cuda")
    types = np.random.default_rng(5).integers(0, 2, B * T).astype(np.int32)
    model.encode(dev(ids).data_ptr(), B, T, out.data_ptr(), stream(), types_dev=dev(types).data_ptr())
    return host(out)


def _dec_out(model, ids, B, T):
    import torch
    out = torch.empty((B, model.hp["n_embd"]), dtype=torch.float32, device="cuda")
    model.encode(dev(ids).data_ptr(), B, T, out.data_ptr(), stream())
    return host(out)


def _rewrite(src, dst, rename=None, retype=None):
    """Copy a GGUF with tensors renamed (dict or function) or re-encoded (name -> (type, bytes))."""
    with gguf.GGUFFile(src) as g:
        w = gguf.GGUFWriter()
        for k in g.keys():
            t, v = g.value(k)
            getattr(w, {gguf.UINT32: "add_uint32", gguf.FLOAT32: "add_float32", gguf.STRING: "add_string",
                        gguf.BOOL: "add_bool"}[t])(k, v)
        for n in g.tensor_names():
            t, ne, d = g.tensor(n)
            raw = d.tobytes()
            if retype and n in retype:
                t, raw = retype[n]
            nn = rename(n) if callable(rename) else (rename or {}).get(n, n)
            if nn is not None:
                w.add_tensor(nn, raw, t, ne)
    w.write(dst)


@pytest.mark.parametrize("wtype", [O.Q8_0, O.F16])
def test_bert_gguf_matches_upload(tmp_path, wtype):
    W = bert.synthetic_weights(BERT_HP, wtype, name="gg")
    p = tmp_path / "bert.gguf"
    gguf.write_bert_gguf(p, BERT_HP, wtype, W)
    ids = _ids(3, 20, BERT_HP["n_vocab"], 1)
    ref = _bert_out(bert.BertEncoder(BERT_HP, wtype, W), ids, 3, 20)
    m = bert.BertEncoder.from_gguf(p)
    assert m.hp["n_layer"] == 2 and m.hp["n_embd"] == 128 and m.hp["n_ff"] == 256 and m.hp["wtype"] == wtype
    assert m.hp["n_type"] == 2 and m.hp["n_max_pos"] == 64 and m.hp["n_vocab"] == 300
    assert np.array_equal(_bert_out(m, ids, 3, 20), ref)

    # llama.cpp names, and q|k|v fused into one tensor
    p2 = tmp_path / "bert_blk.gguf"
    tbl = {"token_embd_norm": "embd_ln", "attn_q": "attn.q", "attn_k": "attn.k", "attn_v": "attn.v",
           "attn_output": "attn.o", "ffn_up": "ffn.fc1", "ffn_down": "ffn.fc2", "attn_output_norm": "ln1",
           "layer_output_norm": "ln2"}
    inv = {v: k for k, v in tbl.items()}

    def blk(n):
        if n.startswith("embd_ln."):
            return "token_embd_norm." + n.split(".")[1]
        if n.startswith("enc."):
            _, i, *rest = n.split(".")
            body, suffix = ".".join(rest[:-1]), rest[-1]
            return f"blk.{i}.{inv[body]}.{suffix}"
        return n
    _rewrite(p, p2, rename=blk)
    assert np.array_equal(_bert_out(bert.BertEncoder.from_gguf(p2), ids, 3, 20), ref)

    p3 = tmp_path / "bert_qkv.gguf"
    with gguf.GGUFFile(p) as g:
        w = gguf.GGUFWriter(arch="bert")
        for k in g.keys():
            if k == "general.architecture":
                continue
            t, v = g.value(k)
            getattr(w, {gguf.UINT32: "add_uint32", gguf.FLOAT32: "add_float32", gguf.STRING: "add_string"}[t])(k, v)
        for n in g.tensor_names():
            t, ne, d = g.tensor(n)
            if ".attn.k." in n or ".attn.v." in n:
                continue
            if ".attn.q." in n:
                parts = [g.tensor(n.replace(".attn.q.", f".attn.{x}."))[2].tobytes() for x in "qkv"]
                nn = n.replace(".attn.q.", ".attn.qkv.")
                w.add_tensor(nn, b"".join(parts), t, [ne[0], 3 * ne[1]] if len(ne) == 2 else [3 * ne[0]])
            else:
                w.add_tensor(n, d.tobytes(), t, ne)
    w.write(p3)
    assert np.array_equal(_bert_out(bert.BertEncoder.from_gguf(p3), ids, 3, 20), ref)


@pytest.mark.parametrize("table_type", [O.F16, O.Q8_0])
def test_bert_gguf_quantized_table(oracle, tmp_path, table_type):
    """token_embd stored as F16 / Q8_0: the loaded model equals the model uploaded with the
    table dequantized by the oracle (ggml's dequantize_row)."""
    W = bert.synthetic_weights(BERT_HP, O.Q8_0, name="gq")
    p = tmp_path / "b.gguf"
    gguf.write_bert_gguf(p, BERT_HP, O.Q8_0, W)
    H, V = BERT_HP["n_embd"], BERT_HP["n_vocab"]
    tq = oracle.quantize_chunk(table_type, W["tok"])
    W2 = dict(W)
    W2["tok"] = oracle.dequantize(table_type, tq, H)
    p2 = tmp_path / "b2.gguf"
    _rewrite(p, p2, retype={"token_embd.weight": (table_type, np.ascontiguousarray(tq).tobytes())})
    ids = _ids(2, 16, V, 2)
    ref = _bert_out(bert.BertEncoder(BERT_HP, O.Q8_0, W2), ids, 2, 16)
    assert np.array_equal(_bert_out(bert.BertEncoder.from_gguf(p2), ids, 2, 16), ref)


@pytest.mark.parametrize("wtype", [O.Q4_K, O.Q6_K, O.Q8_0])
def test_decoder_gguf_matches_upload(tmp_path, wtype):
    W = decoder.synthetic_weights(DEC_HP, wtype, name="gd")
    p = tmp_path / "dec.gguf"
    gguf.write_decoder_gguf(p, DEC_HP, wtype, W)
    ids = _ids(2, 40, DEC_HP["n_vocab"], 3)
    ref = _dec_out(decoder.DecoderEmbedder(DEC_HP, wtype, W), ids, 2, 40)
    m = decoder.DecoderEmbedder.from_gguf(p)
    for k in ("n_layer", "n_embd", "n_head", "n_kv_head", "head_dim", "n_ff", "n_vocab", "causal", "pooling"):
        assert m.hp[k] == DEC_HP[k], k
    assert m.hp["wtype"] == wtype and m.hp["rope_theta"] == 1e6
    assert np.array_equal(_dec_out(m, ids, 2, 40), ref)

    # llama.cpp names
    tbl = {"attn.q": "attn_q", "attn.k": "attn_k", "attn.v": "attn_v", "attn.o": "attn_output",
           "attn.q_norm": "attn_q_norm", "attn.k_norm": "attn_k_norm", "ffn.gate": "ffn_gate", "ffn.up": "ffn_up",
           "ffn.down": "ffn_down", "attn_norm": "attn_norm", "ffn_norm": "ffn_norm"}

    def blk(n):
        if n.startswith("dec."):
            _, i, *rest = n.split(".")
            return f"blk.{i}.{tbl['.'.join(rest[:-1])]}.{rest[-1]}"
        return n
    p2 = tmp_path / "dec_blk.gguf"
    _rewrite(p, p2, rename=blk)
    assert np.array_equal(_dec_out(decoder.DecoderEmbedder.from_gguf(p2), ids, 2, 40), ref)


def test_decoder_gguf_mean_pool_bidirectional(tmp_path):
    hp = dict(DEC_HP, causal=0, pooling=1)
    W = decoder.synthetic_weights(hp, O.Q8_0, name="gm")
    p = tmp_path / "decm.gguf"
    gguf.write_decoder_gguf(p, hp, O.Q8_0, W)
    ids = _ids(2, 33, hp["n_vocab"], 4)
    m = decoder.DecoderEmbedder.from_gguf(p)
    assert m.hp["causal"] == 0 and m.hp["pooling"] == 1
    assert np.array_equal(_dec_out(m, ids, 2, 33), _dec_out(decoder.DecoderEmbedder(hp, O.Q8_0, W), ids, 2, 33))
