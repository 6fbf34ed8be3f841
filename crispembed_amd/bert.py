"""Host side of the BERT-encoder runner (include/mq_bert.h): a synthetic model of a
given shape and its upload through the C ABI.

The synthetic model follows the CrispEmbed GGUF tensor set (src/crispembed.cpp:803-845:
token_embd, position_embd, token_type_embd, embd_ln, enc.N.{attn.q/k/v/o, ln1, ffn.fc1,
ffn.fc2, ln2}): embeddings and biases fp32 N(0, 0.02), LayerNorm weight 1 and bias 0,
linear weights N(0, 0.02) quantized to the chosen GGUF type by the host quantizer.
"""
import ctypes

import numpy as np

from . import mq, synth

MINILM_L6 = dict(n_layer=6, n_embd=384, n_head=12, n_ff=1536, n_vocab=30522, n_max_pos=512, n_type=2,
                 layer_norm_eps=1e-12)


def _quantize(L, wtype, w):
    n, k = w.shape
    out = np.empty(L.mq_row_size(wtype, k) * n, dtype=np.uint8)
    got = L.mq_quantize_chunk(wtype, np.ascontiguousarray(w).ctypes.data_as(ctypes.c_void_p),
                              out.ctypes.data_as(ctypes.c_void_p), n, k)
    if got != out.size:
        raise mq.MQError("weight quantization failed")
    return out.reshape(n, -1)


def synthetic_weights(hp, wtype, name="minilm"):
    """Host tensors of a random-init encoder: dict of fp32 arrays and GGUF weight bytes."""
    L = mq.lib()
    H, F = hp["n_embd"], hp["n_ff"]
    W = {
        "tok": synth.normal(f"{name}/token_embd", (hp["n_vocab"], H), std=0.02),
        "pos": synth.normal(f"{name}/position_embd", (hp["n_max_pos"], H), std=0.02),
        "type": synth.normal(f"{name}/token_type_embd", (max(hp["n_type"], 1), H), std=0.02),
        "ln_w": np.ones(H, np.float32), "ln_b": np.zeros(H, np.float32),
        "layers": [],
    }
    for il in range(hp["n_layer"]):
        lay = {}
        for nm, shape in (("q", (H, H)), ("k", (H, H)), ("v", (H, H)), ("o", (H, H)), ("fc1", (F, H)), ("fc2", (H, F))):
            lay["w" + nm] = _quantize(L, wtype, synth.normal(f"{name}/enc.{il}.{nm}.weight", shape, std=0.02))
            lay["b" + nm] = synth.normal(f"{name}/enc.{il}.{nm}.bias", (shape[0],), std=0.02)
        for nm in ("ln1", "ln2"):
            lay[nm + "_w"] = np.ones(H, np.float32)
            lay[nm + "_b"] = np.zeros(H, np.float32)
        W["layers"].append(lay)
    return W


class BertEncoder:
    """A model resident on the current GPU; encode() runs on device ids."""

    def __init__(self, hp, wtype, weights):
        self.L = mq.lib()
        self.hp = dict(hp)
        c = mq.BertHparams(hp["n_layer"], hp["n_embd"], hp["n_head"], hp["n_ff"], hp["n_vocab"], hp["n_max_pos"],
                           hp["n_type"], hp["layer_norm_eps"], wtype)
        self.h = self.L.mq_bert_create(ctypes.byref(c))
        if not self.h:
            raise mq.MQError(self.L.mq_last_error().decode())
        p = lambda a: np.ascontiguousarray(a).ctypes.data_as(ctypes.c_void_p)  # noqa: E731
        W = weights
        mq.check(self.L.mq_bert_set_embeddings(self.h, p(W["tok"]), p(W["pos"]), p(W["type"]), p(W["ln_w"]),
                                               p(W["ln_b"])))
        for il, lay in enumerate(W["layers"]):
            mq.check(self.L.mq_bert_set_layer(
                self.h, il, p(lay["wq"]), p(lay["wk"]), p(lay["wv"]), p(lay["wo"]), p(lay["wfc1"]), p(lay["wfc2"]),
                p(lay["bq"]), p(lay["bk"]), p(lay["bv"]), p(lay["bo"]), p(lay["bfc1"]), p(lay["bfc2"]),
                p(lay["ln1_w"]), p(lay["ln1_b"]), p(lay["ln2_w"]), p(lay["ln2_b"])))

    @classmethod
    def from_gguf(cls, path):
        """A model loaded from a CrispEmbed BERT GGUF by the native loader (mq_bert_load)."""
        self = cls.__new__(cls)
        self.L = mq.lib()
        self.h = self.L.mq_bert_load(str(path).encode())
        if not self.h:
            raise mq.MQError(self.L.mq_last_error().decode())
        c = mq.BertHparams()
        mq.check(self.L.mq_bert_get_hparams(self.h, ctypes.byref(c)))
        self.hp = {f: getattr(c, f) for f, _ in c._fields_}
        return self

    def encode(self, ids_dev, B, T, out_dev, stream, types_dev=None, hidden_dev=None):
        mq.check(self.L.mq_bert_encode(self.h, ctypes.c_void_p(ids_dev), ctypes.c_void_p(types_dev or 0), B, T,
                                       ctypes.c_void_p(out_dev), ctypes.c_void_p(hidden_dev or 0), stream))

    def __del__(self):
        if getattr(self, "h", None):
            self.L.mq_bert_free(self.h)
            self.h = None
