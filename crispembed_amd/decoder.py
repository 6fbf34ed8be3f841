"""Host side of the decoder-embedder runner (include/mq_decoder.h): a synthetic model of a
given shape and its upload through the C ABI.

The synthetic model follows CrispEmbed's decoder tensor set (src/decoder_embed.cpp:286-313:
token_embd, output_norm, dec.N.{attn_norm, attn.q/k/v/o, attn.q_norm, attn.k_norm, ffn_norm,
ffn.gate/up/down}): token embedding fp32 N(0, 0.02), RMS-norm weights N(1, 0.02),
linear weights N(0, 0.02) quantized to the chosen GGUF type by the host quantizer.
"""
import ctypes

import numpy as np

from . import mq, synth
from .bert import _quantize

QWEN3_EMBED_0_6B = dict(n_layer=28, n_embd=1024, n_head=16, n_kv_head=8, head_dim=128, n_ff=3072, n_vocab=151643,
                        rms_norm_eps=1e-6, rope_theta=1e6, causal=1, pooling=2)


def synthetic_weights(hp, wtype, name="qwen3"):
    """Host tensors of a random-init decoder: dict of fp32 arrays and GGUF weight bytes."""
    L = mq.lib()
    H, F, hd = hp["n_embd"], hp["n_ff"], hp["head_dim"]
    qd, kvd = hp["n_head"] * hd, hp["n_kv_head"] * hd
    norm = lambda nm, n: (1.0 + synth.normal(nm, (n,), std=0.02)).astype(np.float32)  # noqa: E731
    W = {"tok": synth.normal(f"{name}/token_embd", (hp["n_vocab"], H), std=0.02),
         "out_norm": norm(f"{name}/output_norm", H), "layers": []}
    for il in range(hp["n_layer"]):
        lay = {}
        for nm, shape in (("q", (qd, H)), ("k", (kvd, H)), ("v", (kvd, H)), ("o", (H, qd)), ("gate", (F, H)),
                          ("up", (F, H)), ("down", (H, F))):
            lay["w" + nm] = _quantize(L, wtype, synth.normal(f"{name}/dec.{il}.{nm}.weight", shape, std=0.02))
        lay["attn_norm"] = norm(f"{name}/dec.{il}.attn_norm", H)
        lay["ffn_norm"] = norm(f"{name}/dec.{il}.ffn_norm", H)
        lay["q_norm"] = norm(f"{name}/dec.{il}.attn_q_norm", hd)
        lay["k_norm"] = norm(f"{name}/dec.{il}.attn_k_norm", hd)
        W["layers"].append(lay)
    return W


class DecoderEmbedder:
    """A model resident on the current GPU; encode() runs on device ids."""

    def __init__(self, hp, wtype, weights):
        self.L = mq.lib()
        self.hp = dict(hp)
        c = mq.DecoderHparams(hp["n_layer"], hp["n_embd"], hp["n_head"], hp["n_kv_head"], hp["head_dim"], hp["n_ff"],
                              hp["n_vocab"], hp["rms_norm_eps"], hp["rope_theta"], hp["causal"], hp["pooling"], wtype)
        self.h = self.L.mq_decoder_create(ctypes.byref(c))
        if not self.h:
            raise mq.MQError(self.L.mq_last_error().decode())
        p = lambda a: None if a is None else np.ascontiguousarray(a).ctypes.data_as(ctypes.c_void_p)  # noqa: E731
        W = weights
        mq.check(self.L.mq_decoder_set_embeddings(self.h, p(W["tok"]), p(W["out_norm"])))
        for il, lay in enumerate(W["layers"]):
            mq.check(self.L.mq_decoder_set_layer(
                self.h, il, p(lay["wq"]), p(lay["wk"]), p(lay["wv"]), p(lay["wo"]), p(lay["wgate"]), p(lay["wup"]),
                p(lay["wdown"]), p(lay["attn_norm"]), p(lay["ffn_norm"]), p(lay.get("q_norm")), p(lay.get("k_norm"))))

    @classmethod
    def from_gguf(cls, path):
        """A model loaded from a CrispEmbed decoder GGUF by the native loader (mq_decoder_load)."""
        self = cls.__new__(cls)
        self.L = mq.lib()
        self.h = self.L.mq_decoder_load(str(path).encode())
        if not self.h:
            raise mq.MQError(self.L.mq_last_error().decode())
        c = mq.DecoderHparams()
        mq.check(self.L.mq_decoder_get_hparams(self.h, ctypes.byref(c)))
        self.hp = {f: getattr(c, f) for f, _ in c._fields_}
        return self

    def encode(self, ids_dev, B, T, out_dev, stream, hidden_dev=None):
        mq.check(self.L.mq_decoder_encode(self.h, ctypes.c_void_p(ids_dev), B, T, ctypes.c_void_p(out_dev),
                                          ctypes.c_void_p(hidden_dev or 0), stream))

    def __del__(self):
        if getattr(self, "h", None):
            self.L.mq_decoder_free(self.h)
            self.h = None
