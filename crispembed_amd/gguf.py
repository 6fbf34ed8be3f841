"""GGUF v3 files in CrispEmbed's naming: a writer, a reader over the native one, and synthetic
model files for the encoder and decoder runners.

Writer (GGUFWriter).  Stands in for the `gguf` Python package's GGUFWriter as CrispEmbed's
converters use it (models/convert-bert-to-gguf.py:438-470, models/convert-decoder-embed-to-gguf.py:
438-480): typed metadata (add_uint32 / add_int32 / add_float32 / add_bool / add_string /
add_array ...), tensors with their ggml type, written as header, metadata, tensor infos,
padding to general.alignment (32 unless set) and the tensor data, each tensor at an offset that
is a multiple of the alignment.

Reader (GGUFFile).  The native reader of include/mq_gguf.h (mmap, bounds-checked), with the
metadata as Python values and tensors as numpy views of the mapped bytes.

Synthetic models (write_bert_gguf, write_decoder_gguf).  The random-init weights of
crispembed_amd.bert / crispembed_amd.decoder written under the names and keys CrispEmbed's own
converters use (bert.* keys and enc.N.* tensors; qwen3.* keys and dec.N.* tensors), so that
mq_bert_load / mq_decoder_load build the same model as the in-memory upload.

Command line: python -m crispembed_amd.gguf synth {minilm,qwen3-0.6b} --type q8_0 OUT.gguf
"""
import argparse
import ctypes
import struct

import numpy as np

from . import mq

UINT8, INT8, UINT16, INT16, UINT32, INT32, FLOAT32, BOOL, STRING, ARRAY, UINT64, INT64, FLOAT64 = range(13)
_SCALAR = {UINT8: "<B", INT8: "<b", UINT16: "<H", INT16: "<h", UINT32: "<I", INT32: "<i", FLOAT32: "<f", BOOL: "<?",
           UINT64: "<Q", INT64: "<q", FLOAT64: "<d"}
_NP = {UINT8: np.uint8, INT8: np.int8, UINT16: np.uint16, INT16: np.int16, UINT32: np.uint32, INT32: np.int32,
       FLOAT32: np.float32, BOOL: np.uint8, UINT64: np.uint64, INT64: np.int64, FLOAT64: np.float64}

# ggml type id -> (values per block, bytes per block), the types this package writes or reads back
GGML_BLOCK = {mq.TYPE_F32: (1, 4), mq.TYPE_F16: (1, 2), mq.TYPE_Q8_0: (32, 34), mq.TYPE_Q4_K: (256, 144),
              mq.TYPE_Q6_K: (256, 210), 24: (1, 1), 26: (1, 4)}


def _gguf_str(s):
    b = s.encode() if isinstance(s, str) else bytes(s)
    return struct.pack("<Q", len(b)) + b


class GGUFWriter:
    """Collects metadata and tensors, then writes one GGUF v3 file."""

    def __init__(self, arch=None, alignment=32):
        self.kv = []  # (key, type, value, array element type)
        self.tensors = []  # (name, ggml type, ne, bytes)
        self.alignment = alignment
        if alignment != 32:
            self.add_uint32("general.alignment", alignment)
        if arch is not None:
            self.add_string("general.architecture", arch)

    def _add(self, key, vtype, value, etype=None):
        if any(k == key for k, *_ in self.kv):
            raise ValueError(f"duplicate key {key}")
        self.kv.append((key, vtype, value, etype))

    def add_uint8(self, k, v): self._add(k, UINT8, v)
    def add_int8(self, k, v): self._add(k, INT8, v)
    def add_uint16(self, k, v): self._add(k, UINT16, v)
    def add_int16(self, k, v): self._add(k, INT16, v)
    def add_uint32(self, k, v): self._add(k, UINT32, v)
    def add_int32(self, k, v): self._add(k, INT32, v)
    def add_float32(self, k, v): self._add(k, FLOAT32, v)
    def add_uint64(self, k, v): self._add(k, UINT64, v)
    def add_int64(self, k, v): self._add(k, INT64, v)
    def add_float64(self, k, v): self._add(k, FLOAT64, v)
    def add_bool(self, k, v): self._add(k, BOOL, bool(v))
    def add_string(self, k, v): self._add(k, STRING, v)

    def add_array(self, k, values, etype):
        """An array of one element type (STRING or a scalar type)."""
        self._add(k, ARRAY, list(values), etype)

    def add_tensor(self, name, data, ggml_type=None, ne=None):
        """data: a numpy array (F32 / F16 / int8 / int32 inferred, ne its reversed shape) or
        raw GGUF bytes with their ggml_type and ne (ne[0] the fastest axis)."""
        if any(n == name for n, *_ in self.tensors):
            raise ValueError(f"duplicate tensor {name}")
        if isinstance(data, np.ndarray) and ggml_type is None:
            ggml_type = {np.dtype(np.float32): mq.TYPE_F32, np.dtype(np.float16): mq.TYPE_F16,
                         np.dtype(np.int8): 24, np.dtype(np.int32): 26}[data.dtype]
            ne = list(reversed(data.shape))
        raw = np.ascontiguousarray(data).tobytes() if isinstance(data, np.ndarray) else bytes(data)
        blck, bpb = GGML_BLOCK[ggml_type]
        ne = [int(x) for x in ne]
        if not 1 <= len(ne) <= 4 or ne[0] % blck:
            raise ValueError(f"{name}: bad shape {ne} for type {ggml_type}")
        if len(raw) != int(np.prod(ne)) // blck * bpb:
            raise ValueError(f"{name}: {len(raw)} bytes for shape {ne} of type {ggml_type}")
        self.tensors.append((name, ggml_type, ne, raw))

    def _value(self, vtype, v, etype):
        if vtype == STRING:
            return _gguf_str(v)
        if vtype == ARRAY:
            out = struct.pack("<IQ", etype, len(v))
            if etype == STRING:
                return out + b"".join(_gguf_str(x) for x in v)
            return out + np.asarray(v, dtype=_NP[etype]).tobytes()
        return struct.pack(_SCALAR[vtype], v)

    def tobytes(self):
        al = self.alignment
        out = bytearray(b"GGUF" + struct.pack("<IQQ", 3, len(self.tensors), len(self.kv)))
        for k, t, v, et in self.kv:
            out += _gguf_str(k) + struct.pack("<I", t) + self._value(t, v, et)
        off = 0
        offsets = []
        for name, t, ne, raw in self.tensors:
            offsets.append(off)
            out += _gguf_str(name) + struct.pack("<I", len(ne)) + struct.pack(f"<{len(ne)}Q", *ne)
            out += struct.pack("<IQ", t, off)
            off += (len(raw) + al - 1) // al * al
        out += b"\0" * (-len(out) % al)
        for (name, t, ne, raw), o in zip(self.tensors, offsets):
            out += raw + b"\0" * (-len(raw) % al)
        return bytes(out)

    def write(self, path):
        with open(path, "wb") as f:
            f.write(self.tobytes())


class GGUFFile:
    """A GGUF file opened by the native reader; close() (or the context manager) unmaps it."""

    def __init__(self, path):
        self.L = mq.lib()
        self.h = self.L.mq_gguf_open(str(path).encode())
        if not self.h:
            raise mq.MQError(self.L.mq_last_error().decode())

    def close(self):
        if self.h:
            self.L.mq_gguf_close(self.h)
            self.h = None

    def __enter__(self):
        return self

    def __exit__(self, *a):
        self.close()

    def __del__(self):
        self.close()

    @property
    def version(self):
        return self.L.mq_gguf_version(self.h)

    @property
    def alignment(self):
        return self.L.mq_gguf_alignment(self.h)

    @property
    def data_offset(self):
        return self.L.mq_gguf_data_offset(self.h)

    def keys(self):
        return [self.L.mq_gguf_kv_key(self.h, i).decode() for i in range(self.L.mq_gguf_n_kv(self.h))]

    def value(self, key):
        """The metadata value as (type, python value); KeyError when absent."""
        i = self.L.mq_gguf_find_key(self.h, key.encode())
        if i < 0:
            raise KeyError(key)
        t = self.L.mq_gguf_kv_type(self.h, i)
        if t == STRING:
            return t, self.L.mq_gguf_get_str(self.h, key.encode(), None).decode()
        if t == ARRAY:
            et, n = self.L.mq_gguf_arr_type(self.h, i), self.L.mq_gguf_arr_n(self.h, i)
            if et == STRING:
                return t, [self.L.mq_gguf_arr_str(self.h, i, j).decode() for j in range(n)]
            if n == 0:
                return t, np.zeros(0, _NP[et])
            ptr = self.L.mq_gguf_arr_data(self.h, i)
            nb = n * np.dtype(_NP[et]).itemsize
            return t, np.frombuffer(ctypes.string_at(ptr, nb), dtype=_NP[et]).copy()
        raw = ctypes.string_at(self.L.mq_gguf_kv_data(self.h, i), struct.calcsize(_SCALAR[t]))
        v = struct.unpack(_SCALAR[t], raw)[0]
        return t, bool(v) if t == BOOL else v

    def tensor_names(self):
        return [self.L.mq_gguf_tensor_name(self.h, i).decode() for i in range(self.L.mq_gguf_n_tensors(self.h))]

    def tensor(self, name):
        """(ggml type, ne list, uint8 array of the tensor's bytes); KeyError when absent."""
        i = self.L.mq_gguf_find_tensor(self.h, name.encode())
        if i < 0:
            raise KeyError(name)
        t, nd = ctypes.c_int(), ctypes.c_int()
        ne = (ctypes.c_int64 * 4)()
        off, nb = ctypes.c_size_t(), ctypes.c_size_t()
        mq.check(self.L.mq_gguf_tensor_info(self.h, i, ctypes.byref(t), ctypes.byref(nd), ne, ctypes.byref(off),
                                            ctypes.byref(nb)))
        data = np.frombuffer(ctypes.string_at(self.L.mq_gguf_tensor_data(self.h, i), nb.value), dtype=np.uint8)
        return t.value, list(ne[:nd.value]), data

    def tensor_offset(self, name):
        i = self.L.mq_gguf_find_tensor(self.h, name.encode())
        off = ctypes.c_size_t()
        mq.check(self.L.mq_gguf_tensor_info(self.h, i, None, None, None, ctypes.byref(off), None))
        return off.value


def _rows(w):
    """GGUF bytes of a quantized [rows, row_bytes] array, its ne [k, rows] comes separately."""
    return np.ascontiguousarray(w).tobytes()


def write_bert_gguf(path, hp, wtype, W, name="minilm-synthetic"):
    """The encoder weights of crispembed_amd.bert.synthetic_weights as a CrispEmbed BERT GGUF
    (CrispEmbed-native keys, models/convert-bert-to-gguf.py:459-469; tensors
    src/crispembed.cpp:748-845)."""
    H, F = hp["n_embd"], hp["n_ff"]
    w = GGUFWriter(arch="bert")
    w.add_string("general.name", name)
    w.add_uint32("bert.vocab_size", hp["n_vocab"])
    w.add_uint32("bert.max_position_embeddings", hp["n_max_pos"])
    w.add_uint32("bert.hidden_size", H)
    w.add_uint32("bert.num_attention_heads", hp["n_head"])
    w.add_uint32("bert.num_hidden_layers", hp["n_layer"])
    w.add_uint32("bert.intermediate_size", F)
    w.add_float32("bert.layer_norm_eps", hp["layer_norm_eps"])
    w.add_uint32("bert.output_dim", H)
    w.add_uint32("bert.position_offset", 0)
    w.add_uint32("bert.pooling_method", 0)
    w.add_string("bert.model_type", "bert")
    w.add_tensor("token_embd.weight", W["tok"])
    w.add_tensor("position_embd.weight", W["pos"])
    if hp["n_type"] > 0:
        w.add_tensor("token_type_embd.weight", W["type"][:hp["n_type"]])
    w.add_tensor("embd_ln.weight", W["ln_w"])
    w.add_tensor("embd_ln.bias", W["ln_b"])
    for il, lay in enumerate(W["layers"]):
        p = f"enc.{il}."
        for nm, (n, k) in (("attn.q", (H, H)), ("attn.k", (H, H)), ("attn.v", (H, H)), ("attn.o", (H, H)),
                           ("ffn.fc1", (F, H)), ("ffn.fc2", (H, F))):
            key = "w" + nm.split(".")[1]
            w.add_tensor(p + nm + ".weight", _rows(lay[key]), wtype, [k, n])
            w.add_tensor(p + nm + ".bias", lay["b" + nm.split(".")[1]])
        for nm in ("ln1", "ln2"):
            w.add_tensor(p + nm + ".weight", lay[nm + "_w"])
            w.add_tensor(p + nm + ".bias", lay[nm + "_b"])
    w.write(path)


def write_decoder_gguf(path, hp, wtype, W, name="qwen3-synthetic"):
    """The decoder weights of crispembed_amd.decoder.synthetic_weights as a CrispEmbed decoder
    GGUF (qwen3.* keys as models/convert-decoder-embed-to-gguf.py:453-477 writes them; tensors
    src/decoder_embed.cpp:253-313)."""
    H, F, hd = hp["n_embd"], hp["n_ff"], hp["head_dim"]
    qd, kvd = hp["n_head"] * hd, hp["n_kv_head"] * hd
    a = "qwen3"
    w = GGUFWriter(arch=a)
    w.add_string("general.name", name)
    w.add_uint32(f"{a}.embedding_length", H)
    w.add_uint32(f"{a}.block_count", hp["n_layer"])
    w.add_uint32(f"{a}.attention.head_count", hp["n_head"])
    w.add_uint32(f"{a}.attention.head_count_kv", hp["n_kv_head"])
    w.add_uint32(f"{a}.attention.key_length", hd)
    w.add_uint32(f"{a}.attention.value_length", hd)
    w.add_uint32(f"{a}.feed_forward_length", F)
    w.add_float32(f"{a}.attention.layer_norm_rms_epsilon", hp["rms_norm_eps"])
    w.add_float32(f"{a}.rope.freq_base", hp["rope_theta"])
    w.add_uint32(f"{a}.rope.scaling_type", 0)
    w.add_float32(f"{a}.rope.scaling_factor", 1.0)
    w.add_uint32(f"{a}.context_length", 32768)
    w.add_uint32(f"{a}.pooling_type", {2: 3, 1: 1}[hp["pooling"]])
    if not hp["causal"]:
        w.add_uint32("decoder.is_bidirectional", 1)
    w.add_tensor("token_embd.weight", W["tok"])
    w.add_tensor("output_norm.weight", W["out_norm"])
    for il, lay in enumerate(W["layers"]):
        p = f"dec.{il}."
        w.add_tensor(p + "attn_norm.weight", lay["attn_norm"])
        for nm, key, (n, k) in (("attn.q", "wq", (qd, H)), ("attn.k", "wk", (kvd, H)), ("attn.v", "wv", (kvd, H)),
                                ("attn.o", "wo", (H, qd)), ("ffn.gate", "wgate", (F, H)), ("ffn.up", "wup", (F, H)),
                                ("ffn.down", "wdown", (H, F))):
            w.add_tensor(p + nm + ".weight", _rows(lay[key]), wtype, [k, n])
        if lay.get("q_norm") is not None:
            w.add_tensor(p + "attn.q_norm.weight", lay["q_norm"])
        if lay.get("k_norm") is not None:
            w.add_tensor(p + "attn.k_norm.weight", lay["k_norm"])
        w.add_tensor(p + "ffn_norm.weight", lay["ffn_norm"])
    w.write(path)


def main(argv=None):
    ap = argparse.ArgumentParser(prog="python -m crispembed_amd.gguf")
    sub = ap.add_subparsers(dest="cmd", required=True)
    s = sub.add_parser("synth", help="write a random-init model in CrispEmbed GGUF naming")
    s.add_argument("model", choices=["minilm", "qwen3-0.6b"])
    s.add_argument("out")
    s.add_argument("--type", default="q8_0", choices=["q8_0", "q4_K", "q6_K", "f16"])
    s.add_argument("--layers", type=int, default=None, help="override the layer count")
    s.add_argument("--vocab", type=int, default=None, help="override the token table's row count")
    s.add_argument("--one-layer", action="store_true",
                   help="quantize one random layer and store its bytes in every layer (the same work and bytes "
                        "for a kernel measurement, without quantizing every layer on the host)")
    i = sub.add_parser("ids", help="write synthetic token ids (int32, item-major) for the graph drivers")
    i.add_argument("out")
    i.add_argument("--batch", type=int, default=1)
    i.add_argument("--tokens", type=int, required=True)
    i.add_argument("--low", type=int, default=0)
    i.add_argument("--high", type=int, required=True, help="largest id (inclusive)")
    i.add_argument("--name", default="ids", help="the seed's name (the same name gives the same ids)")
    d = sub.add_parser("dump", help="list a GGUF file's metadata and tensors")
    d.add_argument("path")
    args = ap.parse_args(argv)
    if args.cmd == "dump":
        with GGUFFile(args.path) as g:
            print(f"GGUF v{g.version}, alignment {g.alignment}, data at {g.data_offset}")
            for k in g.keys():
                t, v = g.value(k)
                print(f"  {k} = {v if not isinstance(v, (list, np.ndarray)) or len(v) < 8 else f'[{len(v)} items]'}")
            for n in g.tensor_names():
                t, ne, data = g.tensor(n)
                print(f"  {n}: type {t} ne {ne} {data.nbytes} bytes")
        return 0
    if args.cmd == "ids":
        from . import synth
        ids = synth.integers(args.name, (args.batch * args.tokens,), args.low, args.high).astype(np.int32)
        ids.tofile(args.out)
        print(f"wrote {args.out}: {args.batch} x {args.tokens} ids in [{args.low}, {args.high}]")
        return 0
    wtype = {"q8_0": mq.TYPE_Q8_0, "q4_K": mq.TYPE_Q4_K, "q6_K": mq.TYPE_Q6_K, "f16": mq.TYPE_F16}[args.type]

    def weights(mod, hp):
        if not args.one_layer:
            return mod.synthetic_weights(hp, wtype)
        W = mod.synthetic_weights(dict(hp, n_layer=1), wtype)
        return dict(W, layers=W["layers"] * hp["n_layer"])
    if args.model == "minilm":
        from . import bert
        hp = dict(bert.MINILM_L6)
        if args.layers:
            hp["n_layer"] = args.layers
        if args.vocab:
            hp["n_vocab"] = args.vocab
        write_bert_gguf(args.out, hp, wtype, weights(bert, hp))
    else:
        from . import decoder
        hp = dict(decoder.QWEN3_EMBED_0_6B)
        if args.layers:
            hp["n_layer"] = args.layers
        if args.vocab:
            hp["n_vocab"] = args.vocab
        write_decoder_gguf(args.out, hp, wtype, weights(decoder, hp))
    print(f"wrote {args.out}")
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
