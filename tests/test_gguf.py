"""GGUF v3 files (include/mq_gguf.h, crispembed_amd/gguf.py) on the CPU: no GPU call is made.

Pins of the reader, each independent of the writer where it matters:
  * a file assembled byte by byte here from the published layout (magic, version, counts,
    key/type/value triples, tensor infos, alignment padding) is parsed as laid out;
  * writer -> reader round trips of every scalar type (extremes included), strings, arrays,
    tensors of several types and ranks, default and custom alignment;
  * the typed readers convert exactly like core_gguf's kv_u32 / kv_i32 / kv_f32 / kv_bool /
    kv_str (src/core/gguf_loader.cpp:72-137): which source types each accepts, the rest -> default;
  * malformed files (every truncation of a valid file, bad magic / version / counts / lengths,
    misaligned or out-of-file tensor data, bad ranks and block multiples, duplicates, unknown
    types) fail to open with an error, never a crash;
  * the loaders reject GGUF variants the runners do not implement before touching the GPU.
"""
import struct

import numpy as np
import pytest

from crispembed_amd import gguf, mq


def _s(x):
    b = x.encode()
    return struct.pack("<Q", len(b)) + b


def _hand_file(version=3, alignment=None):
    """A GGUF assembled from the layout, independently of GGUFWriter."""
    kvs = [(_s("general.architecture") + struct.pack("<I", 8) + _s("bert")),
           (_s("x.count") + struct.pack("<I", 4) + struct.pack("<I", 1234)),
           (_s("x.list") + struct.pack("<I", 9) + struct.pack("<IQ", 5, 3) + struct.pack("<3i", -1, 0, 7))]
    if alignment:
        kvs.append(_s("general.alignment") + struct.pack("<I", 4) + struct.pack("<I", alignment))
    al = alignment or 32
    t0 = np.arange(6, dtype=np.float32)                      # ne [6]
    t1 = (np.arange(8, dtype=np.float32) - 3).astype(np.float16).reshape(2, 4)  # ne [4, 2]
    infos = [_s("a") + struct.pack("<I", 1) + struct.pack("<Q", 6) + struct.pack("<IQ", 0, 0),
             _s("b") + struct.pack("<I", 2) + struct.pack("<2Q", 4, 2) + struct.pack("<IQ", 1, al)]
    head = b"GGUF" + struct.pack("<IQQ", version, 2, len(kvs)) + b"".join(kvs) + b"".join(infos)
    head += b"\0" * (-len(head) % al)
    data = t0.tobytes() + b"\0" * (al - 24) + t1.tobytes()
    return head + data, len(head), t0, t1


def test_hand_assembled_file(tmp_path):
    for version, al in ((3, None), (2, None), (3, 64)):
        raw, data_off, t0, t1 = _hand_file(version, al)
        p = tmp_path / f"h{version}_{al}.gguf"
        p.write_bytes(raw)
        with gguf.GGUFFile(p) as g:
            assert g.version == version and g.alignment == (al or 32) and g.data_offset == data_off
            assert g.value("general.architecture") == (gguf.STRING, "bert")
            assert g.value("x.count") == (gguf.UINT32, 1234)
            t, v = g.value("x.list")
            assert t == gguf.ARRAY and v.tolist() == [-1, 0, 7]
            assert g.tensor_names() == ["a", "b"]
            ty, ne, d = g.tensor("a")
            assert ty == mq.TYPE_F32 and ne == [6] and np.array_equal(d.view(np.float32), t0)
            ty, ne, d = g.tensor("b")
            assert ty == mq.TYPE_F16 and ne == [4, 2] and np.array_equal(d.view(np.float16).reshape(2, 4), t1)
            assert g.tensor_offset("b") == (al or 32)


SCALARS = [(gguf.UINT8, 255), (gguf.INT8, -128), (gguf.UINT16, 65535), (gguf.INT16, -32768),
           (gguf.UINT32, 4294967295), (gguf.INT32, -2147483648), (gguf.UINT64, 2**64 - 1), (gguf.INT64, -2**63),
           (gguf.FLOAT32, 3.0e38), (gguf.FLOAT64, -1e-300), (gguf.BOOL, True), (gguf.BOOL, False)]


def _add(w, key, t, v):
    getattr(w, {gguf.UINT8: "add_uint8", gguf.INT8: "add_int8", gguf.UINT16: "add_uint16", gguf.INT16: "add_int16",
                gguf.UINT32: "add_uint32", gguf.INT32: "add_int32", gguf.UINT64: "add_uint64", gguf.INT64: "add_int64",
                gguf.FLOAT32: "add_float32", gguf.FLOAT64: "add_float64", gguf.BOOL: "add_bool",
                gguf.STRING: "add_string"}[t])(key, v)


@pytest.mark.parametrize("alignment", [32, 64, 256])
def test_writer_reader_round_trip(tmp_path, alignment):
    rng = np.random.default_rng(alignment)
    w = gguf.GGUFWriter(arch="qwen3", alignment=alignment)
    for i, (t, v) in enumerate(SCALARS):
        _add(w, f"s.{i}", t, v)
    w.add_string("s.empty", "")
    w.add_string("s.utf8", "café ☃")
    w.add_array("a.u8", np.arange(300) % 256, gguf.UINT8)
    w.add_array("a.f32", [1.5, -2.25], gguf.FLOAT32)
    w.add_array("a.i64", [-(2**40), 2**40], gguf.INT64)
    w.add_array("a.str", ["", "tok", "ü"], gguf.STRING)
    w.add_array("a.empty", [], gguf.INT32)
    f32 = rng.standard_normal((3, 5, 7)).astype(np.float32)
    f16 = rng.standard_normal(33).astype(np.float16)
    i8 = rng.integers(-128, 128, (4, 9), dtype=np.int8)
    q8 = rng.integers(0, 256, 2 * 3 * 34, dtype=np.uint8)  # 2 rows x 96 values of Q8_0 bytes
    w.add_tensor("t.f32", f32)
    w.add_tensor("t.f16", f16)
    w.add_tensor("t.i8", i8)
    w.add_tensor("t.q8", q8.tobytes(), mq.TYPE_Q8_0, [96, 2])
    w.add_tensor("t.4d", np.ones((2, 1, 3, 4), np.float32))
    p = tmp_path / "rt.gguf"
    w.write(p)
    with gguf.GGUFFile(p) as g:
        assert g.alignment == alignment and g.data_offset % alignment == 0
        for i, (t, v) in enumerate(SCALARS):
            tt, vv = g.value(f"s.{i}")
            assert tt == t
            assert vv == (np.float32(v) if t == gguf.FLOAT32 else v)
        assert g.value("s.empty") == (gguf.STRING, "")
        assert g.value("s.utf8") == (gguf.STRING, "café ☃")
        assert g.value("a.u8")[1].tolist() == (np.arange(300) % 256).tolist()
        assert g.value("a.f32")[1].tolist() == [1.5, -2.25]
        assert g.value("a.i64")[1].tolist() == [-(2**40), 2**40]
        assert g.value("a.str")[1] == ["", "tok", "ü"]
        assert g.value("a.empty")[1].size == 0
        for name, arr, ty in (("t.f32", f32, mq.TYPE_F32), ("t.f16", f16, mq.TYPE_F16), ("t.i8", i8, 24)):
            t, ne, d = g.tensor(name)
            assert t == ty and ne == list(reversed(arr.shape))
            assert d.tobytes() == arr.tobytes()
            assert g.tensor_offset(name) % alignment == 0
        t, ne, d = g.tensor("t.q8")
        assert t == mq.TYPE_Q8_0 and ne == [96, 2] and d.tobytes() == q8.tobytes()
        assert g.tensor("t.4d")[1] == [4, 3, 1, 2]
        with pytest.raises(KeyError):
            g.value("missing")
        with pytest.raises(KeyError):
            g.tensor("missing")


def test_typed_readers_match_core_gguf(tmp_path):
    """core_gguf conversions: kv_u32 takes every integer type (truncating), kv_i32 only the
    32/64-bit ones, kv_f32 FLOAT32/FLOAT64, kv_bool BOOL, kv_str STRING; else the default."""
    w = gguf.GGUFWriter()
    w.add_int32("i32", -1)
    w.add_uint8("u8", 200)
    w.add_int8("i8", -3)
    w.add_uint16("u16", 40000)
    w.add_uint64("u64", 2**33 + 5)
    w.add_int64("i64", -7)
    w.add_float64("f64", 0.1)
    w.add_float32("f32", 2.5)
    w.add_bool("b", True)
    w.add_string("s", "hello")
    w.add_array("arr", [1], gguf.UINT32)
    p = tmp_path / "typed.gguf"
    w.write(p)
    L = mq.lib()
    with gguf.GGUFFile(p) as g:
        u32 = lambda k: L.mq_gguf_get_u32(g.h, k.encode(), 99)  # noqa: E731
        i32 = lambda k: L.mq_gguf_get_i32(g.h, k.encode(), 99)  # noqa: E731
        f32 = lambda k: L.mq_gguf_get_f32(g.h, k.encode(), 99.0)  # noqa: E731
        bl = lambda k: L.mq_gguf_get_bool(g.h, k.encode(), 7)  # noqa: E731
        st = lambda k: L.mq_gguf_get_str(g.h, k.encode(), b"dflt")  # noqa: E731
        assert u32("i32") == 0xFFFFFFFF and u32("u8") == 200 and u32("i8") == (-3) & 0xFFFFFFFF
        assert u32("u16") == 40000 and u32("u64") == 5 and u32("i64") == (-7) & 0xFFFFFFFF
        assert u32("f32") == 99 and u32("b") == 99 and u32("s") == 99 and u32("arr") == 99 and u32("none") == 99
        assert i32("i32") == -1 and i32("u64") == 5 and i32("i64") == -7
        assert i32("u8") == 99 and i32("u16") == 99 and i32("i8") == 99 and i32("f32") == 99
        assert f32("f32") == 2.5 and f32("f64") == np.float32(0.1) and f32("i32") == 99.0
        assert bl("b") == 1 and bl("u8") == 7 and bl("none") == 7
        assert st("s") == b"hello" and st("u8") == b"dflt" and st("none") == b"dflt"


def _small_valid():
    w = gguf.GGUFWriter(arch="bert")
    w.add_uint32("k.n", 3)
    w.add_array("k.s", ["ab", "c"], gguf.STRING)
    w.add_tensor("t", np.arange(8, dtype=np.float32))
    return w.tobytes()


def _open_fails(tmp_path, raw, name="bad.gguf"):
    p = tmp_path / name
    p.write_bytes(raw)
    with pytest.raises(mq.MQError):
        gguf.GGUFFile(p)


def test_every_truncation_fails_cleanly(tmp_path):
    raw = _small_valid()
    p = tmp_path / "ok.gguf"  # the full file opens
    p.write_bytes(raw)
    gguf.GGUFFile(p).close()
    for n in range(len(raw)):
        _open_fails(tmp_path, raw[:n])


def _patch(raw, off, fmt, val):
    b = bytearray(raw)
    struct.pack_into(fmt, b, off, val)
    return bytes(b)


def test_malformed_headers(tmp_path):
    raw = _small_valid()
    _open_fails(tmp_path, b"GGUG" + raw[4:])                       # magic
    _open_fails(tmp_path, _patch(raw, 4, "<I", 1))                  # version 1
    _open_fails(tmp_path, _patch(raw, 4, "<I", 4))                  # version 4
    _open_fails(tmp_path, _patch(raw, 8, "<Q", 2**62))              # tensor count
    _open_fails(tmp_path, _patch(raw, 16, "<Q", 2**62))             # kv count
    _open_fails(tmp_path, _patch(raw, 24, "<Q", 2**63))             # first key length
    # first kv (general.architecture STRING): its type field -> unknown type 13
    klen = struct.unpack_from("<Q", raw, 24)[0]
    _open_fails(tmp_path, _patch(raw, 32 + klen, "<I", 13))
    # nested array element type
    w = gguf.GGUFWriter()
    w.add_array("x", [1, 2], gguf.UINT8)
    good = w.tobytes()
    klen = struct.unpack_from("<Q", good, 24)[0]
    _open_fails(tmp_path, _patch(good, 32 + klen + 4, "<I", gguf.ARRAY))
    _open_fails(tmp_path, _patch(good, 32 + klen + 8, "<Q", 2**61))  # array length past the file


def _tensor_file(ne, ttype, offset, nbytes=None, alignment=None, extra=b""):
    kv = b""
    n_kv = 0
    if alignment is not None:
        kv = _s("general.alignment") + struct.pack("<II", 4, alignment)
        n_kv = 1
    info = _s("t") + struct.pack("<I", len(ne)) + struct.pack(f"<{len(ne)}Q", *ne) + struct.pack("<IQ", ttype, offset)
    head = b"GGUF" + struct.pack("<IQQ", 3, 1, n_kv) + kv + info + extra
    head += b"\0" * (-len(head) % 32)
    return head + b"\0" * (nbytes if nbytes is not None else 0)


def test_malformed_tensors(tmp_path):
    p = tmp_path / "ok.gguf"  # the valid reference
    p.write_bytes(_tensor_file([8], 0, 0, 32))
    gguf.GGUFFile(p).close()
    _open_fails(tmp_path, _tensor_file([8], 0, 0, 31))             # data past the end
    _open_fails(tmp_path, _tensor_file([8], 0, 16, 64))            # offset not aligned
    _open_fails(tmp_path, _tensor_file([8], 0, 32, 40))            # aligned offset, data past the end
    _open_fails(tmp_path, _tensor_file([1, 1, 1, 1, 8], 0, 0, 32))  # rank 5
    _open_fails(tmp_path, _tensor_file([0], 0, 0, 32))             # zero extent
    _open_fails(tmp_path, _tensor_file([40], mq.TYPE_Q8_0, 0, 64))  # not a multiple of the block
    _open_fails(tmp_path, _tensor_file([8], 99, 0, 64))            # unknown ggml type
    _open_fails(tmp_path, _tensor_file([2**39, 2**39], 0, 0, 32))  # element count overflow
    _open_fails(tmp_path, _tensor_file([8], 0, 0, 64, alignment=48))  # alignment not a power of two
    _open_fails(tmp_path, _tensor_file([8], 0, 0, 64, alignment=0))


def test_duplicates_rejected(tmp_path):
    raw = _small_valid()
    # duplicate key: rename the second key to the first (same length keys)
    w = gguf.GGUFWriter()
    w.add_uint32("aa", 1)
    w.add_uint32("bb", 2)
    _open_fails(tmp_path, w.tobytes().replace(b"bb", b"aa"))
    w = gguf.GGUFWriter()
    w.add_tensor("x1", np.zeros(8, np.float32))
    w.add_tensor("x2", np.zeros(8, np.float32))
    _open_fails(tmp_path, w.tobytes().replace(b"x2", b"x1"))
    assert raw  # the helper file stays valid
    with pytest.raises(ValueError):
        gguf.GGUFWriter().add_tensor("q", b"\0" * 33, mq.TYPE_Q8_0, [32, 1])  # byte count off by one


def _write_tiny_bert(tmp_path, name, keys=(), drop=(), add_tensors=()):
    from crispembed_amd import bert
    hp = dict(n_layer=1, n_embd=64, n_head=2, n_ff=128, n_vocab=50, n_max_pos=16, n_type=2, layer_norm_eps=1e-12)
    W = bert.synthetic_weights(hp, mq.TYPE_Q8_0, name="tiny")
    p = tmp_path / name
    gguf.write_bert_gguf(p, hp, mq.TYPE_Q8_0, W)
    if not (keys or drop or add_tensors):
        return p
    # re-emit through a writer with the requested edits
    with gguf.GGUFFile(p) as g:
        w = gguf.GGUFWriter()
        for k in g.keys():
            t, v = g.value(k)
            if t == gguf.ARRAY:
                continue
            _add(w, k, t, v)
        for k, t, v in keys:
            if any(kk == k for kk, *_ in w.kv):
                w.kv = [x for x in w.kv if x[0] != k]
            _add(w, k, t, v)
        for n in g.tensor_names():
            if n in drop:
                continue
            t, ne, d = g.tensor(n)
            w.add_tensor(n, d.tobytes(), t, ne)
        for n, arr in add_tensors:
            w.add_tensor(n, arr)
    w.write(p)
    return p


@pytest.mark.parametrize("edit,msg", [
    (dict(keys=[("bert.pre_ln", gguf.UINT32, 1)]), "pre-LN"),
    (dict(keys=[("bert.pooling_method", gguf.UINT32, 1)]), "pooling"),
    (dict(keys=[("bert.ffn_act", gguf.STRING, "silu")]), "activation"),
    (dict(keys=[("bert.position_offset", gguf.UINT32, 2)]), "position offset"),
    (dict(keys=[("bert.num_experts", gguf.UINT32, 4)]), "experts"),
    (dict(drop=["position_embd.weight"]), "position embeddings"),
    (dict(drop=["token_embd.weight"]), "token_embd"),
    (dict(drop=["enc.0.ffn.fc2.weight"]), "ffn.fc2"),
    (dict(add_tensors=[("enc.0.ffn_gate.weight", np.zeros((128, 64), np.float32))]), "gated"),
])
def test_bert_loader_rejects_before_gpu(tmp_path, edit, msg):
    p = _write_tiny_bert(tmp_path, "edit.gguf", **edit)
    L = mq.lib()
    assert not L.mq_bert_load(str(p).encode())
    assert msg in L.mq_last_error().decode()


def test_loaders_reject_non_gguf(tmp_path):
    p = tmp_path / "not.gguf"
    p.write_bytes(b"\0" * 100)
    L = mq.lib()
    assert not L.mq_bert_load(str(p).encode()) and "magic" in L.mq_last_error().decode()
    assert not L.mq_decoder_load(str(p).encode())
    assert not L.mq_bert_load(str(tmp_path / "absent.gguf").encode())


def _write_tiny_decoder(tmp_path, name, keys=(), drop=(), add_tensors=()):
    from crispembed_amd import decoder
    hp = dict(n_layer=1, n_embd=256, n_head=2, n_kv_head=1, head_dim=128, n_ff=256, n_vocab=40, rms_norm_eps=1e-6,
              rope_theta=1e6, causal=1, pooling=2)
    W = decoder.synthetic_weights(hp, mq.TYPE_Q8_0, name="tinyd")
    p = tmp_path / name
    gguf.write_decoder_gguf(p, hp, mq.TYPE_Q8_0, W)
    with gguf.GGUFFile(p) as g:
        w = gguf.GGUFWriter()
        for k in g.keys():
            t, v = g.value(k)
            if any(k == kk for kk, *_ in keys):
                continue
            _add(w, k, t, v)
        for k, t, v in keys:
            _add(w, k, t, v)
        for n in g.tensor_names():
            if n in drop:
                continue
            t, ne, d = g.tensor(n)
            w.add_tensor(n, d.tobytes(), t, ne)
        for n, arr in add_tensors:
            w.add_tensor(n, arr)
    w.write(p)
    return p


@pytest.mark.parametrize("edit,msg", [
    (dict(keys=[("general.architecture", gguf.STRING, "gemma3")]), "Gemma"),
    (dict(keys=[("qwen3.rope.scaling_type", gguf.UINT32, 1)]), "RoPE scaling"),
    (dict(keys=[("decoder.activation", gguf.UINT32, 2)]), "activation"),
    (dict(keys=[("decoder.normalize_embeddings", gguf.UINT32, 0)]), "unnormalised"),
    (dict(add_tensors=[("dec.0.attn.q.bias", np.zeros(256, np.float32))]), "biases"),
    (dict(add_tensors=[("dense.0.weight", np.zeros((4, 256), np.float32))]), "dense"),
    (dict(drop=["dec.0.ffn.down.weight"]), "ffn.down"),
])
def test_decoder_loader_rejects_before_gpu(tmp_path, edit, msg):
    p = _write_tiny_decoder(tmp_path, "edit.gguf", **edit)
    L = mq.lib()
    assert not L.mq_decoder_load(str(p).encode())
    assert msg in L.mq_last_error().decode()
