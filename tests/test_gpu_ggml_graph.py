"""CrispEmbed's BERT encoder graph (build_encoder_graph, src/crispembed.cpp:1043-1468) built with
ggml's graph API and computed entirely by the MI355X ggml backend (every node claimed by
supports_op), checked against the CPU reference encoder on the same GGUF bytes.

Cases: separate and fused q|k|v projections, equal-length batches (no mask) and the rectangular
padded batch of encode_tokens_group_4d (src/crispembed.cpp:2052-2127: F16 padding mask, each
item compared with the reference encoding that item alone at its own length), and the graph
with the backend's fusion switched off (MQ_GGML_NO_FUSION) giving the same result to fp32
rounding.  Gate: cosine >= 0.99999 per token row and for the pooled embedding."""
import json
import os
import subprocess

import numpy as np
import pytest

import bert_oracle
import oracle_ffi as O
from crispembed_amd import bert, gguf

pytestmark = pytest.mark.gpu
ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
EXE = os.path.join(ROOT, "crispembed_amd", "bin", "test-bert-graph-mi355")
COSINE_MIN = 0.99999
HP = dict(n_layer=2, n_embd=128, n_head=4, n_ff=512, n_vocab=500, n_max_pos=64, n_type=2, layer_norm_eps=1e-12)


def _run(tmp_path, model, B, T, ids, types, lens, extra=(), env=None):
    for name, a in (("ids", ids), ("types", types), ("lens", lens)):
        np.ascontiguousarray(a, dtype=np.int32).tofile(tmp_path / f"{name}.i32")
    out = tmp_path / "out.f32"
    r = subprocess.run([EXE, str(model), str(B), str(T), str(tmp_path / "ids.i32"), str(tmp_path / "types.i32"),
                        str(tmp_path / "lens.i32"), str(out), *extra], capture_output=True, text=True, timeout=300,
                       env=dict(os.environ, **(env or {})))
    print(r.stderr[-2000:])
    res = json.loads(r.stdout.strip().splitlines()[-1])
    assert r.returncode == 0 and res["ok"], res
    assert res["unsupported"] == 0
    y = np.fromfile(out, dtype=np.float32)
    return (y if "--packed" in extra else y.reshape(B * T, -1)), res


def _cos_rows(a, b):
    a, b = a.astype(np.float64), b.astype(np.float64)
    return (a * b).sum(-1) / (np.linalg.norm(a, axis=-1) * np.linalg.norm(b, axis=-1))


def _pool(h):
    p = h.astype(np.float64).mean(0)
    return p / np.linalg.norm(p)


@pytest.mark.parametrize("wtype,hd,T", [(O.Q8_0, 32, 40), (O.Q8_0, 64, 40), (O.Q4_K, 64, 40), (O.Q6_K, 32, 40),
                                        (O.F16, 32, 40), (O.Q8_0, 32, 64), (O.Q8_0, 64, 64), (O.Q4_K, 32, 64)])
def test_bert_graph_matches_reference(oracle, tmp_path, wtype, hd, T):
    """T = 64 (whole 32-key blocks): the q/k/v GEMM stores k and v as attention fragments."""
    hp = dict(HP, n_head=HP["n_embd"] // hd)
    if wtype in (O.Q4_K, O.Q6_K):
        hp.update(n_embd=256, n_head=256 // hd)
    W = bert.synthetic_weights(hp, wtype, name=f"graph{wtype}_{hd}")
    model = tmp_path / "m.gguf"
    gguf.write_bert_gguf(model, hp, wtype, W)
    B = 3
    rng = np.random.default_rng(wtype + hd)
    ids = rng.integers(0, hp["n_vocab"], (B, T)).astype(np.int32)
    types = rng.integers(0, 2, (B, T)).astype(np.int32)
    _, ref = bert_oracle.encode(oracle, hp, wtype, W, ids, types)
    for extra in ((), ("--fused-qkv",)):
        got, _ = _run(tmp_path, model, B, T, ids, types, np.full(B, T), extra)
        cos = _cos_rows(got, ref)
        print(wtype, hd, extra, "min row cosine", cos.min())
        assert np.isfinite(got).all() and cos.min() >= COSINE_MIN
        for b in range(B):
            assert _pool(got[b * T:(b + 1) * T]) @ _pool(ref[b * T:(b + 1) * T]) >= COSINE_MIN


@pytest.mark.parametrize("lens", [[37, 5, 20, 1], [64, 5, 33, 1]])
def test_bert_graph_padded_batch(oracle, tmp_path, lens):
    """encode_tokens_group_4d: items padded to T_max with a -inf key mask; every item's real rows
    equal the reference encoding of that item alone (T_max 64: k and v as GEMM-stored fragments
    under the mask)."""
    hp = dict(HP)
    W = bert.synthetic_weights(hp, O.Q8_0, name="graphpad")
    model = tmp_path / "m.gguf"
    gguf.write_bert_gguf(model, hp, O.Q8_0, W)
    lens = np.array(lens, dtype=np.int32)
    B, T = len(lens), int(lens.max())
    rng = np.random.default_rng(7)
    ids = np.zeros((B, T), np.int32)
    types = np.zeros((B, T), np.int32)
    for b, n in enumerate(lens):
        ids[b, :n] = rng.integers(0, hp["n_vocab"], n)
        types[b, :n] = rng.integers(0, 2, n)
    got, _ = _run(tmp_path, model, B, T, ids, types, lens)
    for b, n in enumerate(lens):
        _, ref = bert_oracle.encode(oracle, hp, O.Q8_0, W, ids[b:b + 1, :n], types[b:b + 1, :n])
        rows = got[b * T:b * T + n]
        cos = _cos_rows(rows, ref)
        assert np.isfinite(rows).all() and cos.min() >= COSINE_MIN, (b, cos.min())
        assert _pool(rows) @ _pool(ref) >= COSINE_MIN


@pytest.mark.parametrize("hd,lens,maxtok", [(32, [37, 5, 20, 1, 64, 64, 33], 100), (64, [40, 40, 40, 3], 384),
                                            (32, [130, 7], 100)])
def test_bert_graph_packed_batch(oracle, tmp_path, hd, lens, maxtok):
    """The reference's default GPU batching (encode_tokens_packed, src/crispembed.cpp:1870-2008, with
    its greedy grouping :2192-2216): items packed end to end into groups of at most maxtok tokens
    (an item longer than that alone), positions restarting per item, the block-diagonal F16
    seg_mask; a group of one item runs unmasked.  Every item's rows against the CPU encoder's
    encoding of that item alone, per row and pooled, at cosine >= 0.99999."""
    hp = dict(HP, n_head=HP["n_embd"] // hd, n_max_pos=160)
    W = bert.synthetic_weights(hp, O.Q8_0, name=f"graphpack{hd}")
    model = tmp_path / "m.gguf"
    gguf.write_bert_gguf(model, hp, O.Q8_0, W)
    lens = np.array(lens, dtype=np.int32)
    B, T = len(lens), int(lens.max())
    rng = np.random.default_rng(hd + B)
    ids = rng.integers(0, hp["n_vocab"], (B, T)).astype(np.int32)
    types = rng.integers(0, 2, (B, T)).astype(np.int32)
    got, res = _run(tmp_path, model, B, T, ids, types, lens, ("--packed", "--pack-maxtok", str(maxtok)))
    groups, i = [], 0
    while i < B:  # the reference's greedy grouping, restated
        j, tsum = i, 0
        while j < B and not (j > i and tsum + lens[j] > maxtok):
            tsum += lens[j]
            j += 1
        groups.append(tsum)
        i = j
    assert res["groups"] == len(groups) and res["group_tokens"] == groups
    got = got.reshape(-1, hp["n_embd"])
    assert got.shape[0] == lens.sum() and np.isfinite(got).all()
    at = 0
    for b, n in enumerate(lens):
        _, ref = bert_oracle.encode(oracle, hp, O.Q8_0, W, ids[b:b + 1, :n], types[b:b + 1, :n])
        rows = got[at:at + n]
        at += n
        cos = _cos_rows(rows, ref)
        assert cos.min() >= COSINE_MIN, (b, cos.min())
        assert _pool(rows) @ _pool(ref) >= COSINE_MIN


@pytest.mark.parametrize("maxtok", [384, 4096])
def test_bert_graph_packed_minilm_full_shape(oracle, tmp_path, maxtok):
    """The MiniLM-L6 32 x 128 batch through the packed path at the reference's default budget of
    384 tokens (10 groups of 3 items and one of 2, each a 384- or 256-token graph with its
    block-diagonal mask) and at CRISPEMBED_ENCODER_PACK_MAXTOK=4096 (one 4096-token graph, a
    4096 x 4096 mask): sampled items against the CPU encoder, and every item against the same batch
    through the unmasked 4-D batch graph."""
    hp = dict(bert.MINILM_L6)
    W = bert.synthetic_weights(hp, O.Q8_0, name="minilm")
    model = tmp_path / "m.gguf"
    gguf.write_bert_gguf(model, hp, O.Q8_0, W)
    B, T = 32, 128
    ids = np.random.default_rng(32128).integers(1000, 30521, (B, T)).astype(np.int32)
    types = np.zeros((B, T), np.int32)
    got, res = _run(tmp_path, model, B, T, ids, types, np.full(B, T), ("--packed", "--pack-maxtok", str(maxtok)))
    assert res["group_tokens"] == ([384] * 10 + [256] if maxtok == 384 else [4096])
    got = got.reshape(B * T, -1)
    plain, _ = _run(tmp_path, model, B, T, ids, types, np.full(B, T))
    assert _cos_rows(got, plain).min() >= COSINE_MIN
    for b in (0, 2, 3, 31):
        _, ref = bert_oracle.encode(oracle, hp, O.Q8_0, W, ids[b:b + 1], types[b:b + 1])
        rows = got[b * T:(b + 1) * T]
        assert _cos_rows(rows, ref).min() >= COSINE_MIN, b
        assert _pool(rows) @ _pool(ref) >= COSINE_MIN, b


def test_bert_graph_fusion_off_agrees(tmp_path):
    """The fused chains (NORM-MUL-ADD, ADD-GELU_ERF-MUL_MAT) against the node-by-node graph."""
    W = bert.synthetic_weights(HP, O.Q8_0, name="graphfuse")
    model = tmp_path / "m.gguf"
    gguf.write_bert_gguf(model, HP, O.Q8_0, W)
    B, T = 2, 33
    ids = np.random.default_rng(8).integers(0, HP["n_vocab"], (B, T)).astype(np.int32)
    types = np.zeros((B, T), np.int32)
    a, _ = _run(tmp_path, model, B, T, ids, types, np.full(B, T))
    b, _ = _run(tmp_path, model, B, T, ids, types, np.full(B, T), env={"MQ_GGML_NO_FUSION": "1"})
    assert _cos_rows(a, b).min() >= COSINE_MIN


# ------------------------------------------------------------------- decoder ----
DEC_EXE = os.path.join(ROOT, "crispembed_amd", "bin", "test-decoder-graph-mi355")
DEC_HP = dict(n_layer=2, n_embd=256, n_head=4, n_kv_head=2, head_dim=128, n_ff=512, n_vocab=300, rms_norm_eps=1e-6,
              rope_theta=1e6, causal=1, pooling=2)


def _run_dec(tmp_path, model, ids):
    T = ids.size
    np.ascontiguousarray(ids, dtype=np.int32).tofile(tmp_path / "ids.i32")
    out = tmp_path / "dout.f32"
    r = subprocess.run([DEC_EXE, str(model), str(T), str(tmp_path / "ids.i32"), str(out)], capture_output=True,
                       text=True, timeout=300)
    print(r.stderr[-2000:])
    res = json.loads(r.stdout.strip().splitlines()[-1])
    assert r.returncode == 0 and res["ok"], res
    assert res["unsupported"] == 0
    return np.fromfile(out, dtype=np.float32).reshape(T, -1)


@pytest.mark.parametrize("wtype,hd,causal", [(O.Q8_0, 128, 1), (O.Q4_K, 128, 1), (O.Q6_K, 64, 1), (O.Q8_0, 64, 0)])
def test_decoder_graph_matches_reference(oracle, tmp_path, wtype, hd, causal):
    """CrispEmbed's Qwen3 decoder graph (ROPE_EXT NEOX, per-head RMS norms, causal
    FLASH_ATTN_EXT mask, SiLU gate) computed by the backend against the CPU decoder: the normed
    last hidden state's last-token row (last-token pooling) and mean at cosine >= 0.9999 (the
    decoder bar: every mul_mat requantizes its input, and one flipped quant is not averaged
    away by last-token pooling)."""
    import decoder_oracle
    from crispembed_amd import decoder
    hp = dict(DEC_HP, head_dim=hd, causal=causal, pooling=2 if causal else 1)
    if hd == 64:
        hp.update(n_head=4, n_kv_head=4, n_embd=256)
    W = decoder.synthetic_weights(hp, wtype, name=f"dgraph{wtype}_{hd}_{causal}")
    model = tmp_path / "d.gguf"
    gguf.write_decoder_gguf(model, hp, wtype, W)
    T = 45
    ids = np.random.default_rng(wtype + hd).integers(0, hp["n_vocab"], (1, T)).astype(np.int32)
    got = _run_dec(tmp_path, model, ids)
    _, x = decoder_oracle.encode(oracle, hp, wtype, W, ids)
    ref = decoder_oracle.rms_norm(x, W["out_norm"], hp["rms_norm_eps"])
    cos = _cos_rows(got, ref)
    print(wtype, hd, causal, "row cosine min / median", cos.min(), np.median(cos))
    assert np.isfinite(got).all()
    # the median row: the CPU decoder rotates by exact angles, the graph by ggml's rope cache
    # (an fp32 product chain, up to ~1.7e-4 rad off at position 44), which with full attention
    # reaches every row
    assert np.median(cos) >= 0.99995
    assert cos[-1] >= 0.9999
    assert _pool(got) @ _pool(ref) >= 0.9999


@pytest.mark.parametrize("wtype", [O.Q4_K, O.Q6_K])
def test_decoder_graph_decode_size(oracle, tmp_path, monkeypatch, wtype):
    """The decoder graph at decode size (T = 5 tokens: every mat-mul on the self-quantizing GEMV
    path, q|k|v and gate|up as grouped launches) against the CPU decoder, and against the same
    graph run node by node (MQ_GGML_NO_FUSION=1: every MUL_MAT on its own, its input quantized by
    a separate launch)."""
    import decoder_oracle
    from crispembed_amd import decoder
    hp = dict(DEC_HP)
    W = decoder.synthetic_weights(hp, wtype, name=f"dgraph_decode{wtype}")
    model = tmp_path / "d.gguf"
    gguf.write_decoder_gguf(model, hp, wtype, W)
    ids = np.random.default_rng(wtype + 5).integers(0, hp["n_vocab"], (1, 5)).astype(np.int32)
    got = _run_dec(tmp_path, model, ids)
    monkeypatch.setenv("MQ_GGML_NO_FUSION", "1")
    plain = _run_dec(tmp_path, model, ids)
    _, x = decoder_oracle.encode(oracle, hp, wtype, W, ids)
    ref = decoder_oracle.rms_norm(x, W["out_norm"], hp["rms_norm_eps"])
    assert np.isfinite(got).all()
    assert _cos_rows(got, ref).min() >= 0.9999
    assert _cos_rows(got, plain).min() >= 0.99999


def test_bert_graph_hip_graph_replay(tmp_path):
    """With MQ_GGML_GRAPH=1 the backend captures a graph computed twice in a row and replays
    it: replays with different inputs uploaded in between (eager copies and readbacks between
    the replays) equal the first results bit for bit, and the captured second input equals its
    eager computation."""
    W = bert.synthetic_weights(HP, O.Q8_0, name="graphreplay")
    model = tmp_path / "m.gguf"
    gguf.write_bert_gguf(model, HP, O.Q8_0, W)
    B, T = 2, 29
    ids = np.random.default_rng(11).integers(0, HP["n_vocab"] - 1, (B, T)).astype(np.int32)
    types = np.zeros((B, T), np.int32)
    a, res = _run(tmp_path, model, B, T, ids, types, np.full(B, T), ("--check-replay", "--iters", "5"),
                  env={"MQ_GGML_GRAPH": "1"})
    assert res["replay_identical"] == 1
    second = np.fromfile(tmp_path / "out.f32.second", dtype=np.float32)
    a_eager, _ = _run(tmp_path, model, B, T, ids, types, np.full(B, T), ("--check-replay",))
    second_eager = np.fromfile(tmp_path / "out.f32.second", dtype=np.float32)
    assert np.array_equal(a, a_eager) and np.array_equal(second, second_eager)


@pytest.mark.parametrize("fused_qkv", [False, True])
@pytest.mark.parametrize("T", [40, 64])
def test_imatrix_observer_reads_every_src1(tmp_path, fused_qkv, T):
    """The MUL_MAT observer contract (src/imatrix.cpp:57-99, installed at src/crispembed.cpp:723):
    with an eval callback the scheduler computes the graph in pieces that end at each observed
    MUL_MAT and then reads its src1.  Every graph tensor starts as NaN bytes, so a src1 a fusion
    left unwritten shows: none may, every src1 must equal the node-by-node run's (to the last
    bits of the fused norm's lane order) and so must the imatrix sums of x^2, and the pieces
    together must compute the same encoder output."""
    W = bert.synthetic_weights(HP, O.Q8_0, name="graphobs")
    model = tmp_path / "m.gguf"
    gguf.write_bert_gguf(model, HP, O.Q8_0, W)
    B = 3
    ids = np.random.default_rng(12).integers(0, HP["n_vocab"], (B, T)).astype(np.int32)
    types = np.zeros((B, T), np.int32)
    extra = ("--observe", "--fused-qkv") if fused_qkv else ("--observe",)
    _, res = _run(tmp_path, model, B, T, ids, types, np.full(B, T), extra)
    per_layer = 4 if fused_qkv else 6
    assert res["observed"] == per_layer * HP["n_layer"]
    assert res["src1_nan"] == 0
    assert res["src1_max_rel"] <= 1e-5 and res["imatrix_max_rel"] <= 1e-5, res
    assert res["out_max_rel"] <= 1e-4, res


def test_bert_graph_minilm_full_shape(oracle, tmp_path):
    """The MiniLM-L6 shape of the end-to-end workload through the ggml graph: 6 layers, H 384,
    12 heads, FFN 1536, 32 sequences x 128 tokens, Q8_0 (the same batch the embeddings/s
    figure is measured on), against the CPU encoder on sampled sequences (each sequence is
    independent: no mask, attention within the item), and every row finite."""
    hp = dict(bert.MINILM_L6)
    W = bert.synthetic_weights(hp, O.Q8_0, name="minilm")
    model = tmp_path / "m.gguf"
    gguf.write_bert_gguf(model, hp, O.Q8_0, W)
    B, T = 32, 128
    ids = np.random.default_rng(32128).integers(1000, 30521, (B, T)).astype(np.int32)
    types = np.zeros((B, T), np.int32)
    got, _ = _run(tmp_path, model, B, T, ids, types, np.full(B, T))
    assert np.isfinite(got).all()
    for b in (0, 17, 31):
        _, ref = bert_oracle.encode(oracle, hp, O.Q8_0, W, ids[b:b + 1], types[b:b + 1])
        rows = got[b * T:(b + 1) * T]
        assert _cos_rows(rows, ref).min() >= COSINE_MIN, b
        assert _pool(rows) @ _pool(ref) >= COSINE_MIN, b
