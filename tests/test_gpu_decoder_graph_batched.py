"""CrispEmbed's batched decoder graph on the MI355X backend: decoder_encode_tokens_batch
(src/decoder_embed.cpp:1322-1641, called from src/crispembed.cpp:2967) encodes B sequences as one
graph of T_total tokens with a T_total x T_total F16 mask (:1406-1443, passed to every layer's
FLASH_ATTN_EXT at :1517), built with ggml's graph API by test-decoder-graph-mi355 --batch.

At the Qwen3-Embedding-0.6B workload (28 layers, H 1024, 16 query / 8 key-value heads of 128,
SwiGLU FFN 3072, Q4_K linears, 16 sequences x 512 tokens: T_total 8192, a 128 MB mask) the checks
follow tests/test_gpu_decoder_full.py, which makes them for the repository's own runner:

* the graph computes entirely on the GPU, every node claimed by supports_op;
* (1) every quantized activation a product reads -- q/k/v, o, gate/up and down inputs, all 8192
  rows of all 28 layers -- seen through the backend's activation observer, equals the oracle's
  quantize_row_q8_K of the graph's own fp32 src1 byte for byte (quants, scales, min-term
  operands); the down projection's, formed inside the quantizer from silu(gate) * up with the
  device expf, on at least 99.9 % of its quants against the host expf;
* (2) teacher forcing on two sampled sequences: each layer computed by the CPU decoder from the
  GPU's own quantized activations matches every fp32 tensor the graph wrote within 1e-5 of its
  scale;
* the sampled sequences end to end against the free-running CPU decoder (pooled cosine
  >= 0.9999), and all 16 against the runner's encoding of the same batch;
* the scheduler's observed form: the graph in pieces that end at every MUL_MAT, with every src1
  written (no NaN left from the fill) and equal to the node-by-node run.

Smaller models cover the layout's other cases: ragged items with padding positions, the
prefix-sharing layout (positions continuing the prefix), and the same graphs without the mask
block lists (MQ_GGML_NO_MASK_BLOCKS=1).

Weights: four random layers, each uploaded to seven of the 28 layers, token table N(0, 0.02)
over the full 151643-token vocabulary.
"""
import json
import os
import subprocess

import numpy as np
import pytest

import decoder_oracle
import oracle_ffi as O
from bert_oracle import _w_deq
from gpu_util import host, stream

pytestmark = pytest.mark.gpu
ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
EXE = os.path.join(ROOT, "crispembed_amd", "bin", "test-decoder-graph-mi355")
B, T = 16, 512
SAMPLED = (0, 9)


def _run(model, ids, T, extra=(), env=None, out=None, timeout=900):
    """The driver on ids [B, T] (item-major slots); returns (hidden [T_total, H], JSON result)."""
    d = os.path.dirname(str(model))
    ids_p, out = os.path.join(d, "ids.i32"), out or os.path.join(d, "out.f32")
    np.ascontiguousarray(ids, dtype=np.int32).tofile(ids_p)
    cmd = [EXE, str(model), str(T), ids_p, out, "--batch", str(ids.shape[0]), *extra]
    print("running:", " ".join(cmd), flush=True)
    # the driver's progress lines (stderr) pass straight through
    r = subprocess.run(cmd, stdout=subprocess.PIPE, text=True, timeout=timeout, env=dict(os.environ, **(env or {})))
    res = json.loads(r.stdout.strip().splitlines()[-1])
    assert r.returncode == 0 and res["ok"], res
    assert res["unsupported"] == 0
    return np.fromfile(out, dtype=np.float32).reshape(res["T_total"], -1), res


def _l2(x):
    x = x.astype(np.float64)
    return x / np.linalg.norm(x, axis=-1, keepdims=True)


def _last_rows(res, lens):
    """The row of each item's last token in the layout the driver reports."""
    P, slot = res["prefix"], res["slot"]
    return np.array([P + b * slot + (n - P) - 1 for b, n in enumerate(lens)])


@pytest.fixture(scope="module")
def batched(oracle, tmp_path_factory):
    """The model as a CrispEmbed decoder GGUF, the 16 x 512 batch through the batched graph once
    with the activation observer checking every quantized activation, and the sampled sequences'
    rows of every layer's tensors and quantized activations dumped for teacher forcing."""
    from crispembed_amd import decoder, gguf, synth
    hp = dict(decoder.QWEN3_EMBED_0_6B)
    sets = [decoder.synthetic_weights(dict(hp, n_layer=1, n_vocab=1), O.Q4_K, name=f"qwen3_full{j}")["layers"][0]
            for j in range(4)]
    tok = np.random.default_rng(20261202).standard_normal((hp["n_vocab"], hp["n_embd"]), dtype=np.float32) * 0.02
    out_norm = (1.0 + 0.02 * np.random.default_rng(7).standard_normal(hp["n_embd"])).astype(np.float32)
    W = {"tok": tok, "out_norm": out_norm, "layers": [sets[il % 4] for il in range(hp["n_layer"])]}
    d = tmp_path_factory.mktemp("batched")
    model = d / "qwen3.gguf"
    gguf.write_decoder_gguf(model, hp, O.Q4_K, W)
    ids = synth.integers(f"qwen3/ids_{B}x{T}", (B, T), 0, hp["n_vocab"] - 1).astype(np.int32)
    rows = np.concatenate([np.arange(b * T, (b + 1) * T) for b in SAMPLED]).astype(np.int32)
    rows.tofile(d / "rows.i32")
    dump = d / "dump"
    dump.mkdir()
    hidden, res = _run(model, ids, T, ("--act-check", "--dump", str(d / "rows.i32"), str(dump)))
    print("driver:", res)
    return dict(hp=hp, W=W, ids=ids, model=model, hidden=hidden, res=res, dump=dump, rows=rows)


def _dump(bt, name, il, cols, dtype=np.float32):
    return np.fromfile(bt["dump"] / f"{name}_{il}.{'i8' if dtype == np.int8 else 'f32'}",
                       dtype=dtype).reshape(len(bt["rows"]), cols)


def test_batched_graph_full_shape_on_gpu(batched):
    res, hidden = batched["res"], batched["hidden"]
    assert res["T_total"] == B * T and res["prefix"] == 0 and res["slot"] == T
    assert hidden.shape == (B * T, batched["hp"]["n_embd"])
    assert np.isfinite(hidden).all()
    pooled = _l2(hidden[_last_rows(res, [T] * B)])
    cos = pooled @ pooled.T
    assert (cos[~np.eye(B, dtype=bool)] < 0.9999).all()  # 16 distinct sequences, 16 distinct embeddings


def test_glu_fusion_is_the_separate_nodes(batched):
    """Without an observer the backend forms silu(gate) * up in one gate|up GEMM over a combined
    weight image (the gate, SiLU, up and MUL nodes as one launch) and leaves the attention and FFN
    norms' float rows unwritten (their readers take the Q8_K copy): the 16 x 512 batch's hidden
    states equal, bit for bit, those of the graph with the nodes computed separately and every
    norm written (MQ_GGML_NO_GLU=1, MQ_GGML_WRITE_NORMS=1), and those of each change alone."""
    model, ids = batched["model"], batched["ids"]
    d = os.path.dirname(str(model))
    runs = {}
    for name, env in (("fused", {}), ("no_glu", {"MQ_GGML_NO_GLU": "1"}), ("write_norms", {"MQ_GGML_WRITE_NORMS": "1"}),
                      ("plain", {"MQ_GGML_NO_GLU": "1", "MQ_GGML_WRITE_NORMS": "1"})):
        runs[name] = _run(model, ids, T, ("--iters", "3"), env=env, out=os.path.join(d, f"{name}.f32"))
    print("batched graph ms:", {k: round(v[1]["ms_per_graph"], 3) for k, v in runs.items()})
    for name in ("no_glu", "write_norms", "plain"):
        assert np.array_equal(runs["fused"][0], runs[name][0]), name


def test_quantized_activations_are_the_oracles(batched):
    """(1): every product's quantized activation, every row, against the oracle."""
    res, n_layer = batched["res"], batched["hp"]["n_layer"]
    assert res["act_calls"] == 7 * n_layer  # q, k, v, o, gate, up, down
    assert res["act_checked"] == 4 * n_layer and res["act_unchecked"] == 0
    assert res["act_rows_checked"] == 4 * n_layer * B * T
    assert res["act_rows_bad"] == 0, res["act_first_bad"]
    assert res["silu_calls"] == n_layer
    print(f"silu(gate) * up quants identical to the oracle's: worst layer {res['silu_min_same']:.6f}")
    assert res["silu_min_same"] >= 0.999


def test_teacher_forced_layers(batched):
    """(2): each layer of the sampled sequences from the graph's own quantized activations."""
    hp, W, ids = batched["hp"], batched["W"], batched["ids"]
    ids2 = ids[list(SAMPLED)]
    Bs = ids2.shape[0]
    H, F, eps = hp["n_embd"], hp["n_ff"], hp["rms_norm_eps"]
    qd = hp["n_head"] * hp["head_dim"]
    cols = {"attn_norm": H, "attn_out": qd, "ffn_norm": H, "ffn_gate_up": F}
    deq, worst = {}, {}
    x = W["tok"][ids2.ravel()].astype(np.float32)
    for il, lay in enumerate(W["layers"]):
        key = id(lay)
        if key not in deq:
            deq[key] = {"qkv": np.concatenate([_w_deq(O.Q4_K, lay[w], H) for w in ("wq", "wk", "wv")]),
                        "o": _w_deq(O.Q4_K, lay["wo"], qd),
                        "gu": np.concatenate([_w_deq(O.Q4_K, lay[w], H) for w in ("wgate", "wup")]),
                        "down": _w_deq(O.Q4_K, lay["wdown"], F)}
        acts = {}
        for n, k in cols.items():
            q = _dump(batched, "act_" + n, il, k, np.int8)
            d = _dump(batched, "act_" + n, il, k // 256)
            acts[n] = (q.reshape(q.shape[0], -1, 256).astype(np.float64) *
                       d[:, :, None].astype(np.float64)).reshape(q.shape[0], -1)
        ref = decoder_oracle.layer_from_quants(hp, lay, deq[key], x, acts, Bs, T)
        ref["attn_norm"] = decoder_oracle.rms_norm(x, lay["attn_norm"], eps)
        got = {"attn_norm": _dump(batched, "attn_norm", il, H), "attn_out": _dump(batched, "attn_out", il, qd),
               "ffn_norm": _dump(batched, "ffn_norm", il, H),
               "ffn_gate_up": np.concatenate([_dump(batched, "gate", il, F), _dump(batched, "up", il, F)], axis=1)}
        if il + 1 < len(W["layers"]):
            got["l_out"] = _dump(batched, "l_out", il, H)
        else:  # the last residual sum has one reader, the output norm, which forms it: not written
            ref["out"] = decoder_oracle.rms_norm(ref["l_out"], W["out_norm"], eps)
            got["out"] = batched["hidden"][batched["rows"]]
        for name, g in got.items():
            r = ref[name]
            err = float(np.abs(g.astype(np.float64) - r).max() / np.abs(r).max())
            worst[name] = max(worst.get(name, 0.0), err)
            assert err <= 1e-5, (name, il, err)
        x = got.get("l_out")
    print("teacher-forced worst relative error per tensor:", worst)


def test_sampled_sequences_end_to_end(oracle, batched):
    """The sampled sequences against the free-running CPU decoder (last-token pooling)."""
    hp, W, ids = batched["hp"], batched["W"], batched["ids"]
    ids2 = ids[list(SAMPLED)]
    ref, _ = decoder_oracle.encode(oracle, hp, O.Q4_K, W, ids2)
    rows = _last_rows(batched["res"], [T] * B)[list(SAMPLED)]
    got = _l2(batched["hidden"][rows])
    cos = (got * ref).sum(-1)
    print("free-running pooled cosine per sequence:", cos)
    assert cos.min() >= 0.9999


def test_batched_graph_matches_runner(batched):
    """All 16 sequences against the runner's encoding of the same batch (per-sequence causal
    attention, another GEMM grouping): the same computation up to fp32 rounding."""
    import torch
    from crispembed_amd import decoder
    hp, W, ids = batched["hp"], batched["W"], batched["ids"]
    dec = decoder.DecoderEmbedder(hp, O.Q4_K, W)
    ids_d = torch.from_numpy(ids.ravel().copy()).cuda()
    out = torch.empty((B, hp["n_embd"]), dtype=torch.float32, device="cuda")
    dec.encode(ids_d.data_ptr(), B, T, out.data_ptr(), stream())
    runner = host(out).astype(np.float64)
    del dec
    got = _l2(batched["hidden"][_last_rows(batched["res"], [T] * B)])
    cos = (got * runner).sum(-1)
    print("batched graph against the runner, pooled cosine:", cos.min(), np.median(cos))
    assert cos.min() >= 0.9999


def test_observed_split_full_shape(batched):
    """The eval-callback form at the full workload: 196 pieces, each ending at a MUL_MAT whose
    src1 is read after its piece (every graph tensor first filled with NaN bytes).  Every src1 was
    written (none keeps the fill), and the observed run is exact in its own terms: every quantized
    activation it reads equals the oracle's quantization of its own src1 (as the unobserved run's
    do).  Against the node-by-node run: the first products' src1, the normed embeddings before any
    quantization, to fp32 rounding; past the first quantization the two runs' fp32 rows differ by
    ulps (different norm kernels inside and outside the pieces), and an activation they round an ulp
    apart can land on another quant, which later layers carry -- so the src1, the imatrix sums and
    the output agree at the decoder's end-to-end bar (pooled cosine per item >= 0.9999), with the
    largest relative differences printed."""
    _, res = _run(batched["model"], batched["ids"], T, ("--observe", "--act-check"), timeout=1200,
                  out=str(batched["dump"] / "observed.f32"))
    print("observed:", {k: res[k] for k in ("observed", "src1_nan", "src1_max_rel", "src1_max_rel_first",
                                            "src1_max_rel_norm0", "imatrix_max_rel", "out_max_rel",
                                            "obs_pooled_cos_min", "obs_act_checked", "obs_act_rows_bad",
                                            "obs_silu_min_same")})
    n_layer = batched["hp"]["n_layer"]
    assert res["observed"] == 7 * n_layer
    assert res["src1_nan"] == 0
    assert res["obs_act_checked"] >= 4 * n_layer and res["obs_act_unchecked"] == 0
    assert res["obs_act_rows_bad"] == 0 and res["obs_silu_min_same"] >= 0.999
    assert res["src1_max_rel_norm0"] <= 1e-6
    assert res["obs_pooled_cos_min"] >= 0.9999
    assert res["src1_max_rel"] <= 0.05 and res["imatrix_max_rel"] <= 0.05


# ------------------------------------------------------------------ smaller layouts ----
SMALL = dict(n_layer=2, n_embd=256, n_head=4, n_kv_head=2, head_dim=128, n_ff=512, n_vocab=300, rms_norm_eps=1e-6,
             rope_theta=1e6, causal=1, pooling=2)


@pytest.mark.parametrize("layout", ["ragged", "prefix", "prefix_ragged"])
def test_batched_graph_layouts(oracle, tmp_path, layout):
    """Ragged items (padding positions attend only to themselves), and items sharing a prefix of
    at least 4 tokens (one prefix copy, positions continuing it): each item's rows against the
    CPU decoder's encoding of that item alone, and the graph without mask block lists (the
    attention then classifies every mask block itself) against the graph with them."""
    from crispembed_amd import decoder, gguf
    hp = dict(SMALL)
    W = decoder.synthetic_weights(hp, O.Q4_K, name=f"dbatch_{layout}")
    model = tmp_path / "d.gguf"
    gguf.write_decoder_gguf(model, hp, O.Q4_K, W)
    rng = np.random.default_rng(len(layout))
    Tm = 70
    lens = np.array({"ragged": [70, 23, 41, 1], "prefix": [70, 70, 70], "prefix_ragged": [70, 12, 55]}[layout],
                    np.int32)
    ids = rng.integers(0, hp["n_vocab"], (len(lens), Tm)).astype(np.int32)
    if layout.startswith("prefix"):
        ids[:, :10] = ids[0, :10]
    lens.tofile(tmp_path / "lens.i32")
    got, res = _run(model, ids, Tm, ("--lens", str(tmp_path / "lens.i32")))
    assert (res["prefix"] == 10) == layout.startswith("prefix")
    plain, _ = _run(model, ids, Tm, ("--lens", str(tmp_path / "lens.i32")), env={"MQ_GGML_NO_MASK_BLOCKS": "1"},
                    out=str(tmp_path / "plain.f32"))
    assert np.isfinite(got).all()
    a, b = _l2(got), _l2(plain)
    assert (a * b).sum(-1).min() >= 0.99999
    P, slot = res["prefix"], res["slot"]
    for it, n in enumerate(lens):
        _, x = decoder_oracle.encode(oracle, hp, O.Q4_K, W, ids[it:it + 1, :n])
        ref = decoder_oracle.rms_norm(x, W["out_norm"], hp["rms_norm_eps"])
        rows = np.concatenate([np.arange(P), P + it * slot + np.arange(n - P)]) if P else it * slot + np.arange(n)
        cos = (_l2(got[rows]) * _l2(ref)).sum(-1)
        print(layout, it, "row cosine min / median", cos.min(), np.median(cos))
        assert np.median(cos) >= 0.99995 and cos[-1] >= 0.9999, (it, cos.min())
