#!/usr/bin/env python3
"""Writes the golden fixtures of the quantized mul_mat path into tests/golden/.

The reference holds no golden vectors or known-answer tests for this path (its
tests are end-to-end against downloaded models), so these fixtures are written
by the oracle (oracle/liboracle.so, ggml semantics restated in C) from fixed
seeds and frozen here.  Each expected output is also pinned independently of
the oracle by tests/test_golden.py (numpy decoders written from the block
format description, the closed-form quantizers, an fp64 product of the
quantized operands).

Files (numpy .npz, no pickles) and manifest.json with their SHA-256:
  act_q8_0.npz       x fp32 [24,256] -> Q8_0 blocks, the x86 / NEON / _ref rounding variants
  act_q8_K.npz       x fp32 [12,512] -> Q8_K blocks (d, qs, bsums)
  dequant_<t>.npz    GGUF rows (quantized and random-byte blocks) -> fp32 (Q4_K: fused and not)
  weight_<t>.npz     fp32 rows -> GGUF rows by the _ref weight quantizers
  mulmat_<t>.npz     W [40 x 512] GGUF, X fp32 [20 x 512] -> Y fp32 (oracle) and Y fp64 (exact)

Usage: python tests/golden/make_golden.py   (rewrites the files and the manifest)
"""
import hashlib
import json
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(HERE))

import oracle_ffi as O  # noqa: E402

TYPES = {"q8_0": O.Q8_0, "q4_K": O.Q4_K, "q6_K": O.Q6_K, "f16": O.F16}


def crafted_rows(k):
    """Rows that separate rounding modes and hit the quantizers' special cases."""
    rows = [np.zeros(k, np.float32)]
    r = np.zeros(k, np.float32)
    r[:32] = np.array([127.0] + [i + 0.5 for i in range(-15, 16)], np.float32)  # x*id = j+0.5 exactly
    rows += [r, -r]
    r = np.full(k, 1e-6, np.float32); r[0] = -2e-6; rows.append(r)              # negative max
    rows.append(np.full(k, 3e-8, np.float32))                                    # fp16-subnormal scale
    r = np.random.default_rng(7).standard_normal(k).astype(np.float32)
    r[17], r[200 % k] = -9.0, 9.0                                                # |max| tie: first wins
    rows.append(r)
    rows.append((np.arange(k) % 256 - 127.0).astype(np.float32))
    rows.append(np.full(k, 1e-30, np.float32))                                   # scale underflows to 0
    return np.stack(rows)


def random_blocks(t, nblocks, rng):
    """Random block bytes with finite, moderate fp16 scales (other bytes arbitrary)."""
    b = rng.integers(0, 256, size=(nblocks, O.TSIZE[t]), dtype=np.uint8)
    def f16(vals):
        return np.asarray(vals, np.float16).view(np.uint8).reshape(nblocks, 2)
    if t == O.Q8_0:
        b[:, 0:2] = f16(rng.uniform(-0.01, 0.01, nblocks))
    elif t == O.Q4_K:
        b[:, 0:2] = f16(rng.uniform(0.0, 0.002, nblocks))
        b[:, 2:4] = f16(rng.uniform(0.0, 0.001, nblocks))
    elif t == O.Q6_K:
        b[:, 208:210] = f16(rng.uniform(-0.002, 0.002, nblocks))
    return b


def make(orc):
    out = {}
    rng = np.random.default_rng(20260601)

    x = np.concatenate([rng.standard_normal((16, 256)).astype(np.float32), crafted_rows(256)])
    out["act_q8_0.npz"] = dict(x=x, **{f"y_{v}": orc.quantize_act(O.Q8_0, x, i)
                                       for i, v in enumerate(["x86", "neon", "ref"])})

    x = np.concatenate([rng.standard_normal((4, 512)).astype(np.float32) * 3, crafted_rows(512)])
    out["act_q8_K.npz"] = dict(x=x, y=orc.quantize_act(O.Q4_K, x))

    for name, t in (("q8_0", O.Q8_0), ("q4_K", O.Q4_K), ("q6_K", O.Q6_K)):
        k = 512
        wf = (rng.standard_normal((6, k)) * 0.02).astype(np.float32)
        wq = orc.quantize_chunk(t, wf)
        nb = k // O.BLCK[t]
        rb = random_blocks(t, 6 * nb, rng).reshape(6, -1)
        w = np.concatenate([wq, rb])
        d = dict(w=w, k=np.int64(k), y=orc.dequantize(t, w, k, 0))
        if t == O.Q4_K:
            d["y_fused"] = orc.dequantize(t, w, k, 1)
        out[f"dequant_{name}.npz"] = d

        wf = np.concatenate([(rng.standard_normal((6, k)) * 0.02).astype(np.float32),
                             np.zeros((1, k), np.float32),
                             np.linspace(-1, 1, k, dtype=np.float32)[None]])
        out[f"weight_{name}.npz"] = dict(x=wf, w=orc.quantize_chunk(t, wf))

    for name, t in TYPES.items():
        n, k, m = 40, 512, 20
        wf = (rng.standard_normal((n, k)) * 0.02).astype(np.float32)
        w = orc.quantize_chunk(t, wf) if t != O.F16 else orc.fp32_to_fp16(wf).view(np.uint8).reshape(n, -1)
        x = rng.standard_normal((m, k)).astype(np.float32)
        xq = orc.quantize_act(t, x)
        out[f"mulmat_{name}.npz"] = dict(w=w, x=x, y=orc.mul_mat(t, w, x, nthreads=1),
                                         y_exact=orc.mul_mat_exact(t, w, xq, k))
    return out


def sha256(path):
    return hashlib.sha256(open(path, "rb").read()).hexdigest()


def main():
    orc = O.Oracle()
    files = make(orc)
    manifest = {}
    for fname, arrays in files.items():
        path = os.path.join(HERE, fname)
        np.savez_compressed(path, **arrays)
        manifest[fname] = sha256(path)
    with open(os.path.join(HERE, "manifest.json"), "w") as f:
        json.dump(manifest, f, indent=1, sort_keys=True)
        f.write("\n")
    total = sum(os.path.getsize(os.path.join(HERE, f)) for f in files)
    print(f"wrote {len(files)} fixtures, {total / 1024:.0f} KiB")


if __name__ == "__main__":
    main()
