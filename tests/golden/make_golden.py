#!/usr/bin/env python3
"""Writes the golden fixtures in this directory from the oracle (the plain-C
restatement of furnace's CPU path under oracle/), on seeded synthetic inputs:

  dequant.npz   per format: raw bytes of 4 seeded blocks -> f32 values
                (quant.rs:17-133 dequantizers)
  gemv.npz      per decode GEMV shape, the first 16 weight rows: raw rows,
                x ~ N(0, 1), oracle y = matmul_quant (quant.rs:170-258)
  tiny.npz      a 2-layer Q4_K_M model (synthetic GGUF from its spec and
                seed; its SHA-256 pins the writer): prompt, last-position
                logits after the prompt (first 4096 and the top 8), and 32
                greedy ids
                (model.rs:579-600, generate.rs:69-157)
  qwen2-0.5b-q8_0.npz   the same for the Qwen2-0.5B-shape Q8_0 model:
                16-token prompt, 32 greedy ids, last logits after the prompt

The oracle itself is pinned by the reference's own known-answer tests and
closed forms (tests/test_oracle_*.py); these files freeze its outputs so the
HIP path and any later oracle change are compared against the same numbers.
Usage: python3 tests/golden/make_golden.py  (a few minutes on 8 cores)."""
import hashlib
import os
import sys
import tempfile

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)

import furnace_amd as fa  # noqa: E402  (synthetic encoders and GGUF writer only)
from oracle import oracle as orc  # noqa: E402

FORMATS = {"q8_0": fa.Q8_0, "q5_0": fa.Q5_0, "q4_k": fa.Q4_K, "q6_k": fa.Q6_K}
GEMV_SHAPES = [("q4_k", 8960, 1536), ("q4_k", 1536, 8960), ("q6_k", 1536, 8960), ("q8_0", 1536, 1536),
               ("q6_k", 151936, 1536), ("q8_0", 4864, 896), ("q8_0", 896, 4864)]
GEMV_ROWS = 16
TINY = dict(n_layers=2, n_heads=4, n_kv_heads=2, hidden=256, ffn=512, vocab=1000, mix=fa.MIX_Q4_K_M, tied=1,
            embd_type=fa.Q6_K, output_type=fa.Q6_K)
TINY_SEED, Q8_05B_SEED = 23, 0xF0E1 + 1


def sha256(path):
    h = hashlib.sha256()
    with open(path, "rb") as f:
        for chunk in iter(lambda: f.read(1 << 24), b""):
            h.update(chunk)
    return h.hexdigest()


def dequant():
    out = {}
    for name, t in FORMATS.items():
        be, bb = fa.BLOCK[t]
        x = fa.gaussian(100 + t, 0.5, 4 * be)
        raw = fa.quantize(t, x)
        out[name + "_raw"] = raw
        out[name + "_y"] = orc.dequantize(t, raw, 4 * be)
    np.savez_compressed(os.path.join(HERE, "dequant.npz"), **out)


def gemv():
    out = {}
    for i, (name, d_out, d_in) in enumerate(GEMV_SHAPES):
        t = FORMATS[name]
        be, bb = fa.BLOCK[t]
        raw = fa.quantize(t, fa.gaussian(200 + i, 0.02, GEMV_ROWS * d_in))
        x = fa.gaussian(300 + i, 1.0, d_in)
        y = orc.matmul_quant(x.reshape(1, d_in), raw, GEMV_ROWS, d_in, t).ravel()
        key = "%s_%dx%d" % (name, d_out, d_in)
        out[key + "_raw"], out[key + "_x"], out[key + "_y"] = raw, x, y
    np.savez_compressed(os.path.join(HERE, "gemv.npz"), **out)


def model_fixture(fname, spec, seed, prompt_len, max_ctx):
    tmp = tempfile.mkdtemp(prefix="frn_golden_")
    path = os.path.join(tmp, "m.gguf")
    fa.synth_write(path, seed=seed, threads=min(8, os.cpu_count() or 1), **spec)
    rng = np.random.default_rng(seed)
    prompt = rng.integers(0, min(spec["vocab"], 151643), prompt_len).astype(np.uint32)
    m = orc.Model(path)
    m.new_cache(max_ctx)
    logits = m.forward_cached(prompt)
    m.close()
    m = orc.Model(path)
    ids, _, _ = m.generate_greedy(prompt, 32, max_ctx, stop_ids=[])
    m.close()
    top = np.argsort(-logits, kind="stable")[:8]
    np.savez_compressed(os.path.join(HERE, fname), seed=np.int64(seed), prompt=prompt, logits=logits[:4096],
                        top_ids=top.astype(np.uint32), top_logits=logits[top],
                        ids=np.asarray(ids, dtype=np.uint32), gguf_sha256=np.array(sha256(path)),
                        spec_keys=np.array(sorted(spec)), spec_vals=np.array([spec[k] for k in sorted(spec)]))
    os.remove(path)
    os.rmdir(tmp)


def main():
    orc.set_threads(os.cpu_count() or 1)
    dequant()
    gemv()
    model_fixture("tiny.npz", TINY, TINY_SEED, 12, 64)
    model_fixture("qwen2-0.5b-q8_0.npz", fa.PRESETS["qwen2-0.5b-q8_0"], Q8_05B_SEED, 16, 64)


if __name__ == "__main__":
    main()
