"""The committed golden fixtures (tests/golden/, written by make_golden.py
from the oracle) against the oracle (CPU) and the HIP path through the C ABI
(GPU): dequantization bit-exact, GEMV rows within 1e-4 relative, the tiny
Q4_K_M model's and the Qwen2-0.5B-shape Q8_0 model's last-position logits
within 1e-3 max-abs and their 32 greedy ids identical."""
import hashlib
import os

import numpy as np
import pytest

import furnace_amd as fa
from oracle import oracle as orc

HERE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
FORMATS = {"q8_0": fa.Q8_0, "q5_0": fa.Q5_0, "q4_k": fa.Q4_K, "q6_k": fa.Q6_K}
GEMV_TOL, LOGIT_TOL = 1e-4, 1e-3


def fixture(name):
    return np.load(os.path.join(HERE, name))  # allow_pickle stays False


def gemv_cases():
    g = fixture("gemv.npz")
    return sorted({k.rsplit("_", 1)[0] for k in g.files})


def rel_err(got, ref):
    ref64 = ref.astype(np.float64)
    scale = np.maximum(np.abs(ref64), np.sqrt(np.mean(ref64 ** 2)))
    return float(np.max(np.abs(got.astype(np.float64) - ref64) / scale))


def model_spec(f):
    return {str(k): int(v) for k, v in zip(f["spec_keys"], f["spec_vals"])}


def write_model(f, path):
    fa.synth_write(path, seed=int(f["seed"]), threads=min(8, os.cpu_count() or 1), **model_spec(f))
    h = hashlib.sha256()
    with open(path, "rb") as fh:
        for chunk in iter(lambda: fh.read(1 << 24), b""):
            h.update(chunk)
    assert h.hexdigest() == str(f["gguf_sha256"]), "synthetic GGUF writer output changed"


# ---- oracle (CPU) --------------------------------------------------------------
@pytest.mark.parametrize("name", list(FORMATS))
def test_oracle_dequant_matches_golden(name):
    f = fixture("dequant.npz")
    raw, want = f[name + "_raw"], f[name + "_y"]
    got = orc.dequantize(FORMATS[name], raw, want.size)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("key", gemv_cases())
def test_oracle_gemv_matches_golden(key):
    f = fixture("gemv.npz")
    name, shape = key.rsplit("_", 1)
    d_in = int(shape.split("x")[1])
    raw, x, want = f[key + "_raw"], f[key + "_x"], f[key + "_y"]
    got = orc.matmul_quant(x.reshape(1, d_in), raw, want.size, d_in, FORMATS[name]).ravel()
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("fname", ["tiny.npz", "qwen2-0.5b-q8_0.npz"])
def test_oracle_model_matches_golden(tmp_path, fname):
    f = fixture(fname)
    path = str(tmp_path / "m.gguf")
    write_model(f, path)
    orc.set_threads(os.cpu_count() or 1)
    m = orc.Model(path)
    m.new_cache(64)
    logits = m.forward_cached(f["prompt"])
    m.close()
    assert np.array_equal(logits[:4096].view(np.uint32), f["logits"].view(np.uint32))
    m = orc.Model(path)
    ids, _, _ = m.generate_greedy(f["prompt"], 32, 64, stop_ids=[])
    m.close()
    assert ids == f["ids"].tolist()


# ---- HIP path (GPU) --------------------------------------------------------------
@pytest.mark.gpu
@pytest.mark.parametrize("name", list(FORMATS))
def test_gpu_dequant_matches_golden(hip, name):
    f = fixture("dequant.npz")
    raw, want = f[name + "_raw"], f[name + "_y"]
    print("golden dequant %s" % name, flush=True)
    d_raw, d_out = hip.to_device(raw), hip.malloc(want.size * 4)
    fa.dequant_dev(hip, FORMATS[name], d_raw, raw.size, want.size, d_out)
    got = hip.from_device(d_out, want.size, np.float32)
    hip.free(d_raw)
    hip.free(d_out)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


@pytest.mark.gpu
@pytest.mark.parametrize("key", gemv_cases())
def test_gpu_gemv_matches_golden(hip, key):
    f = fixture("gemv.npz")
    name, shape = key.rsplit("_", 1)
    d_in = int(shape.split("x")[1])
    raw, x, want = f[key + "_raw"], f[key + "_x"], f[key + "_y"]
    print("golden gemv %s" % key, flush=True)
    d_w, d_x, d_y = hip.to_device(raw), hip.to_device(x), hip.malloc(want.size * 4)
    fa.matmul_quant_dev(FORMATS[name], d_w, raw.size, d_x, 1, d_y, want.size, d_in)
    got = hip.from_device(d_y, want.size, np.float32)
    for p in (d_w, d_x, d_y):
        hip.free(p)
    assert rel_err(got, want) <= GEMV_TOL


@pytest.mark.gpu
@pytest.mark.parametrize("fname", ["tiny.npz", "qwen2-0.5b-q8_0.npz"])
def test_gpu_model_matches_golden(hip, tmp_path, fname):
    f = fixture(fname)
    path = str(tmp_path / "m.gguf")
    print("golden model %s" % fname, flush=True)
    write_model(f, path)
    m = fa.Model(path, max_ctx=64)
    nxt = m.prefill(f["prompt"])
    logits = m.logits()
    assert np.max(np.abs(logits[:4096] - f["logits"])) <= LOGIT_TOL
    assert np.array_equal(np.argsort(-logits, kind="stable")[:1], f["top_ids"][:1])
    assert np.max(np.abs(logits[f["top_ids"]] - f["top_logits"])) <= LOGIT_TOL
    ids = [nxt]
    while len(ids) < 32:
        ids.append(m.decode(ids[-1]))
    m.close()
    assert ids == f["ids"].tolist()
