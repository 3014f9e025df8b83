"""The furnace-hip CLI's `run` against furnace's `run` output
(src/generate.rs:98-155, src/perf.rs:69-96): the generated ids equal the
oracle's loop, one `[decode N: seq M, X ms/token]` line per decode forward,
and with --timings the decode-only op breakdown with its "unaccounted" row.
At temperature 0 a repeat penalty still applies (sampler.rs:86-108: the
argmax of the penalized logits)."""
import os
import re
import subprocess

import numpy as np
import pytest

import furnace_amd as fa
from oracle import oracle as orc

pytestmark = pytest.mark.gpu

CLI = os.path.join(os.path.dirname(fa.LIB_PATH), "..", "bin", "furnace-hip")
SPEC = dict(n_layers=2, n_heads=4, n_kv_heads=2, hidden=256, ffn=512, vocab=3000, mix=fa.MIX_Q4_K_M, tied=1,
            embd_type=fa.Q6_K, output_type=fa.Q6_K)
STEP_RE = re.compile(r"^\[decode +(\d+): seq +(\d+), +([0-9.]+) ms/token\]$")
ROW_RE = re.compile(r"^  (\S+) +([-0-9.]+) ms +([-0-9.]+)%(?: +(\d+) calls)?$")


def _model(tmpdir_models):
    path = os.path.join(tmpdir_models, "cli-tiny.gguf")
    if not os.path.exists(path):
        fa.synth_write(path, seed=23, **SPEC)
    return path


def _run(path, prompt, n, *extra):
    cmd = [CLI, "run", path, "--prompt-ids", ",".join(str(int(i)) for i in prompt), "-n", str(n)] + list(extra)
    print(" ".join(cmd[:2] + cmd[3:4] + ["..."] + cmd[5:]), flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stderr
    lines = r.stderr.splitlines()
    ids_line = [l for l in lines if l.startswith("generated ids: [")]
    assert len(ids_line) == 1, r.stderr
    body = ids_line[0][len("generated ids: ["):-1]
    ids = [int(x) for x in body.split(",")] if body.strip() else []
    return ids, lines


def _oracle_loop(path, prompt, n, temp, top_k, top_p, penalty, seed):
    """generate.rs:110-136 with the oracle's forward and Sampler."""
    ref = orc.Model(path)
    ref.new_cache(len(prompt) + n + 1)
    logits = ref.forward_cached(prompt)
    s = orc.Sampler(temp, top_k, top_p, penalty, seed=seed)
    stop = set(ref.stop_ids())
    ctx, out = [int(i) for i in prompt], []
    for step in range(n):
        w = max(0, len(ctx) - 64)
        nxt = s.sample(logits, np.array(ctx[w:], np.uint32))
        if nxt in stop:
            break
        out.append(nxt)
        ctx.append(nxt)
        if step + 1 == n:
            break
        logits = ref.forward_cached([nxt])
    ref.close()
    return out


def test_run_greedy_step_lines_and_timings(hip, tmpdir_models):
    path = _model(tmpdir_models)
    prompt = np.random.default_rng(3).integers(0, SPEC["vocab"], 11).astype(np.uint32)
    n = 12
    ids, lines = _run(path, prompt, n, "--temp", "0", "--timings")
    assert ids == _oracle_loop(path, prompt, n, 0.0, 40, 0.9, 1.0, 1)
    steps = [STEP_RE.match(l) for l in lines if l.startswith("[decode")]
    assert all(steps) and len(steps) == n - 1
    for k, m in enumerate(steps):
        assert int(m.group(1)) == k and int(m.group(2)) == prompt.size + k + 1 and float(m.group(3)) > 0
    head = [i for i, l in enumerate(lines) if l.startswith("decode op breakdown (")]
    assert len(head) == 1
    wall = float(re.match(r"decode op breakdown \(([0-9.]+) ms wall\):", lines[head[0]]).group(1))
    rows = {}
    for l in lines[head[0] + 1:]:
        m = ROW_RE.match(l)
        if not m:
            break
        rows[m.group(1)] = (float(m.group(2)), m.group(4))
    assert "unaccounted" in rows and rows["unaccounted"][1] is None
    # the counters were reset after the prefill: per-layer kernels ran once
    # per layer per decode forward, the per-step kernels once per forward
    for name in ("qkv", "attention", "o_proj", "gate_up", "down"):
        assert int(rows[name][1]) == (n - 1) * SPEC["n_layers"], (name, rows[name])
    for name in ("embed", "lm_head"):
        assert int(rows[name][1]) == n - 1, (name, rows[name])
    accounted = sum(ms for k, (ms, calls) in rows.items() if k != "unaccounted")
    assert 0 < accounted <= wall
    assert abs(wall - accounted - rows["unaccounted"][0]) < 0.01


def test_run_without_timings_prints_no_breakdown(hip, tmpdir_models):
    path = _model(tmpdir_models)
    prompt = np.random.default_rng(4).integers(0, SPEC["vocab"], 6).astype(np.uint32)
    ids, lines = _run(path, prompt, 5, "--temp", "0")
    assert ids == _oracle_loop(path, prompt, 5, 0.0, 40, 0.9, 1.0, 1)
    assert sum(1 for l in lines if STEP_RE.match(l)) == 4
    assert not any(l.startswith("decode op breakdown") for l in lines)


def test_run_temperature_zero_keeps_the_repeat_penalty(hip, tmpdir_models):
    path = _model(tmpdir_models)
    prompt = np.random.default_rng(5).integers(0, SPEC["vocab"], 9).astype(np.uint32)
    n = 16
    ids, lines = _run(path, prompt, n, "--temp", "0", "--repeat-penalty", "1.3", "--seed", "9")
    want = _oracle_loop(path, prompt, n, 0.0, 40, 0.9, 1.3, 9)
    assert ids == want
    # the penalty matters here: plain greedy decoding differs
    assert want != _oracle_loop(path, prompt, n, 0.0, 40, 0.9, 1.0, 9)
    assert sum(1 for l in lines if STEP_RE.match(l)) == n - 1
