#!/usr/bin/env python3
"""Decode throughput of the MI355X token loop on the Qwen2-1.5B-shaped Q4_K_M
synthetic model (128-token random prompt, greedy decode), plus the fraction
of the 8 TB/s HBM roofline it reaches.

One step = one decode forward (embedding, 28 layers, lm_head, argmax) for one
token, with the weights already resident in HBM.  Prints one JSON line.
"""
import argparse
import ctypes
import json
import os
import subprocess
import sys
import tempfile
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

import numpy as np  # noqa: E402

import furnace_amd as fa  # noqa: E402

HBM_PEAK_GBS = 8000.0
METRIC = "decode tokens/s + % of HBM peak (Qwen2-1.5B-shape Q4_K_M, 1 GPU)"


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def tensor_bytes(gguf, name):
    t, nd, p, b = ctypes.c_uint32(), ctypes.c_uint32(), ctypes.c_void_p(), ctypes.c_size_t()
    dims = (ctypes.c_uint64 * 4)()
    fa.check(fa.load().frn_gguf_tensor(gguf, name.encode(), ctypes.byref(t), dims, ctypes.byref(nd),
                                       ctypes.byref(p), ctypes.byref(b)))
    return b.value, t.value


def algorithmic_bytes(model):
    """Bytes one decode step must move at minimum: every weight once
    (quantized size), norms and biases, one embedding row, the lm_head, and
    per attended position 2 * L * kv_dim * 4 bytes of f32 KV cache."""
    c = model.cfg
    g = model.gguf
    w = 0
    per = {}
    for l in range(c.n_layers):
        for n in ("attn_q.weight", "attn_k.weight", "attn_v.weight", "attn_output.weight", "ffn_gate.weight",
                  "ffn_up.weight", "ffn_down.weight", "attn_norm.weight", "ffn_norm.weight", "attn_q.bias",
                  "attn_k.bias", "attn_v.bias"):
            b, _ = tensor_bytes(g, "blk.%d.%s" % (l, n))
            w += b
            per.setdefault(n, []).append(b)
    eb, et = tensor_bytes(g, "token_embd.weight")
    w += eb // c.vocab  # one row
    w += tensor_bytes(g, "output_norm.weight")[0]
    lm = tensor_bytes(g, "output.weight")[0] if not c.tied_lm_head else eb
    w += lm
    kv_per_pos = 2 * c.n_layers * c.n_kv_heads * c.head_dim * 4
    return w, kv_per_pos, per, lm


def host_cpu():
    """(logical cores this process may use, CPU model name)."""
    n = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else (os.cpu_count() or 1)
    model = "unknown"
    try:
        out = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10).stdout
        for line in out.splitlines():
            if line.lower().startswith("model name"):
                model = line.split(":", 1)[1].strip()
                break
    except (OSError, ValueError, subprocess.SubprocessError):
        pass
    if model == "unknown" and os.path.exists("/proc/cpuinfo"):
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.lower().startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    return n, model


def cpu_baseline(path, prompt, budget_s, threads):
    """The oracle (plain-C restatement of furnace's CPU path) on the host
    cores, as generate.rs:109-141 runs it: the whole prompt as one prefill
    forward (timed), then greedy decode steps until about budget_s of decode
    work.  threads: the worker count (all logical cores unless
    RAYON_NUM_THREADS says otherwise, as main.rs:167-176 chooses)."""
    from oracle import oracle as orc
    orc.set_threads(threads)
    m = orc.Model(path)
    m.new_cache(len(prompt) + 300)
    t0 = time.perf_counter()
    logits = m.forward_cached(prompt)
    prefill_s = time.perf_counter() - t0
    tok = orc.argmax(logits)
    steps, dec = 0, 0.0
    while dec < budget_s and steps < 256:
        t1 = time.perf_counter()
        logits = m.forward_cached([tok])
        dec += time.perf_counter() - t1
        tok = orc.argmax(logits)
        steps += 1
    m.close()
    return steps / dec, steps, dec, prefill_s


GEMV_SHAPES = [("Q4_K", fa.Q4_K, 8960, 1536), ("Q4_K", fa.Q4_K, 1536, 8960), ("Q6_K", fa.Q6_K, 1536, 8960),
               ("Q8_0", fa.Q8_0, 1536, 1536), ("Q6_K", fa.Q6_K, 151936, 1536)]


def gemv_microbench(seed, reps=200):
    """frn_matmul_quant at batch 1 on each shape: weights N(0, 0.02) quantized
    by the synthetic-model encoders, x ~ N(0, 1).  The timed launches rotate
    over copies of the weights totalling >= 512 MB, so they stream from HBM
    rather than the 256 MB last-level cache.  Bytes = weights + x + y."""
    hip = fa.Hip()
    ev0, ev1 = hip.event(), hip.event()
    for name, t, out, inn in GEMV_SHAPES:
        w = fa.quantize(t, fa.gaussian(seed + out, 0.02, out * inn))
        copies = max(1, min(64, -(-(512 << 20) // w.nbytes)))
        wd = [hip.to_device(w) for _ in range(copies)]
        xd = hip.to_device(fa.gaussian(seed + 1, 1.0, inn))
        yd = hip.malloc(out * 4)
        fa.matmul_quant_dev(t, wd[0], w.nbytes, xd, 1, yd, out, inn)
        best = 1e30
        for _ in range(3):
            hip.record(ev0)
            for i in range(reps):
                fa.matmul_quant_dev(t, wd[i % copies], w.nbytes, xd, 1, yd, out, inn)
            hip.record(ev1)
            best = min(best, hip.elapsed_ms(ev0, ev1) * 1e3 / reps)
        nbytes = w.nbytes + 4 * (inn + out)
        gbs = nbytes / best * 1e-3
        log("gemv %s [%d, %d]: %.2f us/launch, %.1f GB/s (%.1f%% of HBM peak), %d weight copies" %
            (name, out, inn, best, gbs, 100 * gbs / HBM_PEAK_GBS, copies))
        print(json.dumps({"metric": "fused dequant-GEMV bandwidth", "shape": "%s [%d, %d]" % (name, out, inn),
                          "us_per_launch": round(best, 3), "bytes": nbytes, "value": round(gbs, 1),
                          "unit": "GB/s", "hbm_frac": round(gbs / HBM_PEAK_GBS, 4), "batch": 1,
                          "data": "synthetic N(0,0.02) weights, N(0,1) x"}), flush=True)
        for p in wd + [xd, yd]:
            hip.free(p)


def main():
    ap = argparse.ArgumentParser(description=__doc__)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=255, help="timed decode steps (256-token decode = 255 forwards)")
    ap.add_argument("--warmup", type=int, default=16)
    ap.add_argument("--model", default="qwen2-1.5b-q4_k_m", choices=sorted(fa.PRESETS))
    ap.add_argument("--prompt", type=int, default=128)
    ap.add_argument("--seed", type=int, default=0xF0E1)
    ap.add_argument("--timing-steps", type=int, default=32, help="eager steps with per-kernel events")
    ap.add_argument("--cpu-seconds", type=float, default=10.0, help="decode seconds of the CPU baseline")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--gguf", default=None, help="use this GGUF instead of writing the synthetic one")
    ap.add_argument("--eager", action="store_true", help="launch kernels one by one (for profilers) instead of "
                    "replaying the captured decode graph")
    ap.add_argument("--engine", choices=["auto", "graphs", "resident"], default="auto",
                    help="decode engine: the per-step graphs, the resident decode kernel, or the engine's choice")
    ap.add_argument("--copy-probe", type=int, default=0, metavar="BYTES",
                    help="only run a plain device-to-device copy of BYTES, 5 times (calibrates the HBM byte "
                         "counters of rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE against a known size), then exit")
    ap.add_argument("--gemv", action="store_true",
                    help="instead of the decode loop, run the single-op fused dequant-GEMV microbench (batch 1, "
                         "the five weight shapes of the decode step) and print one JSON line per shape")
    ap.add_argument("--traffic", default=os.path.join(ROOT, "profiles", "traffic.json"),
                    help="measured HBM bytes per launch (from rocprofv3 --pmc runs) to report as roofline.traffic")
    args = ap.parse_args()
    if args.gemv:
        gemv_microbench(args.seed)
        return
    if args.copy_probe:
        import torch
        src = torch.empty(args.copy_probe // 4, dtype=torch.float32, device="cuda").fill_(1.0)
        dst = torch.empty_like(src)
        for _ in range(5):
            dst.copy_(src)
        torch.cuda.synchronize()
        log("copied %d bytes 5 times" % args.copy_probe)
        return
    if args.gpus != 1:
        print("bench.py: this engine runs on one GPU; --gpus %d is not supported (sharding is design-only)" %
              args.gpus, file=sys.stderr)
        sys.exit(2)

    tmp = tempfile.mkdtemp(prefix="frn_bench_")
    path = args.gguf or os.path.join(tmp, args.model + ".gguf")
    if not args.gguf:
        t0 = time.perf_counter()
        fa.synth_write(path, seed=args.seed, threads=min(16, os.cpu_count() or 1), **fa.PRESETS[args.model])
        log("synthetic %s written in %.1f s" % (args.model, time.perf_counter() - t0))
    rng = np.random.default_rng(args.seed)
    prompt = rng.integers(0, 151643, args.prompt).astype(np.uint32)
    max_ctx = args.prompt + args.steps + args.timing_steps + max(args.warmup, 8) + 2

    t0 = time.perf_counter()
    model = fa.Model(path, max_ctx=max_ctx, eager=args.eager,
                     resident={"auto": None, "graphs": False, "resident": True}[args.engine])
    engine_on, engine_why = model.decode_engine()
    log("decode engine: %s%s" % ("resident kernel" if engine_on else "step graphs",
                                  "" if engine_on else " (%s)" % engine_why))
    log("weights uploaded in %.2f s" % (time.perf_counter() - t0))
    w_bytes, kv_per_pos, per, lm_bytes = algorithmic_bytes(model)
    hip = fa.Hip()

    # warm-up: compile caches, first graph launches
    tok = model.prefill(prompt[:8])
    for _ in range(args.warmup):
        tok = model.decode(tok)
    model.reset()

    # prefill of the whole prompt, then the timed decode steps
    hip.sync()
    t0 = time.perf_counter()
    tok = model.prefill(prompt)
    hip.sync()
    prefill_s = time.perf_counter() - t0
    # the timed steps: frn_decode_greedy, the argmax fed back on the device
    # and one host synchronisation per batch of steps
    hip.sync()
    t0 = time.perf_counter()
    ids = model.decode_greedy(tok, args.steps)
    hip.sync()
    dec_s = time.perf_counter() - t0
    assert len(ids) == args.steps
    tok = ids[-1]
    ms_per_step = dec_s * 1000.0 / args.steps
    # positions attended by the timed steps: prompt+1 .. prompt+steps
    avg_attended = args.prompt + (args.steps + 1) / 2.0
    step_bytes = w_bytes + kv_per_pos * avg_attended
    step_gbs = step_bytes / (ms_per_step * 1e-3) / 1e9
    log("decode: %d steps, %.4f ms/token, %.1f tokens/s, %.1f GB/s (%.1f%% of HBM peak)" %
        (args.steps, ms_per_step, 1000 / ms_per_step, step_gbs, 100 * step_gbs / HBM_PEAK_GBS))
    log("prefill: %d tokens in %.3f s (%.1f tokens/s)" % (args.prompt, prefill_s, args.prompt / prefill_s))
    # the same steps through the one-step call (a host round trip per id)
    model.reset()
    tok = model.prefill(prompt)
    hip.sync()
    t0 = time.perf_counter()
    loop_ids = []
    for _ in range(args.steps):
        tok = model.decode(tok)
        loop_ids.append(tok)
    hip.sync()
    loop_ms = (time.perf_counter() - t0) * 1000.0 / args.steps
    assert loop_ids == ids, "frn_decode loop and frn_decode_greedy disagree"
    log("decode, one frn_decode call per step: %.4f ms/token (%.1f tokens/s); same ids" % (loop_ms, 1000 / loop_ms))

    # live per-kernel durations (HIP events around each kernel, eager steps)
    model.timings_reset()
    model.timings_enable(True)
    for _ in range(args.timing_steps):
        tok = model.decode(tok)
    model.timings_enable(False)
    tm = model.timings()
    c = model.cfg
    log("per-kernel (eager, %d steps):" % args.timing_steps)
    for k, (ms, calls) in tm.items():
        if calls:
            log("  %-10s %9.3f ms  %6d calls  %8.2f us/call" % (k, ms, calls, 1000 * ms / calls))
    # per-kernel algorithmic bytes and replayed launch durations.  Each
    # category is replayed over every layer in turn (the weights then stream
    # from HBM, as in a decode step), so the mean per launch carries no
    # per-launch event overhead; rocprofv3's kernel trace of the same run
    # gives the same means (profiles/).
    L = c.n_layers
    pos = model.cache_len()
    ns = pos // 64 + 1
    qd, kvd = c.n_heads * c.head_dim, c.n_kv_heads * c.head_dim
    part_b = ns * c.n_heads * (c.head_dim + 2) * 4
    avg = lambda names: sum(sum(per[n]) for n in names) / L
    kbytes = {
        "qkv": avg(["attn_q.weight", "attn_k.weight", "attn_v.weight", "attn_q.bias", "attn_k.bias", "attn_v.bias",
                    "attn_norm.weight"]) + 4 * (c.hidden + qd + 2 * kvd),
        "attention": 2 * (pos + 1) * kvd * 4 + 4 * (qd + 2 * kvd) + part_b,
        "o_proj": avg(["attn_output.weight"]) + part_b + 2 * 4 * c.hidden,
        "gate_up": avg(["ffn_gate.weight", "ffn_up.weight", "ffn_norm.weight"]) + 4 * (c.hidden + c.ffn),
        "down": avg(["ffn_down.weight"]) + 4 * (c.ffn + 2 * c.hidden),
        "lm_head": lm_bytes + 4 * (2 * c.hidden + c.vocab),
    }
    per_step = {"qkv": L, "attention": L, "o_proj": L, "gate_up": L, "down": L, "lm_head": 1}
    kern = {}
    for k in kbytes:
        us = model.bench_kernel(k, None, 2 if k == "lm_head" else 4)
        kern[k] = {"avg_us": round(us, 3), "bytes": int(kbytes[k]), "gbs": round(kbytes[k] / us * 1e-3, 1),
                   "us_per_step": round(us * per_step[k], 1)}
        log("  replay %-10s %8.2f us/launch  %8.1f GB/s  %7.1f us/step" %
            (k, us, kbytes[k] / us * 1e-3, us * per_step[k]))
    model.reset()
    dom = max(kern, key=lambda k: kern[k]["us_per_step"])
    dk = kern[dom]
    traffic = None
    if os.path.exists(args.traffic):
        with open(args.traffic) as f:
            tr = json.load(f).get("bytes_per_launch", {})
        traffic = tr.get("%s/%s" % (args.model, dom))

    cpu = None
    if not args.no_cpu:
        cores, cpu_model = host_cpu()
        env = os.environ.get("RAYON_NUM_THREADS", "")
        threads = int(env) if env.isdigit() and int(env) > 0 else cores
        tps, steps, dec, pf = cpu_baseline(path, prompt, args.cpu_seconds, threads)
        log("cpu baseline (%s, %d logical cores, %d threads): %d-token prefill %.2f s (%.1f tokens/s); "
            "decode %.2f tokens/s (%d steps in %.1f s)" %
            (cpu_model, cores, threads, len(prompt), pf, len(prompt) / pf, tps, steps, dec))
        cpu = {"value": round(tps, 3), "unit": "tokens/s", "cores": threads, "kind": "port",
               "prefill_tokens_per_s": round(len(prompt) / pf, 2), "nproc": cores, "cpu_model": cpu_model,
               "sample": "oracle (C restatement of furnace's CPU path) on the same %s GGUF: the %d-token prompt "
                         "as one prefill forward, then %d greedy decode steps (%.1f s of decode)"
                         % (args.model, len(prompt), steps, dec)}
    model.close()
    if not args.gguf:
        os.remove(path)
        os.rmdir(tmp)

    out = {
        "metric": METRIC, "value": round(1000.0 / ms_per_step, 2), "unit": "tokens/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms_per_step, 5),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "f32",
        "data": "synthetic (seeded N(0,0.02) weights, uniform random prompt ids)",
        "config": {"workload": "%s greedy decode after a %d-token prompt" % (args.model, args.prompt),
                   "weights": "Q4_K_M mix (Q4_K; Q6_K attn_v/ffn_down on even layers; Q6_K tied lm_head)"
                   if "q4_k_m" in args.model else "Q8_0", "prompt_tokens": args.prompt,
                   "decode_tokens": args.steps, "bytes_per_token": int(step_bytes),
                   "hbm_frac_per_token": round(step_gbs / HBM_PEAK_GBS, 4),
                   "prefill_tokens_per_s": round(args.prompt / prefill_s, 1),
                   "decode_api": "frn_decode_greedy (%s)" % ("resident decode kernel, 128 steps per launch"
                                                             if engine_on else "step graphs, 32 steps per host sync"),
                   "per_call_decode_tokens_per_s": round(1000.0 / loop_ms, 1)},
        "roofline": {"bound": "hbm", "kernel": dom, "achieved": dk["gbs"], "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(dk["gbs"] / HBM_PEAK_GBS, 4), "traffic": traffic,
                     "bytes_per_launch": dk["bytes"], "avg_us": dk["avg_us"]},
        "kernels": kern,
        "cpu_baseline": cpu,
    }
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
