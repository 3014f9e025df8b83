"""Phase timeline of the resident decode kernel (frn_resident_trace): every
block stamps a 100 MHz clock at the end of each phase of each layer for
the first steps of a launch; this prints, per phase, the median over the
traced steps and layers of the block median and block maximum since the
layer's start, the layer period and the lm_head/argmax tail.

    python3 -m furnace_amd.resident_trace --model qwen2-1.5b-q4_k_m --prompt 128
"""
import argparse
import os
import sys
import tempfile
import time

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

import furnace_amd as fa  # noqa: E402

# stamp slots of a layer (resident.hpp RES_TR_*), in phase order
PHASES = [(0, "layer start"), (12, "A: x arrived"), (1, "A: x staged"), (2, "A: q|k|v rows"), (3, "B: attention"),
          (15, "C: partials arrived"), (4, "C: merged"), (5, "C: o-proj partial"), (6, "D: x' rows (cross-XCD)"),
          (13, "E: x' arrived"), (7, "E: x' staged"), (8, "E: gate/up + SwiGLU"), (14, "F: act arrived"),
          (9, "F: act staged"), (10, "F: down partial"), (11, "G: x'' rows (cross-XCD)")]


def main():
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--model", default="qwen2-1.5b-q4_k_m", choices=sorted(fa.PRESETS))
    ap.add_argument("--prompt", type=int, default=128)
    ap.add_argument("--steps", type=int, default=4, help="traced decode steps (the first is not counted)")
    ap.add_argument("--seed", type=int, default=0xF0E1)
    args = ap.parse_args()
    tmp = tempfile.mkdtemp(prefix="frn_rt_")
    path = os.path.join(tmp, args.model + ".gguf")
    fa.synth_write(path, seed=args.seed, threads=min(16, os.cpu_count() or 1), **fa.PRESETS[args.model])
    prompt = np.random.default_rng(args.seed).integers(0, 151643, args.prompt).astype(np.uint32)
    m = fa.Model(path, max_ctx=args.prompt + 256 + args.steps, resident=True)
    on, why = m.decode_engine()
    if not on:
        raise SystemExit("the resident decode kernel does not serve this model here: " + why)
    tok = m.prefill(prompt)
    m.decode_greedy(tok, 32)
    m.reset()
    tok = m.prefill(prompt)
    t0 = time.perf_counter()
    ids = m.decode_greedy(tok, 128)
    dt = time.perf_counter() - t0
    print("resident decode: 128 steps, %.1f tokens/s" % (128 / dt))
    m.reset()
    tok = m.prefill(prompt)
    m.resident_trace(args.steps)
    m.decode_greedy(tok, args.steps)
    tr = m.resident_trace(args.steps, read=True).astype(np.int64)
    L = m.cfg.n_layers
    print("%-26s %10s %10s" % ("phase end", "median us", "max us"))
    for k, name in PHASES:
        med, mx = [], []
        for s in range(1, args.steps):
            for l in range(1, L):
                d = (tr[s, l, k] - tr[s, l, 0]) * 0.01
                med.append(np.median(d))
                mx.append(np.max(d))
        print("%-26s %10.2f %10.2f" % (name, np.median(med), np.median(mx)))
    per = [np.median(tr[s, l, 0] - tr[s, l - 1, 0]) * 0.01 for s in range(1, args.steps) for l in range(1, L)]
    print("layer period: %.2f us" % np.median(per))
    for k, name in [(1, "lm_head input staged"), (2, "lm_head rows"), (3, "argmax")]:
        d = [np.median(tr[s, L, k] - tr[s, L - 1, 0]) * 0.01 for s in range(1, args.steps)]
        print("%s: %.2f us after the last layer's start" % (name, np.median(d)))
    m.close()
    os.remove(path)
    os.rmdir(tmp)


if __name__ == "__main__":
    main()
