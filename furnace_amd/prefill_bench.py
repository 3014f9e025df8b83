"""Prefill throughput of the engine on a synthetic model: one prompt of
`--prompt` random ids through frn_prefill (blocks of rows through the MFMA
GEMMs and the MFMA attention), timed after a warm-up prefill, `--reps`
times.  Prints one line per timed prefill.

    python3 -m furnace_amd.prefill_bench --model qwen2-7b-q4_k_m --prompt 2048
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


def main():
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--model", default="qwen2-7b-q4_k_m", choices=sorted(fa.PRESETS))
    ap.add_argument("--prompt", type=int, default=2048)
    ap.add_argument("--reps", type=int, default=3)
    ap.add_argument("--seed", type=int, default=0xF0E5)
    args = ap.parse_args()
    tmp = tempfile.mkdtemp(prefix="frn_pf_")
    path = os.path.join(tmp, args.model + ".gguf")
    fa.synth_write(path, seed=args.seed, threads=min(16, os.cpu_count() or 1), **fa.PRESETS[args.model])
    prompt = np.random.default_rng(args.seed).integers(0, 151643, args.prompt).astype(np.uint32)
    m = fa.Model(path, max_ctx=args.prompt + 8)
    hip = fa.Hip()
    m.prefill(prompt)
    m.reset()
    hip.sync()
    for _ in range(args.reps):
        t0 = time.perf_counter()
        tok = m.prefill(prompt)
        hip.sync()
        dt = time.perf_counter() - t0
        print("prefill %s, %d tokens: %.1f ms, %.0f tokens/s, first id %d" %
              (args.model, args.prompt, dt * 1e3, args.prompt / dt, tok), flush=True)
        m.reset()
    m.close()
    os.remove(path)
    os.rmdir(tmp)


if __name__ == "__main__":
    main()
