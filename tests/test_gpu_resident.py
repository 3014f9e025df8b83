"""The resident decode kernel (the whole greedy loop in one persistent launch,
include/furnace_hip.h frn_decode_engine) against the oracle and against the
per-step graphs on the same seeded models: greedy ids identical, last
logits within 1e-3 max-abs, stop ids honoured as generate.rs:125-127 does,
and runs longer than one launch."""
import os

import numpy as np
import pytest

import furnace_amd as fa
from oracle import oracle as orc

pytestmark = pytest.mark.gpu

LOGIT_TOL = 1e-3

SPECS = {
    # Q4_K_M mix (v/down Q6_K on even layers), head_dim 64, some XCDs own no head
    "tiny-q4_k_m": dict(n_layers=3, n_heads=4, n_kv_heads=2, hidden=256, ffn=512, vocab=3000, mix=fa.MIX_Q4_K_M,
                        tied=1, embd_type=fa.Q6_K, output_type=fa.Q6_K),
    # 12 query heads over 2 kv heads, head_dim 128 (the 1.5B head shape), small FFN and vocab
    "tiny-hd128-gq6": dict(n_layers=2, n_heads=12, n_kv_heads=2, hidden=1536, ffn=1280, vocab=2048,
                           mix=fa.MIX_Q4_K_M, tied=1, embd_type=fa.Q6_K, output_type=fa.Q6_K),
    # all Q8_0, 14 heads over 2 kv heads (the 0.5B head shape)
    "tiny-q8_0-gq7": dict(n_layers=2, n_heads=14, n_kv_heads=2, hidden=896, ffn=640, vocab=1500,
                          mix=fa.MIX_ALL_Q8_0, tied=1, embd_type=fa.Q8_0, output_type=fa.Q8_0),
}


def _path(tmpdir_models, name):
    path = os.path.join(tmpdir_models, "res-" + name + ".gguf")
    if not os.path.exists(path):
        fa.synth_write(path, seed=41, **SPECS[name])
    return path


@pytest.mark.parametrize("name", list(SPECS))
def test_resident_matches_oracle_and_graphs(hip, tmpdir_models, name):
    path = _path(tmpdir_models, name)
    cfg = SPECS[name]
    prompt = np.random.default_rng(7).integers(0, cfg["vocab"], 13).astype(np.uint32)
    n = 40
    print("model %s" % name, flush=True)
    ref = orc.Model(path)
    ref_ids, _, ref_logits = ref.generate_greedy(prompt, n, 256, stop_ids=[])
    ref.close()
    runs = []
    for resident in (True, False):
        m = fa.Model(path, max_ctx=256, resident=resident)
        on, why = m.decode_engine()
        assert on == (1 if resident else 0), why
        ids, _ = m.generate_greedy(prompt, n, stop_ids=[])
        runs.append((ids, m.logits()))
        m.close()
    (rids, rlog), (gids, glog) = runs
    print("resident", rids[:16], flush=True)
    print("oracle  ", ref_ids[:16], flush=True)
    assert rids == ref_ids
    assert gids == ref_ids
    assert np.max(np.abs(rlog - ref_logits)) <= LOGIT_TOL
    assert np.max(np.abs(rlog - glog)) <= LOGIT_TOL


def test_resident_single_steps_and_stop_ids(hip, tmpdir_models):
    path = _path(tmpdir_models, "tiny-q4_k_m")
    prompt = np.random.default_rng(9).integers(0, 3000, 10).astype(np.uint32)
    m = fa.Model(path, max_ctx=256, resident=True)
    assert m.decode_engine()[0] == 1
    first = m.prefill(prompt)
    steps = []
    tok = first
    for _ in range(12):  # one resident launch per frn_decode
        tok = m.decode(tok)
        steps.append(tok)
    m.reset()
    assert m.prefill(prompt) == first
    batch = m.decode_greedy(first, 12)
    assert batch == steps
    assert m.cache_len() == prompt.size + 12
    # a stop id ends the loop after the step that produced it
    m.reset()
    m.prefill(prompt)
    k = 5
    stop = steps[k]
    got = m.decode_greedy(first, 12, stop_ids=[stop, 2999 if stop != 2999 else 2998])
    j = steps.index(stop)
    assert got == steps[:j + 1]
    assert m.cache_len() == prompt.size + j + 1
    # decoding continues from there as the step loop would
    assert m.decode_greedy(got[-1], 3) == steps[j + 1:j + 4]
    m.close()


def test_resident_runs_across_launches(hip, tmpdir_models):
    """More steps than one launch runs (128), compared with the graphs."""
    path = _path(tmpdir_models, "tiny-q4_k_m")
    prompt = np.random.default_rng(11).integers(0, 3000, 8).astype(np.uint32)
    outs = []
    for resident in (True, False):
        m = fa.Model(path, max_ctx=512, resident=resident)
        first = m.prefill(prompt)
        ids = m.decode_greedy(first, 300)
        outs.append((ids, m.logits(), m.cache_len()))
        m.close()
    assert outs[0][0] == outs[1][0]
    assert outs[0][2] == outs[1][2] == prompt.size + 300
    assert np.max(np.abs(outs[0][1] - outs[1][1])) <= LOGIT_TOL


def test_resident_refuses_unsupported_formats(hip, tmpdir_models):
    path = os.path.join(tmpdir_models, "res-q5.gguf")
    fa.synth_write(path, seed=3, n_layers=2, n_heads=2, n_kv_heads=2, hidden=256, ffn=512, vocab=1000,
                   mix=fa.MIX_ALL_Q5_0, tied=0, embd_type=fa.Q5_0, output_type=fa.Q8_0)
    m = fa.Model(path, max_ctx=64, resident=True)
    on, why = m.decode_engine()
    assert on == 0 and "format" in why
    m.close()
