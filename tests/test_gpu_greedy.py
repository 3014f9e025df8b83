"""frn_decode_greedy (steps enqueued back to back, argmax fed back on the
device) gives the ids of the frn_decode loop, across several host
synchronisation batches, and a stop id ends the loop with the position
rolled back so that decoding continues exactly as the step loop would."""
import os

import numpy as np
import pytest

import furnace_amd as fa

pytestmark = pytest.mark.gpu

SPEC = dict(n_layers=3, n_heads=4, n_kv_heads=2, hidden=256, ffn=512, vocab=3000, mix=fa.MIX_Q4_K_M,
            tied=1, embd_type=fa.Q6_K, output_type=fa.Q6_K)
N_STEPS = 70  # three batches of the host synchronisation


def _model(tmpdir_models):
    path = os.path.join(tmpdir_models, "greedy.gguf")
    if not os.path.exists(path):
        fa.synth_write(path, seed=23, **SPEC)
    return fa.Model(path, max_ctx=256)


def _loop(m, prompt, n):
    tok = m.prefill(prompt)
    first = tok
    ids = []
    for _ in range(n):
        tok = m.decode(tok)
        ids.append(tok)
    return first, ids, m.logits()


def test_greedy_batches_match_the_step_loop(hip, tmpdir_models):
    prompt = np.random.default_rng(3).integers(0, SPEC["vocab"], 11).astype(np.uint32)
    m = _model(tmpdir_models)
    first, ref, ref_logits = _loop(m, prompt, N_STEPS)
    m.reset()
    print("greedy batches: %d steps" % N_STEPS, flush=True)
    assert m.prefill(prompt) == first
    got = m.decode_greedy(first, N_STEPS)
    assert got == ref
    assert m.cache_len() == prompt.size + N_STEPS
    assert np.array_equal(m.logits(), ref_logits)
    assert m.decode_greedy(got[-1], 0) == []
    m.close()


def test_greedy_stop_id_rolls_back(hip, tmpdir_models):
    m = _model(tmpdir_models)
    # a prompt whose greedy ids hold a stop candidate inside the first batch
    # (not at its end): an id that first occurs at step k >= 1
    for seed in range(4, 24):
        prompt = np.random.default_rng(seed).integers(0, SPEC["vocab"], 7).astype(np.uint32)
        first, ref, _ = _loop(m, prompt, 40)
        m.reset()
        ks = [i for i in range(1, 30) if ref[i] not in ref[:i] and ref[i] != first]
        if ks:
            k = ks[-1]
            break
    else:
        pytest.fail("no prompt with a fresh greedy id in steps 1..29")
    print("greedy stop at step %d (id %d)" % (k, ref[k]), flush=True)
    assert m.prefill(prompt) == first
    got = m.decode_greedy(first, 40, stop_ids=[ref[k], SPEC["vocab"] + 5])
    assert got == ref[:k + 1]
    assert m.cache_len() == prompt.size + k + 1
    with pytest.raises(fa.FrnError):
        m.logits()  # the batch ran past the stop id: its logits are not the stop step's
    # decoding on from the stop id repeats the step loop's continuation
    tok = ref[k]
    for i in range(k + 1, 40):
        tok = m.decode(tok)
        assert tok == ref[i], i
    m.close()


def test_exact_split_graphs_across_split_boundaries(hip, tmpdir_models):
    """Below 1024 positions each decode step replays the graph whose
    attention grid is exactly its 64-position splits (four-step graphs only
    where the four steps share the count).  150 steps from a 50-token prompt
    cross the 64 and 128 boundaries at every offset of the four-step
    groups; the ids and logits equal the eager steps' (one grid of all
    splits) and the oracle's (model.rs:371-438)."""
    from oracle import oracle as orc
    path = os.path.join(tmpdir_models, "greedy.gguf")
    if not os.path.exists(path):
        fa.synth_write(path, seed=23, **SPEC)
    prompt = np.random.default_rng(17).integers(0, SPEC["vocab"], 50).astype(np.uint32)
    n = 150
    ref = orc.Model(path)
    ref_ids, _, ref_logits = ref.generate_greedy(prompt, n + 1, 256, stop_ids=[])
    ref.close()
    runs = []
    for eager in (False, True):
        m = fa.Model(path, max_ctx=256, eager=eager)
        first = m.prefill(prompt)
        ids = [first] + m.decode_greedy(first, n)
        runs.append((ids, m.logits()))
        m.close()
    assert runs[0][0] == runs[1][0] == ref_ids
    assert np.max(np.abs(runs[0][1] - runs[1][1])) <= 1e-3
    assert np.max(np.abs(runs[0][1] - ref_logits)) <= 1e-3
