"""The device sampler (frn_sampler_init / frn_sample) draws the ids the
oracle's Sampler (src/sampler.rs) draws from the same logits and seed:
temperature, top-k, top-p, repeat penalty, the argmax short-circuits, the
draw count, and a sampled generation loop.  The oracle is fed the device
logits, so the comparison is of the sampler alone (the logits themselves
are pinned to 1e-3 by the model tests)."""
import os

import numpy as np
import pytest

import furnace_amd as fa
from oracle import oracle as orc

pytestmark = pytest.mark.gpu

# one layer and a Qwen2-size vocabulary: 149 candidate blocks, the last partial
SPEC = dict(n_layers=1, n_heads=4, n_kv_heads=2, hidden=256, ffn=512, vocab=151936, mix=fa.MIX_Q4_K_M,
            tied=1, embd_type=fa.Q6_K, output_type=fa.Q6_K)
CASES = [  # temperature, top_k, top_p, repeat_penalty, n_recent
    (0.7, 40, 0.9, 1.0, 0),    # the reference CLI's defaults
    (1.3, 64, 1.0, 1.1, 64),
    (0.5, 5, 0.5, 1.3, 40),
    (0.05, 17, 0.95, 0.8, 10),
    (0.0, 40, 0.9, 1.5, 64),   # temperature 0: argmax of the penalized logits, no draw
    (0.8, 1, 0.9, 1.2, 64),    # top_k 1: the same
    # the whole-vocabulary path: every candidate sorted, then the sequential sums
    (0.7, 0, 0.9, 1.0, 0),     # top_k 0 (no cut) with the default top_p
    (1.0, 0, 1.0, 1.1, 20),    # no cut at all: the draw walks the sorted vocabulary
    (0.8, 100, 0.95, 1.0, 0),  # top_k above the 64 the candidate path keeps
]


def _model(tmpdir_models):
    path = os.path.join(tmpdir_models, "sampler-vocab.gguf")
    if not os.path.exists(path):
        fa.synth_write(path, seed=31, **SPEC)
    return fa.Model(path, max_ctx=256)


@pytest.mark.parametrize("case", CASES)
def test_device_sampler_matches_the_oracle(hip, tmpdir_models, case):
    temp, k, p, pen, n_recent = case
    print("sampler case T=%g k=%d p=%g penalty=%g recent=%d" % case, flush=True)
    rng = np.random.default_rng(5)
    m = _model(tmpdir_models)
    prompt = rng.integers(0, SPEC["vocab"], 9).astype(np.uint32)
    m.prefill(prompt)
    logits = m.logits()
    # recent ids: some of the top logits (so the penalty changes the
    # candidates), with repeats (penalized once)
    top = np.argsort(-logits)[:32]
    recent = np.concatenate([top[:n_recent // 2], rng.integers(0, SPEC["vocab"], n_recent - n_recent // 2),
                             top[:3]])[:n_recent].astype(np.uint32) if n_recent else np.zeros(0, np.uint32)
    m.sampler_init(temp, k, p, pen, seed=1234)
    ref = orc.Sampler(temp, k, p, pen, seed=1234)
    got = [m.sample(recent) for _ in range(200)]
    want = [ref.sample(logits, recent) for _ in range(200)]
    assert got == want
    assert m.sampler_draws() == ref.draws
    if temp == 0.0 or k == 1:
        assert ref.draws == 0 and len(set(got)) == 1
    elif temp >= 0.5:  # a flat enough distribution that the draws must differ
        assert len(set(got)) > 1
    m.close()


def test_sampled_generation_loop(hip, tmpdir_models):
    # generate.rs:121-136 with the sampler: recent = the last 64 context ids
    m = _model(tmpdir_models)
    prompt = list(np.random.default_rng(6).integers(0, SPEC["vocab"], 70).astype(np.uint32))
    m.sampler_init(0.9, 40, 0.9, 1.1, seed=99)
    ref = orc.Sampler(0.9, 40, 0.9, 1.1, seed=99)
    m.prefill(np.array(prompt, np.uint32))
    context = list(prompt)
    for step in range(40):
        logits = m.logits()
        recent = np.array(context[-64:], np.uint32)
        t = m.sample(recent)
        assert t == ref.sample(logits, recent), step
        context.append(t)
        m.decode(t)
    assert m.sampler_draws() == ref.draws == 40
    m.close()


def test_sampler_rejects_unsupported_settings(hip, tmpdir_models):
    m = _model(tmpdir_models)
    with pytest.raises(fa.FrnError):
        m.sampler_init(-1.0, 40, 0.9)
    with pytest.raises(fa.FrnError):
        m.sampler_init(0.7, 40, float("nan"))
    with pytest.raises(fa.FrnError):
        m.sampler_init(0.7, 40, 0.9, 0.0)  # repeat penalty must be > 0
    m.sampler_init(0.7, 40, 0.9)
    with pytest.raises(fa.FrnError):
        m.sample()                    # no logits yet
    m.prefill([1, 2, 3])
    with pytest.raises(fa.FrnError):
        m.sample([SPEC["vocab"]])     # recent id out of range
    m.close()


@pytest.mark.parametrize("top_k", [40, 0])
def test_generate_sampled_is_the_sampling_loop(hip, tmpdir_models, top_k):
    # frn_generate_sampled (the host layer's generate.rs loop) against the
    # same loop driven step by step: prefill, sample over the last 64 ids,
    # stop check, decode (top_k 0: the whole-vocabulary path)
    m = _model(tmpdir_models)
    prompt = list(np.random.default_rng(8).integers(0, SPEC["vocab"], 12).astype(np.uint32))
    ids, st, draws = m.generate_sampled(prompt, 30, 0.8, top_k, 0.9, 1.1, seed=5, stop_ids=[])
    assert len(ids) == 30 and st.decode_steps == 29 and draws == 30
    m.reset()
    m.sampler_init(0.8, top_k, 0.9, 1.1, seed=5)
    m.prefill(np.array(prompt, np.uint32))
    context, loop = list(prompt), []
    for step in range(30):
        t = m.sample(np.array(context[-64:], np.uint32))
        loop.append(t)
        context.append(t)
        if step + 1 < 30:
            m.decode(t)
    assert ids == loop
    m.close()
