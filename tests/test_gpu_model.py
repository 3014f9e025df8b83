"""End-to-end parity of the device token loop against the oracle on seeded
synthetic GGUF models: last-position logits within 1e-3 max-abs, KV cache
rows, and greedy (temperature 0) ids identical for the first 32 tokens."""
import os
import struct

import numpy as np
import pytest

import furnace_amd as fa
from oracle import oracle as orc

pytestmark = pytest.mark.gpu

LOGIT_TOL = 1e-3  # max-abs on last-position logits
N_IDS = 32        # greedy ids that must match exactly


def small_models():
    return {
        "tiny-q4_k_m": dict(n_layers=3, n_heads=4, n_kv_heads=2, hidden=256, ffn=512, vocab=3000, mix=fa.MIX_Q4_K_M,
                            tied=1, embd_type=fa.Q6_K, output_type=fa.Q6_K),
        "tiny-q8_0-hd64": dict(n_layers=2, n_heads=4, n_kv_heads=1, hidden=256, ffn=256 + 32, vocab=2000,
                               mix=fa.MIX_ALL_Q8_0, tied=1, embd_type=fa.Q8_0, output_type=fa.Q8_0),
        "tiny-q5_0-untied": dict(n_layers=2, n_heads=2, n_kv_heads=2, hidden=256, ffn=512, vocab=1000,
                                 mix=fa.MIX_ALL_Q5_0, tied=0, embd_type=fa.Q5_0, output_type=fa.Q8_0),
        "tiny-q4_k-gq8": dict(n_layers=2, n_heads=8, n_kv_heads=1, hidden=1024, ffn=768, vocab=500,
                              mix=fa.MIX_ALL_Q4_K, tied=1, embd_type=fa.Q4_K, output_type=fa.Q4_K),
        # llama.cpp's Q4_K_M layer mix over 16 layers, untied Q6_K output,
        # general.alignment 256
        "tiny-llama-q4_k_m": dict(n_layers=16, n_heads=4, n_kv_heads=2, hidden=256, ffn=512, vocab=1500,
                                  mix=fa.MIX_Q4_K_M_LLAMA, tied=0, embd_type=fa.Q4_K, output_type=fa.Q6_K,
                                  alignment=256),
        # F16 weights (beyond the reference, which rejects them): the oracle
        # widens them exactly to f32 under its F16 extension
        "tiny-f16-tied": dict(n_layers=2, n_heads=4, n_kv_heads=2, hidden=256, ffn=512, vocab=1000,
                              mix=fa.MIX_ALL_F16, tied=1, embd_type=fa.F16, output_type=fa.F16),
    }


@pytest.mark.parametrize("name", list(small_models()))
def test_small_model_prefill_decode(hip, tmpdir_models, name):
    path = os.path.join(tmpdir_models, name + ".gguf")
    fa.synth_write(path, seed=17, **small_models()[name])
    rng = np.random.default_rng(5)
    cfg = small_models()[name]
    prompt = rng.integers(0, cfg["vocab"], 300 if name == "tiny-q4_k-gq8" else 9).astype(np.uint32)
    print("model %s prompt %d" % (name, prompt.size), flush=True)
    if cfg["mix"] == fa.MIX_ALL_F16:
        with orc.f16_extension():
            ref = orc.Model(path)
    else:
        ref = orc.Model(path)
    ref.new_cache(512)
    ref_logits = ref.forward_cached(prompt)
    m = fa.Model(path, max_ctx=512)
    nxt = m.prefill(prompt)
    got = m.logits()
    assert np.max(np.abs(got - ref_logits)) <= LOGIT_TOL
    assert nxt == orc.argmax(got)
    assert m.cache_len() == prompt.size
    for layer in (0, cfg["n_layers"] - 1):
        for which in (0, 1):
            gk = m.cache_read(layer, which, prompt.size)
            rk = ref.cache_read(layer, which, prompt.size)
            assert np.max(np.abs(gk - rk)) <= 1e-4 * max(1.0, float(np.abs(rk).max()))
    # greedy decode, step by step against the oracle's logits
    tok = orc.argmax(ref_logits)
    assert tok == nxt
    for step in range(6):
        ref_logits = ref.forward_cached([tok])
        nxt = m.decode(tok)
        got = m.logits()
        assert np.max(np.abs(got - ref_logits)) <= LOGIT_TOL, step
        assert nxt == orc.argmax(ref_logits), step
        tok = nxt
    m.close()
    ref.close()


def test_errors_from_the_device_context(hip, tmpdir_models):
    path = os.path.join(tmpdir_models, "err.gguf")
    fa.synth_write(path, seed=2, **small_models()["tiny-q4_k_m"])
    m = fa.Model(path, max_ctx=8)
    with pytest.raises(fa.FrnError) as e:
        m.prefill([3000])  # vocab is 3000
    assert e.value.status == 5
    with pytest.raises(fa.FrnError) as e:
        m.prefill(list(range(9)))
    assert e.value.status == 4
    m.prefill(list(range(8)))
    with pytest.raises(fa.FrnError) as e:
        m.decode(1)
    assert e.value.status == 4
    m.reset()
    assert m.cache_len() == 0
    m.prefill([1, 2])
    m.close()


def test_load_rejects_a_zero_row_length(hip, tmpdir_models):
    """A 2-D tensor whose first dimension is 0 is refused with FRN_ESHAPE
    (Model::load errors on it, src/model.rs:111-123), not a division by
    zero."""
    path = os.path.join(tmpdir_models, "zero-dim.gguf")
    fa.synth_write(path, seed=2, **small_models()["tiny-q4_k_m"])
    data = bytearray(open(path, "rb").read())
    name = b"blk.0.ffn_gate.weight"
    at = data.index(struct.pack("<Q", len(name)) + name) + 8 + len(name)
    assert struct.unpack_from("<I", data, at)[0] == 2  # n_dims
    struct.pack_into("<Q", data, at + 4, 0)  # dims[0] = 0
    open(path, "wb").write(bytes(data))
    with pytest.raises(fa.FrnError) as e:
        fa.Model(path, max_ctx=8)
    assert e.value.status == 3 and "dimension 0 is zero" in str(e.value)


def _greedy_parity(path, prompt, max_new, max_ctx):
    ref = orc.Model(path)
    ref_ids, _, ref_last = ref.generate_greedy(prompt, max_new, max_ctx)
    ref.close()
    m = fa.Model(path, max_ctx=max_ctx)
    ids, st = m.generate_greedy(prompt, max_new)
    got_last = m.logits()
    m.close()
    return ids, ref_ids, got_last, ref_last


@pytest.mark.parametrize("preset,n_prompt", [("qwen2-0.5b-q8_0", 16), ("qwen2-1.5b-q4_k_m", 128)])
def test_full_model_greedy_ids_and_logits(hip, tmpdir_models, preset, n_prompt):
    path = os.path.join(tmpdir_models, preset + ".gguf")
    print("writing %s" % preset, flush=True)
    fa.synth_write(path, seed=0xF0E1, **fa.PRESETS[preset])
    prompt = np.random.default_rng(0xF0E1).integers(0, 151643, n_prompt).astype(np.uint32)
    orc.set_threads(min(16, os.cpu_count() or 1))
    print("running %s prompt %d" % (preset, n_prompt), flush=True)
    ids, ref_ids, got_last, ref_last = _greedy_parity(path, prompt, N_IDS + 1, 512)
    print("gpu ids", ids[:N_IDS], flush=True)
    print("ref ids", ref_ids[:N_IDS], flush=True)
    assert ids[:N_IDS] == ref_ids[:N_IDS]
    assert np.max(np.abs(got_last - ref_last)) <= LOGIT_TOL
    os.remove(path)


@pytest.mark.parametrize("mix", ["q4_k_m", "q6_k", "q8_0"])
def test_prefill_block_sizes(hip, tmpdir_models, mix):
    """Prompt lengths that run each prefill GEMM tile height (32, 64 and 128
    token rows, full and partial), for the formats
    with their own weight loaders (Q4_K, Q6_K) and the generic one (Q8_0):
    the last-position logits and the KV cache against the oracle."""
    spec = dict(n_layers=2, n_heads=4, n_kv_heads=2, hidden=512, ffn=768, vocab=1000, tied=1,
                mix={"q4_k_m": fa.MIX_Q4_K_M, "q6_k": fa.MIX_ALL_Q6_K, "q8_0": fa.MIX_ALL_Q8_0}[mix],
                embd_type=fa.Q6_K if mix != "q8_0" else fa.Q8_0, output_type=fa.Q8_0)
    path = os.path.join(tmpdir_models, "blocks-%s.gguf" % mix)
    fa.synth_write(path, seed=53, **spec)
    for n in (2, 31, 40, 64, 100, 257):
        prompt = np.random.default_rng(n).integers(0, spec["vocab"], n).astype(np.uint32)
        print("%s prompt %d" % (mix, n), flush=True)
        ref = orc.Model(path)
        ref.new_cache(300)
        ref_logits = ref.forward_cached(prompt)
        m = fa.Model(path, max_ctx=300)
        nxt = m.prefill(prompt)
        dl = float(np.max(np.abs(m.logits() - ref_logits)))
        print("%s prompt %d: max |dlogit| %.2e" % (mix, n, dl), flush=True)
        assert dl <= LOGIT_TOL, n
        assert nxt == orc.argmax(ref_logits), n
        got_k = m.cache_read(1, 0, n)
        want_k = ref.cache_read(1, False, n)
        assert np.max(np.abs(got_k - want_k)) <= 1e-3 * max(1.0, float(np.max(np.abs(want_k)))), n
        m.close()
        ref.close()
    os.remove(path)


@pytest.mark.parametrize("mix", ["q4_k_m", "q6_k", "q8_0", "q5_0", "f16"])
def test_prefill_split_k(hip, tmpdir_models, mix):
    """Short prompts on a model whose GEMMs give fewer than 128 output tiles
    and at least 32 k-steps (hidden 1024, FFN 2048): the prefill splits K
    over blocks for the q/k/v store, the residual adds and the SwiGLU pair,
    and adds the partial products afterwards.  Last-position logits, the
    argmax and the KV cache against the oracle (tensor.rs:114-135)."""
    mixes = {"q4_k_m": fa.MIX_Q4_K_M, "q6_k": fa.MIX_ALL_Q6_K, "q8_0": fa.MIX_ALL_Q8_0, "q5_0": fa.MIX_ALL_Q5_0,
             "f16": fa.MIX_ALL_F16}
    spec = dict(n_layers=2, n_heads=8, n_kv_heads=2, hidden=1024, ffn=2048, vocab=1000, tied=1, mix=mixes[mix],
                embd_type=fa.Q8_0, output_type=fa.Q8_0)
    path = os.path.join(tmpdir_models, "splitk-%s.gguf" % mix)
    fa.synth_write(path, seed=61, **spec)
    for n in (2, 40, 100):
        prompt = np.random.default_rng(100 + n).integers(0, spec["vocab"], n).astype(np.uint32)
        if mix == "f16":  # beyond the reference: the oracle widens F16 exactly under its extension
            with orc.f16_extension():
                ref = orc.Model(path)
        else:
            ref = orc.Model(path)
        ref.new_cache(128)
        ref_logits = ref.forward_cached(prompt)
        m = fa.Model(path, max_ctx=128)
        nxt = m.prefill(prompt)
        dl = float(np.max(np.abs(m.logits() - ref_logits)))
        print("%s prompt %d: max |dlogit| %.2e" % (mix, n, dl), flush=True)
        assert dl <= LOGIT_TOL, n
        assert nxt == orc.argmax(ref_logits), n
        for layer in (0, 1):
            for which in (0, 1):
                got = m.cache_read(layer, which, n)
                want = ref.cache_read(layer, bool(which), n)
                assert np.max(np.abs(got - want)) <= 1e-3 * max(1.0, float(np.max(np.abs(want)))), (n, layer, which)
        m.close()
        ref.close()
    os.remove(path)


def test_7b_greedy_ids_and_logits(hip, tmpdir_models):
    """Qwen2-7B shape (hidden 3584, FFN 18944, 7 query heads per kv head,
    untied Q6_K lm_head, Q4_K embedding): a 16-token prompt keeps the
    oracle's run to seconds; the shapes are the full model's."""
    path = os.path.join(tmpdir_models, "qwen2-7b-q4_k_m.gguf")
    print("writing qwen2-7b-q4_k_m", flush=True)
    fa.synth_write(path, seed=0xF0E1 + 4, threads=min(16, os.cpu_count() or 1), **fa.PRESETS["qwen2-7b-q4_k_m"])
    prompt = np.random.default_rng(0xF0E1 + 4).integers(0, 151643, 16).astype(np.uint32)
    orc.set_threads(min(16, os.cpu_count() or 1))
    print("running 7b prompt 16", flush=True)
    ids, ref_ids, got_last, ref_last = _greedy_parity(path, prompt, N_IDS + 1, 64)
    print("gpu ids", ids[:N_IDS], flush=True)
    print("ref ids", ref_ids[:N_IDS], flush=True)
    assert ids[:N_IDS] == ref_ids[:N_IDS]
    assert np.max(np.abs(got_last - ref_last)) <= LOGIT_TOL
    os.remove(path)


def test_long_context_small_model(hip, tmpdir_models):
    """Past 4096 positions (the long-context workload's length) on a small
    model, so the oracle's single-threaded attention stays cheap: prefill
    of 4200 ids in blocks, then decode steps over 66+ attention splits."""
    cfg = dict(small_models()["tiny-q4_k_m"], n_layers=2, vocab=1000)
    path = os.path.join(tmpdir_models, "tiny-long.gguf")
    fa.synth_write(path, seed=31, **cfg)
    prompt = np.random.default_rng(31).integers(0, cfg["vocab"], 4200).astype(np.uint32)
    print("long context prompt %d" % prompt.size, flush=True)
    ref = orc.Model(path)
    ref.new_cache(4300)
    ref_logits = ref.forward_cached(prompt)
    m = fa.Model(path, max_ctx=4300)
    nxt = m.prefill(prompt)
    dl = float(np.max(np.abs(m.logits() - ref_logits)))
    print("prefill of %d tokens: max |dlogit| %.2e" % (prompt.size, dl), flush=True)
    assert dl <= LOGIT_TOL
    tok = orc.argmax(ref_logits)
    assert nxt == tok
    for step in range(8):
        ref_logits = ref.forward_cached([tok])
        nxt = m.decode(tok)
        assert np.max(np.abs(m.logits() - ref_logits)) <= LOGIT_TOL, step
        assert nxt == orc.argmax(ref_logits), step
        tok = nxt
    m.close()
    ref.close()


def test_long_context_1p5b_head_shape(hip, tmpdir_models):
    """The long-context form at the Qwen2-1.5B head shape (12 query heads
    over 2 kv heads, head_dim 128; model.rs:371-438) against the oracle:
    a 4200-token prompt through the prefill's row blocks, then 8 decode
    steps whose attention runs past 4096 positions in up to 128 splits per
    head, merged per head.  Two layers, FFN 1280 and a 2048-id vocabulary
    keep the oracle's run to seconds."""
    cfg = dict(n_layers=2, n_heads=12, n_kv_heads=2, hidden=1536, ffn=1280, vocab=2048, mix=fa.MIX_Q4_K_M,
               tied=1, embd_type=fa.Q6_K, output_type=fa.Q6_K)
    path = os.path.join(tmpdir_models, "hd128-long.gguf")
    fa.synth_write(path, seed=37, **cfg)
    prompt = np.random.default_rng(37).integers(0, cfg["vocab"], 4200).astype(np.uint32)
    orc.set_threads(min(16, os.cpu_count() or 1))
    print("1.5B head shape, prompt %d: oracle prefill" % prompt.size, flush=True)
    ref = orc.Model(path)
    ref.new_cache(4300)
    ref_logits = ref.forward_cached(prompt)
    print("device prefill", flush=True)
    m = fa.Model(path, max_ctx=4300)
    nxt = m.prefill(prompt)
    dl = float(np.max(np.abs(m.logits() - ref_logits)))
    print("prefill of %d tokens: max |dlogit| %.2e" % (prompt.size, dl), flush=True)
    assert dl <= LOGIT_TOL
    tok = orc.argmax(ref_logits)
    assert nxt == tok
    for step in range(8):
        ref_logits = ref.forward_cached([tok])
        nxt = m.decode(tok)
        assert np.max(np.abs(m.logits() - ref_logits)) <= LOGIT_TOL, step
        assert nxt == orc.argmax(ref_logits), step
        tok = nxt
    m.close()
    ref.close()
    os.remove(path)


def test_7b_shape_prompt_scale_prefill(hip, tmpdir_models):
    """The Qwen2-7B layer shapes (hidden 3584, FFN 18944, 7 query heads per
    kv head, untied Q6_K lm_head [152064, 3584]) at prompt scale: a
    640-token prompt runs the prefill's 128-row GEMM tiles at their real K
    (3584 and 18944; tensor.rs:114-135), then 8 greedy decode steps, all
    against the oracle.  Two layers keep the oracle's run to about half a
    minute."""
    cfg = dict(fa.PRESETS["qwen2-7b-q4_k_m"], n_layers=2)
    path = os.path.join(tmpdir_models, "qwen2-7b-2layer.gguf")
    print("writing 2-layer 7b-shape model", flush=True)
    fa.synth_write(path, seed=41, threads=min(16, os.cpu_count() or 1), **cfg)
    prompt = np.random.default_rng(41).integers(0, 151643, 640).astype(np.uint32)
    orc.set_threads(min(16, os.cpu_count() or 1))
    print("7b shape, prompt %d: oracle prefill" % prompt.size, flush=True)
    ref = orc.Model(path)
    ref.new_cache(700)
    ref_logits = ref.forward_cached(prompt)
    print("device prefill", flush=True)
    m = fa.Model(path, max_ctx=700)
    nxt = m.prefill(prompt)
    dl = float(np.max(np.abs(m.logits() - ref_logits)))
    print("prefill of %d tokens: max |dlogit| %.2e" % (prompt.size, dl), flush=True)
    assert dl <= LOGIT_TOL
    tok = orc.argmax(ref_logits)
    assert nxt == tok
    ids, ref_ids = [], []
    for step in range(8):
        ref_logits = ref.forward_cached([tok])
        ref_ids.append(orc.argmax(ref_logits))
        ids.append(m.decode(tok))
        assert np.max(np.abs(m.logits() - ref_logits)) <= LOGIT_TOL, step
        tok = ref_ids[-1]
    assert ids == ref_ids
    m.close()
    ref.close()
    os.remove(path)


def test_long_context_full_size_paths_agree(hip, tmpdir_models):
    """The long-context workload's shape (1.5B Q4_K_M, 4096-token prompt) is
    beyond the oracle's reach in a test, so the two device paths are
    checked against each other: blocks of rows through the MFMA GEMMs vs
    one decode step per position, then 16 greedy decode steps from each."""
    path = os.path.join(tmpdir_models, "qwen2-1.5b-q4_k_m-long.gguf")
    fa.synth_write(path, seed=0xF0E1 + 3, threads=min(16, os.cpu_count() or 1), **fa.PRESETS["qwen2-1.5b-q4_k_m"])
    prompt = np.random.default_rng(0xF0E1 + 3).integers(0, 151643, 4096).astype(np.uint32)
    outs = []
    for stepwise in (False, True):
        print("4096-token prefill, stepwise=%s" % stepwise, flush=True)
        m = fa.Model(path, max_ctx=4096 + 32, stepwise_prefill=stepwise)
        nxt = m.prefill(prompt)
        logits = m.logits()
        ids = [nxt]
        for _ in range(15):
            ids.append(m.decode(ids[-1]))
        m.close()
        outs.append((logits, ids))
    assert np.max(np.abs(outs[0][0] - outs[1][0])) <= LOGIT_TOL
    assert outs[0][1] == outs[1][1]
    os.remove(path)
