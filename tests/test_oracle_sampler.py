"""Oracle sampler (src/sampler.rs), pinned by the reference's own tests
(src/sampler.rs:169-250), by O'Neill's published PCG32 demo stream, and by
the empirical distribution of many draws against filtered()."""
import math

import numpy as np

from oracle import oracle as orc


def close(got, want, tol=1e-5):  # sampler.rs:164-166
    assert abs(float(got) - float(want)) < tol, (got, want)


def test_pcg32_published_stream():
    # pcg32_srandom_r(&rng, 42u, 54u) in O'Neill's pcg-c-basic demo prints
    # these six 32-bit outputs first
    r = orc.Pcg32(42, 54)
    assert [r.next_u32() for _ in range(6)] == [0xa15c02b7, 0x7b47f409, 0xba1d3330, 0x83d2f293, 0xbfa4784b,
                                               0xcbed606e]


def test_pcg32_f32_is_the_top_24_bits():  # sampler.rs:31-33
    a, b = orc.Pcg32(1234), orc.Pcg32(1234)
    for _ in range(1000):
        u = a.next_u32()
        f = b.next_f32()
        assert f == (u >> 8) / float(1 << 24)
        assert 0.0 <= f < 1.0


def test_temperature_reshapes_the_distribution():  # sampler.rs:168-181
    logits = [0.0, math.log(3.0)]
    ids, p = orc.Sampler(1.0, 0, 1.0).filtered(logits)
    assert ids[0] == 1
    close(p[0], 0.75)
    close(p[1], 0.25)
    ids, p = orc.Sampler(0.5, 0, 1.0).filtered(logits)
    close(p[0], 0.9)
    close(p[1], 0.1)


def test_top_k_keeps_exactly_k():  # sampler.rs:183-190
    ids, p = orc.Sampler(1.0, 2, 1.0).filtered([5.0, 1.0, 4.0, 2.0, 3.0])
    assert ids.tolist() == [0, 2]
    close(p.sum(), 1.0)


def test_top_p_cuts_at_the_crossing_token():  # sampler.rs:192-203
    logits = [math.log(p) for p in np.array([0.5, 0.3, 0.15, 0.05], np.float32)]
    ids, p = orc.Sampler(1.0, 0, 0.8).filtered(np.array(logits, np.float32))
    assert len(ids) == 2
    assert (ids[0], ids[1]) == (0, 1)
    close(p[0], 0.625)
    close(p[1], 0.375)


def test_repeat_penalty_follows_llama_cpp_sign_convention():  # sampler.rs:205-213
    out = orc.apply_repeat_penalty([2.0, -2.0, 1.0], [0, 1, 0], 2.0)
    assert out.tolist() == [1.0, -4.0, 1.0]
    assert orc.apply_repeat_penalty([2.0, -2.0], [0, 1], 1.0).tolist() == [2.0, -2.0]


def test_degenerate_filters_disable_cleanly():  # sampler.rs:215-222
    ids, p = orc.Sampler(1.0, 0, 1.0).filtered([1.0, 0.5, 0.0, -0.5])
    assert len(ids) == 4
    close(p.sum(), 1.0)


def test_temperature_zero_is_argmax_with_no_rng_draw():  # sampler.rs:224-238
    logits = [0.1, 3.0, 0.2]
    s = orc.Sampler(0.0, 40, 0.9)
    assert s.sample(logits) == 1 and s.draws == 0
    s = orc.Sampler(0.7, 1, 0.9)
    assert s.sample(logits) == 1 and s.draws == 0
    s = orc.Sampler(0.7, 40, 0.9)
    s.sample(logits)
    assert s.draws == 1


def test_same_seed_same_stream_different_seed_different_stream():  # sampler.rs:240-249
    logits = np.array([(i % 7) * 0.01 for i in range(100)], np.float32)

    def run(seed):
        s = orc.Sampler(1.0, 0, 1.0, 1.0, seed)
        return [s.sample(logits) for _ in range(20)]

    assert run(42) == run(42)
    assert run(42) != run(43)


def test_draws_follow_the_filtered_distribution():
    # 40 000 draws from a 6-candidate distribution (top-k 6 of 50, top-p
    # 0.9): every empirical frequency within 5 sigma of filtered()'s
    # probability, and no id outside the filtered set
    rng = np.random.default_rng(11)
    logits = rng.normal(0, 2, 50).astype(np.float32)
    s = orc.Sampler(0.8, 6, 0.9, 1.0, 99)
    ids, p = s.filtered(logits)
    assert 1 <= len(ids) <= 6 and abs(float(p.sum()) - 1.0) < 1e-6
    assert np.all(np.diff(p) <= 0)
    counts = {}
    n = 40000
    for _ in range(n):
        t = s.sample(logits)
        counts[t] = counts.get(t, 0) + 1
    assert set(counts) <= set(ids.tolist())
    for i, pi in zip(ids.tolist(), p.tolist()):
        sigma = math.sqrt(n * pi * (1 - pi)) + 1
        assert abs(counts.get(i, 0) - n * pi) < 5 * sigma, (i, counts.get(i, 0), n * pi)
    assert s.draws == n


def test_top_p_crossing_invariant_on_random_logits():
    # the kept prefix is the shortest one whose f32 cumulative sum reaches p
    rng = np.random.default_rng(12)
    for trial in range(20):
        logits = rng.normal(0, 3, 300).astype(np.float32)
        top_p = float(rng.uniform(0.3, 0.99))
        s = orc.Sampler(float(rng.uniform(0.3, 1.5)), int(rng.integers(0, 60)), top_p)
        full = orc.Sampler(s.st.temperature, s.st.top_k, 1.0)
        ids_all, p_all = full.filtered(logits)
        ids, _ = s.filtered(logits)
        cum = np.cumsum(p_all.astype(np.float32), dtype=np.float32)
        keep = int(np.argmax(cum >= np.float32(top_p))) + 1 if np.any(cum >= np.float32(top_p)) else len(p_all)
        assert ids.tolist() == ids_all[:keep].tolist(), trial
