"""Oracle f32 ops and attention, pinned by furnace's known-answer and
invariant tests (src/tensor.rs:258-337, src/model.rs:614-743,
src/generate.rs:225-229) and by f64 recomputation."""
import math

import numpy as np
import pytest

from oracle import oracle as orc


def close(got, want, tol):
    assert np.all(np.abs(np.asarray(got, np.float64) - np.asarray(want, np.float64)) <= tol), (got, want)


def test_matmul_hand_computed():  # tensor.rs:258-269
    a = np.array([[1, 2, 3], [4, 5, 6]], np.float32)
    w = np.array([[1, 0, 1], [0, 1, 0]], np.float32)
    assert orc.matmul_f32(a, w).tolist() == [[4, 2], [10, 5]]


def test_rmsnorm_hand_computed():  # tensor.rs:279-287
    close(orc.rmsnorm(np.array([[3, 4]]), np.array([2, 0.5]), 0.0), [[1.69706, 0.56569]], 1e-5)


def test_rmsnorm_zero_row_stays_finite():  # tensor.rs:289-297
    y = orc.rmsnorm(np.zeros((1, 3)), np.ones(3), 1e-5)
    assert np.isfinite(y).all() and (y == 0).all()


def test_softmax_hand_computed():  # tensor.rs:299-305
    close(orc.softmax(np.array([[0.0, math.log(2)]])), [[1 / 3, 2 / 3]], 1e-6)


def test_softmax_survives_large_logits():  # tensor.rs:307-316
    p = orc.softmax(np.array([[1000.0, 1001.0]]))
    assert np.isfinite(p).all() and abs(p.sum() - 1) < 1e-6 and p[0, 1] > p[0, 0]


def test_silu_and_swiglu_known_points():  # tensor.rs:318-329
    close(orc.silu(np.array([0.0, 1.0, -1.0])), [0.0, 0.731059, -0.268941], 1e-5)
    close(orc.swiglu(np.array([1.0]), np.array([2.0])), [1.462117], 1e-5)


def test_add_elementwise():  # tensor.rs:331-337
    assert orc.add(np.array([1, 2]), np.array([10, 0.5])).tolist() == [11, 2.5]


def test_rope_position_zero_is_identity():  # model.rs:614-620
    assert orc.rope(np.array([[1, 2, 3, 4]]), 1, 4, 1e6, 0).tolist() == [[1, 2, 3, 4]]


def test_rope_known_vector_at_position_one():  # model.rs:622-637
    x = orc.rope(np.array([[9, 9, 9, 9], [1, 2, 3, 4]]), 1, 4, 4.0, 0)
    close(x[1], [-1.9841108, -0.1625368, 2.4623778, 4.4691815], 1e-5)


def test_rope_matches_f64_at_long_positions():
    # angle = pos * theta^(-2i/hd) in f32 before sin/cos: compare with f64
    # evaluation of the same f32 angle
    hd, theta = 128, 1e6
    x = np.random.default_rng(5).standard_normal((1, hd)).astype(np.float32)
    for pos in (0, 1, 17, 4095, 4607):
        got = orc.rope(x, 1, hd, theta, pos)[0]
        half = hd // 2
        i = np.arange(half, dtype=np.float32)
        freq = np.power(np.float32(theta), (np.float32(-2.0) * i) / np.float32(hd), dtype=np.float32)
        ang = (np.float32(pos) * freq).astype(np.float64)
        a, b = x[0, :half].astype(np.float64), x[0, half:].astype(np.float64)
        want = np.concatenate([a * np.cos(ang) - b * np.sin(ang), a * np.sin(ang) + b * np.cos(ang)])
        # one ulp of freq (numpy's float32 power vs libm powf) moves the
        # angle by up to pos * 2^-23 rad
        close(got, want, 1e-6 + pos * 2.4e-7 * float(np.abs(x).max()))


def test_causal_mask_zeroes_future_tokens():  # model.rs:639-656
    q = np.array([[1, 0], [0, 1], [1, 1]])
    k = np.array([[1, 1], [0, 1], [1, 0]])
    p = orc.attention_scores(q, k, 1, 1, 2).ravel()
    assert p[0] == 1.0 and p[1] == 0.0 and p[2] == 0.0 and p[5] == 0.0
    for row in p.reshape(3, 3):
        assert abs(row.sum() - 1) < 1e-6


def test_gqa_maps_q_heads_to_shared_kv_heads():  # model.rs:731-743
    probs = orc.attention_scores(np.ones((1, 8)), np.ones((1, 4)), 4, 2, 2)
    out = orc.attention_apply(probs, np.array([[10, 20, 30, 40]]), 4, 2, 2)
    assert out.tolist() == [[10, 20, 10, 20, 30, 40, 30, 40]]


def _fill(n, salt):  # model.rs:658-661
    return (np.sin(np.arange(n, dtype=np.float32) * np.float32(0.37) + np.float32(salt)) * np.float32(0.5)).astype(np.float32)


def _tiny():  # model.rs:663-694
    c = orc.Config(n_layers=1, n_heads=2, n_kv_heads=1, hidden=8, ffn=16, head_dim=4, vocab=1, context_length=32,
                   rope_theta=100.0, rms_eps=1e-6)
    h, f, qd, kd = 8, 16, 8, 4
    arrs = dict(attn_norm=_fill(h, 1), wq=_fill(qd * h, 2), bq=_fill(qd, 3), wk=_fill(kd * h, 4), bk=_fill(kd, 5),
                wv=_fill(kd * h, 6), bv=_fill(kd, 7), wo=_fill(h * qd, 8), ffn_norm=_fill(h, 9),
                w_gate=_fill(f * h, 10), w_up=_fill(f * h, 11), w_down=_fill(h * f, 12))
    layer = orc.F32Layer(**{k: v.ctypes.data for k, v in arrs.items()})
    return c, layer, arrs


def test_cached_path_is_bit_identical_to_uncached():  # model.rs:696-729
    c, layer, keep = _tiny()
    x = _fill(5 * 8, 20).reshape(5, 8)
    unc = np.empty((5, 8), np.float32)
    orc.lib().orc_layer_forward_f32(x.ctypes.data, 5, layer, c, unc.ctypes.data)
    kc = np.zeros(32 * 4, np.float32)
    vc = np.zeros(32 * 4, np.float32)
    pre = np.empty((3, 8), np.float32)
    x3 = np.ascontiguousarray(x[:3])
    orc.lib().orc_layer_forward_cached_f32(x3.ctypes.data, 3, layer, c, kc.ctypes.data, vc.ctypes.data, 32, 0,
                                           pre.ctypes.data)
    assert np.array_equal(pre, unc[:3])
    for s in (3, 4):
        row = np.ascontiguousarray(x[s:s + 1])
        out = np.empty((1, 8), np.float32)
        orc.lib().orc_layer_forward_cached_f32(row.ctypes.data, 1, layer, c, kc.ctypes.data, vc.ctypes.data, 32, s,
                                               out.ctypes.data)
        assert np.array_equal(out[0], unc[s]), "decode step for position %d diverged from uncached" % s


def test_argmax_first_max_wins_ties():  # generate.rs:225-229
    assert orc.argmax(np.array([1.0, 5.0, 5.0, 2.0])) == 1
    assert orc.argmax(np.array([-3.0, -1.0, -2.0])) == 1


def test_dot_vs_f64():
    rng = np.random.default_rng(3)
    for n in (1, 7, 8, 9, 64, 1000, 1536):
        a, b = rng.standard_normal(n).astype(np.float32), rng.standard_normal(n).astype(np.float32)
        ref = float(a.astype(np.float64) @ b.astype(np.float64))
        assert abs(orc.dot(a, b) - ref) <= 1e-5 * max(1.0, float(np.abs(a) @ np.abs(b)))


def test_softmax_vs_f64():
    x = np.random.default_rng(4).standard_normal((3, 300)).astype(np.float32) * 4
    e = np.exp(x.astype(np.float64) - x.max(1, keepdims=True))
    close(orc.softmax(x), e / e.sum(1, keepdims=True), 1e-6)
