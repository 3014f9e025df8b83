"""Oracle dequantizers and fused matmul, pinned by furnace's own known-answer
tests (src/quant.rs:283-464), by exhaustive f16 decoding against numpy, and
by closed-form checks on blocks packed from chosen integer fields."""
import math

import numpy as np
import pytest

from oracle import oracle as orc


def f16_bytes(v):
    return np.array([v], dtype=np.float16).tobytes()


def q8_block(scale, quants):  # quant.rs:288-292
    return f16_bytes(scale) + bytes((q & 0xFF) for q in quants)


# ---- quant.rs:294-328 ----------------------------------------------------------
def test_one_block_with_negative_quants():
    out = orc.dequantize(orc.Q8_0, q8_block(0.5, [i - 16 for i in range(32)]), 32)
    assert out.tolist() == [0.5 * (i - 16) for i in range(32)]


def test_zero_scale_gives_exact_zeros():
    out = orc.dequantize(orc.Q8_0, q8_block(0.0, [127] * 32), 32)
    assert (out == 0.0).all()


def test_two_blocks_use_their_own_scales():
    out = orc.dequantize(orc.Q8_0, q8_block(1.0, [3] * 32) + q8_block(2.0, [3] * 32), 64)
    assert out[0] == 3.0 and out[32] == 6.0


def test_rejects_wrong_length():
    raw = q8_block(1.0, [0] * 32)
    for data, n in ((raw[:33], 32), (raw, 64), (raw, 31)):
        with pytest.raises(ValueError):
            orc.dequantize(orc.Q8_0, data, n)


# ---- quant.rs:330-357 ----------------------------------------------------------
def test_fused_q8_matmul_matches_dequant_reference():
    raw = b""
    for o in range(3):
        for b in range(2):
            quants = [((j * 7 + o * 13 + b * 5) % 255 - 127) for j in range(32)]
            raw += q8_block(0.5 + o * 0.25, quants)
    x = np.sin(np.arange(2 * 64, dtype=np.float32) * np.float32(0.31)).reshape(2, 64)
    w = orc.dequantize(orc.Q8_0, raw, 3 * 64).reshape(3, 64)
    ref = orc.matmul_f32(x, w)
    fused = orc.matmul_quant(x, np.frombuffer(raw, np.uint8), 3, 64, orc.Q8_0)
    assert fused.shape == ref.shape == (2, 3)
    assert np.all(np.abs(fused - ref) < 1e-4)


# ---- quant.rs:359-413 (hand-computed blocks) ---------------------------------
def test_q4_k_block_hand_computed():
    b = bytearray(144)
    b[0:2] = bytes([0x00, 0x3C])
    b[2:4] = bytes([0x00, 0x38])
    b[4], b[8], b[5], b[9], b[12] = 3, 2, 5, 1, 7
    b[16] = 0x51
    b[16 + 64] = 0x04
    out = orc.dequantize(orc.Q4_K, bytes(b), 256)
    assert out[0] == 2.0 and out[32] == 24.5 and out[128] == 28.0 and out[1] == -1.0


def test_q6_k_block_hand_computed():
    b = bytearray(210)
    b[208:210] = bytes([0x00, 0x38])
    b[192], b[194], b[196], b[198] = 2, 1, 3, 0xFF
    b[0] = 0x21
    b[128] = 0xC4
    out = orc.dequantize(orc.Q6_K, bytes(b), 256)
    assert (out[0], out[32], out[64], out[96]) == (-31.0, -8.0, -45.0, -8.0)


def test_q5_0_block_hand_computed():  # quant.rs:415-431
    b = bytearray(22)
    b[0:2] = bytes([0x00, 0x38])
    b[2] = 0b1
    b[6] = 0x51
    out = orc.dequantize(orc.Q5_0, bytes(b), 32)
    assert (out[0], out[16], out[1]) == (0.5, -5.5, -8.0)


# ---- quant.rs:433-454 ----------------------------------------------------------
def test_fused_k_matmul_matches_dequant_reference():
    raw = np.array([(i * 37 + 11) % 251 for i in range(2 * 144)], dtype=np.uint8)
    x = np.sin(np.arange(3 * 256, dtype=np.float32) * np.float32(0.17)).reshape(3, 256)
    w = orc.dequantize(orc.Q4_K, raw, 2 * 256).reshape(2, 256)
    ref = orc.matmul_f32(x, w)
    fused = orc.matmul_quant(x, raw, 2, 256, orc.Q4_K)
    assert np.all(np.abs(fused - ref) <= 1e-3 * np.maximum(np.abs(ref), 1.0))


def test_f32_passthrough_reads_le():  # quant.rs:456-464
    raw = np.array([1.5, -2.25, 0.0], dtype="<f4").tobytes()
    assert orc.dequantize(orc.F32, raw, 3).tolist() == [1.5, -2.25, 0.0]


def test_unsupported_type_is_an_error():  # quant.rs:279
    with pytest.raises(ValueError, match="not implemented"):
        orc.dequantize(orc.F16, b"\x00\x3c", 1)


def test_f16_extension_widens_exactly_and_switches_off():
    # beyond the reference: with the switch on, F16 data widens as numpy's
    # float16 -> float32 cast does, for every bit pattern (NaNs by class)
    bits = np.arange(1 << 16, dtype=np.uint16)
    with orc.f16_extension():
        got = orc.dequantize(orc.F16, bits.tobytes(), bits.size)
        with pytest.raises(ValueError, match="expected"):
            orc.dequantize(orc.F16, bits[:3].tobytes(), 4)
    want = bits.view(np.float16).astype(np.float32)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))
    with pytest.raises(ValueError, match="not implemented"):
        orc.dequantize(orc.F16, b"\x00\x3c", 1)


# ---- f16 widening: every bit pattern against numpy's IEEE conversion ----------
def test_f16_to_f32_exhaustive():
    bits = np.arange(65536, dtype=np.uint16)
    want = bits.view(np.float16).astype(np.float32)
    got = np.array([orc.lib().orc_f16_to_f32(int(b)) for b in bits], dtype=np.float32)
    finite = np.isfinite(want)
    assert np.array_equal(got[finite].view(np.uint32), want[finite].view(np.uint32))
    assert np.array_equal(np.isnan(got), np.isnan(want))
    assert np.array_equal(np.isinf(got), np.isinf(want))


# ---- closed forms on blocks packed from chosen fields --------------------------
# The packers below follow the byte layout described in quant.rs's comments
# (:3-6, :46-52, :67-77, :70-72, :111-113); the expected values are computed
# from the chosen integer fields, never from the bytes.
rng = np.random.default_rng(1234)


def _f16(v):
    return np.float16(v)


def test_q4_k_closed_form_random_fields():
    for _ in range(200):
        d, dmin = _f16(rng.uniform(-2, 2)), _f16(rng.uniform(-2, 2))
        sc = rng.integers(0, 64, 8)
        m = rng.integers(0, 64, 8)
        q = rng.integers(0, 16, 256)
        s = bytearray(12)
        for j in range(4):
            s[j] = sc[j] | ((sc[j + 4] >> 4) << 6)
            s[j + 4] = m[j] | ((m[j + 4] >> 4) << 6)
            s[j + 8] = (sc[j + 4] & 15) | ((m[j + 4] & 15) << 4)
        qs = bytearray(128)
        for j64 in range(4):
            for l in range(32):
                qs[32 * j64 + l] = q[64 * j64 + l] | (q[64 * j64 + 32 + l] << 4)
        blk = np.float16(d).tobytes() + np.float16(dmin).tobytes() + bytes(s) + bytes(qs)
        out = orc.dequantize(orc.Q4_K, blk, 256)
        sub = np.arange(256) // 32
        want = (np.float32(d) * sc[sub].astype(np.float32)) * q.astype(np.float32) - \
               np.float32(dmin) * m[sub].astype(np.float32)
        assert np.array_equal(out, want.astype(np.float32))


def test_q6_k_closed_form_random_fields():
    for _ in range(200):
        d = _f16(rng.uniform(-1, 1))
        sc = rng.integers(-128, 128, 16)
        q = rng.integers(-32, 32, 256)
        b = bytearray(210)
        for e in range(256):
            u = int(q[e]) + 32
            h, r = divmod(e, 128)
            k, l = divmod(r, 32)
            idx = 64 * h + l + (32 if k & 1 else 0)
            b[idx] |= (u & 15) << (4 if k & 2 else 0)
            b[128 + 32 * h + l] |= (u >> 4) << (2 * k)
        for j in range(16):
            b[192 + j] = sc[j] & 0xFF
        b[208:210] = np.float16(d).tobytes()
        out = orc.dequantize(orc.Q6_K, bytes(b), 256)
        want = (np.float32(d) * sc[np.arange(256) // 16].astype(np.float32)) * q.astype(np.float32)
        assert np.array_equal(out, want.astype(np.float32))


def test_q5_0_and_q8_0_closed_form_random_fields():
    for _ in range(200):
        d = _f16(rng.uniform(-1, 1))
        q5 = rng.integers(0, 32, 32)
        qh = 0
        qs = bytearray(16)
        for j in range(16):
            qs[j] = (q5[j] & 15) | ((q5[j + 16] & 15) << 4)
            qh |= ((int(q5[j]) >> 4) & 1) << j
            qh |= ((int(q5[j + 16]) >> 4) & 1) << (j + 16)
        blk = np.float16(d).tobytes() + qh.to_bytes(4, "little") + bytes(qs)
        out = orc.dequantize(orc.Q5_0, blk, 32)
        assert np.array_equal(out, (np.float32(d) * (q5 - 16).astype(np.float32)).astype(np.float32))
        q8 = rng.integers(-128, 128, 32)
        out = orc.dequantize(orc.Q8_0, q8_block(float(d), q8), 32)
        assert np.array_equal(out, (np.float32(d) * q8.astype(np.float32)).astype(np.float32))


# ---- fused matmul against an f64 dequantize-then-dot -----------------------------
@pytest.mark.parametrize("gtype,d_in", [(orc.Q8_0, 96), (orc.Q5_0, 64), (orc.Q5_0, 96), (orc.Q4_K, 512),
                                        (orc.Q6_K, 768)])
def test_fused_matmul_vs_f64(gtype, d_in):
    be, bb = orc.BLOCK[gtype]
    d_out, seq = 37, 3
    raw = rng.integers(0, 256, d_out * d_in // be * bb).astype(np.uint8)
    # keep every f16 scale finite and modest
    for blk in range(raw.size // bb):
        base = blk * bb
        offs = [208] if gtype == orc.Q6_K else ([0, 2] if gtype == orc.Q4_K else [0])
        for o in offs:
            raw[base + o:base + o + 2] = np.frombuffer(np.float16(rng.uniform(-0.1, 0.1)).tobytes(), np.uint8)
    x = rng.standard_normal((seq, d_in)).astype(np.float32)
    w = orc.dequantize(gtype, raw, d_out * d_in).reshape(d_out, d_in).astype(np.float64)
    ref = x.astype(np.float64) @ w.T
    got = orc.matmul_quant(x, raw, d_out, d_in, gtype)
    scale = np.maximum(np.abs(ref), np.sqrt(np.mean(ref ** 2)))
    assert np.max(np.abs(got - ref) / scale) < 1e-5


def test_matmul_rejects_bad_shapes():
    raw = np.zeros(144, np.uint8)
    with pytest.raises(ValueError, match="not a multiple"):
        orc.matmul_quant(np.zeros((1, 100), np.float32), raw, 1, 100, orc.Q4_K)
    with pytest.raises(ValueError, match="bad weight byte count"):
        orc.matmul_quant(np.zeros((1, 256), np.float32), raw, 2, 256, orc.Q4_K)
