"""GPU parity of the single-op entry points against the oracle:
dequantization bit-exact in f32, fused dequant-GEMV within 1e-4 relative
(max |g - c| / max(|c|, rms(c))), device argmax with the first-max rule."""
import numpy as np
import pytest

import furnace_amd as fa
from oracle import oracle as orc

pytestmark = pytest.mark.gpu

GEMV_TOL = 1e-4  # single-op GEMV gate, relative


def rel_err(got, ref):
    ref64 = ref.astype(np.float64)
    scale = np.maximum(np.abs(ref64), np.sqrt(np.mean(ref64 ** 2)))
    return float(np.max(np.abs(got.astype(np.float64) - ref64) / scale))


def random_blocks(rng, gtype, n_blocks):
    """Arbitrary bytes with finite, modest f16 scales: every bit pattern of
    the quant fields is exercised."""
    be, bb = fa.BLOCK[gtype]
    raw = rng.integers(0, 256, n_blocks * bb).astype(np.uint8).reshape(n_blocks, bb)
    offs = {fa.Q8_0: [0], fa.Q5_0: [0], fa.Q4_K: [0, 2], fa.Q6_K: [208]}[gtype]
    for o in offs:
        raw[:, o:o + 2] = np.frombuffer(rng.uniform(-1, 1, n_blocks).astype(np.float16).tobytes(),
                                        np.uint8).reshape(n_blocks, 2)
    return raw.ravel()


@pytest.mark.parametrize("gtype", [fa.Q8_0, fa.Q5_0, fa.Q4_K, fa.Q6_K])
def test_dequant_bit_exact(hip, gtype):
    rng = np.random.default_rng(100 + gtype)
    be, bb = fa.BLOCK[gtype]
    for n_blocks in (1, 3, 1000):
        raw = random_blocks(rng, gtype, n_blocks)
        n = n_blocks * be
        print("dequant type %d blocks %d" % (gtype, n_blocks), flush=True)
        d_raw = hip.to_device(raw)
        d_out = hip.malloc(n * 4)
        fa.dequant_dev(hip, gtype, d_raw, raw.size, n, d_out)
        got = hip.from_device(d_out, n, np.float32)
        want = orc.dequantize(gtype, raw, n)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
        hip.free(d_raw)
        hip.free(d_out)


def test_dequant_f16_every_bit_pattern(hip):
    # F16 (beyond the reference): exact widening, against the oracle's F16
    # extension, for all 65536 halves
    bits = np.arange(1 << 16, dtype=np.uint16)
    d_raw = hip.to_device(bits.view(np.uint8))
    d_out = hip.malloc(bits.size * 4)
    fa.dequant_dev(hip, fa.F16, d_raw, bits.size * 2, bits.size, d_out)
    got = hip.from_device(d_out, bits.size, np.float32)
    with orc.f16_extension():
        want = orc.dequantize(orc.F16, bits.tobytes(), bits.size)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))
    hip.free(d_raw)
    hip.free(d_out)


def test_dequant_reference_known_answers(hip):
    # quant.rs:359-387 Q4_K block through the device path
    b = bytearray(144)
    b[0:2] = bytes([0x00, 0x3C]); b[2:4] = bytes([0x00, 0x38])
    b[4], b[8], b[5], b[9], b[12] = 3, 2, 5, 1, 7
    b[16] = 0x51; b[16 + 64] = 0x04
    d_raw = hip.to_device(np.frombuffer(bytes(b), np.uint8))
    d_out = hip.malloc(256 * 4)
    fa.dequant_dev(hip, fa.Q4_K, d_raw, 144, 256, d_out)
    out = hip.from_device(d_out, 256, np.float32)
    assert (out[0], out[32], out[128], out[1]) == (2.0, 24.5, 28.0, -1.0)


def _gemv_case(hip, gtype, d_out, d_in, seed, seq=1):
    rng = np.random.default_rng(seed)
    w = fa.gaussian(seed, 0.02, d_out * d_in)
    raw = fa.quantize(gtype, w)
    x = rng.standard_normal((seq, d_in)).astype(np.float32)
    print("gemv type %d [%d x %d] seq %d" % (gtype, d_out, d_in, seq), flush=True)
    d_w, d_x, d_y = hip.to_device(raw), hip.to_device(x), hip.malloc(seq * d_out * 4)
    fa.matmul_quant_dev(gtype, d_w, raw.size, d_x, seq, d_y, d_out, d_in)
    got = hip.from_device(d_y, (seq, d_out), np.float32)
    for p in (d_w, d_x, d_y):
        hip.free(p)
    if gtype == fa.F32:  # F32 weights take tensor::matmul (tensor.rs:74-80)
        return got, orc.matmul_f32(x, raw.view(np.float32).reshape(d_out, d_in))
    if gtype == fa.F16:  # widened exactly to f32, then as F32 weights
        return got, orc.matmul_f32(x, raw.view(np.float16).astype(np.float32).reshape(d_out, d_in))
    return got, orc.matmul_quant(x, raw, d_out, d_in, gtype)


# The single-op microbench shapes (Q4_K 8960x1536 and 1536x8960, Q6_K
# 1536x8960, Q8_0 1536x1536, Q6_K lm_head 151936x1536) plus the other
# decode shapes of the 0.5B/1.5B/7B models and odd-block rows.
@pytest.mark.parametrize("gtype,d_out,d_in", [
    (fa.Q4_K, 8960, 1536), (fa.Q4_K, 1536, 8960), (fa.Q6_K, 1536, 8960), (fa.Q8_0, 1536, 1536),
    (fa.Q6_K, 151936, 1536),
    (fa.Q4_K, 256, 1536), (fa.Q6_K, 256, 1536), (fa.Q8_0, 4864, 896), (fa.Q8_0, 896, 4864), (fa.Q8_0, 128, 896),
    (fa.Q4_K, 3584, 18944), (fa.Q6_K, 512, 3584),
    (fa.Q5_0, 1000, 1536), (fa.Q5_0, 100, 96), (fa.Q8_0, 100, 96), (fa.F32, 300, 512),
    (fa.F16, 1536, 1536), (fa.F16, 300, 512), (fa.F16, 100, 96)])
def test_gemv_within_tolerance(hip, gtype, d_out, d_in):
    got, ref = _gemv_case(hip, gtype, d_out, d_in, seed=d_out * 7 + d_in)
    assert rel_err(got, ref) <= GEMV_TOL


def test_matmul_multi_row(hip):
    got, ref = _gemv_case(hip, fa.Q4_K, 512, 1536, seed=9, seq=5)
    assert rel_err(got, ref) <= GEMV_TOL


def test_argmax_first_max_rule(hip):
    import ctypes
    lib = fa.load()
    cases = [np.array([1.0, 5.0, 5.0, 2.0], np.float32), np.array([-3.0, -1.0, -2.0], np.float32),
             np.random.default_rng(1).standard_normal(151936).astype(np.float32)]
    big = np.random.default_rng(2).standard_normal(300000).astype(np.float32)
    big[[1234, 250000]] = 9.0  # tie: first index wins
    cases.append(big)
    for x in cases:
        d_x, d_o = hip.to_device(x), hip.malloc(4)
        fa.check(lib.frn_argmax(d_x, x.size, d_o, None))
        got = int(hip.from_device(d_o, 1, np.uint32)[0])
        assert got == orc.argmax(x)
        hip.free(d_x)
        hip.free(d_o)
