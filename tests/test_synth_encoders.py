"""The synthetic-model encoders produce blocks the CPU path decodes back to
the input within each format's step size."""
import numpy as np
import pytest

import furnace_amd as fa
from oracle import oracle as orc


@pytest.mark.parametrize("gtype,rel", [(fa.Q8_0, 1 / 127), (fa.Q5_0, 1 / 15), (fa.Q4_K, 1 / 7), (fa.Q6_K, 1 / 30)])
def test_encode_decode_roundtrip(gtype, rel):
    be, _ = fa.BLOCK[gtype]
    x = fa.gaussian(11, 0.02, 64 * be)
    raw = fa.quantize(gtype, x)
    y = orc.dequantize(gtype, raw, x.size)
    blocks = np.abs(x).reshape(-1, be).max(1, keepdims=True)
    err = np.abs(y - x).reshape(-1, be)
    # within about one quantization step of the block's range
    assert np.all(err <= 1.05 * rel * blocks + 1e-7)
    # and clearly better than nothing: correlation with the input
    assert np.corrcoef(x, y)[0, 1] > 0.97


def test_f16_encoder_rounds_to_nearest_even():
    # IEEE binary16 round-to-nearest-even, as numpy's float32 -> float16 cast
    # (normals, subnormals, overflow to inf, signed zero, ties)
    rng = np.random.default_rng(3)
    x = np.concatenate([
        fa.gaussian(12, 0.02, 4096),
        rng.uniform(-70000, 70000, 1024).astype(np.float32),
        np.float32(2.0 ** -24) * rng.uniform(-3, 3, 512).astype(np.float32),
        np.array([0.0, -0.0, 65504.0, 65520.0, 65519.0, -1e9, 1 + 2 ** -11, 1 + 3 * 2 ** -11], np.float32),
    ]).astype(np.float32)
    raw = fa.quantize(fa.F16, x)
    with np.errstate(over="ignore"):
        want = x.astype("<f2")
    assert raw.tobytes() == want.tobytes()


def test_gaussian_statistics():
    x = fa.gaussian(5, 0.02, 1 << 18)
    assert abs(x.mean()) < 2e-4 and abs(x.std() - 0.02) < 2e-4
    assert np.array_equal(fa.gaussian(5, 0.02, 1000), x[:1000])
