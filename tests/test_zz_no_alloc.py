"""frn_argmax_noalloc (include/furnace_hip.h: frn_argmax without allocation,
its running key in a static per-device array) against frn_argmax and the
oracle's argmax (generate.rs:69-77): two calls in a row, the second on a
smaller input whose maximum lies below the first call's, so a key left over
from the first call would win if it were not cleared."""
import numpy as np
import pytest

import furnace_amd as fa
from oracle import oracle as orc

pytestmark = pytest.mark.gpu


def _run(hip, lib, fn, x):
    d_x, d_o = hip.to_device(x), hip.malloc(4)
    try:
        fa.check(fn(d_x, x.size, d_o, None))
        return int(hip.from_device(d_o, 1, np.uint32)[0])
    finally:
        hip.free(d_x)
        hip.free(d_o)


def test_noalloc_argmax_matches_allocating_entry_point(hip):
    lib = fa.load()
    rng = np.random.default_rng(77)
    first = rng.standard_normal(151936).astype(np.float32)
    first[[100000, 140000]] = 50.0  # tie far past the second input's end: first index wins
    second = rng.standard_normal(1000).astype(np.float32)  # all far below 50
    second[[17, 600]] = 4.5
    third = np.array([np.nan, 1.0, 2.0], np.float32)  # NaN at index 0 wins (strict > never replaces it)
    for i, x in enumerate((first, second, third)):
        print("noalloc argmax call %d, n=%d" % (i, x.size), flush=True)
        want = orc.argmax(x)
        got_alloc = _run(hip, lib, lib.frn_argmax, x)
        got_static = _run(hip, lib, lib.frn_argmax_noalloc, x)
        assert got_alloc == want
        assert got_static == want
    assert orc.argmax(first) == 100000 and orc.argmax(second) == 17


def test_noalloc_argmax_rejects_bad_arguments(hip):
    lib = fa.load()
    d_o = hip.malloc(4)
    try:
        assert lib.frn_argmax_noalloc(None, 10, d_o, None) != 0
        assert lib.frn_argmax_noalloc(d_o, 0, d_o, None) != 0
        assert lib.frn_argmax_noalloc(d_o, 1 << 32, d_o, None) == 3  # FRN_ESHAPE
    finally:
        hip.free(d_o)
