"""The engine library loads, exports every entry point declared in
include/*.h, and rejects bad arguments before touching a device."""
import ctypes
import os
import re

import numpy as np
import pytest

import furnace_amd as fa

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared_symbols():
    names = set()
    for h in ("furnace_hip.h", "furnace_host.h"):
        text = open(os.path.join(ROOT, "include", h)).read()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        names |= set(re.findall(r"\b(frn_[a-z0-9_]+)\s*\(", text))
    return names


def test_every_declared_symbol_is_exported():
    lib = fa.load()
    decl = declared_symbols()
    assert len(decl) >= 25
    missing = [n for n in sorted(decl) if not hasattr(lib, n)]
    assert not missing, missing
    # and the Python binding covers exactly the declared set
    assert set(fa.SIGNATURES) == decl


def test_dequant_validates_before_launch():
    lib = fa.load()
    assert lib.frn_dequant(99, None, 0, 0, None, None) == 2  # EDTYPE
    assert lib.frn_dequant(fa.Q4_K, None, 144, 255, None, None) == 3  # not a multiple of 256
    assert lib.frn_dequant(fa.Q4_K, None, 143, 256, None, None) == 3  # byte count
    assert b"expected 144" in lib.frn_last_error()
    assert lib.frn_dequant(fa.Q8_0, None, 34, 32, None, None) == 1  # null pointers


def test_matmul_validates_before_launch():
    lib = fa.load()
    assert lib.frn_matmul_quant(2, None, 0, None, 1, None, 1, 32, None) == 2  # Q4_0: no kernel
    assert lib.frn_matmul_quant(fa.Q4_K, None, 144, None, 1, None, 1, 100, None) == 3
    assert lib.frn_matmul_quant(fa.Q4_K, None, 100, None, 1, None, 1, 256, None) == 3
    assert b"bad weight byte count" in lib.frn_last_error()


def test_context_calls_reject_null():
    lib = fa.load()
    nxt = ctypes.c_uint32()
    assert lib.frn_decode(None, 0, ctypes.byref(nxt)) == 1
    assert lib.frn_decode_greedy(None, 0, 4, None, 0, None, ctypes.byref(nxt)) == 1
    assert lib.frn_sampler_init(None, 0.7, 40, 0.9, 1.0, 7) == 1
    assert lib.frn_sample(None, None, 0, ctypes.byref(nxt)) == 1
    assert lib.frn_sampler_draws(None, None) == 1
    assert lib.frn_prefill(None, None, 0, ctypes.byref(nxt)) == 1
    assert lib.frn_finalize(None) == 1
    assert lib.frn_reset(None) == 1
    assert lib.frn_logits(None, None, 0) == 1
    lib.frn_destroy(None)


def test_create_rejects_bad_configs():
    lib = fa.load()
    ctx = ctypes.c_void_p()
    c = fa.Config(n_layers=1, n_heads=3, n_kv_heads=1, hidden=256, ffn=256, head_dim=64, vocab=10, max_ctx=8)
    assert lib.frn_create(ctypes.byref(c), 0, ctypes.byref(ctx)) == 3  # head_dim != hidden / heads
    c = fa.Config(n_layers=0, n_heads=4, n_kv_heads=1, hidden=256, ffn=256, head_dim=64, vocab=10, max_ctx=8)
    assert lib.frn_create(ctypes.byref(c), 0, ctypes.byref(ctx)) == 1
    c = fa.Config(n_layers=1, n_heads=4, n_kv_heads=3, hidden=256, ffn=256, head_dim=64, vocab=10, max_ctx=8)
    assert lib.frn_create(ctypes.byref(c), 0, ctypes.byref(ctx)) == 3


def test_create_without_device_reports_enodev():
    h = fa.Hip()
    if h.device_count() > 0:
        pytest.skip("a device is visible")
    lib = fa.load()
    ctx = ctypes.c_void_p()
    c = fa.Config(n_layers=1, n_heads=4, n_kv_heads=2, hidden=256, ffn=256, head_dim=64, vocab=10, max_ctx=8,
                  rope_theta=1e6, rms_eps=1e-6)
    assert lib.frn_create(ctypes.byref(c), 0, ctypes.byref(ctx)) == 8


def test_product_path_does_not_touch_the_oracle():
    # the product package must never load or mention the oracle
    pkg = os.path.join(ROOT, "furnace_amd")
    for dirpath, _, files in os.walk(pkg):
        for f in files:
            if f.endswith((".py", ".hip", ".hpp", ".cpp", ".h")):
                text = open(os.path.join(dirpath, f)).read()
                assert "oracle" not in text and "liboracle" not in text, f
