"""GGUF parsing: the product reader (frn_gguf_*) and the oracle's, against
the hand-assembled file of furnace's src/gguf.rs:532-609 and its negative
tests (bad magic, truncation), plus the synthetic writer's output."""
import ctypes
import os
import struct

import numpy as np
import pytest

import furnace_amd as fa
from oracle import oracle as orc


def _s(b):
    return struct.pack("<Q", len(b)) + b


def synthetic_file():  # gguf.rs:532-564
    b = b"GGUF" + struct.pack("<IQQ", 3, 1, 3)
    b += _s(b"general.architecture") + struct.pack("<I", 8) + _s(b"qwen2")
    b += _s(b"qwen2.rope.freq_base") + struct.pack("<If", 6, 1e6)
    b += _s(b"tokenizer.ggml.tokens") + struct.pack("<IIQ", 9, 8, 2) + _s(b"a") + _s(b"b")
    b += _s(b"blk.0.attn_q.weight") + struct.pack("<IQQIQ", 2, 896, 896, 8, 0)
    b += b"\x00" * ((32 - len(b) % 32) % 32)
    return b + b"\xab" * 64


def _open(path):
    g = ctypes.c_void_p()
    st = fa.load().frn_gguf_open(path.encode(), ctypes.byref(g))
    return st, g


def test_parses_synthetic_file(tmp_path):  # gguf.rs:566-596
    p = tmp_path / "s.gguf"
    data = synthetic_file()
    p.write_bytes(data)
    st, g = _open(str(p))
    assert st == 0, fa.load().frn_last_error()
    try:
        t, nd, ptr, nb = ctypes.c_uint32(), ctypes.c_uint32(), ctypes.c_void_p(), ctypes.c_size_t()
        dims = (ctypes.c_uint64 * 4)()
        # the tensor is declared Q8_0 896x896 but the blob is 64 bytes: the
        # slice must be refused (gguf.rs:420-432)
        st = fa.load().frn_gguf_tensor(g, b"blk.0.attn_q.weight", ctypes.byref(t), dims, ctypes.byref(nd),
                                       ctypes.byref(ptr), ctypes.byref(nb))
        assert st != 0 and b"past end of file" in fa.load().frn_last_error()
        assert fa.load().frn_gguf_tensor(g, b"missing", None, None, None, None, None) != 0
        # metadata: a float is not a u32
        v = ctypes.c_uint32()
        assert fa.load().frn_gguf_meta_u32(g, b"qwen2.rope.freq_base", ctypes.byref(v)) != 0
    finally:
        fa.load().frn_gguf_close(g)


def test_rejects_bad_magic(tmp_path):  # gguf.rs:598-602
    p = tmp_path / "bad.gguf"
    p.write_bytes(b"GGML\x03\x00\x00\x00")
    st, _ = _open(str(p))
    assert st != 0 and b"bad magic" in fa.load().frn_last_error()
    assert orc.lib().orc_model_load(str(p).encode()) is None
    assert "bad magic" in orc.err()


def test_rejects_truncated_file(tmp_path):  # gguf.rs:604-609
    p = tmp_path / "t.gguf"
    p.write_bytes(synthetic_file()[:40])
    st, _ = _open(str(p))
    assert st != 0 and b"EOF" in fa.load().frn_last_error()
    assert orc.lib().orc_model_load(str(p).encode()) is None
    assert "EOF" in orc.err()


def test_rejects_bad_version_and_alignment(tmp_path):
    p = tmp_path / "v.gguf"
    p.write_bytes(b"GGUF" + struct.pack("<IQQ", 1, 0, 0))
    st, _ = _open(str(p))
    assert st != 0 and b"version" in fa.load().frn_last_error()
    b = b"GGUF" + struct.pack("<IQQ", 3, 0, 1) + _s(b"general.alignment") + struct.pack("<II", 4, 48)
    p.write_bytes(b)
    st, _ = _open(str(p))
    assert st != 0 and b"power of two" in fa.load().frn_last_error()


def test_synthetic_writer_roundtrip(tmp_path):
    p = str(tmp_path / "m.gguf")
    fa.synth_write(p, seed=7, n_layers=2, n_heads=4, n_kv_heads=2, hidden=256, ffn=512, vocab=300,
                   mix=fa.MIX_Q4_K_M, tied=0, embd_type=fa.Q4_K, output_type=fa.Q6_K)
    st, g = _open(p)
    assert st == 0
    cfg, ctx_len = fa.Config(), ctypes.c_uint32()
    assert fa.load().frn_gguf_config(g, ctypes.byref(cfg), ctypes.byref(ctx_len)) == 0
    assert (cfg.n_layers, cfg.n_heads, cfg.n_kv_heads, cfg.hidden, cfg.ffn, cfg.head_dim, cfg.vocab) == \
        (2, 4, 2, 256, 512, 64, 300)
    assert abs(cfg.rope_theta - 1e6) < 1 and abs(cfg.rms_eps - 1e-6) < 1e-12 and cfg.tied_lm_head == 0
    fa.load().frn_gguf_close(g)
    m = orc.Model(p)
    # Q4_K_M mix: Q6_K attn_v / ffn_down on even layers, Q4_K elsewhere
    assert m.tensor("blk.0.attn_v.weight")[0] == orc.Q6_K and m.tensor("blk.1.attn_v.weight")[0] == orc.Q4_K
    assert m.tensor("blk.0.ffn_down.weight")[0] == orc.Q6_K and m.tensor("blk.1.ffn_down.weight")[0] == orc.Q4_K
    assert m.tensor("blk.0.attn_q.weight")[0] == orc.Q4_K and m.tensor("output.weight")[0] == orc.Q6_K
    t, dims, raw = m.tensor("blk.1.ffn_down.weight")
    assert dims == [512, 256]
    assert m.tensor("blk.0.attn_norm.weight")[2].view(np.float32).tolist() == [1.0] * 256
    m.close()


def test_synthetic_writer_is_deterministic(tmp_path):
    a, b = str(tmp_path / "a.gguf"), str(tmp_path / "b.gguf")
    kw = dict(n_layers=1, n_heads=2, n_kv_heads=1, hidden=256, ffn=256, vocab=64, mix=fa.MIX_ALL_Q8_0, tied=1,
              embd_type=fa.Q8_0, output_type=fa.Q8_0)
    fa.synth_write(a, seed=3, threads=1, **kw)
    fa.synth_write(b, seed=3, threads=4, **kw)
    assert open(a, "rb").read() == open(b, "rb").read()
    fa.synth_write(b, seed=4, **kw)
    assert open(a, "rb").read() != open(b, "rb").read()


def test_llama_cpp_q4_k_m_layer_mix(tmp_path):
    # llama.cpp's Q4_K_M (use_more_bits): Q6_K attn_v / ffn_down on layers
    # i < n/8, i >= 7n/8 and (i - n/8) % 3 == 2; with n = 16 that is
    # 0, 1, 4, 7, 10, 13, 14, 15
    path = str(tmp_path / "llama-mix.gguf")
    fa.synth_write(path, seed=3, n_layers=16, n_heads=2, n_kv_heads=1, hidden=256, ffn=256, vocab=300,
                   mix=fa.MIX_Q4_K_M_LLAMA, tied=0, embd_type=fa.Q4_K, output_type=fa.Q6_K)
    m = orc.Model(path)
    more = {0, 1, 4, 7, 10, 13, 14, 15}
    for layer in range(16):
        for name in ("attn_v", "ffn_down"):
            t, _, _ = m.tensor("blk.%d.%s.weight" % (layer, name))
            assert t == (fa.Q6_K if layer in more else fa.Q4_K), (layer, name)
        for name in ("attn_q", "attn_k", "attn_output", "ffn_gate", "ffn_up"):
            assert m.tensor("blk.%d.%s.weight" % (layer, name))[0] == fa.Q4_K
    assert m.tensor("output.weight")[0] == fa.Q6_K
    m.close()


@pytest.mark.parametrize("align", [64, 256, 4096])
def test_general_alignment_moves_the_data(tmp_path, align):  # gguf.rs:344-354
    # the same tensors written with the default and with a larger
    # general.alignment: both loaders must find identical bytes in both
    # files, at offsets that follow the alignment
    kw = dict(n_layers=1, n_heads=2, n_kv_heads=1, hidden=256, ffn=288, vocab=70, mix=fa.MIX_ALL_Q5_0, tied=0,
              embd_type=fa.Q8_0, output_type=fa.Q6_K)
    a, b = str(tmp_path / "a.gguf"), str(tmp_path / ("b%d.gguf" % align))
    fa.synth_write(a, seed=9, **kw)
    fa.synth_write(b, seed=9, alignment=align, **kw)
    assert os.path.getsize(b) > os.path.getsize(a)
    names = ["token_embd.weight", "blk.0.attn_q.bias", "blk.0.attn_v.weight", "blk.0.ffn_norm.weight",
             "blk.0.ffn_down.weight", "output.weight"]
    ma, mb = orc.Model(a), orc.Model(b)
    st, g = _open(b)
    assert st == 0, fa.load().frn_last_error()
    try:
        for name in names:
            ta, mb_t = ma.tensor(name), mb.tensor(name)
            assert ta[0] == mb_t[0] and ta[1] == mb_t[1] and np.array_equal(ta[2], mb_t[2]), name
            t, nd, ptr, nb = ctypes.c_uint32(), ctypes.c_uint32(), ctypes.c_void_p(), ctypes.c_size_t()
            dims = (ctypes.c_uint64 * 4)()
            assert fa.load().frn_gguf_tensor(g, name.encode(), ctypes.byref(t), dims, ctypes.byref(nd),
                                             ctypes.byref(ptr), ctypes.byref(nb)) == 0
            assert ptr.value % align == 0, name  # the file is mapped at a page boundary
            got = np.ctypeslib.as_array(ctypes.cast(ptr, ctypes.POINTER(ctypes.c_uint8)), (nb.value,))
            assert np.array_equal(got, ta[2].view(np.uint8)), name
    finally:
        fa.load().frn_gguf_close(g)
        ma.close()
        mb.close()
    with pytest.raises(fa.FrnError, match="power of two"):
        fa.synth_write(str(tmp_path / "c.gguf"), seed=9, alignment=48, **kw)
