"""ctypes view of oracle/liboracle.so -- test infrastructure only.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg import
this module, as the test oracle.  The product (furnace_amd/) never does.
"""
import ctypes
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")

F32, F16, Q5_0, Q8_0, Q4_K, Q6_K = 0, 1, 6, 8, 12, 14
BLOCK = {F32: (1, 4), F16: (1, 2), Q5_0: (32, 22), Q8_0: (32, 34), Q4_K: (256, 144), Q6_K: (256, 210)}


class Config(ctypes.Structure):
    _fields_ = [(n, ctypes.c_uint32) for n in
                ("n_layers", "n_heads", "n_kv_heads", "hidden", "ffn", "head_dim", "vocab", "context_length")] + \
               [("rope_theta", ctypes.c_float), ("rms_eps", ctypes.c_float)]


class F32Layer(ctypes.Structure):
    _fields_ = [(n, ctypes.c_void_p) for n in
                ("attn_norm", "wq", "bq", "wk", "bk", "wv", "bv", "wo", "ffn_norm", "w_gate", "w_up", "w_down")]


class Pcg32State(ctypes.Structure):
    _fields_ = [("state", ctypes.c_uint64), ("inc", ctypes.c_uint64)]


class SamplerState(ctypes.Structure):
    _fields_ = [("temperature", ctypes.c_float), ("top_k", ctypes.c_uint32), ("top_p", ctypes.c_float),
                ("repeat_penalty", ctypes.c_float), ("repeat_window", ctypes.c_uint32), ("rng", Pcg32State),
                ("draws", ctypes.c_uint64)]


_P, _SZ, _U32, _F = ctypes.c_void_p, ctypes.c_size_t, ctypes.c_uint32, ctypes.c_float
_SIG = {
    "orc_set_f16_extension": (None, [ctypes.c_int]),
    "orc_pcg32_seed": (None, [ctypes.POINTER(Pcg32State), ctypes.c_uint64, ctypes.c_uint64]),
    "orc_pcg32_next_u32": (_U32, [ctypes.POINTER(Pcg32State)]),
    "orc_pcg32_next_f32": (_F, [ctypes.POINTER(Pcg32State)]),
    "orc_apply_repeat_penalty": (None, [_P, _P, _SZ, _F]),
    "orc_sampler_new": (None, [ctypes.POINTER(SamplerState), _F, _U32, _F, _F, ctypes.c_uint64]),
    "orc_sampler_filtered": (_SZ, [ctypes.POINTER(SamplerState), _P, _SZ, _P, _P]),
    "orc_sampler_sample": (_U32, [ctypes.POINTER(SamplerState), _P, _SZ, _P, _SZ]),
    "orc_f16_to_f32": (ctypes.c_float, [ctypes.c_uint16]),
    "orc_dequantize": (ctypes.c_int, [_U32, _P, _SZ, _SZ, _P]),
    "orc_matmul_quant": (ctypes.c_int, [_P, _SZ, _P, _SZ, _SZ, _SZ, _U32, _P]),
    "orc_matmul_f32": (None, [_P, _SZ, _P, _SZ, _SZ, _P]),
    "orc_dot": (ctypes.c_float, [_P, _P, _SZ]),
    "orc_rmsnorm": (None, [_P, _SZ, _SZ, _P, _F, _P]),
    "orc_softmax": (None, [_P, _SZ, _SZ]),
    "orc_silu": (None, [_P, _SZ, _P]),
    "orc_swiglu": (None, [_P, _P, _SZ, _P]),
    "orc_add": (None, [_P, _P, _SZ, _P]),
    "orc_rope": (None, [_P, _SZ, _SZ, _SZ, _F, _SZ]),
    "orc_attention_scores": (None, [_P, _P, _SZ, _SZ, _SZ, _SZ, _P]),
    "orc_attention_apply": (None, [_P, _P, _SZ, _SZ, _SZ, _SZ, _P]),
    "orc_argmax": (_U32, [_P, _SZ]),
    "orc_model_load": (_P, [ctypes.c_char_p]),
    "orc_model_free": (None, [_P]),
    "orc_model_get_config": (ctypes.c_int, [_P, ctypes.POINTER(Config)]),
    "orc_model_meta_u32": (ctypes.c_int64, [_P, ctypes.c_char_p]),
    "orc_model_tensor": (ctypes.c_int, [_P, ctypes.c_char_p, ctypes.POINTER(_U32), ctypes.POINTER(ctypes.c_uint64),
                                        ctypes.POINTER(_U32), ctypes.POINTER(_P), ctypes.POINTER(_SZ)]),
    "orc_model_param_bytes": (_SZ, [_P]),
    "orc_cache_new": (_P, [_P, _SZ]),
    "orc_cache_free": (None, [_P]),
    "orc_cache_len": (_SZ, [_P]),
    "orc_cache_read": (ctypes.c_int, [_P, _SZ, ctypes.c_int, _SZ, _P]),
    "orc_forward_cached": (ctypes.c_int, [_P, _P, _P, _SZ, _P]),
    "orc_forward_cached_hidden": (ctypes.c_int, [_P, _P, _P, _SZ, _P]),
    "orc_forward_last": (ctypes.c_int, [_P, _P, _SZ, _P]),
    "orc_generate_greedy": (ctypes.c_long, [_P, _P, _SZ, _SZ, _SZ, _P, _SZ, _P, ctypes.POINTER(ctypes.c_double),
                                            ctypes.POINTER(ctypes.c_double), ctypes.POINTER(_SZ), _P]),
    "orc_set_threads": (None, [ctypes.c_int]),
    "orc_get_threads": (ctypes.c_int, []),
    "orc_last_error": (ctypes.c_char_p, []),
    "orc_layer_forward_f32": (None, [_P, _SZ, ctypes.POINTER(F32Layer), ctypes.POINTER(Config), _P]),
    "orc_layer_forward_cached_f32": (None, [_P, _SZ, ctypes.POINTER(F32Layer), ctypes.POINTER(Config), _P, _P, _SZ,
                                            _SZ, _P]),
}

_lib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise ImportError("oracle: %s is missing; run `make -C oracle`" % LIB_PATH)
        l = ctypes.CDLL(LIB_PATH)
        for n, (r, a) in _SIG.items():
            f = getattr(l, n)
            f.restype, f.argtypes = r, a
        _lib = l
    return _lib


def _p(a):
    return ctypes.c_void_p(a.ctypes.data)


def f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


def err():
    return lib().orc_last_error().decode()


def dequantize(gtype, raw, n):
    raw = np.ascontiguousarray(np.frombuffer(bytes(raw), dtype=np.uint8) if not isinstance(raw, np.ndarray) else raw,
                               dtype=np.uint8)
    out = np.empty(n, dtype=np.float32)
    if lib().orc_dequantize(gtype, _p(raw), raw.size, n, _p(out)) != 0:
        raise ValueError(err())
    return out


def matmul_quant(a, raw, d_out, d_in, gtype):
    a = f32(a).reshape(-1, d_in)
    raw = np.ascontiguousarray(raw, dtype=np.uint8)
    out = np.empty((a.shape[0], d_out), dtype=np.float32)
    if lib().orc_matmul_quant(_p(a), a.shape[0], _p(raw), raw.size, d_out, d_in, gtype, _p(out)) != 0:
        raise ValueError(err())
    return out


def matmul_f32(a, w):
    a, w = f32(a), f32(w)
    out = np.empty((a.shape[0], w.shape[0]), dtype=np.float32)
    lib().orc_matmul_f32(_p(a), a.shape[0], _p(w), w.shape[0], w.shape[1], _p(out))
    return out


def dot(a, b):
    a, b = f32(a), f32(b)
    return lib().orc_dot(_p(a), _p(b), a.size)


def rmsnorm(x, w, eps):
    x, w = f32(x), f32(w)
    out = np.empty_like(x)
    rows = x.size // x.shape[-1]
    lib().orc_rmsnorm(_p(x), rows, x.shape[-1], _p(w), eps, _p(out))
    return out


def softmax(x):
    x = f32(x).copy()
    lib().orc_softmax(_p(x), x.size // x.shape[-1], x.shape[-1])
    return x


def silu(x):
    x = f32(x)
    out = np.empty_like(x)
    lib().orc_silu(_p(x), x.size, _p(out))
    return out


def swiglu(g, u):
    g, u = f32(g), f32(u)
    out = np.empty_like(g)
    lib().orc_swiglu(_p(g), _p(u), g.size, _p(out))
    return out


def add(a, b):
    a, b = f32(a), f32(b)
    out = np.empty_like(a)
    lib().orc_add(_p(a), _p(b), a.size, _p(out))
    return out


def rope(x, n_heads, head_dim, theta, start_pos):
    x = f32(x).copy()
    lib().orc_rope(_p(x), x.shape[0], n_heads, head_dim, theta, start_pos)
    return x


def attention_scores(q, k, n_heads, n_kv_heads, head_dim):
    q, k = f32(q), f32(k)
    seq = q.shape[0]
    out = np.empty((n_heads, seq, seq), dtype=np.float32)
    lib().orc_attention_scores(_p(q), _p(k), seq, n_heads, n_kv_heads, head_dim, _p(out))
    return out


def attention_apply(probs, v, n_heads, n_kv_heads, head_dim):
    probs, v = f32(probs), f32(v)
    seq = v.shape[0]
    out = np.empty((seq, n_heads * head_dim), dtype=np.float32)
    lib().orc_attention_apply(_p(probs), _p(v), seq, n_heads, n_kv_heads, head_dim, _p(out))
    return out


class Pcg32:
    """Pcg32 (sampler.rs:5-35); seed(initstate, initseq) is O'Neill's
    pcg32_srandom_r, and Pcg32(seed) the reference's Pcg32::new(seed)."""

    def __init__(self, seed=None, initseq=0xda3e39cb94b95bdb):
        self.st = Pcg32State()
        if seed is not None:
            lib().orc_pcg32_seed(ctypes.byref(self.st), seed, initseq)

    def next_u32(self):
        return lib().orc_pcg32_next_u32(ctypes.byref(self.st))

    def next_f32(self):
        return lib().orc_pcg32_next_f32(ctypes.byref(self.st))


def apply_repeat_penalty(logits, recent, penalty):
    x = f32(logits).copy()
    r = np.ascontiguousarray(recent, dtype=np.uint32)
    lib().orc_apply_repeat_penalty(_p(x), _p(r) if r.size else None, r.size, penalty)
    return x


class Sampler:
    """Sampler (sampler.rs:57-155)."""

    def __init__(self, temperature, top_k, top_p, repeat_penalty=1.0, seed=7):
        self.st = SamplerState()
        lib().orc_sampler_new(ctypes.byref(self.st), temperature, top_k, top_p, repeat_penalty, seed)

    @property
    def draws(self):
        return self.st.draws

    def filtered(self, logits):
        x = f32(logits)
        ids = np.empty(x.size, dtype=np.uint32)
        pr = np.empty(x.size, dtype=np.float32)
        n = lib().orc_sampler_filtered(ctypes.byref(self.st), _p(x), x.size, _p(ids), _p(pr))
        return ids[:n], pr[:n]

    def sample(self, logits, recent=()):
        x = f32(logits)
        r = np.ascontiguousarray(recent, dtype=np.uint32)
        return int(lib().orc_sampler_sample(ctypes.byref(self.st), _p(x), x.size, _p(r) if r.size else None, r.size))


def argmax(x):
    x = f32(x)
    return lib().orc_argmax(_p(x), x.size)


def set_threads(n):
    lib().orc_set_threads(int(n))


class f16_extension:
    """Context manager: F16 tensors widen exactly to f32 inside it (the
    engine's F16 support, which the reference does not have: quant.rs:279);
    outside it F16 is the reference's "not implemented" error."""

    def __enter__(self):
        lib().orc_set_f16_extension(1)
        return self

    def __exit__(self, *exc):
        lib().orc_set_f16_extension(0)
        return False


class Model:
    """Model::load over a GGUF file, plus its KvCache (model.rs:321-592)."""

    def __init__(self, path):
        self.h = lib().orc_model_load(path.encode())
        if not self.h:
            raise ValueError(err())
        self.cfg = Config()
        lib().orc_model_get_config(self.h, ctypes.byref(self.cfg))
        self.cache = None

    def meta_u32(self, key):
        v = lib().orc_model_meta_u32(self.h, key.encode())
        return None if v < 0 else int(v)

    def stop_ids(self):
        return [v for v in (self.meta_u32("tokenizer.ggml.eos_token_id"),
                            self.meta_u32("tokenizer.ggml.bos_token_id")) if v is not None]

    def tensor(self, name):
        t, nd, p, b = ctypes.c_uint32(), ctypes.c_uint32(), ctypes.c_void_p(), ctypes.c_size_t()
        dims = (ctypes.c_uint64 * 4)()
        if lib().orc_model_tensor(self.h, name.encode(), ctypes.byref(t), dims, ctypes.byref(nd), ctypes.byref(p),
                                  ctypes.byref(b)) != 0:
            raise ValueError(err())
        raw = np.ctypeslib.as_array((ctypes.c_uint8 * b.value).from_address(p.value)).copy()
        return t.value, [dims[i] for i in range(nd.value)], raw

    def new_cache(self, max_ctx):
        if self.cache:
            lib().orc_cache_free(self.cache)
        self.cache = lib().orc_cache_new(self.h, max_ctx)
        if not self.cache:
            raise ValueError(err())

    def forward_cached(self, tokens):
        t = np.ascontiguousarray(tokens, dtype=np.uint32)
        out = np.empty(self.cfg.vocab, dtype=np.float32)
        if lib().orc_forward_cached(self.h, self.cache, _p(t), t.size, _p(out)) != 0:
            raise ValueError(err())
        return out

    def forward_last(self, tokens):
        t = np.ascontiguousarray(tokens, dtype=np.uint32)
        out = np.empty(self.cfg.vocab, dtype=np.float32)
        if lib().orc_forward_last(self.h, _p(t), t.size, _p(out)) != 0:
            raise ValueError(err())
        return out

    def cache_read(self, layer, which_v, n):
        kvd = self.cfg.n_kv_heads * self.cfg.head_dim
        out = np.empty((n, kvd), dtype=np.float32)
        if lib().orc_cache_read(self.cache, layer, 1 if which_v else 0, n, _p(out)) != 0:
            raise ValueError(err())
        return out

    def generate_greedy(self, prompt, max_new, max_ctx, stop_ids=None):
        p = np.ascontiguousarray(prompt, dtype=np.uint32)
        stop = np.ascontiguousarray(self.stop_ids() if stop_ids is None else stop_ids, dtype=np.uint32)
        out = np.zeros(max(max_new, 1), dtype=np.uint32)
        pf, dc, steps = ctypes.c_double(), ctypes.c_double(), ctypes.c_size_t()
        logits = np.empty(self.cfg.vocab, dtype=np.float32)
        n = lib().orc_generate_greedy(self.h, _p(p), p.size, max_new, max_ctx, _p(stop) if stop.size else None,
                                      stop.size, _p(out), ctypes.byref(pf), ctypes.byref(dc), ctypes.byref(steps),
                                      _p(logits))
        if n < 0:
            raise ValueError(err())
        return out[:n].tolist(), dict(prefill_s=pf.value, decode_s=dc.value, decode_steps=steps.value), logits

    def close(self):
        if self.cache:
            lib().orc_cache_free(self.cache)
            self.cache = None
        if self.h:
            lib().orc_model_free(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
