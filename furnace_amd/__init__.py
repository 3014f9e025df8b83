"""furnace_amd: MI355X (gfx950) engine for furnace's token loop.

Python view of the C ABI in include/furnace_hip.h and include/furnace_host.h,
through ctypes.  The compute path is the HIP library built by
furnace_amd/_build.py; importing this package never falls back to a CPU
implementation -- if the library is missing, load() raises.
"""
import ctypes
import os

import numpy as np

_PKG = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_PKG, "lib", "libfurnace_hip.so")
CLI_PATH = os.path.join(_PKG, "bin", "furnace-hip")

# ggml type codes (src/gguf.rs:180-201)
F32, F16, Q5_0, Q8_0, Q4_K, Q6_K = 0, 1, 6, 8, 12, 14
BLOCK = {F32: (1, 4), F16: (1, 2), Q5_0: (32, 22), Q8_0: (32, 34), Q4_K: (256, 144), Q6_K: (256, 210)}

FLAG_EAGER = 1  # FRN_FLAG_EAGER
FLAG_STEPWISE_PREFILL = 2  # FRN_FLAG_STEPWISE_PREFILL
FLAG_NO_RESIDENT = 4  # FRN_FLAG_NO_RESIDENT
FLAG_RESIDENT = 8  # FRN_FLAG_RESIDENT

MIX_ALL_Q8_0, MIX_Q4_K_M, MIX_ALL_Q4_K, MIX_ALL_Q6_K, MIX_ALL_Q5_0, MIX_ALL_F32, MIX_Q4_K_M_LLAMA, MIX_ALL_F16 = range(8)

STATUS = {0: "FRN_OK", 1: "FRN_EINVAL", 2: "FRN_EDTYPE", 3: "FRN_ESHAPE", 4: "FRN_ECTX_OVERFLOW",
          5: "FRN_ETOKEN", 6: "FRN_EOOM", 7: "FRN_EHIP", 8: "FRN_ENODEV"}


class FrnError(RuntimeError):
    def __init__(self, status, msg):
        super().__init__("%s: %s" % (STATUS.get(status, status), msg))
        self.status = status


class Config(ctypes.Structure):
    _fields_ = [(n, ctypes.c_uint32) for n in
                ("n_layers", "n_heads", "n_kv_heads", "hidden", "ffn", "head_dim", "vocab", "max_ctx")] + \
               [("rope_theta", ctypes.c_float), ("rms_eps", ctypes.c_float),
                ("tied_lm_head", ctypes.c_uint32), ("flags", ctypes.c_uint32)]


class GenStats(ctypes.Structure):
    _fields_ = [("prefill_s", ctypes.c_double), ("decode_s", ctypes.c_double),
                ("decode_steps", ctypes.c_uint32), ("n_generated", ctypes.c_uint32)]


class SynthSpec(ctypes.Structure):
    _fields_ = [(n, ctypes.c_uint32) for n in
                ("n_layers", "n_heads", "n_kv_heads", "hidden", "ffn", "vocab", "context_length")] + \
               [("rope_theta", ctypes.c_float), ("rms_eps", ctypes.c_float)] + \
               [(n, ctypes.c_uint32) for n in ("mix", "tied", "embd_type", "output_type")] + \
               [("seed", ctypes.c_uint64), ("weight_std", ctypes.c_float), ("threads", ctypes.c_uint32),
                ("alignment", ctypes.c_uint32)]


class Timing(ctypes.Structure):
    _fields_ = [("name", ctypes.c_char * 16), ("ms", ctypes.c_double), ("calls", ctypes.c_uint64)]


# Every entry point of include/furnace_hip.h and include/furnace_host.h.
_P, _U32, _U64, _SZ, _I, _F = (ctypes.c_void_p, ctypes.c_uint32, ctypes.c_uint64, ctypes.c_size_t,
                                ctypes.c_int, ctypes.c_float)
SIGNATURES = {
    "frn_create": (_I, [ctypes.POINTER(Config), _I, ctypes.POINTER(_P)]),
    "frn_upload": (_I, [_P, ctypes.c_char_p, _U32, _U64, _U64, _P, _SZ]),
    "frn_finalize": (_I, [_P]),
    "frn_prefill": (_I, [_P, _P, _U32, ctypes.POINTER(_U32)]),
    "frn_decode": (_I, [_P, _U32, ctypes.POINTER(_U32)]),
    "frn_decode_greedy": (_I, [_P, _U32, _U32, _P, _U32, _P, ctypes.POINTER(_U32)]),
    "frn_decode_engine": (_I, [_P, ctypes.POINTER(_U32), ctypes.c_char_p, _SZ]),
    "frn_resident_trace": (_I, [_P, _U32, _P, _SZ]),
    "frn_sampler_init": (_I, [_P, ctypes.c_float, _U32, ctypes.c_float, ctypes.c_float, ctypes.c_uint64]),
    "frn_sample": (_I, [_P, _P, _U32, ctypes.POINTER(_U32)]),
    "frn_sampler_draws": (_I, [_P, ctypes.POINTER(ctypes.c_uint64)]),
    "frn_logits": (_I, [_P, _P, _SZ]),
    "frn_reset": (_I, [_P]),
    "frn_cache_len": (_I, [_P, ctypes.POINTER(_U32)]),
    "frn_cache_read": (_I, [_P, _U32, _U32, _U32, _P]),
    "frn_destroy": (None, [_P]),
    "frn_last_error": (ctypes.c_char_p, []),
    "frn_timings_enable": (_I, [_P, _I]),
    "frn_timings_reset": (_I, [_P]),
    "frn_step_times_enable": (_I, [_P, ctypes.c_int]),
    "frn_step_times": (_I, [_P, _P, _U32, ctypes.POINTER(_U32)]),
    "frn_timings": (_I, [_P, ctypes.POINTER(Timing), _U32, ctypes.POINTER(_U32)]),
    "frn_bench_kernel": (_I, [_P, ctypes.c_char_p, _U32, _U32, ctypes.POINTER(ctypes.c_float)]),
    "frn_dequant": (_I, [_U32, _P, _SZ, _SZ, _P, _P]),
    "frn_matmul_quant": (_I, [_U32, _P, _SZ, _P, _U32, _P, _U32, _U32, _P]),
    "frn_argmax": (_I, [_P, _SZ, _P, _P]),
    "frn_argmax_noalloc": (_I, [_P, _SZ, _P, _P]),
    "frn_gguf_open": (_I, [ctypes.c_char_p, ctypes.POINTER(_P)]),
    "frn_gguf_close": (None, [_P]),
    "frn_gguf_config": (_I, [_P, ctypes.POINTER(Config), ctypes.POINTER(_U32)]),
    "frn_gguf_meta_u32": (_I, [_P, ctypes.c_char_p, ctypes.POINTER(_U32)]),
    "frn_gguf_tensor": (_I, [_P, ctypes.c_char_p, ctypes.POINTER(_U32), ctypes.POINTER(_U64),
                             ctypes.POINTER(_U32), ctypes.POINTER(_P), ctypes.POINTER(_SZ)]),
    "frn_model_load": (_I, [_P, _I, _U32, _U32, ctypes.POINTER(_P)]),
    "frn_generate_greedy": (_I, [_P, _P, _U32, _U32, _P, _U32, _P, ctypes.POINTER(GenStats)]),
    "frn_generate_sampled": (_I, [_P, _P, _U32, _U32, ctypes.c_float, _U32, ctypes.c_float, ctypes.c_float,
                                  ctypes.c_uint64, _P, _U32, _P, ctypes.POINTER(GenStats),
                                  ctypes.POINTER(ctypes.c_uint64)]),
    "frn_synth_write": (_I, [ctypes.POINTER(SynthSpec), ctypes.c_char_p]),
    "frn_quantize": (_I, [_U32, _P, _SZ, _P]),
    "frn_gaussian": (_I, [_U64, _F, _SZ, _P]),
}

_lib = None


def load():
    """Load the engine library (raises if it has not been built)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise ImportError("furnace_amd: %s is missing; run __graft_entry__.build()" % LIB_PATH)
        lib = ctypes.CDLL(LIB_PATH, mode=ctypes.RTLD_GLOBAL)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        _lib = lib
    return _lib


def check(status):
    if status != 0:
        raise FrnError(status, load().frn_last_error().decode(errors="replace"))


def _ptr(a):
    return ctypes.c_void_p(a.ctypes.data)


# ---- device memory plumbing (HIP runtime the engine links) -------------------
class Hip:
    """Minimal hipMalloc/hipMemcpy/hipEvent access through the runtime the
    engine library itself links (no second runtime in the process)."""
    H2D, D2H, D2D = 1, 2, 3

    def __init__(self):
        load()
        self.rt = ctypes.CDLL("libamdhip64.so", mode=ctypes.RTLD_GLOBAL)
        self.rt.hipMalloc.argtypes = [ctypes.POINTER(ctypes.c_void_p), ctypes.c_size_t]
        self.rt.hipFree.argtypes = [ctypes.c_void_p]
        self.rt.hipMemcpy.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int]
        self.rt.hipMemset.argtypes = [ctypes.c_void_p, ctypes.c_int, ctypes.c_size_t]
        self.rt.hipGetDeviceCount.argtypes = [ctypes.POINTER(ctypes.c_int)]
        self.rt.hipEventCreate.argtypes = [ctypes.POINTER(ctypes.c_void_p)]
        self.rt.hipEventRecord.argtypes = [ctypes.c_void_p, ctypes.c_void_p]
        self.rt.hipEventSynchronize.argtypes = [ctypes.c_void_p]
        self.rt.hipEventElapsedTime.argtypes = [ctypes.POINTER(ctypes.c_float), ctypes.c_void_p, ctypes.c_void_p]
        self.rt.hipEventDestroy.argtypes = [ctypes.c_void_p]
        self.rt.hipDeviceSynchronize.argtypes = []

    def device_count(self):
        n = ctypes.c_int(0)
        return n.value if self.rt.hipGetDeviceCount(ctypes.byref(n)) == 0 else 0

    def _ok(self, e, what):
        if e != 0:
            raise RuntimeError("%s failed with hipError %d" % (what, e))

    def malloc(self, nbytes):
        p = ctypes.c_void_p()
        self._ok(self.rt.hipMalloc(ctypes.byref(p), max(int(nbytes), 1) + 256), "hipMalloc")
        return p.value

    def free(self, p):
        self.rt.hipFree(p)

    def to_device(self, arr):
        arr = np.ascontiguousarray(arr)
        p = self.malloc(arr.nbytes)
        self._ok(self.rt.hipMemcpy(p, arr.ctypes.data, arr.nbytes, self.H2D), "hipMemcpy H2D")
        return p

    def from_device(self, p, shape, dtype):
        out = np.empty(shape, dtype=dtype)
        self.sync()
        self._ok(self.rt.hipMemcpy(out.ctypes.data, p, out.nbytes, self.D2H), "hipMemcpy D2H")
        return out

    def copy_d2d(self, dst, src, nbytes):
        self._ok(self.rt.hipMemcpy(dst, src, nbytes, self.D2D), "hipMemcpy D2D")

    def sync(self):
        self._ok(self.rt.hipDeviceSynchronize(), "hipDeviceSynchronize")

    def event(self):
        e = ctypes.c_void_p()
        self._ok(self.rt.hipEventCreate(ctypes.byref(e)), "hipEventCreate")
        return e.value

    def record(self, ev, stream=None):
        self._ok(self.rt.hipEventRecord(ev, stream), "hipEventRecord")

    def elapsed_ms(self, a, b):
        self._ok(self.rt.hipEventSynchronize(b), "hipEventSynchronize")
        ms = ctypes.c_float()
        self._ok(self.rt.hipEventElapsedTime(ctypes.byref(ms), a, b), "hipEventElapsedTime")
        return ms.value


# ---- single ops ----------------------------------------------------------------
def quantize(gtype, x):
    """Encode float32 values into ggml blocks (the synthetic-model encoders)."""
    x = np.ascontiguousarray(x, dtype=np.float32).ravel()
    be, bb = BLOCK[gtype]
    out = np.empty(x.size // be * bb, dtype=np.uint8)
    check(load().frn_quantize(gtype, _ptr(x), x.size, _ptr(out)))
    return out


def gaussian(seed, std, n):
    out = np.empty(n, dtype=np.float32)
    check(load().frn_gaussian(seed, std, n, _ptr(out)))
    return out


def dequant_dev(hip, gtype, raw_dev, raw_bytes, n, out_dev, stream=None):
    check(load().frn_dequant(gtype, raw_dev, raw_bytes, n, out_dev, stream))


def matmul_quant_dev(gtype, w_dev, w_bytes, a_dev, seq, out_dev, d_out, d_in, stream=None):
    check(load().frn_matmul_quant(gtype, w_dev, w_bytes, a_dev, seq, out_dev, d_out, d_in, stream))


# ---- synthetic models -----------------------------------------------------------
PRESETS = {
    # Qwen2-0.5B shape, all linear weights Q8_0, tied embeddings
    "qwen2-0.5b-q8_0": dict(n_layers=24, n_heads=14, n_kv_heads=2, hidden=896, ffn=4864, vocab=151936,
                            mix=MIX_ALL_Q8_0, tied=1, embd_type=Q8_0, output_type=Q8_0),
    # Qwen2-1.5B shape, Q4_K_M mix (Q6_K attn_v/ffn_down on even layers), tied Q6_K embedding
    "qwen2-1.5b-q4_k_m": dict(n_layers=28, n_heads=12, n_kv_heads=2, hidden=1536, ffn=8960, vocab=151936,
                              mix=MIX_Q4_K_M, tied=1, embd_type=Q6_K, output_type=Q6_K),
    # Qwen2-7B shape, Q4_K_M mix, untied Q6_K lm_head, Q4_K embedding
    "qwen2-7b-q4_k_m": dict(n_layers=28, n_heads=28, n_kv_heads=4, hidden=3584, ffn=18944, vocab=152064,
                            mix=MIX_Q4_K_M, tied=0, embd_type=Q4_K, output_type=Q6_K),
}


def synth_write(path, seed, threads=0, weight_std=0.02, rope_theta=1e6, rms_eps=1e-6, context_length=32768,
                **shape):
    s = SynthSpec()
    for k, v in shape.items():
        setattr(s, k, v)
    s.seed, s.threads, s.weight_std = seed, threads, weight_std
    s.rope_theta, s.rms_eps, s.context_length = rope_theta, rms_eps, context_length
    check(load().frn_synth_write(ctypes.byref(s), path.encode()))
    return path


# ---- model / token loop -----------------------------------------------------------
class Model:
    """A GGUF model loaded onto one GPU: Model::load + KvCache in one context."""

    def __init__(self, path, device=0, max_ctx=4096, eager=False, stepwise_prefill=False, resident=None):
        lib = load()
        self.gguf = ctypes.c_void_p()
        check(lib.frn_gguf_open(path.encode(), ctypes.byref(self.gguf)))
        self.cfg = Config()
        ctx_len = ctypes.c_uint32()
        check(lib.frn_gguf_config(self.gguf, ctypes.byref(self.cfg), ctypes.byref(ctx_len)))
        self.context_length = ctx_len.value
        self.ctx = ctypes.c_void_p()
        flags = ((FLAG_EAGER if eager else 0) | (FLAG_STEPWISE_PREFILL if stepwise_prefill else 0) |
                 (0 if resident is None else FLAG_RESIDENT if resident else FLAG_NO_RESIDENT))
        check(lib.frn_model_load(self.gguf, device, max_ctx, flags, ctypes.byref(self.ctx)))
        self.cfg.max_ctx = max_ctx
        self.vocab = self.cfg.vocab

    def meta_u32(self, key):
        v = ctypes.c_uint32()
        st = load().frn_gguf_meta_u32(self.gguf, key.encode(), ctypes.byref(v))
        return v.value if st == 0 else None

    def stop_ids(self):
        return [v for v in (self.meta_u32("tokenizer.ggml.eos_token_id"),
                            self.meta_u32("tokenizer.ggml.bos_token_id")) if v is not None]

    def prefill(self, ids):
        ids = np.ascontiguousarray(ids, dtype=np.uint32)
        nxt = ctypes.c_uint32()
        check(load().frn_prefill(self.ctx, _ptr(ids), ids.size, ctypes.byref(nxt)))
        return nxt.value

    def decode(self, tok):
        nxt = ctypes.c_uint32()
        check(load().frn_decode(self.ctx, int(tok), ctypes.byref(nxt)))
        return nxt.value

    def decode_engine(self):
        """(resident, reason): 1 when the resident decode kernel serves
        decode steps, else 0 and why not (frn_decode_engine)."""
        on = ctypes.c_uint32()
        why = ctypes.create_string_buffer(256)
        check(load().frn_decode_engine(self.ctx, ctypes.byref(on), why, 256))
        return on.value, why.value.decode()

    def resident_trace(self, n_steps, read=False):
        """Arm (read=False) or read (read=True) the resident kernel's phase
        timestamps: [n_steps][n_layers + 1][16][256] uint64 at 100 MHz."""
        if not read:
            check(load().frn_resident_trace(self.ctx, n_steps, None, 0))
            return None
        shape = (n_steps, self.cfg.n_layers + 1, 16, 256)
        out = np.zeros(shape, dtype=np.uint64)
        check(load().frn_resident_trace(self.ctx, n_steps, out.ctypes.data, out.size))
        return out

    def decode_greedy(self, tok, n, stop_ids=()):
        """n greedy steps from token tok (frn_decode_greedy): the ids of the
        frn_decode loop, with one host synchronisation per batch of steps;
        ends early after a step whose argmax is in stop_ids."""
        out = np.zeros(max(int(n), 1), dtype=np.uint32)
        stop = np.asarray(list(stop_ids), dtype=np.uint32)
        done = ctypes.c_uint32()
        check(load().frn_decode_greedy(self.ctx, int(tok), int(n),
                                       stop.ctypes.data if len(stop) else None, len(stop),
                                       out.ctypes.data, ctypes.byref(done)))
        return [int(v) for v in out[:done.value]]

    def sampler_init(self, temperature, top_k, top_p, repeat_penalty=1.0, seed=7):
        """Sampler::new on the device (frn_sampler_init)."""
        check(load().frn_sampler_init(self.ctx, float(temperature), int(top_k), float(top_p),
                                      float(repeat_penalty), int(seed)))

    def sample(self, recent=()):
        """Sampler::sample on the last step's device logits (frn_sample)."""
        r = np.ascontiguousarray(list(recent), dtype=np.uint32)
        nxt = ctypes.c_uint32()
        check(load().frn_sample(self.ctx, r.ctypes.data if r.size else None, r.size, ctypes.byref(nxt)))
        return nxt.value

    def sampler_draws(self):
        d = ctypes.c_uint64()
        check(load().frn_sampler_draws(self.ctx, ctypes.byref(d)))
        return d.value

    def logits(self):
        out = np.empty(self.vocab, dtype=np.float32)
        check(load().frn_logits(self.ctx, _ptr(out), out.size))
        return out

    def reset(self):
        check(load().frn_reset(self.ctx))

    def cache_len(self):
        v = ctypes.c_uint32()
        check(load().frn_cache_len(self.ctx, ctypes.byref(v)))
        return v.value

    def cache_read(self, layer, which_v, n):
        kvd = self.cfg.n_kv_heads * self.cfg.head_dim
        out = np.empty((n, kvd), dtype=np.float32)
        check(load().frn_cache_read(self.ctx, layer, 1 if which_v else 0, n, _ptr(out)))
        return out

    def generate_greedy(self, prompt, max_new, stop_ids=None):
        prompt = np.ascontiguousarray(prompt, dtype=np.uint32)
        stop = np.ascontiguousarray(self.stop_ids() if stop_ids is None else stop_ids, dtype=np.uint32)
        out = np.zeros(max(max_new, 1), dtype=np.uint32)
        st = GenStats()
        check(load().frn_generate_greedy(self.ctx, _ptr(prompt), prompt.size, max_new,
                                         _ptr(stop) if stop.size else None, stop.size, _ptr(out),
                                         ctypes.byref(st)))
        return out[:st.n_generated].tolist(), st

    def generate_sampled(self, prompt, max_new, temperature=0.7, top_k=40, top_p=0.9, repeat_penalty=1.0, seed=7,
                         stop_ids=None):
        """generate (generate.rs:83-157) with the device sampler; returns
        (ids, stats, draws)."""
        prompt = np.ascontiguousarray(prompt, dtype=np.uint32)
        stop = np.ascontiguousarray(self.stop_ids() if stop_ids is None else stop_ids, dtype=np.uint32)
        out = np.zeros(max(max_new, 1), dtype=np.uint32)
        st = GenStats()
        draws = ctypes.c_uint64()
        check(load().frn_generate_sampled(self.ctx, _ptr(prompt), prompt.size, max_new, float(temperature),
                                          int(top_k), float(top_p), float(repeat_penalty), int(seed),
                                          _ptr(stop) if stop.size else None, stop.size, _ptr(out),
                                          ctypes.byref(st), ctypes.byref(draws)))
        return out[:st.n_generated].tolist(), st, draws.value

    def timings_enable(self, on=True):
        check(load().frn_timings_enable(self.ctx, 1 if on else 0))

    def timings_reset(self):
        check(load().frn_timings_reset(self.ctx))

    def timings(self):
        arr = (Timing * 32)()
        n = ctypes.c_uint32()
        check(load().frn_timings(self.ctx, arr, 32, ctypes.byref(n)))
        return {arr[i].name.decode(): (arr[i].ms, arr[i].calls) for i in range(n.value)}

    def step_times_enable(self, on=True):
        check(load().frn_step_times_enable(self.ctx, 1 if on else 0))

    def step_times(self, max_n=1 << 16):
        """Per-step decode durations (ms) kept since the last read."""
        arr = (ctypes.c_float * max_n)()
        n = ctypes.c_uint32()
        check(load().frn_step_times(self.ctx, arr, max_n, ctypes.byref(n)))
        return list(arr[:n.value])

    def bench_kernel(self, name, layer=None, reps=10):
        """Mean time per launch (us) of one kernel category replayed back to
        back (layer None: every layer in turn, reps rounds); leaves the
        context state undefined (reset() afterwards)."""
        layer = 0xFFFFFFFF if layer is None else layer
        us = ctypes.c_float()
        check(load().frn_bench_kernel(self.ctx, name.encode(), layer, reps, ctypes.byref(us)))
        return us.value

    def close(self):
        lib = load()
        if self.ctx:
            lib.frn_destroy(self.ctx)
            self.ctx = ctypes.c_void_p()
        if self.gguf:
            lib.frn_gguf_close(self.gguf)
            self.gguf = ctypes.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
