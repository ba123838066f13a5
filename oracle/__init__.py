"""ctypes binding of the CPU parity oracle (oracle/liboracle.so).

TEST INFRASTRUCTURE ONLY.  Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
import this package, and only as the checker or the timed CPU baseline; the product (wavo_amd) never
does.  The C sources restate wavo's CPU backend (src/cpu/) in its portable f16-rounded arithmetic;
see oracle.h for the per-function citations.
"""

import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")

F32, F16, Q4_0, Q8_0 = 0, 1, 2, 8
BIAS, SILU, RELU, RESIDUAL, GELU, GELU_RESIDUAL, TANH = range(7)

_lib = None
_fp = ctypes.POINTER(ctypes.c_float)
_u32p = ctypes.POINTER(ctypes.c_uint32)
_ip = ctypes.POINTER(ctypes.c_int)


def build():
    """Compiles liboracle.so with its Makefile (gcc, OpenMP)."""
    subprocess.run(["make", "-s", "-C", HERE], check=True)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        L = ctypes.CDLL(LIB_PATH)
        sig = {
            "ox_to_half": (ctypes.c_float, [ctypes.c_float]),
            "ox_half_to_float": (ctypes.c_float, [ctypes.c_uint16]),
            "ox_float_to_half_bits": (ctypes.c_uint16, [ctypes.c_float]),
            "ox_exp": (ctypes.c_float, [ctypes.c_float]),
            "ox_silu": (ctypes.c_float, [ctypes.c_float]),
            "ox_gelu": (ctypes.c_float, [ctypes.c_float]),
            "ox_dot": (ctypes.c_float, [_fp, _fp, ctypes.c_size_t]),
            "ox_type_size": (ctypes.c_size_t, [ctypes.c_int, ctypes.c_size_t]),
            "ox_dequant": (ctypes.c_int, [ctypes.c_int, ctypes.c_void_p, _fp, ctypes.c_size_t]),
            "ox_quantize_q8_0": (None, [_fp, ctypes.c_void_p, ctypes.c_size_t]),
            "ox_quantize_q4_0": (None, [_fp, ctypes.c_void_p, ctypes.c_size_t]),
            "ox_linear_new": (ctypes.c_void_p, [ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                                ctypes.POINTER(ctypes.c_void_p), _ip, _fp]),
            "ox_linear_free": (None, [ctypes.c_void_p]),
            "ox_gemm": (None, [_fp, ctypes.c_void_p, _fp, ctypes.c_int, ctypes.c_int, ctypes.c_float]),
            "ox_gemm_wide": (None, [_fp, ctypes.c_void_p, _fp, ctypes.c_int, ctypes.c_int,
                                    ctypes.c_float, _fp, ctypes.c_int]),
            "ox_gemv": (None, [_fp, ctypes.c_void_p, _fp, ctypes.c_int, ctypes.c_float]),
            "ox_layer_norm": (None, [_fp, _fp, _fp, _fp, ctypes.c_int, ctypes.c_int, _fp, _fp,
                                     ctypes.c_int]),
            "ox_im2col": (None, [_fp, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                 ctypes.c_int, _fp, ctypes.c_int]),
            "ox_conv_glu": (None, [_fp, _fp, _fp, ctypes.c_int, _fp, _fp, ctypes.c_int, _fp,
                                   ctypes.c_int, ctypes.c_int, ctypes.c_int]),
            "ox_attention": (None, [_fp, ctypes.c_int, _fp, ctypes.c_int, _fp, ctypes.c_int,
                                    ctypes.c_int, ctypes.c_int, ctypes.c_int]),
            "ox_relative_attention": (None, [_fp, _fp, _fp, _fp, _fp, ctypes.c_int, ctypes.c_int,
                                             ctypes.c_int, ctypes.c_int]),
            "ox_attend": (None, [_fp, _fp, ctypes.c_int, ctypes.c_int, _fp, ctypes.c_int,
                                 ctypes.c_int]),
            "ox_pack": (None, [_fp, ctypes.c_int, ctypes.c_int, _u32p, ctypes.c_int, ctypes.c_int,
                               ctypes.c_int, ctypes.c_int]),
            "ox_rope_table": (None, [ctypes.c_int, ctypes.c_int, ctypes.c_double, _fp]),
            "ox_rel_positions": (None, [ctypes.c_int, ctypes.c_long, ctypes.c_int, _fp]),
            "ox_batch_norm": (None, [_fp, _fp, _fp, _fp, ctypes.c_int, _fp, _fp]),
            "ox_sub_first": (None, [_fp, ctypes.c_int, ctypes.c_int, _fp, _fp, _fp, _fp,
                                    ctypes.c_int, _fp, ctypes.c_int, ctypes.c_int]),
            "ox_depthwise": (None, [_fp, _fp, _fp, ctypes.c_int, ctypes.c_int, ctypes.c_int, _fp,
                                    ctypes.c_int, ctypes.c_int]),
            "ox_flatten": (None, [_fp, _fp, ctypes.c_int, ctypes.c_int, ctypes.c_int]),
            "ox_argmax": (ctypes.c_int, [_fp, ctypes.c_int]),
            "ox_ctc": (ctypes.c_int, [_fp, ctypes.c_int, ctypes.c_int, ctypes.c_int, _u32p]),
            "ox_tdt_scripted": (ctypes.c_int, [ctypes.c_int, ctypes.c_int, _ip, ctypes.c_int,
                                               ctypes.c_int, _ip, ctypes.c_int, _u32p, _ip, _ip]),
            "ox_model_load": (ctypes.c_void_p, [ctypes.c_char_p, ctypes.c_char_p, ctypes.c_size_t]),
            "ox_model_free": (None, [ctypes.c_void_p]),
            "ox_model_encode": (ctypes.c_int, [ctypes.c_void_p, _fp, ctypes.c_int, ctypes.c_int,
                                               _fp, _ip, _ip]),
            "ox_model_blocks": (ctypes.c_int, [ctypes.c_void_p, _fp, ctypes.c_int, ctypes.c_int]),
            "ox_model_info": (ctypes.c_int, [ctypes.c_void_p, _ip, _ip, _ip, _ip, _ip]),
            "ox_model_tdt": (ctypes.c_int, [ctypes.c_void_p, _fp, ctypes.c_int, ctypes.c_int,
                                            _u32p, ctypes.c_int]),
            "ox_model_tdt_trace": (ctypes.c_int, [ctypes.c_void_p, _fp, ctypes.c_int, ctypes.c_int,
                                                  _u32p, ctypes.c_int, _ip, _fp, ctypes.c_int]),
            "ox_model_tdt_lipschitz": (ctypes.c_float, [ctypes.c_void_p]),
            "ox_model_predict": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_int, _fp, _fp, _fp]),
            "ox_model_joint": (ctypes.c_int, [ctypes.c_void_p, _fp, _fp, _fp]),
            "ox_whisper_begin": (ctypes.c_int, [ctypes.c_void_p, _fp, ctypes.c_int]),
            "ox_whisper_step": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_int, ctypes.c_int, _fp]),
            "ox_model_whisper_ids": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_void_p]),
            "ox_model_context": (ctypes.c_int, [ctypes.c_void_p]),
            "ox_timestamp_rules": (None, [ctypes.c_void_p, _fp, ctypes.c_int, _u32p, ctypes.c_int]),
            "ox_whisper_argmax": (ctypes.c_int, [_fp, ctypes.c_int, ctypes.c_int, _fp]),
            "ox_whisper_pick": (ctypes.c_int, [ctypes.c_void_p, _fp, ctypes.c_int, _u32p, ctypes.c_int,
                                               ctypes.c_int, _fp]),
            "ox_probability": (ctypes.c_float, [_fp, ctypes.c_int, ctypes.c_int]),
            "ox_whisper_decode": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_void_p, _fp, ctypes.c_int,
                                                 ctypes.c_int, ctypes.c_int, _u32p, ctypes.c_int, _fp, _fp]),
            "ox_top2_gap": (ctypes.c_float, [_fp, ctypes.c_int, ctypes.c_void_p, _u32p, ctypes.c_int]),
            "ox_whisper_retrieve": (ctypes.c_int, [ctypes.c_void_p, _u32p, ctypes.c_int, ctypes.c_int,
                                                   _ip, ctypes.c_int, _ip]),
            "ox_fft": (ctypes.c_int, [ctypes.c_int, ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p]),
            "ox_fft_tables": (ctypes.c_int, [ctypes.c_int, _ip, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p,
                                             ctypes.c_void_p, _ip, _ip]),
            "ox_parakeet_filterbank": (None, [_fp]),
            "ox_mel_raw": (None, [ctypes.c_int]),
            "ox_parakeet_log_mel": (ctypes.c_int, [_fp, ctypes.c_int, ctypes.c_int, ctypes.c_int, _fp]),
            "ox_parakeet_mel": (ctypes.c_int, [_fp, ctypes.c_int, _fp]),
            "ox_gigaam_mel": (ctypes.c_int, [_fp, ctypes.c_int, _fp, _fp, ctypes.c_int, _fp]),
            "ox_whisper_mel": (ctypes.c_int, [_fp, ctypes.c_int, _fp, _fp, ctypes.c_int, _fp]),
            "ox_threads": (ctypes.c_int, []),
            "ox_set_threads": (None, [ctypes.c_int]),
        }
        for name, (res, args) in sig.items():
            f = getattr(L, name)
            f.restype = res
            f.argtypes = args
        _lib = L
    return _lib


def f32(a):
    """A C-contiguous float32 copy/view of `a` and its pointer."""
    a = np.ascontiguousarray(a, dtype=np.float32)
    return a, a.ctypes.data_as(_fp)


def _ptr(a):
    return None if a is None else a.ctypes.data_as(_fp)


def to_half(x):
    L = lib()
    x = np.asarray(x, dtype=np.float32)
    return np.array([L.ox_to_half(float(v)) for v in x.ravel()], dtype=np.float32).reshape(x.shape)


def quantize(x, wtype):
    """GGUF bytes of the rows of x (float32) in type wtype (convert.py's quantizers for Q8_0)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    n = x.size
    if wtype == F32:
        return x.tobytes()
    if wtype == F16:
        return x.astype(np.float16).tobytes()
    L = lib()
    out = ctypes.create_string_buffer(L.ox_type_size(wtype, n))
    if wtype == Q8_0:
        L.ox_quantize_q8_0(_ptr(x), out, n)
    elif wtype == Q4_0:
        L.ox_quantize_q4_0(_ptr(x), out, n)
    else:
        raise ValueError(wtype)
    return out.raw


def dequant(raw, wtype, n):
    L = lib()
    out = np.zeros(n, np.float32)
    buf = ctypes.create_string_buffer(bytes(raw), len(raw))
    if L.ox_dequant(wtype, buf, _ptr(out), n):
        raise ValueError(wtype)
    return out


class Linear:
    """ox_linear: weights [n][k] in GGUF bytes, stacked, with a bias (src/cpu/gemm.rs:35-72)."""

    def __init__(self, wtype, k, tensors, bias=None):
        L = lib()
        self._keep = [ctypes.create_string_buffer(bytes(t), len(t)) for t, _ in tensors]
        rows = [r for _, r in tensors]
        ws = (ctypes.c_void_p * len(tensors))(*[ctypes.cast(b, ctypes.c_void_p) for b in self._keep])
        rr = (ctypes.c_int * len(rows))(*rows)
        self.n = sum(rows)
        self.k = k
        b = None if bias is None else np.ascontiguousarray(bias, np.float32)
        self.h = L.ox_linear_new(wtype, k, len(tensors), ws, rr, _ptr(b))
        if not self.h:
            raise ValueError("bad linear layer")

    def __del__(self):
        if getattr(self, "h", None):
            lib().ox_linear_free(self.h)
            self.h = None


def gemm(a, l, m, epi, alpha=0.0, c=None):
    a, pa = f32(a)
    c = np.zeros((m, l.n), np.float32) if c is None else np.ascontiguousarray(c, np.float32).copy()
    lib().ox_gemm(pa, l.h, _ptr(c), m, epi, alpha)
    return c


def gemm_wide(a, l, m, epi, alpha=0.0, c=None, bias2=None, dual=0):
    a, pa = f32(a)
    cols = l.n if l.n % 32 == 0 else (l.n + 63) // 64 * 64
    c = np.zeros((m, cols + dual), np.float32) if c is None else np.ascontiguousarray(c, np.float32).copy()
    b2 = None if bias2 is None else np.ascontiguousarray(bias2, np.float32)
    lib().ox_gemm_wide(pa, l.h, _ptr(c), m, epi, alpha, _ptr(b2), dual)
    return c


def gemv(x, l, epi, alpha=0.0, c=None):
    x, px = f32(x)
    c = np.zeros(l.n, np.float32) if c is None else np.ascontiguousarray(c, np.float32).copy()
    lib().ox_gemv(px, l.h, _ptr(c), epi, alpha)
    return c


def layer_norm(x, g, b, table=None, head_dim=0):
    x, px = f32(x)
    rows, cols = x.shape
    y = np.zeros_like(x)
    yr = np.zeros_like(x) if table is not None else None
    tb = None if table is None else np.ascontiguousarray(table, np.float32)
    lib().ox_layer_norm(px, _ptr(f32(g)[0]), _ptr(f32(b)[0]), _ptr(y), rows, cols, _ptr(tb),
                        _ptr(yr), head_dim)
    return (y, yr) if table is not None else y


def im2col(x, t, ch, kernel, stride, pad, width=None):
    x, px = f32(x)
    rows = (t + 2 * pad - kernel) // stride + 1
    width = width or ch * kernel
    col = np.zeros((rows, width), np.float32)
    lib().ox_im2col(px, t, ch, kernel, stride, pad, _ptr(col), width)
    return col


def conv_glu(h, taps, tb, kernel, g, beta, layer_norm_, t, ch, valid=-1):
    """taps [kernel][ch] (the CPU layout)."""
    h = np.ascontiguousarray(h, np.float32).copy()
    y = np.zeros((t, ch), np.float32)
    lib().ox_conv_glu(_ptr(h), _ptr(f32(taps)[0]), _ptr(f32(tb)[0]), kernel, _ptr(f32(g)[0]),
                      _ptr(f32(beta)[0]), int(layer_norm_), _ptr(y), t, ch, valid)
    return y


def attention(qk, ld, v, ldv, t, heads, hd, valid=-1):
    qk, pq = f32(qk)
    v, pv = f32(v)
    o = np.zeros((t, heads * hd), np.float32)
    lib().ox_attention(pq, ld, pv, ldv, _ptr(o), t, heads, hd, valid)
    return o


def relative_attention(qkv, pos, u, vb, t, heads, hd, valid=-1):
    qkv, pq = f32(qkv)
    pos, pp = f32(pos)
    o = np.zeros((t, heads * hd), np.float32)
    lib().ox_relative_attention(pq, pp, _ptr(f32(u)[0]), _ptr(f32(vb)[0]), _ptr(o), t, heads, hd,
                                valid)
    return o


def attend(q, kv, cols, n, heads, hd):
    q, pq = f32(q)
    kv, pk = f32(kv)
    o = np.zeros(heads * hd, np.float32)
    lib().ox_attend(pq, pk, cols, n, _ptr(o), heads, hd)
    return o


def pack(x, src, stride, cache, rows, d, cols, col):
    x, px = f32(x)
    cache = np.ascontiguousarray(cache, np.uint32).copy()
    lib().ox_pack(px, src, stride, cache.ctypes.data_as(_u32p), rows, d, cols, col)
    return cache


def rope_table(frames, hd, theta):
    out = np.zeros((frames, hd), np.float32)
    lib().ox_rope_table(frames, hd, theta, _ptr(out))
    return out


def rel_positions(d, first, rows):
    out = np.zeros((rows, d), np.float32)
    lib().ox_rel_positions(d, first, rows, _ptr(out))
    return out


def half_len(n):
    return (n - 1) // 2 + 1


def sub_first(mel, valid, mels, w0, b0, w2, b2, ch, rows, t0):
    mel, pm = f32(mel)
    y = np.zeros((rows, half_len(half_len(mels)), ch), np.float32)
    lib().ox_sub_first(pm, valid, mels, _ptr(f32(w0)[0]), _ptr(f32(b0)[0]), _ptr(f32(w2)[0]),
                       _ptr(f32(b2)[0]), ch, _ptr(y), rows, t0)
    return y


def depthwise(x, w, b, t, f, ch, n, t0):
    x, px = f32(x)
    y = np.zeros((n, half_len(f), ch), np.float32)
    lib().ox_depthwise(px, _ptr(f32(w)[0]), _ptr(f32(b)[0]), t, f, ch, _ptr(y), n, t0)
    return y


def flatten(x, t, f, ch):
    x, px = f32(x)
    y = np.zeros((t, f * ch), np.float32)
    lib().ox_flatten(px, _ptr(y), t, f, ch)
    return y


def fft(x, f64=True):
    """Fft::forward (src/fft.rs:72-104) of real x: (re, im) in float64 or float32."""
    dt = np.float64 if f64 else np.float32
    x = np.ascontiguousarray(x, dt)
    re, im = np.zeros(len(x), dt), np.zeros(len(x), dt)
    lib().ox_fft(len(x), int(f64), x.ctypes.data, re.ctypes.data, im.ctypes.data)
    return re, im


def mel_raw(on):
    """on: the frontends return each filter's sum before the logarithm (no normalization or scale)."""
    lib().ox_mel_raw(int(on))


def parakeet_filterbank():
    out = np.zeros((128, 257), np.float32)
    lib().ox_parakeet_filterbank(_ptr(out))
    return out


def parakeet_log_mel(pcm, t0, t1):
    """Frontend::log_mel (src/parakeet/frontend.rs:74-108): frames [t0, t1) of the whole pcm."""
    pcm, pp = f32(pcm)
    out = np.zeros((max(t1 - t0, 0), 128), np.float32)
    if lib().ox_parakeet_log_mel(pp, len(pcm), t0, t1, _ptr(out)) < 0:
        raise ValueError("bad frame range")
    return out


def parakeet_mel(pcm):
    """Frontend::compute (src/parakeet/frontend.rs:52-72): [len / 160 + 1][128], empty below 3 frames."""
    pcm, pp = f32(pcm)
    n = lib().ox_parakeet_mel(pp, len(pcm), None)
    out = np.zeros((n, 128), np.float32)
    if n:
        lib().ox_parakeet_mel(pp, len(pcm), _ptr(out))
    return out


def gigaam_mel(pcm, window, filters):
    """Frontend::compute (src/gigaam/frontend.rs:50-71) with the GGUF's window and filterbank [mels][161]."""
    pcm, pp = f32(pcm)
    w, pw = f32(window)
    f, pf = f32(filters)
    n = lib().ox_gigaam_mel(pp, len(pcm), pw, pf, f.shape[0], None)
    out = np.zeros((n, f.shape[0]), np.float32)
    if n:
        lib().ox_gigaam_mel(pp, len(pcm), pw, pf, f.shape[0], _ptr(out))
    return out


def whisper_mel(pcm, window, filters):
    """Frontend::compute (src/whisper/frontend.rs:45-85) with the GGUF's window and filterbank [mels][201]."""
    pcm, pp = f32(pcm)
    w, pw = f32(window)
    f, pf = f32(filters)
    n = lib().ox_whisper_mel(pp, len(pcm), pw, pf, f.shape[0], None)
    out = np.zeros((n, f.shape[0]), np.float32)
    lib().ox_whisper_mel(pp, len(pcm), pw, pf, f.shape[0], _ptr(out))
    return out


def ctc(logits, blank):
    logits, pl = f32(logits)
    frames, classes = logits.shape
    out = np.zeros(2 * frames, np.uint32)
    n = lib().ox_ctc(pl, frames, classes, blank, out.ctypes.data_as(_u32p))
    return [(int(out[2 * i]), int(out[2 * i + 1])) for i in range(n)]


def tdt_scripted(frames, blank, durations, max_symbols, global_, script):
    """The TDT loop over scripted (token, duration index) decisions: (pairs, calls)."""
    d = (ctypes.c_int * len(durations))(*durations)
    flat = [v for pair in script for v in pair]
    sc = (ctypes.c_int * max(1, len(flat)))(*flat)
    out = np.zeros(2 * 4096, np.uint32)
    calls = (ctypes.c_int * (2 * 4096))()
    used = ctypes.c_int()
    n = lib().ox_tdt_scripted(frames, blank, d, max_symbols, int(global_), sc, len(script),
                              out.ctypes.data_as(_u32p), calls, ctypes.byref(used))
    pairs = [(int(out[2 * i]), int(out[2 * i + 1])) for i in range(n)]
    cl = [(calls[2 * i], None if calls[2 * i + 1] < 0 else calls[2 * i + 1]) for i in range(used.value)]
    return pairs, cl


class WhisperIds(ctypes.Structure):
    """ox_whisper_ids: the reference's `Ids` (src/whisper/search.rs:16-23) plus SOT."""

    _fields_ = [("eot", ctypes.c_int), ("no_timestamps", ctypes.c_int), ("begin", ctypes.c_int),
                ("sot", ctypes.c_int), ("suppress", _ip), ("n_suppress", ctypes.c_int),
                ("begin_suppress", _ip), ("n_begin_suppress", ctypes.c_int)]

    @classmethod
    def make(cls, eot, no_timestamps, begin, suppress=(), begin_suppress=(), sot=-1):
        ids = cls()
        ids.eot, ids.no_timestamps, ids.begin, ids.sot = eot, no_timestamps, begin, sot
        ids._s = (ctypes.c_int * max(1, len(suppress)))(*suppress)
        ids._b = (ctypes.c_int * max(1, len(begin_suppress)))(*begin_suppress)
        ids.suppress, ids.n_suppress = ctypes.cast(ids._s, _ip), len(suppress)
        ids.begin_suppress, ids.n_begin_suppress = ctypes.cast(ids._b, _ip), len(begin_suppress)
        return ids


def _gen(generated):
    g = np.ascontiguousarray(np.asarray(list(generated) or [0], np.uint32))
    return g, g.ctypes.data_as(_u32p)


def timestamp_rules(ids, logits, generated):
    l = np.ascontiguousarray(logits, np.float32).copy()
    g, pg = _gen(generated)
    lib().ox_timestamp_rules(ctypes.byref(ids), _ptr(l), l.size, pg, len(generated))
    return l


def whisper_pick(ids, logits, generated, logprob=False):
    """(id, log-probability, logits after the rules)."""
    l = np.ascontiguousarray(logits, np.float32).copy()
    g, pg = _gen(generated)
    lp = ctypes.c_float()
    i = lib().ox_whisper_pick(ctypes.byref(ids), _ptr(l), l.size, pg, len(generated), int(logprob), ctypes.byref(lp))
    return i, lp.value, l


def probability(logits, i):
    l, pl = f32(logits)
    return float(lib().ox_probability(pl, l.size, i))


def whisper_retrieve(ids, generated, frames):
    """(segments [(start, text ids)], advance)."""
    g, pg = _gen(generated)
    n = len(generated)
    seg = (ctypes.c_int * (3 * (n + 2)))()
    adv = ctypes.c_int()
    c = lib().ox_whisper_retrieve(ctypes.byref(ids), pg, n, frames, seg, n + 2, ctypes.byref(adv))
    out = []
    for i in range(c):
        s, lo, hi = seg[3 * i], seg[3 * i + 1], seg[3 * i + 2]
        out.append((s, [int(x) for x in generated[lo:hi] if x < ids.eot]))
    return out, adv.value


class Model:
    """ox_model: a whole encoder (and decoder) restated on the CPU, loaded from a GGUF file."""

    def __init__(self, path):
        err = ctypes.create_string_buffer(512)
        self.h = lib().ox_model_load(path.encode(), err, 512)
        if not self.h:
            raise ValueError(err.value.decode())
        a, d, layers, mels, width = (ctypes.c_int() for _ in range(5))
        lib().ox_model_info(self.h, ctypes.byref(a), ctypes.byref(d), ctypes.byref(layers),
                            ctypes.byref(mels), ctypes.byref(width))
        self.arch, self.d, self.layers, self.mels, self.width = (v.value for v in (a, d, layers, mels, width))

    def __del__(self):
        if getattr(self, "h", None):
            lib().ox_model_free(self.h)
            self.h = None

    def encode(self, mel, valid=None):
        mel, pm = f32(mel)
        frames, width = ctypes.c_int(), ctypes.c_int()
        mf = mel.shape[0]
        valid = mf if valid is None else valid
        lib().ox_model_encode(self.h, pm, mf, valid, None, ctypes.byref(frames), ctypes.byref(width))
        out = np.zeros((frames.value, width.value), np.float32)
        rc = lib().ox_model_encode(self.h, pm, mf, valid, _ptr(out), ctypes.byref(frames),
                                   ctypes.byref(width))
        if rc:
            raise ValueError("encode failed")
        return out

    def blocks(self, x, layers):
        x = np.ascontiguousarray(x, np.float32).copy()
        if lib().ox_model_blocks(self.h, _ptr(x), x.shape[0], layers):
            raise ValueError("blocks failed")
        return x

    def tdt(self, enc):
        enc, pe = f32(enc)
        out = np.zeros(2 * 16384, np.uint32)
        n = lib().ox_model_tdt(self.h, pe, enc.shape[0], enc.shape[1], out.ctypes.data_as(_u32p), 16384)
        if n < 0:
            raise ValueError("tdt failed")
        return [(int(out[2 * i]), int(out[2 * i + 1])) for i in range(min(n, 16384))]

    def tdt_trace(self, enc):
        """TDT tokens and, per decision, (frame, token, duration index) and the smaller top-2 gap of
        its token/duration logits."""
        enc, pe = f32(enc)
        cap = 16384
        out = np.zeros(2 * cap, np.uint32)
        frames = np.zeros(3 * 4 * cap, np.int32)
        gaps = np.full(4 * cap, -1.0, np.float32)  # a gap is >= 0: the decisions are the leading run
        n = lib().ox_model_tdt_trace(self.h, pe, enc.shape[0], enc.shape[1], out.ctypes.data_as(_u32p), cap,
                                     frames.ctypes.data_as(_ip), _ptr(gaps), 4 * cap)
        if n < 0:
            raise ValueError("tdt failed")
        toks = [(int(out[2 * i]), int(out[2 * i + 1])) for i in range(min(n, cap))]
        d = int(np.argmax(gaps < 0)) if (gaps < 0).any() else len(gaps)
        return toks, frames.reshape(-1, 3)[:d], gaps[:d]

    def predict(self, token, state, hidden, joint, layers):
        """One predictor step: (next state, joint's predictor projection)."""
        st, ps = f32(state)
        nxt = np.zeros(2 * layers * hidden, np.float32)
        pred = np.zeros(joint, np.float32)
        if lib().ox_model_predict(self.h, token, ps, _ptr(nxt), _ptr(pred)):
            raise ValueError("predict failed")
        return nxt, pred

    def joint(self, enc_row, pred, outputs):
        e, pe = f32(enc_row)
        p, pp = f32(pred)
        out = np.zeros(outputs, np.float32)
        if lib().ox_model_joint(self.h, pe, pp, _ptr(out)):
            raise ValueError("joint failed")
        return out

    def tdt_lipschitz(self):
        return float(lib().ox_model_tdt_lipschitz(self.h))

    def whisper_begin(self, enc):
        enc, pe = f32(enc)
        if lib().ox_whisper_begin(self.h, pe, enc.shape[0]):
            raise ValueError("whisper_begin failed")

    def whisper_ids(self):
        ids = WhisperIds()
        if lib().ox_model_whisper_ids(self.h, ctypes.byref(ids)):
            raise ValueError("not a Whisper model")
        return ids

    def whisper_decode(self, logits, prompt=1, logprobs=False, cap=512):
        """search::decode from the prompt's last logits: (generated ids, avg log-prob, per-pick top-2
        gaps after the rules)."""
        ids = self.whisper_ids()
        l = np.ascontiguousarray(logits, np.float32).copy()
        out = np.zeros(cap, np.uint32)
        gaps = np.zeros(cap + 1, np.float32)
        avg = ctypes.c_float()
        n = lib().ox_whisper_decode(self.h, ctypes.byref(ids), _ptr(l), l.size, prompt, int(logprobs),
                                    out.ctypes.data_as(_u32p), cap, ctypes.byref(avg), _ptr(gaps))
        if n < 0:
            raise ValueError("whisper_decode failed")
        return [int(x) for x in out[:n]], avg.value, gaps[:n + 1]

    def whisper_step(self, token, pos, vocab):
        out = np.zeros(vocab, np.float32)
        if lib().ox_whisper_step(self.h, token, pos, _ptr(out)):
            raise ValueError("whisper_step failed")
        return out
