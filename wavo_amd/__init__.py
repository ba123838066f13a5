"""Python binding of the MI355X backend's C ABI (include/wavo_hip.h, libwavo_hip.so).

It mirrors the reference's crate-internal GPU operator API (src/gpu/mod.rs): `Gpu` (device,
buffers, weights), `Linear`, `Epilogue` codes, and the `Pass` ops as `Gpu` methods queued on the
device's stream; `Model` drives the family encoders (GigaAM, Parakeet, Whisper).  Every op calls
the hand-written gfx950 kernels in libwavo_hip.so; there is no CPU or PyTorch fallback — importing
this package without the built library raises.
"""

import ctypes
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libwavo_hip.so")

# ggml types (src/gguf.rs:14-38 + Q4_0) and Epilogue::params (src/gpu/mod.rs:445-455).
F32, F16, Q4_0, Q8_0 = 0, 1, 2, 8
BIAS, SILU, RELU, RESIDUAL, GELU, GELU_RESIDUAL, TANH = range(7)
EOK, EARG, EGPU, EOOM = 0, -1, -2, -3

_vp = ctypes.c_void_p
_i = ctypes.c_int
_f = ctypes.c_float
_sz = ctypes.c_size_t

# Every symbol the header declares, with its ctypes signature (restype, argtypes).
SIGNATURES = {
    "wh_open": (_i, [_i, ctypes.POINTER(_vp)]),
    "wh_close": (None, [_vp]),
    "wh_last_error": (ctypes.c_char_p, [_vp]),
    "wh_device_info": (_i, [_vp, ctypes.c_char_p, _sz, ctypes.POINTER(_i), ctypes.POINTER(_i)]),
    "wh_alloc": (_i, [_vp, _sz, ctypes.POINTER(_vp)]),
    "wh_free": (_i, [_vp, _vp]),
    "wh_host_alloc": (_i, [_vp, _sz, ctypes.POINTER(_vp)]),
    "wh_host_free": (_i, [_vp, _vp]),
    "wh_write": (_i, [_vp, _vp, _vp, _sz]),
    "wh_copy": (_i, [_vp, _vp, _vp, _sz]),
    "wh_zero": (_i, [_vp, _vp, _sz]),
    "wh_read": (_i, [_vp, _vp, _vp, _sz]),
    "wh_sync": (_i, [_vp]),
    "wh_stream": (_vp, [_vp]),
    "wh_tune": (_i, [_vp, ctypes.c_char_p, ctypes.c_char_p]),
    "wh_profile": (_i, [_vp, _i]),
    "wh_profile_read": (_i, [_vp, ctypes.c_char_p, _sz]),
    "wh_region": (_i, [_vp, ctypes.c_char_p, ctypes.c_double, ctypes.c_double]),
    "wh_record_begin": (_i, [_vp]),
    "wh_record_end": (_i, [_vp, ctypes.POINTER(_vp)]),
    "wh_replay": (_i, [_vp, _vp]),
    "wh_pass_free": (None, [_vp]),
    "wh_linear_new": (_i, [_vp, _vp, _i, _vp, _i, _i, ctypes.POINTER(_vp)]),
    "wh_linear_width": (_i, [_vp]),
    "wh_linear_k": (_i, [_vp]),
    "wh_linear_type": (_i, [_vp]),
    "wh_linear_free": (None, [_vp, _vp]),
    "wh_gemm": (_i, [_vp, _vp, _vp, _vp, _i, _i, _f]),
    "wh_gemm_h": (_i, [_vp, _vp, _vp, _vp, _i, _i, _f, _i]),
    "wh_gemm_noalloc": (_i, [_vp, _vp, _vp, _vp, _i, _i, _f]),
    "wh_gemm_noalloc_limit": (_sz, []),
    "wh_gemv": (_i, [_vp, _vp, _vp, _vp, _i, _f, _i]),
    "wh_embed": (_i, [_vp, _vp, _vp, _vp, _vp, _i, _i]),
    "wh_layer_norm": (_i, [_vp, _vp, _vp, _vp, _vp, _i, _i, _vp, _vp, _i]),
    "wh_attend": (_i, [_vp, _vp, _vp, _vp, _vp, _i, _i, _i, _i]),
    "wh_attend_len": (_sz, [_i, _i, _i]),
    "wh_pack": (_i, [_vp, _vp, _i, _i, _vp, _i, _i, _i, _i]),
    "wh_im2col": (_i, [_vp, _vp, _vp, _i, _i, _i, _i, _i]),
    "wh_conv_glu": (_i, [_vp, _vp, _vp, _vp, _i, _vp, _vp, _i, _vp, _i, _i, _i]),
    "wh_attention": (_i, [_vp, _vp, _vp, _vp, _vp, _i, _i, _i, _i]),
    "wh_depthwise": (_i, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _i, _i, _i, _i, _i]),
    "wh_flatten": (_i, [_vp, _vp, _vp, _i, _i, _i]),
    "wh_argmax": (_i, [_vp, _vp, _vp, _i]),
    "wh_model_load": (_i, [_vp, ctypes.c_char_p, ctypes.POINTER(_vp)]),
    "wh_model_free": (None, [_vp]),
    "wh_model_info": (_i, [_vp] + [ctypes.POINTER(_i)] * 5),
    "wh_model_frames": (_i, [_vp, _i, ctypes.POINTER(_i), ctypes.POINTER(_i)]),
    "wh_model_encode": (_i, [_vp, _vp, _i, _i, _vp]),
    "wh_model_encode_batch": (_i, [_vp, _vp, _i, _i, _vp, _vp]),
    "wh_model_graphs": (_i, [_vp, _i]),
    "wh_model_blocks": (_i, [_vp, _vp, _i, _i]),
    "wh_model_greedy": (_i, [_vp, _vp, _i, _i, _vp, _i]),
    "wh_model_greedy_device": (_i, [_vp, _vp, _i, _i, _vp, _i]),
    "wh_model_mel": (_i, [_vp, _vp, _i, _vp, ctypes.POINTER(_i)]),
    "wh_whisper_begin": (_i, [_vp, _vp, _i]),
    "wh_whisper_step": (_i, [_vp, _i, _i, _vp]),
    "wh_whisper_ids_of": (_i, [_vp, _vp]),
    "wh_whisper_pick": (_i, [_vp, _vp, _i, _vp, _i, _vp]),
    "wh_whisper_probability": (_f, [_vp, _i, _i]),
    "wh_whisper_retrieve": (_i, [_vp, _vp, _i, _i, _vp, _i, _vp]),
    "wh_whisper_decode": (_i, [_vp, _vp, _i, _vp, _i, _vp, _i, _vp, _vp]),
}

_lib = None


class WavoError(RuntimeError):
    """Error::Gpu (fatal: reload) or Error::Model (bad shape/argument), by `code`."""

    def __init__(self, code, msg):
        super().__init__(msg)
        self.code = code

    @property
    def fatal(self):
        return self.code in (EGPU, EOOM)


def lib():
    """The loaded libwavo_hip.so; raises if it is not built (no fallback path exists)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise ImportError(f"{LIB_PATH} is not built: run __graft_entry__.build()")
        L = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


class Buffer:
    """Device memory from wh_alloc (Gpu::buffer, src/gpu/mod.rs:675-684)."""

    def __init__(self, gpu, nbytes):
        self.gpu = gpu
        self.nbytes = nbytes
        p = _vp()
        gpu._check(lib().wh_alloc(gpu.h, (nbytes + 3) // 4, ctypes.byref(p)))
        self.ptr = p.value

    def free(self):
        if getattr(self, "ptr", None) and self.gpu.h:
            lib().wh_free(self.gpu.h, self.ptr)
            self.ptr = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass

    def offset(self, floats):
        """A raw pointer `floats` f32 into the buffer."""
        return self.ptr + 4 * floats


class HostArray:
    """Page-locked host memory from wh_host_alloc, viewed as a numpy array (`.array`)."""

    def __init__(self, gpu, shape, dtype=np.float32):
        self.gpu = gpu
        n = int(np.prod(shape)) * np.dtype(dtype).itemsize
        p = _vp()
        gpu._check(lib().wh_host_alloc(gpu.h, n, ctypes.byref(p)))
        self.ptr = p.value
        buf = (ctypes.c_uint8 * max(n, 1)).from_address(self.ptr)
        self.array = np.frombuffer(buf, dtype=dtype, count=int(np.prod(shape))).reshape(shape)

    def free(self):
        if getattr(self, "ptr", None) and self.gpu.h:
            self.array = None
            lib().wh_host_free(self.gpu.h, self.ptr)
            self.ptr = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class Linear:
    """A linear layer on the device (src/gpu/mod.rs:390-413)."""

    def __init__(self, gpu, h):
        self.gpu, self.h = gpu, h
        self.width = lib().wh_linear_width(h)
        self.k = lib().wh_linear_k(h)

    def __del__(self):
        if getattr(self, "h", None) and self.gpu.h:
            lib().wh_linear_free(self.gpu.h, self.h)
            self.h = None


class WhisperIds(ctypes.Structure):
    """wh_whisper_ids: the reference's `Ids` (src/whisper/search.rs:16-23) plus SOT."""

    _fields_ = [("eot", _i), ("no_timestamps", _i), ("begin", _i), ("sot", _i),
                ("suppress", ctypes.POINTER(_i)), ("n_suppress", _i),
                ("begin_suppress", ctypes.POINTER(_i)), ("n_begin_suppress", _i)]

    @classmethod
    def make(cls, eot, no_timestamps, begin, suppress=(), begin_suppress=(), sot=-1):
        ids = cls()
        ids.eot, ids.no_timestamps, ids.begin, ids.sot = eot, no_timestamps, begin, sot
        ids._s = (_i * max(1, len(suppress)))(*suppress)
        ids._b = (_i * max(1, len(begin_suppress)))(*begin_suppress)
        ids.suppress, ids.n_suppress = ctypes.cast(ids._s, ctypes.POINTER(_i)), len(suppress)
        ids.begin_suppress = ctypes.cast(ids._b, ctypes.POINTER(_i))
        ids.n_begin_suppress = len(begin_suppress)
        return ids


def _ids_array(generated):
    g = np.ascontiguousarray(np.asarray(list(generated) or [0], np.uint32))
    return g


def whisper_pick(ids, logits, generated, logprob=False):
    """search::decode's `pick` on host logits (wh_whisper_pick): (id, log-probability or None, the
    logits after the rules).  Needs no GPU."""
    l = np.ascontiguousarray(logits, np.float32).copy()
    g = _ids_array(generated)
    lp = ctypes.c_float()
    i = lib().wh_whisper_pick(ctypes.byref(ids), l.ctypes.data, l.size, g.ctypes.data, len(generated),
                              ctypes.byref(lp) if logprob else None)
    if i < 0:
        raise WavoError(i, "wh_whisper_pick: bad arguments")
    return i, (lp.value if logprob else None), l


def whisper_probability(logits, i):
    l = np.ascontiguousarray(logits, np.float32)
    return float(lib().wh_whisper_probability(l.ctypes.data, l.size, i))


def whisper_retrieve(ids, generated, frames):
    """search::retrieve (wh_whisper_retrieve): ([(start, text ids)], advance).  Needs no GPU."""
    g = _ids_array(generated)
    n = len(generated)
    seg = (_i * (3 * (n + 2)))()
    adv = _i()
    c = lib().wh_whisper_retrieve(ctypes.byref(ids), g.ctypes.data, n, frames, seg, n + 2, ctypes.byref(adv))
    if c < 0:
        raise WavoError(c, "wh_whisper_retrieve: bad arguments")
    return [(seg[3 * i], [int(x) for x in generated[seg[3 * i + 1]:seg[3 * i + 2]] if x < ids.eot])
            for i in range(c)], adv.value


class _Tensor(ctypes.Structure):
    _fields_ = [("data", _vp), ("type", _i), ("k", _i), ("rows", _i)]


def _p(x):
    """A device pointer argument: Buffer, int or None."""
    if x is None:
        return None
    if isinstance(x, Buffer):
        return x.ptr
    return int(x)


class Pass:
    """A recorded pass (wh_record_end): replay() queues it again on its context's stream."""

    def __init__(self, gpu, h):
        self.gpu, self.h = gpu, h

    def replay(self):
        self.gpu._check(lib().wh_replay(self.gpu.h, self.h))

    def free(self):
        if self.h:
            lib().wh_pass_free(self.h)
            self.h = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class Gpu:
    """The device (Gpu, src/gpu/mod.rs:211-577) with the Pass ops (:1394-1678) as methods."""

    def __init__(self, index=0):
        h = _vp()
        rc = lib().wh_open(index, ctypes.byref(h))
        if rc:
            raise WavoError(rc, lib().wh_last_error(None).decode())
        self.h = h.value
        name = ctypes.create_string_buffer(256)
        cus, wave = _i(), _i()
        lib().wh_device_info(self.h, name, 256, ctypes.byref(cus), ctypes.byref(wave))
        self.name, self.cus = name.value.decode(), cus.value

    def close(self):
        if self.h:
            # Models and recorded passes hold device memory and graphs of this context: free them first.
            for m in list(getattr(self, "_models", ())):
                m.free()
            for p in list(getattr(self, "_passes", ())):
                p.free()
            lib().wh_close(self.h)
            self.h = None

    # -- recorded passes (Gpu::record / finish)
    def record_begin(self):
        """Ops queued from here to record_end are recorded into a Pass instead of running."""
        self._check(lib().wh_record_begin(self.h))

    def record_end(self):
        h = _vp()
        self._check(lib().wh_record_end(self.h, ctypes.byref(h)))
        p = Pass(self, h.value)
        if not hasattr(self, "_passes"):
            import weakref

            self._passes = weakref.WeakSet()
        self._passes.add(p)
        return p

    def _check(self, rc):
        if rc:
            raise WavoError(rc, lib().wh_last_error(self.h).decode())

    @property
    def stream(self):
        return lib().wh_stream(self.h)

    def tune(self, key, value):
        """Tuning and measurement overrides (wh_tune): gemm_plan, gemm_shape_plans, gemm_kernel_only,
        gemm_group, attn_split, position_cache, and the check switches mel_raw, whisper_host, whisper_logprobs, attend_merge,
        epilogue_fusion."""
        self._check(lib().wh_tune(self.h, key.encode(), str(value).encode()))

    def profile(self, mode):
        """0 off, 1 (or True) events around every launch, 2 named regions only (wh_region)."""
        self._check(lib().wh_profile(self.h, int(mode)))

    def region_begin(self, name):
        self._check(lib().wh_region(self.h, name.encode(), 0.0, 0.0))

    def region_end(self, flops=0.0, nbytes=0.0):
        self._check(lib().wh_region(self.h, None, float(flops), float(nbytes)))

    def profile_read(self):
        """Per kernel variant: launches, total ms, algorithmic flops and bytes (profiled launches)."""
        import json

        buf = ctypes.create_string_buffer(1 << 20)
        self._check(lib().wh_profile_read(self.h, buf, len(buf)))
        return json.loads(buf.value.decode())

    # -- memory
    def buffer(self, n_f32):
        return Buffer(self, 4 * int(n_f32))

    def upload(self, array):
        a = np.ascontiguousarray(array)
        b = Buffer(self, max(a.nbytes, 4))
        self.write(b, a)
        return b

    def write(self, buf, array, offset_bytes=0):
        a = np.ascontiguousarray(array)
        self._check(lib().wh_write(self.h, _p(buf) + offset_bytes, a.ctypes.data, a.nbytes))

    def read(self, buf, shape, dtype=np.float32, offset_bytes=0):
        out = np.empty(shape, dtype)
        self._check(lib().wh_read(self.h, out.ctypes.data, _p(buf) + offset_bytes, out.nbytes))
        return out

    def host_array(self, shape, dtype=np.float32):
        """Page-locked host memory (HostArray; its numpy view is `.array`)."""
        return HostArray(self, shape, dtype)

    def read_into(self, buf, out, offset_bytes=0):
        """wh_read into an existing C-contiguous numpy array (e.g. a HostArray's)."""
        self._check(lib().wh_read(self.h, out.ctypes.data, _p(buf) + offset_bytes, out.nbytes))

    def copy(self, dst, src, nbytes):
        """Device-to-device copy of nbytes with the library's copy kernel."""
        self._check(lib().wh_copy(self.h, _p(dst), _p(src), int(nbytes)))

    def zero(self, buf, nbytes=None):
        self._check(lib().wh_zero(self.h, _p(buf), buf.nbytes if nbytes is None else nbytes))

    def sync(self):
        self._check(lib().wh_sync(self.h))

    # -- weights
    def linear(self, tensors, bias=None, pad_k=False):
        """tensors: [(raw GGUF bytes, type, k, rows)], stacked along n (Gpu::linear / conv)."""
        arr = (_Tensor * len(tensors))()
        keep = []
        for i, (raw, ty, k, rows) in enumerate(tensors):
            buf = ctypes.create_string_buffer(bytes(raw), len(raw))
            keep.append(buf)
            arr[i] = _Tensor(ctypes.cast(buf, _vp), ty, k, rows)
        b = None if bias is None else np.ascontiguousarray(bias, np.float32)
        out = _vp()
        self._check(lib().wh_linear_new(self.h, arr, len(tensors), None if b is None else b.ctypes.data,
                                        0 if b is None else b.size, int(pad_k), ctypes.byref(out)))
        return Linear(self, out.value)

    # -- Pass ops
    def gemm(self, a, l, c, m, epi, alpha=0.0):
        self._check(lib().wh_gemm(self.h, _p(a), l.h, _p(c), m, epi, alpha))

    def gemm_h(self, a16, l, c, m, epi, alpha=0.0, out16=False):
        """Pass::gemm with `a` already f16 (and f16 outputs with out16)."""
        self._check(lib().wh_gemm_h(self.h, _p(a16), l.h, _p(c), int(m), int(epi), float(alpha), int(out16)))

    def gemv(self, a, l, c, epi, alpha=0.0, offset=0):
        self._check(lib().wh_gemv(self.h, _p(a), l.h, _p(c), epi, alpha, offset))

    def embed(self, l, pos, c, ids, i, offset):
        self._check(lib().wh_embed(self.h, l.h, _p(pos), _p(c), _p(ids), i, offset))

    def layer_norm(self, x, g, b, y, rows, cols, table=None, yr=None, head_dim=0):
        self._check(lib().wh_layer_norm(self.h, _p(x), _p(g), _p(b), _p(y), rows, cols, _p(table),
                                        _p(yr), head_dim))

    def attend(self, q, kv, part, o, n, cols, heads, hd):
        self._check(lib().wh_attend(self.h, _p(q), _p(kv), _p(part), _p(o), n, cols, heads, hd))

    @staticmethod
    def attend_len(n, heads, hd):
        return lib().wh_attend_len(n, heads, hd)

    def pack(self, x, src, stride, y, rows, d, cols, col):
        self._check(lib().wh_pack(self.h, _p(x), src, stride, _p(y), rows, d, cols, col))

    def im2col(self, x, col, t, ch, kernel, stride, pad):
        self._check(lib().wh_im2col(self.h, _p(x), _p(col), t, ch, kernel, stride, pad))

    def conv_glu(self, h, dw_w, dw_b, kernel, g, b, layer_norm, y, t, ch, valid=-1):
        self._check(lib().wh_conv_glu(self.h, _p(h), _p(dw_w), _p(dw_b), kernel, _p(g), _p(b),
                                      int(layer_norm), _p(y), t, ch, valid))

    def attention(self, qk, v, pos, o, t, heads, hd, valid=-1):
        self._check(lib().wh_attention(self.h, _p(qk), _p(v), _p(pos), _p(o), t, heads, hd, valid))

    def depthwise(self, x, first_w, first_b, w, b, y, t, f, ch, t0, rows):
        self._check(lib().wh_depthwise(self.h, _p(x), _p(first_w), _p(first_b), _p(w), _p(b), _p(y),
                                       t, f, ch, t0, rows))

    def flatten(self, x, y, t, f, ch):
        self._check(lib().wh_flatten(self.h, _p(x), _p(y), t, f, ch))

    def argmax(self, x, out, n):
        self._check(lib().wh_argmax(self.h, _p(x), _p(out), n))


class Model:
    """A GGUF model's encoder (and Whisper decoder) on the device (Model::load, src/lib.rs:556-617)."""

    ARCHS = ("gigaam", "parakeet", "whisper")

    def __init__(self, gpu, path):
        self.gpu = gpu
        h = _vp()
        gpu._check(lib().wh_model_load(gpu.h, path.encode(), ctypes.byref(h)))
        self.h = h.value
        if not hasattr(gpu, "_models"):
            import weakref

            gpu._models = weakref.WeakSet()
        gpu._models.add(self)
        vals = [_i() for _ in range(5)]
        lib().wh_model_info(self.h, *[ctypes.byref(v) for v in vals])
        arch, self.d, self.layers, self.mels, self.width = (v.value for v in vals)
        self.arch = self.ARCHS[arch]

    def free(self):
        if getattr(self, "h", None) and self.gpu.h:
            lib().wh_model_free(self.h)
        self.h = None

    def __del__(self):
        self.free()

    def frames(self, mel_frames):
        f, w = _i(), _i()
        self.gpu._check(lib().wh_model_frames(self.h, mel_frames, ctypes.byref(f), ctypes.byref(w)))
        return f.value, w.value

    def encode_device(self, mel_buf, mel_frames, out_buf, valid=None):
        valid = mel_frames if valid is None else valid
        self.gpu._check(lib().wh_model_encode(self.h, _p(mel_buf), mel_frames, valid, _p(out_buf)))

    def encode(self, mel, valid=None):
        """mel [mel_frames][mels] (host) → encoder output [frames][width] (host)."""
        mel = np.ascontiguousarray(mel, np.float32)
        frames, width = self.frames(mel.shape[0])
        mb = self.gpu.upload(mel)
        ob = self.gpu.buffer(frames * width)
        self.encode_device(mb, mel.shape[0], ob, valid)
        return self.gpu.read(ob, (frames, width))

    def encode_batch_device(self, mel_buf, batch, mel_frames, valid, out_buf):
        v = (ctypes.c_int * batch)(*valid)
        self.gpu._check(lib().wh_model_encode_batch(self.h, _p(mel_buf), batch, mel_frames, v, _p(out_buf)))

    def graphs(self, on):
        """Record repeated encoder calls into HIP graphs and replay them (on), or launch eagerly."""
        self.gpu._check(lib().wh_model_graphs(self.h, int(on)))

    def blocks_device(self, x_buf, t, layers):
        self.gpu._check(lib().wh_model_blocks(self.h, _p(x_buf), t, layers))

    def greedy(self, enc):
        """CTC (GigaAM) or TDT (Parakeet) greedy (token, frame) pairs of a host encoder output."""
        enc = np.ascontiguousarray(enc, np.float32)
        cap = 4 * enc.shape[0] + 16
        out = np.zeros(2 * cap, np.uint32)
        n = lib().wh_model_greedy(self.h, enc.ctypes.data, enc.shape[0], enc.shape[1], out.ctypes.data, cap)
        if n < 0:
            self.gpu._check(n)
        return [(int(out[2 * i]), int(out[2 * i + 1])) for i in range(min(n, cap))]

    def mel_frames(self, samples):
        f = _i()
        self.gpu._check(lib().wh_model_mel(self.h, None, samples, None, ctypes.byref(f)))
        return f.value

    def mel_device(self, pcm_buf, samples, mel_buf):
        """The family's log-mel frontend on the device (wh_model_mel): returns the frame count."""
        f = _i()
        self.gpu._check(lib().wh_model_mel(self.h, _p(pcm_buf), samples, _p(mel_buf), ctypes.byref(f)))
        return f.value

    def mel(self, pcm):
        """Log-mel features [frames][mels] of host audio, computed on the device."""
        pcm = np.ascontiguousarray(pcm, np.float32)
        frames = self.mel_frames(len(pcm))
        if frames == 0:
            return np.zeros((0, self.mels), np.float32)
        pb, mb = self.gpu.upload(pcm if len(pcm) else np.zeros(1, np.float32)), self.gpu.buffer(frames * self.mels)
        self.mel_device(pb, len(pcm), mb)
        return self.gpu.read(mb, (frames, self.mels))

    def greedy_device(self, enc_buf, frames, width, cap=None):
        """The same greedy decoders run on the device over an encoder output in device memory
        (wh_model_greedy_device)."""
        cap = 4 * frames + 16 if cap is None else cap
        out = np.zeros(2 * max(cap, 1), np.uint32)
        n = lib().wh_model_greedy_device(self.h, _p(enc_buf), frames, width, out.ctypes.data, cap)
        if n < 0:
            self.gpu._check(n)
        return [(int(out[2 * i]), int(out[2 * i + 1])) for i in range(min(n, cap))]

    def whisper_begin(self, enc_buf, frames):
        self.gpu._check(lib().wh_whisper_begin(self.h, _p(enc_buf), frames))

    def whisper_step(self, token, pos, logits_buf):
        self.gpu._check(lib().wh_whisper_step(self.h, token, pos, _p(logits_buf)))

    def whisper_ids(self):
        ids = WhisperIds()
        self.gpu._check(lib().wh_whisper_ids_of(self.h, ctypes.byref(ids)))
        return ids

    def whisper_decode(self, enc_buf, frames, prompt=(), cap=512):
        """One window's greedy search on the device (wh_whisper_decode): (generated ids, no-speech
        probability, average log-probability)."""
        p = np.ascontiguousarray(np.asarray(list(prompt) or [0], np.uint32))
        out = np.zeros(cap, np.uint32)
        ns, lp = _f(), _f()
        n = lib().wh_whisper_decode(self.h, _p(enc_buf), frames, p.ctypes.data if prompt else None, len(prompt),
                                    out.ctypes.data, cap, ctypes.byref(ns), ctypes.byref(lp))
        if n < 0:
            self.gpu._check(n)
        return [int(x) for x in out[:min(n, cap)]], ns.value, lp.value
