"""Failure handling on the device, forced from the host: allocations larger than the device's memory
return WH_EOOM (Error::Gpu, fatal to the reference's caller, src/error.rs:129-140) with a message, and
bad shapes return WH_EARG; in every case nothing was queued and the context keeps working (a copy
round trip and a GEMM against numpy afterwards)."""

import ctypes

import numpy as np
import pytest

import wavo_amd as wa
from wavo_amd import gguf

pytestmark = pytest.mark.gpu


def still_works(gpu):
    x = np.arange(4096, dtype=np.float32)
    b = gpu.upload(x)
    assert np.array_equal(gpu.read(b, (4096,)), x)
    rng = np.random.default_rng(0)
    w = (rng.standard_normal((64, 64)) * 0.1).astype(np.float32)
    a = rng.standard_normal((8, 64)).astype(np.float32)
    lin = gpu.linear([(w.tobytes(), gguf.F32, 64, 64)])
    ab, cb = gpu.upload(a), gpu.buffer(8 * 64)
    gpu.gemm(ab, lin, cb, 8, wa.BIAS)
    # The GEMM rounds both operands to f16 (Pass::gemm): compare with the f16-rounded product.
    want = a.astype(np.float16).astype(np.float64) @ w.astype(np.float16).astype(np.float64).T
    assert np.allclose(gpu.read(cb, (8, 64)), want, rtol=0, atol=1e-4)


def test_alloc_past_device_memory(gpu):
    p = ctypes.c_void_p()
    rc = wa.lib().wh_alloc(gpu.h, 1 << 40, ctypes.byref(p))  # 4 TiB
    assert rc == wa.EOOM
    assert "hipMalloc" in wa.lib().wh_last_error(gpu.h).decode()
    still_works(gpu)


def test_linear_past_device_memory(gpu):
    # 3·10⁶ rows of 32768 f32 weights (393 GB): the device allocation fails before any weight is read,
    # so a small host buffer stands for the data.
    raw = ctypes.create_string_buffer(64)
    t = wa._Tensor(ctypes.cast(raw, ctypes.c_void_p), gguf.F32, 32768, 3_000_000)
    out = ctypes.c_void_p()
    rc = wa.lib().wh_linear_new(gpu.h, ctypes.byref(t), 1, None, 0, 0, ctypes.byref(out))
    assert rc == wa.EOOM and not out.value
    assert "weights" in wa.lib().wh_last_error(gpu.h).decode()
    still_works(gpu)


def test_bad_shapes_leave_context_usable(gpu):
    w = np.zeros((64, 64), np.float32)
    lin = gpu.linear([(w.tobytes(), gguf.F32, 64, 64)])
    a, c = gpu.buffer(64), gpu.buffer(64)
    with pytest.raises(wa.WavoError) as e:
        gpu.gemm(a, lin, c, -1, wa.BIAS)  # m < 0
    assert e.value.code == wa.EARG
    with pytest.raises(wa.WavoError) as e:
        gpu.gemv(a, lin, c, 99)  # no such epilogue
    assert e.value.code == wa.EARG
    with pytest.raises(wa.WavoError) as e:
        gpu.linear([(w.tobytes(), gguf.F32, 64, 64), (w[:, :32].copy().tobytes(), gguf.F32, 32, 64)])
    assert e.value.code == wa.EARG
    still_works(gpu)


def test_whisper_window_past_the_model(gpu):
    # More encoder frames than the model's window: refused with a message naming both counts, before
    # the decoder's buffers exist; a fitting call afterwards works.
    from wavo_amd import synth

    m = wa.Model(gpu, synth.model_path("whisper", small=True))
    frames, width = m.frames(1)  # Whisper: the model's window, whatever the mel
    enc = gpu.buffer((frames + 64) * width)
    with pytest.raises(wa.WavoError) as e:
        m.whisper_begin(enc, frames + 64)
    assert e.value.code == wa.EARG and f"{frames + 64} encoder frames" in str(e.value)
    gpu.zero(enc)
    m.whisper_begin(enc, frames)
    m.free()
    still_works(gpu)
