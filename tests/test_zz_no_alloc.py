"""wh_gemm_noalloc, the GEMM entry point that allocates nothing (its workspace is a fixed device array),
against wh_gemm, the entry point it varies, through the C ABI: bit for bit equal outputs on two calls in
a row, the second with a smaller input (the workspace keeps the first call's contents), a call whose
workspace would exceed the limit refused without launching, and a call from another stream refused
while the device's previous call may still run."""

import ctypes

import numpy as np
import pytest

import wavo_amd as wa
from wavo_amd import gguf

pytestmark = pytest.mark.gpu


def layer(gpu, n, k, wtype, seed):
    rng = np.random.default_rng(seed)
    w = rng.standard_normal(n * k, dtype=np.float32) * np.float32(0.02)
    bias = rng.standard_normal(n, dtype=np.float32) * np.float32(0.02)
    return gpu.linear([(gguf.encode(w, wtype), wtype, k, n)], bias)


def noalloc(gpu, a, lin, c, m, epi, alpha=0.0):
    L = wa.lib()
    L.wh_gemm_noalloc.restype = ctypes.c_int
    L.wh_gemm_noalloc.argtypes = [ctypes.c_void_p] * 4 + [ctypes.c_int, ctypes.c_int, ctypes.c_float]
    return L.wh_gemm_noalloc(gpu.h, a.ptr, lin.h, c.ptr, m, epi, alpha)


# (m, n, k, type, epilogue) of two calls in a row: the first splits k four ways (partial sums in the
# workspace after the rounded a), the second is smaller and whole; on three weight types.
CASES = [
    [(750, 1024, 4096, wa.Q8_0, wa.RESIDUAL), (300, 1024, 1024, wa.Q8_0, wa.SILU)],
    [(750, 1280, 5120, wa.Q4_0, wa.GELU), (37, 768, 3072, wa.F16, wa.BIAS)],
]


@pytest.mark.parametrize("calls", CASES)
def test_noalloc_equals_gemm(gpu, calls):
    limit = wa.lib().wh_gemm_noalloc_limit()
    assert limit == 32 << 20
    for i, (m, n, k, wtype, epi) in enumerate(calls):
        lin = layer(gpu, n, k, wtype, 10 + i)
        a = gpu.upload(np.random.default_rng(20 + i).standard_normal((m, k), dtype=np.float32))
        c0 = np.random.default_rng(30 + i).standard_normal(m * lin.width, dtype=np.float32)
        want_b, got_b = gpu.upload(c0), gpu.upload(c0)
        gpu.gemm(a, lin, want_b, m, epi, 0.5)
        rc = noalloc(gpu, a, lin, got_b, m, epi, 0.5)
        assert rc == 0, wa.lib().wh_last_error(gpu.h).decode()
        want = gpu.read(want_b, (m, lin.width))
        got = gpu.read(got_b, (m, lin.width))
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), f"call {i}: {m}x{n}x{k}"


def test_noalloc_refuses_past_its_workspace(gpu):
    m, n, k = 12000, 1024, 4096  # the f16 copy of a alone is 98 MB
    lin = layer(gpu, n, k, wa.Q8_0, 3)
    a, c = gpu.buffer(m * k), gpu.buffer(m * lin.width)
    rc = noalloc(gpu, a, lin, c, m, wa.BIAS)
    assert rc == wa.EARG
    assert "workspace" in wa.lib().wh_last_error(gpu.h).decode()
    # The context still works afterwards.
    small = gpu.upload(np.ones((16, k), np.float32))
    assert noalloc(gpu, small, lin, c, 16, wa.BIAS) == 0
    gpu.sync()


def test_noalloc_refuses_an_overlapping_call_from_another_stream(gpu):
    # Two contexts on device 0, each with its own stream: while the first context's queued calls may
    # still run, a call from the second is refused (the workspace is shared); once the first has
    # drained, the second's call runs and equals wh_gemm.
    # ~80 µs of kernels per call (no k split: 8 MB of workspace), more than the ~20 µs a call takes to queue
    m, n, k = 2048, 4096, 2048
    other = wa.Gpu(0)
    try:
        lin1, lin2 = layer(gpu, n, k, wa.Q8_0, 5), layer(other, n, k, wa.Q8_0, 5)
        rng = np.random.default_rng(6)
        x = rng.standard_normal((m, k), dtype=np.float32)
        a1, a2 = gpu.upload(x), other.upload(x)
        c1, c2, want_b = gpu.buffer(m * lin1.width), other.buffer(m * lin2.width), other.buffer(m * lin2.width)
        gpu.sync()
        for _ in range(40):  # a backlog of ~2 ms queued on the first context's stream
            assert noalloc(gpu, a1, lin1, c1, m, wa.BIAS) == 0, wa.lib().wh_last_error(gpu.h).decode()
        rc = noalloc(other, a2, lin2, c2, m, wa.BIAS)
        assert rc == wa.EARG, "an overlapping call from another stream was accepted"
        assert "overlap" in wa.lib().wh_last_error(other.h).decode()
        gpu.sync()
        assert noalloc(other, a2, lin2, c2, m, wa.BIAS) == 0, wa.lib().wh_last_error(other.h).decode()
        other.gemm(a2, lin2, want_b, m, wa.BIAS)
        got, want = other.read(c2, (m, lin2.width)), other.read(want_b, (m, lin2.width))
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
        other.sync()
    finally:
        other.close()
