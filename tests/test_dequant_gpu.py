"""The dequantized weights on the device, bit for bit ("bit-exact on the
dequantized weights"), and the f16 range of GEMM operands.

A GEMM whose rows of `a` are one-hot (a[r][k_r] = 1) returns, with a zero bias, the weights of column
k_r exactly as the kernel fed them to the matrix cores: 1·w is exact and so is its f32 sum with zeros
(a sum that starts from +0 turns a weight of −0 into +0, in the reference's GEMM as here, so the
expected values are the dequantized weights plus +0).
The reference rounds every GEMM weight to f16 after dequantizing (src/cpu/gemm.rs:163-176, to_half at
:209-221; gemm.wgsl:43-51), so the device must return to_half(q·d) for Q8_0 (src/gguf.rs:274-287),
to_half((nibble − 8)·d) for Q4_0 (ggml block_q4_0) and the stored half for F16.  The GEMV does not
round W (src/cpu/gemm.rs:181-208, gemm.wgsl:244-307): a one-hot activation row returns q·d in f32.
"""

import numpy as np
import pytest

import oracle as ox
import wavo_amd as wa
from wavo_amd import gguf

pytestmark = pytest.mark.gpu


def weights(n, k, seed):
    rng = np.random.default_rng(seed)
    w = rng.standard_normal((n, k), dtype=np.float32) * np.float32(0.02)
    # Blocks whose scale is subnormal in f16, and ones with large values (scale near the top of f16).
    w[0, :32] *= np.float32(1e-4)
    w[1, 32:64] *= np.float32(2e5)
    w[2, :] = 0.0
    return w


@pytest.mark.parametrize("wtype", [wa.Q8_0, wa.Q4_0, wa.F16])
@pytest.mark.parametrize("n,k", [(192, 256), (1024, 1024), (64, 4096)])
def test_gemm_weights_bit_exact(gpu, wtype, n, k):
    w = weights(n, k, n + k)
    raw = gguf.encode(w, wtype)
    deq = ox.dequant(raw, wtype, n * k).reshape(n, k)
    want = np.array([ox.lib().ox_to_half(float(x)) for x in deq.ravel()], np.float32).reshape(n, k)
    assert np.array_equal(want, deq.astype(np.float16).astype(np.float32))  # in range: IEEE RNE
    want = want + np.float32(0.0)  # Σ from +0: −0 becomes +0
    lin = gpu.linear([(raw, wtype, k, n)])
    a = np.eye(k, dtype=np.float32)  # row r picks weight column r
    ab, cb = gpu.upload(a), gpu.buffer(k * lin.width)
    gpu.gemm(ab, lin, cb, k, wa.BIAS)
    got = gpu.read(cb, (k, lin.width))[:, :n].T
    bad = np.argwhere(got.view(np.uint32) != want.view(np.uint32))
    assert bad.size == 0, f"{len(bad)} weights differ, first {tuple(bad[0])}: {got[tuple(bad[0])]} vs {want[tuple(bad[0])]}"
    # The same through the f16-input entry point (the graph drivers' form).
    a16 = gpu.upload(a.astype(np.float16))
    gpu.gemm_h(a16, lin, cb, k, wa.BIAS)
    got = gpu.read(cb, (k, lin.width))[:, :n].T
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("wtype", [wa.Q8_0, wa.Q4_0, wa.F16])
def test_gemv_weights_unrounded(gpu, wtype):
    n, k = 256, 1280
    w = weights(n, k, 5)
    raw = gguf.encode(w, wtype)
    deq = ox.dequant(raw, wtype, n * k).reshape(n, k)
    lin = gpu.linear([(raw, wtype, k, n)])
    cb = gpu.buffer(lin.width)
    for col in (0, 33, 700, k - 1):
        x = np.zeros(k, np.float32)
        x[col] = 1.0
        gpu.gemv(gpu.upload(x), lin, cb, wa.BIAS)
        got = gpu.read(cb, (lin.width,))[:n]
        want = deq[:, col] + np.float32(0.0)  # Σ from +0: −0 becomes +0
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), f"column {col}"


def test_activation_past_the_f16_range(gpu):
    """Operands past ±65504 do not fit an f16 MFMA operand: the device rounds them to ±inf (IEEE), where
    the reference's to_half keeps their exponent (src/cpu/gemm.rs:209-221; the oracle does too).  This is
    the documented divergence; in range both give IEEE round-to-nearest-even."""
    assert ox.lib().ox_to_half(70000.0) == 70016.0  # the reference's rule, pinned in the oracle
    n, k, m = 64, 64, 2
    w = np.full((n, k), 0.5, np.float32)
    lin = gpu.linear([(gguf.encode(w, wa.F16), wa.F16, k, n)])
    a = np.zeros((m, k), np.float32)
    a[0, 3] = 70000.0   # past the range: inf
    a[1, 3] = 65504.0   # the largest half: exact
    cb = gpu.buffer(m * n)
    gpu.gemm(gpu.upload(a), lin, cb, m, wa.BIAS)
    got = gpu.read(cb, (m, n))
    assert np.all(np.isposinf(got[0]))
    assert np.all(got[1] == np.float32(65504.0 * 0.5))
