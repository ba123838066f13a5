"""Pins of the CPU oracle (oracle/*.c) before it is trusted as the parity reference.

Each function is checked against the reference's own known answers where its unit tests hold them
(src/gguf.rs:451-483, src/cpu/gemm.rs:567-657, src/cpu/mod.rs:471-527, src/parakeet/decoder.rs:193-258,
src/parakeet/mod.rs:154-164), else against closed forms or brute force in float64 numpy, chosen so a
dropped term, a wrong sign or a transposed operand fails.  CPU only.
"""

import math
import struct

import numpy as np
import pytest

import oracle as ox
from wavo_amd import gguf, synth


def f16_bits(x):
    return struct.unpack("<H", np.float16(x).tobytes())[0]


# ------------------------------------------------------------------------------ formats


def test_q8_0_block_known_answer():
    # src/gguf.rs:451-483: one block with d = 0.5 and q = i − 16 reads as (i − 16)·0.5.
    raw = struct.pack("<H", f16_bits(0.5)) + bytes((i - 16) & 0xFF for i in range(32))
    got = ox.dequant(raw, ox.Q8_0, 32)
    assert np.array_equal(got, (np.arange(32) - 16) * 0.5)
    assert np.array_equal(gguf.dequantize(raw, gguf.Q8_0, 32), got)


def test_q4_0_block_layout():
    # ggml block_q4_0: d, then 16 bytes; element i < 16 is the low nibble of byte i, 16 + i the high.
    qs = bytes((i & 15) | (((15 - i) & 15) << 4) for i in range(16))
    raw = struct.pack("<H", f16_bits(2.0)) + qs
    want = np.concatenate([np.arange(16) - 8, (15 - np.arange(16)) - 8]) * 2.0
    assert np.array_equal(ox.dequant(raw, ox.Q4_0, 32), want)
    assert np.array_equal(gguf.dequantize(raw, gguf.Q4_0, 32), want)


@pytest.mark.parametrize("wtype", [gguf.Q8_0, gguf.Q4_0, gguf.F16, gguf.F32])
def test_quantizers_agree_and_bound_the_error(wtype):
    x = np.random.default_rng(1).normal(0, 1, 32 * 64).astype(np.float32)
    x[:32] = 0.0  # an all-zero block: d = 0
    raw = gguf.encode(x, wtype)
    assert raw == ox.quantize(x, wtype)
    back = ox.dequant(raw, wtype, x.size)
    b = x.reshape(-1, 32)
    err = np.abs(back.reshape(-1, 32) - b).max(axis=1)
    amax = np.abs(b).max(axis=1)
    # Q8_0: half a step of amax/127 (+ the f16 rounding of d); Q4_0: a step of amax/8.
    bound = {gguf.Q8_0: amax / 127 * 0.51 + 1e-3 * amax, gguf.Q4_0: amax / 8 * 1.01 + 1e-6,
             gguf.F16: amax * 2.0 ** -11, gguf.F32: 0 * amax}[wtype]
    assert np.all(err <= bound + 1e-12)


def test_q8_0_quantizer_known_answer():
    # d = 127/127 = 1; q = round-half-away(x): 0.5 → 1, −0.5 → −1, 2.5 → 3, 127 stays.
    x = np.zeros(32, np.float32)
    x[:5] = [127.0, 0.5, -0.5, 2.5, -126.49]
    raw = gguf.quantize_q8_0(x)
    assert struct.unpack("<H", raw[:2])[0] == f16_bits(1.0)
    assert list(np.frombuffer(raw[2:7], np.int8)) == [127, 1, -1, 3, -126]


def test_to_half_matches_ieee_below_the_range():
    # src/cpu/gemm.rs:606-614: to_half == half::f16::from_f32 over normal and subnormal halves.
    bits = np.arange(0x30000000, 0x47700000, 4093, dtype=np.uint32)
    x = bits.view(np.float32)
    for v in (x, -x):
        got = ox.to_half(v)
        assert np.array_equal(got, v.astype(np.float16).astype(np.float32))


def test_to_half_keeps_the_exponent_past_the_range():
    # Values past the f16 range keep their exponent with 10 mantissa bits (gemm.wgsl:43-51).
    for v in (1e6, -3.5e5, 65520.0, 1.0e30):
        b = np.float32(v).view(np.uint32)
        want = np.uint32((int(b) + 0xFFF + ((int(b) >> 13) & 1)) & 0xFFFFE000).view(np.float32)
        assert ox.to_half(np.float32(v)) == want
        assert np.isfinite(ox.to_half(np.float32(v)))


def test_exp_silu_gelu_against_closed_forms():
    x = np.linspace(-20, 20, 4001).astype(np.float32)
    L = ox.lib()
    e = np.array([L.ox_exp(float(v)) for v in x])
    assert np.max(np.abs(e / np.exp(x.astype(np.float64)) - 1)) < 3e-7
    s = np.array([L.ox_silu(float(v)) for v in x])
    assert np.max(np.abs(s - x / (1 + np.exp(-x.astype(np.float64))))) < 1e-5
    g = np.array([L.ox_gelu(float(v)) for v in x])
    exact = np.array([0.5 * v * (1 + math.erf(v / math.sqrt(2))) for v in x.astype(np.float64)])
    # A&S 7.1.26 approximates erf within 1.5e-7.
    assert np.max(np.abs(g - exact) / np.maximum(1, np.abs(x))) < 5e-7
    assert L.ox_gelu(0.0) == 0.0


def test_dot_is_sixteen_lanes_summed_pairwise():
    a = np.random.default_rng(2).normal(size=333).astype(np.float32)
    b = np.random.default_rng(3).normal(size=333).astype(np.float32)
    acc = np.zeros(16, np.float32)
    for i in range(0, 320, 16):
        acc = (acc.astype(np.float64) + a[i:i + 16].astype(np.float64) * b[i:i + 16]).astype(np.float32)
    # fma per lane: the product is exact in f64, one rounding per step as an f32 FMA.
    for w in (8, 4, 2, 1):
        acc[:w] = acc[:w] + acc[w:2 * w]
    tail = np.float32(0)
    for i in range(320, 333):
        tail = np.float32(tail + np.float32(a[i] * b[i]))
    want = np.float32(acc[0] + tail)
    got = ox.lib().ox_dot(a.ctypes.data_as(ox._fp), b.ctypes.data_as(ox._fp), 333)
    assert np.float32(got) == want


# ---------------------------------------------------------------------------------- GEMM


def exact_weights(n, k):
    # src/cpu/gemm.rs:578-604: q/8 with q in −15..=15, exact in all three types; Q8_0 with d = 1/8.
    v = ((np.arange(n * k) * 7919 % 31) / 8 - 15 / 8).astype(np.float32)
    q8 = b"".join(struct.pack("<H", f16_bits(0.125)) + (v[i:i + 32] * 8).astype(np.int8).tobytes()
                  for i in range(0, v.size, 32))
    return v.reshape(n, k), {ox.F32: v.tobytes(), ox.F16: v.astype(np.float16).tobytes(), ox.Q8_0: q8}


@pytest.mark.parametrize("wtype", [ox.F32, ox.F16, ox.Q8_0])
def test_gemm_matches_dot(wtype):
    k, n, m = 64, 40, 13
    v, raws = exact_weights(n, k)
    a = ((np.arange(m * k) * 31 % 17) / 8 - 1).astype(np.float32).reshape(m, k)
    bias = (np.arange(n) / 4).astype(np.float32)
    l = ox.Linear(wtype, k, [(raws[wtype], n)], bias)
    c = ox.gemm(a, l, m, ox.RESIDUAL, 0.5, c=np.ones((m, n), np.float32))
    want = 1 + 0.5 * (a.astype(np.float64) @ v.T.astype(np.float64) + bias)
    # Every product and partial sum is a multiple of 1/64 below 2^10: exact in f32.
    assert np.array_equal(c, want.astype(np.float32))


def test_gemm_rounds_both_operands_to_half():
    # h(a)·h(W): a value between two halves must enter the product rounded (src/cpu/gemm.rs:163-176).
    k, n, m = 32, 1, 1
    a = np.full((m, k), 1 + 2 ** -12, np.float32)   # rounds to 1.0 in f16
    w = np.full((n, k), 1 + 3 * 2 ** -12, np.float32)  # rounds to 1 + 2^-10
    l = ox.Linear(ox.F32, k, [(w.tobytes(), n)])
    c = ox.gemm(a, l, m, ox.BIAS)
    assert c[0, 0] == np.float32(k * (1 + 2 ** -10))


def test_gemm_wide_padding_and_dual_layout():
    # 164 rows: width 192 (rows % 32 != 0 → rounded to 64); columns 164..191 are epi(0); 64 dual
    # outputs repeat the first 64 at 192.. with their own bias and no epilogue (src/gpu/mod.rs:1878-1945).
    k, n, m = 64, 164, 5
    w = np.random.default_rng(4).uniform(-1, 1, (n, k)).astype(np.float32)
    a = np.random.default_rng(5).uniform(-1, 1, (m, k)).astype(np.float32)
    bias = np.random.default_rng(6).uniform(-1, 1, n).astype(np.float32)
    bias2 = np.random.default_rng(7).uniform(-1, 1, 64).astype(np.float32)
    l = ox.Linear(ox.F32, k, [(w.tobytes(), n)], bias)
    c0 = np.random.default_rng(8).uniform(-1, 1, (m, 256)).astype(np.float32)
    got = ox.gemm_wide(a, l, m, ox.RESIDUAL, 0.5, c=c0, bias2=bias2, dual=64)
    dot = ox.to_half(a).astype(np.float64) @ ox.to_half(w).astype(np.float64).T
    want = c0.astype(np.float64).copy()
    want[:, :n] += 0.5 * (dot + bias)
    want[:, 192:] = dot[:, :64] + bias2
    assert np.allclose(got, want, atol=1e-5)


@pytest.mark.parametrize("wtype", [ox.F32, ox.Q8_0])
def test_gemv_is_dot_on_the_dequantized_row(wtype):
    # src/cpu/gemm.rs:616-640: gemv == gelu(dot(row, x) + b), bit for bit; W not rounded.
    k, n = 96, 70
    v, raws = exact_weights(n, k)
    x = ((np.arange(k) * 31 % 17) / 8 - 1).astype(np.float32)
    bias = (np.arange(n) / 4).astype(np.float32)
    l = ox.Linear(wtype, k, [(raws[wtype], n)], bias)
    got = ox.gemv(x, l, ox.GELU)
    L = ox.lib()
    want = [L.ox_gelu(float(np.float32(L.ox_dot(np.ascontiguousarray(v[j]).ctypes.data_as(ox._fp),
                                                  x.ctypes.data_as(ox._fp), k)) + bias[j])) for j in range(n)]
    assert np.array_equal(got, np.array(want, np.float32))


def test_linear_rows_load_every_type():
    # src/cpu/mod.rs:497-527: rows of 64 values exact in every type read back unchanged.
    v, raws = exact_weights(70, 64)
    for wtype, raw in raws.items():
        assert np.array_equal(ox.dequant(raw, wtype, v.size).reshape(v.shape), v)


# ----------------------------------------------------------------------------- row ops


def ln64(x, g, b):
    x = x.astype(np.float64)
    mean = x.mean(axis=1, keepdims=True)
    var = ((x - mean) ** 2).mean(axis=1, keepdims=True)
    return (x - mean) / np.sqrt(var + 1e-5) * g + b


def test_layer_norm_and_rope():
    rows, cols, hd = 9, 96, 48
    x = np.random.default_rng(5).normal(size=(rows, cols)).astype(np.float32)
    g, b = np.random.default_rng(6).normal(size=cols), np.random.default_rng(7).normal(size=cols)
    table = np.random.default_rng(8).normal(size=(rows, hd)).astype(np.float32)
    y, yr = ox.layer_norm(x, g, b, table, hd)
    want = ln64(x, g, b)
    assert np.allclose(y, want, atol=2e-5)
    half = hd // 2
    wr = np.empty_like(want)
    for h0 in range(0, cols, hd):
        y0, y1 = want[:, h0:h0 + half], want[:, h0 + half:h0 + hd]
        c, s = table[:, :half], table[:, half:]
        wr[:, h0:h0 + half] = y0 * c - y1 * s
        wr[:, h0 + half:h0 + hd] = y1 * c + y0 * s
    assert np.allclose(yr, wr, atol=5e-5)


def test_im2col_known_layout():
    t, ch, kernel, stride, pad = 7, 3, 3, 2, 1
    x = np.arange(t * ch, dtype=np.float32).reshape(t, ch) + 1
    col = ox.im2col(x, t, ch, kernel, stride, pad, 32)
    rows = (t + 2 * pad - kernel) // stride + 1
    for i in range(rows):
        for c in range(ch):
            for k in range(kernel):
                s = stride * i + k - pad
                assert col[i, c * kernel + k] == (x[s, c] if 0 <= s < t else 0)
    assert not col[:, ch * kernel:].any()


@pytest.mark.parametrize("layer_norm", [True, False])
@pytest.mark.parametrize("valid", [-1, 11])
def test_conv_glu_brute_force(layer_norm, valid):
    t, ch, kernel = 17, 24, 5
    rng = np.random.default_rng(9)
    h = rng.normal(size=(t, 2 * ch)).astype(np.float32)
    taps, tb = rng.normal(size=(kernel, ch)).astype(np.float32), rng.normal(size=ch).astype(np.float32)
    g, beta = rng.normal(size=ch).astype(np.float32), rng.normal(size=ch).astype(np.float32)
    got = ox.conv_glu(h, taps, tb, kernel, g, beta, layer_norm, t, ch, valid)
    hd = h.astype(np.float64)
    glu = hd[:, :ch] / (1 + np.exp(-hd[:, ch:]))
    if valid >= 0:
        glu[valid:] = 0
    acc = np.tile(tb.astype(np.float64), (t, 1))
    for i in range(t):
        for k in range(kernel):
            s = i + k - kernel // 2
            if 0 <= s < t:
                acc[i] += taps[k] * glu[s]
    y = ln64(acc, g, beta) if layer_norm else acc * g + beta
    want = y / (1 + np.exp(-y))
    assert np.allclose(got, want, atol=1e-5)


def softmax_attn(s, v, valid):
    s = s.copy()
    s[:, valid:] = -np.inf
    p = np.exp(s - s.max(axis=1, keepdims=True))
    return (p / p.sum(axis=1, keepdims=True)) @ v


@pytest.mark.parametrize("valid", [-1, 13])
def test_attention_brute_force(valid):
    t, heads, hd = 29, 3, 16
    d = heads * hd
    rng = np.random.default_rng(10)
    qk, v = rng.normal(size=(t, 2 * d)).astype(np.float32), rng.normal(size=(t, d)).astype(np.float32)
    got = ox.attention(qk, 2 * d, v, d, t, heads, hd, valid)
    nv = t if valid < 0 else valid
    for h in range(heads):
        q = qk[:, h * hd:(h + 1) * hd].astype(np.float64)
        k = qk[:, d + h * hd:d + (h + 1) * hd].astype(np.float64)
        want = softmax_attn(q @ k.T / math.sqrt(hd), v[:, h * hd:(h + 1) * hd].astype(np.float64), nv)
        assert np.allclose(got[:, h * hd:(h + 1) * hd], want, atol=2e-6)


@pytest.mark.parametrize("valid", [-1, 20])
def test_relative_attention_brute_force(valid):
    # score(i, j) = ((q+u)_i·k_j + (q+v)_i·P[j − i + t + 15]) / √hd (src/cpu/ops.rs:223-273).
    t, heads, hd = 23, 2, 16
    d = heads * hd
    rng = np.random.default_rng(11)
    qkv = rng.normal(size=(t, 3 * d)).astype(np.float32)
    pos = rng.normal(size=(2 * t + 15, d)).astype(np.float32)
    u, vb = rng.normal(size=d).astype(np.float32), rng.normal(size=d).astype(np.float32)
    got = ox.relative_attention(qkv, pos, u, vb, t, heads, hd, valid)
    nv = t if valid < 0 else valid
    for h in range(heads):
        sl = slice(h * hd, (h + 1) * hd)
        q, k, v = (qkv[:, o + h * hd:o + (h + 1) * hd].astype(np.float64) for o in (0, d, 2 * d))
        s = np.empty((t, t))
        for i in range(t):
            for j in range(t):
                s[i, j] = (q[i] + u[sl]) @ k[j] + (q[i] + vb[sl]) @ pos[j - i + t + 15, sl]
        want = softmax_attn(s / math.sqrt(hd), v, nv)
        assert np.allclose(got[:, sl], want, atol=2e-6)


def test_attend_rounds_the_query_to_half():
    heads, hd, cols, n = 2, 16, 40, 33
    rng = np.random.default_rng(12)
    q = rng.normal(size=heads * hd).astype(np.float32)
    kv = rng.normal(size=(2 * heads, cols, hd)).astype(np.float16).astype(np.float32)
    got = ox.attend(q, kv, cols, n, heads, hd)
    qh = q.astype(np.float16).astype(np.float64)
    for h in range(heads):
        k, v = kv[h, :n].astype(np.float64), kv[heads + h, :n].astype(np.float64)
        s = k @ qh[h * hd:(h + 1) * hd] / math.sqrt(hd)
        p = np.exp(s - s.max())
        assert np.allclose(got[h * hd:(h + 1) * hd], p @ v / p.sum(), atol=2e-6)


def test_pack_layout_known_answer():
    # decode.wgsl:148-173 and the reference test :2108-2128: K transposed, then V by position.
    x = np.random.default_rng(7).uniform(-1, 1, 3 + 13 * 2).astype(np.float32)
    for rows, col in ((1, 4), (2, 5)):
        y = np.random.default_rng(9).integers(0, 2 ** 32, 42, dtype=np.uint64).astype(np.uint32)
        got = ox.pack(x, 3, 13, y, rows, 6, 7, col)
        want = y.copy()
        h = lambda v: f16_bits(v)
        for j in range(rows):
            pair = lambda i: h(x[3 + 13 * j + 2 * i]) | (h(x[4 + 13 * j + 2 * i]) << 16)
            for i in range(3):
                want[i * 7 + col + j] = pair(i)
                want[3 * 7 + (col + j) * 3 + i] = pair(3 + i)
        assert np.array_equal(got, want)


def test_position_tables_closed_form():
    d, t = 64, 10
    got = ox.rel_positions(d, t + 15, 2 * t + 15)
    pos = (t + 15 - np.arange(2 * t + 15))[:, None].astype(np.float64)
    div = np.exp(np.arange(0, d, 2) * (-math.log(10000.0) / d))
    assert np.allclose(got[:, 0::2], np.sin(pos * div), atol=2e-5)
    assert np.allclose(got[:, 1::2], np.cos(pos * div), atol=2e-5)
    r = ox.rope_table(12, 48, 5000.0)
    ang = np.arange(12)[:, None] * 5000.0 ** (-2.0 * np.arange(24) / 48)
    assert np.allclose(r[:, :24], np.cos(ang), atol=1e-7) and np.allclose(r[:, 24:], np.sin(ang), atol=1e-7)


def depthwise64(x, w, b, t, f, ch):
    fo = (f - 1) // 2 + 1
    out = np.zeros(((t - 1) // 2 + 1, fo, ch))
    for r in range(out.shape[0]):
        for j in range(fo):
            acc = b.astype(np.float64).copy()
            for k in range(9):
                ti, fi = 2 * r + k // 3 - 1, 2 * j + k % 3 - 1
                if 0 <= ti < t and 0 <= fi < f:
                    acc += w[k] * x[ti, fi]
            out[r, j] = acc
    return out


@pytest.mark.parametrize("valid_drop", [0, 1])
def test_subsampling_brute_force(valid_drop):
    # The reference's subsampling test (src/gpu/mod.rs:2256-2295) in float64.
    t, f, ch = 29, 11, 5
    valid = t - valid_drop
    rng = np.random.default_rng(19)
    mel = rng.uniform(-1, 1, (t, f)).astype(np.float32)
    w0, w2, w5 = (rng.uniform(-1, 1, (9, ch)).astype(np.float32) for _ in range(3))
    b0, b2, b5 = (rng.uniform(-1, 1, ch).astype(np.float32) for _ in range(3))
    wide = np.repeat(mel[:, :, None], ch, axis=2)
    first = np.maximum(depthwise64(wide[:valid], w0, b0, valid, f, ch), 0)
    h = lambda n: (n - 1) // 2 + 1
    second = depthwise64(first, w2, b2, h(valid), h(f), ch)
    t2, f2 = h(h(t)), h(h(f))
    sec = np.zeros((t2, f2, ch))
    sec[:second.shape[0]] = second
    want = depthwise64(sec, w5, b5, t2, f2, ch)
    got = np.zeros_like(want)
    for t0 in (0, 2):
        c = ox.sub_first(mel, valid, f, w0, b0, w2, b2, ch, 5, t0)
        # Chunk rows 2·t0 − 1 …: compare the ones inside the image.
        for k in range(5):
            r = 2 * t0 + k - 1
            if 0 <= r < t2:
                assert np.allclose(c[k], sec[r], atol=1e-5)
        got[t0:t0 + 2] = ox.depthwise(c, w5, b5, t2, f2, ch, 2, t0)
    assert np.allclose(got, want, atol=1e-5)
    x = rng.normal(size=(t, f, ch)).astype(np.float32)
    assert np.array_equal(ox.flatten(x, t, f, ch), x.transpose(0, 2, 1).reshape(t, ch * f))


# ------------------------------------------------------------------------- decoders


BLANK = 9


def test_tdt_blank_moves_on_and_tokens_stay():
    # src/parakeet/decoder.rs:234-242.
    out, calls = ox.tdt_scripted(6, BLANK, [0, 1, 3], 10, False, [(BLANK, 0), (5, 0), (6, 2), (BLANK, 1), (7, 1)])
    assert out == [(5, 1), (6, 1), (7, 5)]
    assert calls == [(0, None), (1, None), (1, 5), (4, 6), (5, None)]


def test_tdt_ten_decisions_per_frame():
    # src/parakeet/decoder.rs:244-255.
    script = [(5, 0)] * 19 + [(BLANK, 0), (6, 1)]
    out, calls = ox.tdt_scripted(3, BLANK, [0, 1], 10, False, script)
    assert [f for _, f in out] == [0] * 10 + [1] * 9 + [2]
    assert sum(1 for c in calls if c[0] == 1) == 10
    assert len(calls) == len(script)


def test_tdt_global_budget():
    # src/parakeet/decoder.rs:257-268.
    script = [(5, 0)] * 12 + [(BLANK, 0)] + [(6, 0)] * 7
    out, calls = ox.tdt_scripted(2, BLANK, [0, 1], 10, True, script)
    assert [f for _, f in out] == [0] * 12 + [1] * 7
    assert len(calls) == 20


def test_ctc_collapses_repeats_then_drops_blanks():
    # src/gigaam/decoder.rs:135-151: first-max argmax, repeats of the previous frame dropped, blanks.
    ids = [3, 3, 0, 3, 1, 1, 0, 0, 2, 3]
    logits = np.zeros((len(ids), 5), np.float32)
    for t, i in enumerate(ids):
        logits[t, i] = 1.0
    logits[4, 4] = 1.0  # a tie: the lower index wins
    assert ox.ctc(logits, 0) == [(3, 0), (3, 3), (1, 4), (2, 8), (3, 9)]


def test_encoder_frames_table(tmp_path):
    # src/parakeet/mod.rs:154-164.
    m = ox.Model(synth.write_model(str(tmp_path / "p.gguf"), dict(synth.SMALL["parakeet"], layers=1)))
    import ctypes
    fr, w = ctypes.c_int(), ctypes.c_int()
    for mel_frames, want in [(3, 1), (8, 1), (9, 1), (10, 2), (16, 2), (17, 2), (18, 3), (505, 63), (1057, 132)]:
        ox.lib().ox_model_encode(m.h, None, mel_frames, mel_frames, None, ctypes.byref(fr), ctypes.byref(w))
        assert fr.value == want, mel_frames


def test_model_rejects_a_corrupt_file(tmp_path):
    p = tmp_path / "bad.gguf"
    p.write_bytes(b"GGUF" + struct.pack("<IQQ", 2, 0, 0))
    with pytest.raises(ValueError, match="version"):
        ox.Model(str(p))
    good = synth.write_model(str(tmp_path / "g.gguf"), dict(synth.SMALL["gigaam"], layers=1))
    data = open(good, "rb").read()
    (tmp_path / "trunc.gguf").write_bytes(data[: len(data) // 2])
    with pytest.raises(ValueError, match="bounds"):
        ox.Model(str(tmp_path / "trunc.gguf"))
