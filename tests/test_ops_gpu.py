"""Parity of each Pass op's gfx950 kernel with the CPU oracle, on the cases of the reference's own GPU
tests (src/gpu/mod.rs:1681-2361): shapes, padding columns, dual outputs, all 7 epilogues, every weight
type, at the reference's tolerance 2e-5·max|want| (src/gpu/mod.rs:1741-1751) unless noted.  Inputs are
seeded uniform(-1, 1) rather than the reference's xorshift stream; the checks are the same formulas.
"""

import numpy as np
import pytest

import oracle as ox
import wavo_amd as wa

pytestmark = pytest.mark.gpu

TYPES = [wa.F32, wa.F16, wa.Q8_0, wa.Q4_0]


def rnd(n, seed):
    return np.random.default_rng(seed).uniform(-1.0, 1.0, n).astype(np.float32)


def close(got, want, tol=2e-5, what=""):
    got = np.asarray(got, np.float32).ravel()
    want = np.asarray(want, np.float32).ravel()
    assert got.shape == want.shape
    scale = max(1.0, float(np.abs(want).max()))
    err = np.abs(got - want)
    i = int(err.argmax())
    assert err[i] <= tol * scale, f"{what} [{i}]: {got[i]} vs {want[i]} (err {err[i]:.3g}, tol {tol * scale:.3g})"


def epi_zero(e, c):
    """The epilogue of v = 0 (padding columns): only the residual modes keep c."""
    return c if e in (wa.RESIDUAL, wa.GELU_RESIDUAL) else np.zeros_like(c)


@pytest.mark.parametrize("wtype", TYPES)
@pytest.mark.parametrize("k", [96, 128, 1024])
@pytest.mark.parametrize("n,cols", [(164, 192), (288, 288)])
def test_gemm(gpu, wtype, k, n, cols):
    w = rnd(n * k, 1).reshape(n, k)
    bias = rnd(n, 2)
    dual = np.concatenate([bias, rnd(64, 5)])
    raw = ox.quantize(w, wtype)
    half = len(raw) // 2
    parts = [(raw[:half], wtype, k, n // 2), (raw[half:], wtype, k, n // 2)]
    for b in (bias, None, dual):
        d = 64 if b is dual else 0
        l = gpu.linear(parts, b)
        width = cols + d
        assert l.width == width
        ol = ox.Linear(wtype, k, [(raw[:half], n // 2), (raw[half:], n // 2)], None if b is None else b[:n])
        ms = [1, 37, 70, 2100] if k < 1024 else [37, 300]
        for m in ms:
            a = rnd(m * k, 3).reshape(m, k)
            ab = gpu.upload(a)
            # One float more than the rows written: it must stay as it was.
            c0 = rnd(m * width + 1, 4)
            # Rounding of the sums over k scales with the pre-activations, which tanh squashes:
            # the tolerance is relative to the largest of them (the reference's k = 96 stays < 1).
            pre = ox.gemm_wide(a, ol, m, wa.BIAS, 0.0, c=c0[:-1].reshape(m, width),
                               bias2=dual[n:] if d else None, dual=d)
            for e in range(7):
                cb = gpu.upload(c0)
                alpha = 0.5 if e == wa.RESIDUAL else 0.0
                gpu.gemm(ab, l, cb, m, e, alpha)
                got = gpu.read(cb, c0.shape)
                want = ox.gemm_wide(a, ol, m, e, alpha, c=c0[:-1].reshape(m, width),
                                    bias2=dual[n:] if d else None, dual=d)
                scale = max(1.0, float(np.abs(pre).max()), float(np.abs(want).max()))
                close(got[:-1], want, tol=2e-5 * scale, what=f"type {wtype} k {k} n {n} m {m} epi {e} dual {d}")
                assert got[-1] == c0[-1]


@pytest.mark.parametrize("wtype", [wa.Q8_0, wa.Q4_0, wa.F16])
@pytest.mark.parametrize("m,n,k", [(2048, 4096, 256), (750, 4096, 1024), (750, 1024, 4096), (1515, 1024, 1024),
                                   (4224, 4096, 192)])
def test_gemm_large(gpu, wtype, m, n, k):
    # The tile plans of the main kernel at the encoder's shapes: 128×128 tiles of 8 wavefronts with
    # four LDS stages (one wave of workgroups) or three (4224 rows: several workgroups per CU, the
    # batched-window plan), 64×64 tiles with k split 4 ways (partial sums finished in order).
    w = np.random.default_rng(1).normal(0, 0.02, (n, k)).astype(np.float32)
    raw = ox.quantize(w, wtype)
    bias = rnd(n, 2)
    l = gpu.linear([(raw, wtype, k, n)], bias)
    ol = ox.Linear(wtype, k, [(raw, n)], bias)
    a = rnd(m * k, 3).reshape(m, k)
    ab, cb = gpu.upload(a), gpu.buffer(m * n)
    for e in (wa.BIAS, wa.SILU):
        gpu.gemm(ab, l, cb, m, e)
        want = ox.gemm(a, ol, m, e)
        close(gpu.read(cb, (m, n)), want, tol=2e-5 * max(1.0, float(np.abs(want).max())),
              what=f"type {wtype} {m}x{n}x{k} epi {e}")


@pytest.mark.parametrize("m,n,k", [(1500, 5120, 1280), (1500, 1280, 5120)])
def test_gemm_more_tiles_than_cus(gpu, m, n, k):
    # The 1500-frame plans: 128×128 tiles of 4 wavefronts, three stages, two workgroups per CU
    # (1500 × 5120: 480 tiles), and the same split 4 ways over k (1500 × 1280 × 5120).
    w = np.random.default_rng(1).normal(0, 0.02, (n, k)).astype(np.float32)
    raw = ox.quantize(w, wa.Q8_0)
    bias = rnd(n, 2)
    l = gpu.linear([(raw, wa.Q8_0, k, n)], bias)
    ol = ox.Linear(wa.Q8_0, k, [(raw, n)], bias)
    a = rnd(m * k, 3).reshape(m, k)
    ab, cb = gpu.upload(a), gpu.upload(rnd(m * n, 4).reshape(m, n))
    c0 = gpu.read(cb, (m, n))
    for e in (wa.GELU, wa.RESIDUAL):
        gpu.gemm(ab, l, cb, m, e, 1.0)
        want = ox.gemm(a, ol, m, e, 1.0, c0)
        close(gpu.read(cb, (m, n)), want, tol=2e-5 * max(1.0, float(np.abs(want).max())), what=f"{m}x{n}x{k} epi {e}")
        c0 = gpu.read(cb, (m, n))


# Every kernel variant the GEMM builds: tile, wavefronts per tile row and column, ring slots, k split,
# loop variant (2: ping-pong), k groups — forced through wh_tune("gemm_plan") on one shape with edge
# tiles in both directions and dual columns.
PLANS = ["128,128,2,4,3,1", "64,64,2,2,3,1", "128,128,2,4,2,1", "128,128,2,2,2,1", "256,128,4,2,2,1",
         "96,64,1,2,2,1", "192,128,2,2,2,1", "256,256,2,4,2,1", "96,128,1,4,3,1", "256,256,2,4,3,1,2",
         "64,64,2,2,4,1,0,2", "96,64,1,2,2,1,0,2", "96,128,1,4,3,1,0,2",
         "96,64,1,2,2,4", "128,128,2,2,2,4", "64,64,2,2,3,2", "64,64,2,2,4,2,0,2", "96,64,1,2,2,4,0,2"]


@pytest.mark.parametrize("wtype", [wa.Q8_0, wa.Q4_0, wa.F16])
@pytest.mark.parametrize("plan", PLANS)
def test_gemm_every_plan(gpu, wtype, plan):
    if wtype == wa.F16 and plan.split(",")[6:7] == ["2"]:
        pytest.skip("the ping-pong loop is built for quantized W only (F16 rows need no dequantization)")
    m, n, k, d = 300, 320, 1024, 64
    w = np.random.default_rng(1).normal(0, 0.02, (n, k)).astype(np.float32)
    raw = ox.quantize(w, wtype)
    bias = rnd(n + d, 2)
    ol = ox.Linear(wtype, k, [(raw, n)], bias[:n])
    a = rnd(m * k, 3).reshape(m, k)
    c0 = rnd(m * (n + d), 4).reshape(m, n + d)
    gpu.tune("gemm_plan", plan)
    try:
        l = gpu.linear([(raw, wtype, k, n)], bias)
        assert l.width == n + d
        ab = gpu.upload(a)
        for e, alpha in ((wa.BIAS, 0.0), (wa.RESIDUAL, 0.5), (wa.SILU, 0.0)):
            cb = gpu.upload(c0)
            gpu.gemm(ab, l, cb, m, e, alpha)
            want = ox.gemm_wide(a, ol, m, e, alpha, c=c0, bias2=bias[n:], dual=d)
            close(gpu.read(cb, c0.shape), want, tol=2e-5 * max(1.0, float(np.abs(want).max())),
                  what=f"plan {plan} type {wtype} epi {e}")
    finally:
        gpu.tune("gemm_plan", "")


@pytest.mark.parametrize("plan", ["96,128,1,4,3,1,0,2", "96,64,1,2,2,4", "64,64,2,2,3,1"])
def test_gemm_tile_orders_agree(gpu, plan):
    # The order in which XCDs take the tiles (groups of 1, 2, 3 and all row tiles, column by column
    # inside a group; a ragged last group at 3) changes no bit of the output; n = 960 gives tile
    # counts that are not multiples of the 8 XCDs (the first XCDs take one tile more), checked
    # against the oracle too.
    m, k = 700, 1024
    for n in (1024, 960):
        w = np.random.default_rng(5).normal(0, 0.02, (n, k)).astype(np.float32)
        raw, bias = ox.quantize(w, wa.Q8_0), rnd(n, 6)
        l = gpu.linear([(raw, wa.Q8_0, k, n)], bias)
        a = rnd(m * k, 7).reshape(m, k)
        ab = gpu.upload(a)
        outs = []
        gpu.tune("gemm_plan", plan)
        try:
            for group in (1, 2, 3, 64):
                gpu.tune("gemm_group", str(group))
                cb = gpu.buffer(m * n)
                gpu.gemm(ab, l, cb, m, wa.BIAS, 0.0)
                outs.append(gpu.read(cb, (m, n)))
        finally:
            gpu.tune("gemm_plan", "")
            gpu.tune("gemm_group", "0")
        for group, o in zip((2, 3, 64), outs[1:]):
            assert np.array_equal(o, outs[0]), f"plan {plan}, n {n}: {group} row tiles per group"
        want = ox.gemm(a, ox.Linear(wa.Q8_0, k, [(raw, n)], bias), m, ox.BIAS)
        close(outs[0], want, tol=2e-5 * max(1.0, float(np.abs(want).max())), what=f"plan {plan}, n {n}")


def test_gemm_rejects_internal_epilogues(gpu):
    # The library's own epilogues past WH_TANH (the conv module's GLU) are not callers' to ask for.
    m, n, k = 4, 64, 64
    l = gpu.linear([(ox.quantize(rnd(n * k, 1).reshape(n, k), wa.Q8_0), wa.Q8_0, k, n)], rnd(n, 2))
    ab, cb = gpu.upload(rnd(m * k, 3).reshape(m, k)), gpu.buffer(m * n)
    for epi in (7, -1):
        with pytest.raises(wa.WavoError, match="epilogue"):
            gpu.gemm(ab, l, cb, m, epi)
        with pytest.raises(wa.WavoError, match="epilogue"):
            gpu.gemm_h(ab, l, cb, m, epi)


def test_gemm_padded_k(gpu):
    # k = 40 is padded to 64 by Gpu::conv; input rows are 64 wide with zeros after 40 (from im2col).
    n, k, m = 64, 40, 37
    a = rnd(m * 64, 3).reshape(m, 64)
    a[:, k:] = 0
    w = rnd(n * k, 1).reshape(n, k)
    for wtype in (wa.F32, wa.F16):
        raw = ox.quantize(w, wtype)
        with pytest.raises(wa.WavoError):
            gpu.linear([(raw, wtype, k, n)])
        l = gpu.linear([(raw, wtype, k, n)], pad_k=True)
        assert l.k == 64
        wp = np.zeros((n, 64), np.float32)
        wp[:, :k] = ox.dequant(raw, wtype, n * k).reshape(n, k)
        ol = ox.Linear(ox.F32, 64, [(wp.tobytes(), n)])
        ab, cb = gpu.upload(a), gpu.buffer(m * n)
        gpu.gemm(ab, l, cb, m, wa.BIAS)
        close(gpu.read(cb, (m, n)), ox.gemm(a, ol, m, ox.BIAS))


def test_layer_norm_and_rope(gpu):
    rows, cols, hd = 37, 192, 48
    x = rnd(rows * cols, 5).reshape(rows, cols)
    g, b = rnd(cols, 6), rnd(cols, 7)
    table = rnd(rows * hd, 8).reshape(rows, hd)
    y, yr = ox.layer_norm(x, g, b, table, hd)
    xb, gb, bb, tb = gpu.upload(x), gpu.upload(g), gpu.upload(b), gpu.upload(table)
    out, outr = gpu.buffer(rows * cols), gpu.buffer(rows * cols)
    gpu.layer_norm(xb, gb, bb, out, rows, cols)
    close(gpu.read(out, (rows, cols)), y, what="layer_norm")
    gpu.layer_norm(xb, gb, bb, out, 1, cols)
    close(gpu.read(out, (cols,)), y[0], what="layer_norm_row")
    gpu.layer_norm(xb, gb, bb, out, rows, cols, tb, outr, hd)
    close(gpu.read(outr, (rows, cols)), yr, what="rope")
    # The models' widths (GigaAM 768, Parakeet 1024, Whisper 1280: kernels specialized to the width),
    # with RoPE at 1024, and a long row past the register path.
    for cols in (768, 1024, 1280, 5000):
        x = rnd(5 * cols, 9).reshape(5, cols)
        g, b = rnd(cols, 10), rnd(cols, 11)
        xb, gb, bb, out = gpu.upload(x), gpu.upload(g), gpu.upload(b), gpu.buffer(5 * cols)
        gpu.layer_norm(xb, gb, bb, out, 5, cols)
        close(gpu.read(out, (5, cols)), ox.layer_norm(x, g, b), what=f"cols {cols}")
        if cols == 1024:
            table = rnd(5 * 128, 12).reshape(5, 128)
            tb, outr = gpu.upload(table), gpu.buffer(5 * cols)
            gpu.layer_norm(xb, gb, bb, out, 5, cols, tb, outr, 128)
            close(gpu.read(outr, (5, cols)), ox.layer_norm(x, g, b, table, 128)[1], what="rope 1024")


@pytest.mark.parametrize("t_in,ch,conv", [(37, 20, (5, 2, 2)), (37, 20, (3, 1, 1)), (37, 20, (3, 2, 1)),
                                         (900, 1, (127, 64, 0))])
def test_im2col(gpu, t_in, ch, conv):
    kernel, stride, pad = conv
    x = rnd(t_in * ch, 9).reshape(t_in, ch)
    t_out = (t_in + 2 * pad - kernel) // stride + 1
    width = (ch * kernel + 31) // 32 * 32
    want = ox.im2col(x, t_in, ch, kernel, stride, pad, width)
    xb, cb = gpu.upload(x), gpu.buffer(t_out * width)
    gpu.im2col(xb, cb, t_in, ch, kernel, stride, pad)
    close(gpu.read(cb, (t_out, width)), want)


@pytest.mark.parametrize("wtype", TYPES)
@pytest.mark.parametrize("k", [96, 128])
@pytest.mark.parametrize("n,cols", [(100, 128), (288, 288)])
def test_gemv_and_embed(gpu, wtype, k, n, cols):
    w = rnd(n * k, 1).reshape(n, k)
    bias = rnd(n, 2)
    a = rnd(k, 3)
    pos = rnd(2 * k, 6)
    raw = ox.quantize(w, wtype)
    l = gpu.linear([(raw, wtype, k, n)], bias)
    ol = ox.Linear(wtype, k, [(raw, n)], bias)
    ab = gpu.upload(a)
    c0 = rnd(3 + cols + 1, 4)
    for e in range(7):
        alpha = 0.5 if e == wa.RESIDUAL else 0.0
        cb = gpu.upload(c0)
        gpu.gemv(ab, l, cb, e, alpha, 3)
        got = gpu.read(cb, c0.shape)
        want = c0.copy()
        want[3:3 + n] = ox.gemv(a, ol, e, alpha, c=c0[3:3 + n])
        want[3 + n:3 + cols] = epi_zero(e, c0[3 + n:3 + cols])
        close(got, want, what=f"gemv type {wtype} epi {e}")
    # The embedding row 7 (ids[1]) plus the position row from k plus the bias.
    ids = gpu.upload(np.array([5, 7], np.uint32))
    pb, ob = gpu.upload(pos), gpu.buffer(k)
    gpu.embed(l, pb, ob, ids, 1, k)
    wrow = ox.dequant(raw, wtype, n * k).reshape(n, k)[7]
    padded = np.zeros(max(k, n), np.float32)
    padded[:n] = bias  # the bias is zero past W's rows (upload_linear pads it)
    close(gpu.read(ob, (k,)), wrow + pos[k:] + padded[:k], what="embed")


@pytest.mark.parametrize("wtype", [wa.Q8_0, wa.F16, wa.Q4_0])
@pytest.mark.parametrize("n,k", [(1280, 1280), (3840, 1280), (5120, 1280), (1280, 5120), (51866, 1280), (37, 64)])
def test_gemv_decoder_shapes(gpu, wtype, n, k):
    # Whisper-large-v3-turbo's decoder GEMVs (per layer and the 51866-row head) through the streaming
    # kernel: rows split across workgroups and stages, the last stage partial, padding columns.
    w = np.random.default_rng(21).normal(0, 0.02, (n, k)).astype(np.float32)
    raw = ox.quantize(w, wtype)
    bias = rnd(n, 22)
    l = gpu.linear([(raw, wtype, k, n)], bias)
    ol = ox.Linear(wtype, k, [(raw, n)], bias)
    a = rnd(k, 23)
    ab = gpu.upload(a)
    cols = l.width
    c0 = rnd(cols + 1, 24)
    for e, alpha in ((wa.BIAS, 0.0), (wa.RESIDUAL, 1.0), (wa.GELU, 0.0)):
        cb = gpu.upload(c0)
        gpu.gemv(ab, l, cb, e, alpha)
        got = gpu.read(cb, c0.shape)
        want = c0.copy()
        want[:n] = ox.gemv(a, ol, e, alpha, c=c0[:n])
        want[n:cols] = epi_zero(e, c0[n:cols])
        close(got, want, what=f"gemv {n}x{k} type {wtype} epi {e}")


def test_recorded_pass_replays(gpu):
    # Gpu::record / finish: a recorded chain of ops (layer norm -> GEMV -> GEMV with the residual
    # epilogue -> GEMM) replayed several times, with other work queued between the replays, gives
    # the eager result every time, bit for bit; the pass's buffers are re-initialised before each
    # replay so the residual reads the same input.
    k, n, m = 1280, 1280, 40
    w1 = ox.quantize(np.random.default_rng(31).normal(0, 0.02, (n, k)).astype(np.float32), wa.Q8_0)
    w2 = ox.quantize(np.random.default_rng(32).normal(0, 0.02, (n, n)).astype(np.float32), wa.Q8_0)
    l1 = gpu.linear([(w1, wa.Q8_0, k, n)], rnd(n, 33))
    l2 = gpu.linear([(w2, wa.Q8_0, n, n)], rnd(n, 34))
    x0, g, b, c0 = rnd(k, 35), rnd(k, 36), rnd(k, 37), rnd(n, 38)
    a = rnd(m * k, 39).reshape(m, k)
    xb, gb, bb, ab = gpu.upload(x0), gpu.upload(g), gpu.upload(b), gpu.upload(a)
    yb, hb, cb, ob = gpu.buffer(k), gpu.buffer(n), gpu.buffer(n), gpu.buffer(m * n)

    def ops():
        gpu.layer_norm(xb, gb, bb, yb, 1, k)
        gpu.gemv(yb, l1, hb, wa.GELU, 0.0)
        gpu.gemv(hb, l2, cb, wa.RESIDUAL, 1.0)
        gpu.gemm(ab, l1, ob, m, wa.SILU)

    gpu.write(cb, c0)
    ops()
    want_c, want_o = gpu.read(cb, n), gpu.read(ob, (m, n))
    gpu.record_begin()
    ops()
    p = gpu.record_end()
    for i in range(3):
        gpu.write(cb, c0)
        gpu.zero(ob)
        gpu.zero(hb)
        p.replay()
        assert np.array_equal(gpu.read(cb, n), want_c), i
        assert np.array_equal(gpu.read(ob, (m, n)), want_o), i
        gpu.gemv(yb, l2, hb, wa.BIAS, 0.0)  # unrelated work between replays
    p.free()
    with pytest.raises(wa.WavoError):
        gpu.record_end()  # not recording


@pytest.mark.parametrize("merge", [False, True])
@pytest.mark.parametrize("heads,hd", [(2, 40), (3, 36), (20, 64), (2, 100), (4, 128)])
def test_attend_and_pack(gpu, heads, hd, merge):
    """Parts of 256 keys merged by a second kernel, or (merge) by the launch's last part to finish,
    through the head's counter: 1 to 17 parts in a row on one set of counters."""
    keys = 4100
    d = heads * hd
    kv = rnd(keys * 2 * d, 7).reshape(keys, 2 * d)
    q = rnd(d, 8)
    # The CPU cache layout: K heads then V heads, [2·heads][keys][hd], f16-rounded.
    cpu = kv.reshape(keys, 2 * heads, hd).transpose(1, 0, 2).astype(np.float16).astype(np.float32)
    xb, qb = gpu.upload(kv), gpu.upload(q)
    cache = gpu.buffer(keys * d)
    part = gpu.buffer(gpu.attend_len(keys, heads, hd))
    ob = gpu.buffer(d)
    gpu.pack(xb, 0, 2 * d, cache, keys, d, keys, 0)
    gpu.tune("attend_merge", int(merge))
    try:
        for n in (1, 37, 256, 257, 1500, 2049, keys, 300):
            gpu.attend(qb, cache, part, ob, n, keys, heads, hd)
            close(gpu.read(ob, (d,)), ox.attend(q, cpu, keys, n, heads, hd), what=f"attend n {n}")
    finally:
        gpu.tune("attend_merge", 0)


@pytest.mark.parametrize("merge", [False, True])
def test_attend_long_cache(gpu, merge):
    # 32 to 36 parts of 256 keys per head.
    heads, hd, keys = 2, 64, 9000
    d = heads * hd
    kv = rnd(keys * 2 * d, 17).reshape(keys, 2 * d)
    q = rnd(d, 18)
    cpu = kv.reshape(keys, 2 * heads, hd).transpose(1, 0, 2).astype(np.float16).astype(np.float32)
    xb, qb = gpu.upload(kv), gpu.upload(q)
    cache = gpu.buffer(keys * d)
    part = gpu.buffer(gpu.attend_len(keys, heads, hd))
    ob = gpu.buffer(d)
    gpu.pack(xb, 0, 2 * d, cache, keys, d, keys, 0)
    gpu.tune("attend_merge", int(merge))
    try:
        for n in (8192, 8193, keys):
            gpu.attend(qb, cache, part, ob, n, keys, heads, hd)
            close(gpu.read(ob, (d,)), ox.attend(q, cpu, keys, n, heads, hd), what=f"attend n {n}")
    finally:
        gpu.tune("attend_merge", 0)


def test_pack_layout(gpu):
    # Rows of K then V (d = 6) from x[3..], 13 floats apart, into a cache of 7 positions.
    x = rnd(3 + 13 * 2, 7)
    xb = gpu.upload(x)
    for rows, col in ((1, 4), (2, 5)):
        y = rnd(7 * 6, 9).view(np.uint32)
        yb = gpu.upload(y)
        gpu.pack(xb, 3, 13, yb, rows, 6, 7, col)
        got = gpu.read(yb, y.shape, np.uint32)
        want = ox.pack(x, 3, 13, y, rows, 6, 7, col)
        assert np.array_equal(got, want), f"pack {rows} rows"


@pytest.mark.parametrize("kernel,layer_norm", [(5, True), (9, False)])
@pytest.mark.parametrize("valid", [None, 30])
def test_conv_glu(gpu, kernel, layer_norm, valid):
    t, ch = 37, 192
    h = rnd(t * 2 * ch, 10).reshape(t, 2 * ch)
    g, b = rnd(ch, 13), rnd(ch, 14)
    w, wb = rnd(ch * kernel, 11).reshape(ch, kernel), rnd(ch, 12)
    v = -1 if valid is None else valid
    want = ox.conv_glu(h, w.T.copy(), wb, kernel, g, b, layer_norm, t, ch, v)
    hb, wbuf, wbb, gb, bb, yb = (gpu.upload(x) for x in (h, w, wb, g, b, np.zeros((t, ch), np.float32)))
    gpu.conv_glu(hb, wbuf, wbb, kernel, gb, bb, layer_norm, yb, t, ch, v)
    close(gpu.read(yb, (t, ch)), want)


ATTN = [(37, 48), (100, 48), (100, 56), (5, 36), (70, 52), (100, 64), (40, 80), (275, 48), (300, 128)]

# Attention runs its products on f16 operands with f32 accumulation, as the reference's f16 flash
# tier does; the reference holds that tier to 1e-3·max|want| (src/gpu/mod.rs:2197-2198).
ATT_TOL = 1e-3


@pytest.mark.parametrize("t,hd", ATTN)
def test_attention(gpu, t, hd):
    heads = 2
    d = heads * hd
    qk = rnd(t * 2 * d, 15).reshape(t, 2 * d)
    v = rnd(t * d, 16).reshape(t, d)
    want = ox.attention(qk, 2 * d, v, d, t, heads, hd)
    qb, vb, ob = gpu.upload(qk), gpu.upload(v), gpu.buffer(t * d)
    gpu.attention(qb, vb, None, ob, t, heads, hd)
    close(gpu.read(ob, (t, d)), want, tol=ATT_TOL, what="rotary layout")
    # Whisper's [q | k | v] rows.
    qkv = np.concatenate([qk, v], axis=1)
    want = ox.attention(qkv, 3 * d, v, d, t, heads, hd)
    qb = gpu.upload(qkv)
    gpu.attention(qb, None, None, ob, t, heads, hd)
    close(gpu.read(ob, (t, d)), want, tol=ATT_TOL, what="qkv layout")


# (300, …): keys split over two workgroups per query tile; valid 10 leaves the first split empty.
@pytest.mark.parametrize("t,valid", [(37, 20), (100, 64), (100, 1), (300, 150), (300, 10)])
def test_attention_masked(gpu, t, valid):
    heads, hd = 2, 64
    d = heads * hd
    qk = rnd(t * 2 * d, 15).reshape(t, 2 * d)
    v = rnd(t * d, 16).reshape(t, d)
    want = ox.attention(qk, 2 * d, v, d, t, heads, hd, valid)
    qb, vb, ob = gpu.upload(qk), gpu.upload(v), gpu.buffer(t * d)
    gpu.attention(qb, vb, None, ob, t, heads, hd, valid)
    close(gpu.read(ob, (t, d)), want, tol=ATT_TOL)


def relative_inputs(t, heads, hd, seed=17):
    d = heads * hd
    qkv = rnd(t * 3 * d, seed).reshape(t, 3 * d)
    pos = rnd((2 * t + 15) * d, seed + 1).reshape(2 * t + 15, d)
    u, vb = rnd(d, seed + 2), rnd(d, seed + 3)
    q = qkv[:, :d]
    gpu_rows = np.concatenate([q + u, qkv[:, d:], q + vb], axis=1)
    return qkv, pos, u, vb, gpu_rows


@pytest.mark.parametrize("t,heads,hd,valid", [(5, 2, 40, None), (37, 2, 40, None), (100, 3, 128, None),
                                               (750, 8, 128, None), (275, 16, 48, None), (100, 3, 128, 60),
                                               (750, 8, 128, 400)])
def test_relative_attention(gpu, t, heads, hd, valid):
    d = heads * hd
    qkv, pos, u, vb, rows = relative_inputs(t, heads, hd)
    v = -1 if valid is None else valid
    want = ox.relative_attention(qkv, pos, u, vb, t, heads, hd, v)
    qb, pb, ob = gpu.upload(rows), gpu.upload(pos), gpu.buffer(t * d)
    gpu.attention(qb, None, pb, ob, t, heads, hd, v)
    close(gpu.read(ob, (t, d)), want, tol=ATT_TOL)


@pytest.mark.parametrize("heads", [8, 3])
@pytest.mark.parametrize("valid", [None, 400])
def test_relative_attention_many_splits(valid, heads):
    """Key blocks split 8 ways (more than the merge's group of four: its running-maximum rescale, and
    splits past the valid keys that contribute nothing), through a context opened with the tuning
    override.  8 heads: each XCD merges the heads whose partial outputs it wrote; 3 heads (window-head
    pairs not a multiple of 8): the merge's plain order."""
    t, hd = 750, 128
    g = wa.Gpu(0)
    g.tune("attn_split", 8)
    try:
        d = heads * hd
        qkv, pos, u, vb, rows = relative_inputs(t, heads, hd, seed=23)
        v = -1 if valid is None else valid
        want = ox.relative_attention(qkv, pos, u, vb, t, heads, hd, v)
        qb, pb, ob = g.upload(rows), g.upload(pos), g.buffer(t * d)
        g.attention(qb, None, pb, ob, t, heads, hd, v)
        close(g.read(ob, (t, d)), want, tol=ATT_TOL)
    finally:
        g.close()


@pytest.mark.parametrize("t,f,ch", [(7, 16, 256), (3, 8, 64), (2, 16, 128), (5, 4, 32)])
def test_flatten_power_of_two(gpu, t, f, ch):
    """The LDS transpose path of flatten (f and ch powers of two, f·ch ≤ 4096, as after Parakeet's
    subsampling): a permutation, so bit for bit."""
    x = rnd(t * f * ch, 27).reshape(t, f, ch)
    xb, fb = gpu.upload(x), gpu.buffer(t * f * ch)
    gpu.flatten(xb, fb, t, f, ch)
    assert np.array_equal(gpu.read(fb, (t, f * ch)), ox.flatten(x, t, f, ch))


# ch = 5: one channel per thread; ch % 4 == 0: four channels and four output columns per thread (a
# partial group of columns at f 11, 13 and 40).
@pytest.mark.parametrize("valid_drop", [0, 1])
@pytest.mark.parametrize("t,f,ch", [(29, 11, 5), (29, 11, 8), (29, 13, 12), (37, 32, 64), (29, 40, 4)])
def test_subsampling(gpu, valid_drop, t, f, ch):
    valid = t - valid_drop
    mel = rnd(t * f, 19).reshape(t, f)
    ws = [rnd(ch * 9, 20 + i) if i % 2 == 0 else rnd(ch, 20 + i) for i in range(6)]
    w0, b0, w2, b2, w5, b5 = ws
    t2, f2 = ox.half_len(ox.half_len(t)), ox.half_len(ox.half_len(f))
    want = np.zeros((4, ox.half_len(f2), ch), np.float32)
    mb = gpu.upload(mel)
    dev = [gpu.upload(x) for x in ws]
    chunk = gpu.buffer(5 * f2 * ch)
    yb = gpu.upload(np.zeros(want.shape, np.float32))
    for t0 in (0, 2):
        c = ox.sub_first(mel, valid, f, w0, b0, w2, b2, ch, 5, t0)
        want[t0:t0 + 2] = ox.depthwise(c, w5, b5, t2, f2, ch, 2, t0)
        gpu.depthwise(mb, dev[0], dev[1], dev[2], dev[3], chunk, valid, f, ch, t0, 5)
        close(gpu.read(chunk, c.shape), c, what=f"first t0 {t0}")
        gpu.depthwise(chunk, None, None, dev[4], dev[5], yb, t2, f2, ch, t0, 2)
    close(gpu.read(yb, want.shape), want, what="conv5")
    x = rnd(t * f * ch, 26).reshape(t, f, ch)
    xb, fb = gpu.upload(x), gpu.buffer(t * f * ch)
    gpu.flatten(xb, fb, t, f, ch)
    close(gpu.read(fb, (t, f * ch)), ox.flatten(x, t, f, ch), what="flatten")


def test_argmax(gpu):
    logits = rnd(1000, 35)
    logits[700] = 2.0
    logits[300] = 2.0
    lb, ob = gpu.upload(logits), gpu.buffer(1)
    for n in (1000, 500):
        gpu.argmax(lb, ob, n)
        assert int(gpu.read(ob, (1,), np.uint32)[0]) == 300
