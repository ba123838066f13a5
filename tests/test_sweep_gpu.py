"""BASELINE configs[4], the isolated kernel sweep, on the device against the CPU oracle.

(a) The GEMM over every (N, K) pair of configs 0-2 × M ∈ {1, 16, 275, 750, 1500, 12000} × weights in
    {q4_0, q8_0, f16}, random N(0, 1) activations (the reference ABI passes f32, which the GEMM rounds
    to f16).  Rows of the output are checked against the oracle's GEMM on the same rows of `a` — every
    row for M ≤ 275, a seeded sample of 48 rows (first and last included) above — at the reference's
    GEMM tolerance, 2e-5·max|want| (src/gpu/mod.rs:1741-1751).  The dequantized weights are checked bit
    for bit by tests/test_dequant_gpu.py.
(b) Flash attention with head_dim 48/64/128, 8/16/20 heads, T ∈ {275, 750, 1500, 6000}, with and
    without the relative-position term and a key mask, against float64 softmax attention on the
    query rows sampled the same way, at the reference's f16-tier tolerance 1e-3·max|want|
    (src/gpu/mod.rs:2197-2198).
"""

import numpy as np
import pytest

import oracle as ox
import wavo_amd as wa
from wavo_amd import gguf

pytestmark = pytest.mark.gpu

NK = [(768, 768), (3072, 768), (768, 3072), (1024, 4096), (4096, 1024), (1280, 5120), (5120, 1280), (51866, 1280)]
MS = [1, 16, 275, 750, 1500, 12000]
WTYPES = [wa.Q8_0, wa.Q4_0, wa.F16]

_weights = {}


def weights(gpu, n, k, wtype):
    """One device linear layer (and its oracle twin) per (n, k, type), shared by the M cases."""
    key = (n, k, wtype)
    if key not in _weights:
        _weights.clear()  # one shape at a time on the device
        rng = np.random.default_rng(n * 7 + k)
        w = (rng.standard_normal(n * k, dtype=np.float32) * np.float32(0.02))
        raw = gguf.encode(w, wtype)
        bias = rng.standard_normal(n, dtype=np.float32) * np.float32(0.02)
        _weights[key] = (gpu.linear([(raw, wtype, k, n)], bias), ox.Linear(wtype, k, [(raw, n)], bias))
    return _weights[key]


def sample_rows(m, seed, count=48):
    if m <= 275:
        return np.arange(m)
    rng = np.random.default_rng(seed)
    return np.unique(np.concatenate([[0, m - 1], rng.choice(m, count - 2, replace=False)]))


@pytest.mark.parametrize("wtype", WTYPES)
@pytest.mark.parametrize("n,k", NK)
@pytest.mark.parametrize("m", MS)
def test_gemm_sweep(gpu, n, k, wtype, m):
    lin, olin = weights(gpu, n, k, wtype)
    width = lin.width
    a = np.random.default_rng(m + n + k).standard_normal((m, k), dtype=np.float32)
    ab, cb = gpu.upload(a), gpu.buffer(m * width)
    gpu.gemm(ab, lin, cb, m, wa.BIAS)
    rows = sample_rows(m, n + k)
    gpu.sync()
    got = np.stack([gpu.read(cb, (width,), offset_bytes=4 * int(r) * width) for r in rows])[:, :n]
    want = ox.gemm(a[rows], olin, len(rows), ox.BIAS)
    scale = max(1.0, float(np.abs(want).max()))
    err = np.abs(got - want)
    i = np.unravel_index(int(err.argmax()), err.shape)
    assert err[i] <= 2e-5 * scale, f"{m}x{n}x{k} type {wtype}: row {rows[i[0]]} col {i[1]}: {got[i]} vs {want[i]}"


def attention64(q, k, v, scale, valid, pos_term=None):
    """float64 softmax attention of query rows q [r][hd] over keys k/v [t][hd]; pos_term [r][t] is added
    to the scores before scaling."""
    s = q.astype(np.float64) @ k.astype(np.float64).T
    if pos_term is not None:
        s = s + pos_term
    s = s * scale
    s[:, valid:] = -np.inf
    s -= s.max(axis=1, keepdims=True)
    p = np.exp(s)
    p /= p.sum(axis=1, keepdims=True)
    return p @ v.astype(np.float64)


ATT = [(hd, h, t) for hd in (48, 64, 128) for h in (8, 16, 20) for t in (275, 750, 1500, 6000)]


@pytest.mark.parametrize("hd,heads,t", ATT)
@pytest.mark.parametrize("rel", [False, True])
@pytest.mark.parametrize("masked", [False, True])
def test_attention_sweep(gpu, hd, heads, t, rel, masked):
    d = heads * hd
    rng = np.random.default_rng(hd * 1000 + heads * 10 + t)
    valid = (t * 3) // 5 if masked else t
    scale = 1.0 / np.sqrt(hd)
    rows = sample_rows(t, t + hd, 24)
    if rel:
        q, k, v = (rng.uniform(-1, 1, (t, d)).astype(np.float32) for _ in range(3))
        u, vb = rng.uniform(-1, 1, d).astype(np.float32), rng.uniform(-1, 1, d).astype(np.float32)
        pos = rng.uniform(-1, 1, (2 * t + 15, d)).astype(np.float32)
        x = np.concatenate([q + u, k, v, q + vb], axis=1)
        xb, pb, ob = gpu.upload(x), gpu.upload(pos), gpu.buffer(t * d)
        gpu.attention(xb, None, pb, ob, t, heads, hd, valid if masked else -1)
    else:
        qk = rng.uniform(-1, 1, (t, 2 * d)).astype(np.float32)
        v = rng.uniform(-1, 1, (t, d)).astype(np.float32)
        q, k = qk[:, :d], qk[:, d:]
        qb, vbuf, ob = gpu.upload(qk), gpu.upload(v), gpu.buffer(t * d)
        gpu.attention(qb, vbuf, None, ob, t, heads, hd, valid if masked else -1)
    got = gpu.read(ob, (t, d))[rows]
    want = np.zeros((len(rows), d))
    for h in range(heads):
        sl = slice(h * hd, (h + 1) * hd)
        term = None
        if rel:
            # score(i, j) += (q + v)_i · P[j − i + t + 15]   (src/cpu/ops.rs:228-273)
            j = np.arange(t)
            idx = j[None, :] - rows[:, None] + t + 15
            qv = (q[rows] + vb)[:, sl].astype(np.float64)
            pr = pos[:, sl].astype(np.float64)
            term = np.einsum("rd,rjd->rj", qv, pr[idx])
            want[:, sl] = attention64((q[rows] + u)[:, sl], k[:, sl], v[:, sl], scale, valid, term)
        else:
            want[:, sl] = attention64(q[rows][:, sl], k[:, sl], v[:, sl], scale, valid)
    err = np.abs(got - want)
    tol = 1e-3 * max(1.0, float(np.abs(want).max()))
    i = np.unravel_index(int(err.argmax()), err.shape)
    assert err[i] <= tol, f"hd {hd} heads {heads} t {t} rel {rel} valid {valid}: row {rows[i[0]]}: {got[i]} vs {want[i]}"
