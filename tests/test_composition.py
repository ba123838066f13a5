"""Pins of the oracle's model-level composition (oracle/models.c: ox_model_blocks, ox_model_encode,
ox_whisper_begin/step, ox_model_predict/joint) against float64 restatements written here from the
reference's graph code, reading the GGUF tensors by name with a third reader (tests/ggufread.py).

The restatements follow the reference's CPU backend op by op:
  Conformer block ............ src/cpu/conformer.rs:159-200 (rotary and relative attention, the
                               conv module of src/cpu/ops.rs:137-182, BatchNorm fold
                               src/conformer.rs:130-139, block output norm_out(x))
  relative attention ......... src/cpu/ops.rs:223-273, positions src/conformer.rs:144-153
  rotary LayerNorm ........... src/cpu/ops.rs:64-110, table src/gigaam/mod.rs:86-97
  Parakeet encoder ........... src/parakeet/cpu.rs:67-174 (subsampling with its masking)
  GigaAM encoder ............. src/gigaam/encoder.rs:83-93
  Whisper encoder / step ..... src/whisper/cpu.rs:40-47, src/cpu/transformer.rs:94-117, :161-266
  TDT predictor and joint .... src/parakeet/decoder.rs:107-142
Where the reference rounds GEMM operands to f16 (src/cpu/gemm.rs:163-176) the restatement rounds
them too, so what remains between oracle and restatement is f32 against f64 arithmetic.  The models
are the small synthetic shapes with their norms, BatchNorm statistics and position biases moved away
from identity values (synth's `perturb`), so that a parameter in the wrong place shows.

Each check also runs the restatement with a plausible wiring mistake planted in it (u and v swapped,
the FFN's ½ dropped, the output norm skipped, BatchNorm folded with var instead of √(var + ε), LSTM
gates in another order, RoPE on the projection's output instead of its input, …) and requires that
version to miss the oracle by far more than the tolerance: the check can see such a mistake.
"""

import math

import numpy as np
import pytest

import oracle as ox
from ggufread import Gguf
from wavo_amd import gguf, synth

EPS = 1e-5


def h16(x):
    """The GEMM's to_half of an operand (IEEE round to nearest even inside the f16 range)."""
    return np.asarray(x, np.float32).astype(np.float16).astype(np.float64)


def gemm(a, w, b=None):
    y = h16(a) @ h16(w).T
    return y if b is None else y + b


def gemv(x, w, b=None):
    y = np.asarray(w, np.float64) @ np.asarray(x, np.float64)
    return y if b is None else y + b


def ln(x, g, b):
    x = np.asarray(x, np.float64)
    mu = x.mean(axis=-1, keepdims=True)
    var = ((x - mu) ** 2).mean(axis=-1, keepdims=True)
    return (x - mu) / np.sqrt(var + EPS) * g + b


def silu(v):
    return v / (1.0 + np.exp(-v))


def sigmoid(v):
    return 1.0 / (1.0 + np.exp(-v))


def gelu(v):
    return 0.5 * v * (1.0 + np.vectorize(math.erf)(v / math.sqrt(2.0)))


def softmax_rows(s):
    s = s - s.max(axis=-1, keepdims=True)
    p = np.exp(s)
    return p / p.sum(axis=-1, keepdims=True)


def rel_err(a, b):
    return float(np.linalg.norm(np.asarray(a, np.float64) - b) / np.linalg.norm(b))


class Weights:
    """Tensors of a synthetic model by name, in float64."""

    def __init__(self, path):
        self.g = Gguf(path)

    def t(self, name):
        return self.g.tensor(name).astype(np.float64)

    def m(self, name):
        return self.g.matrix(name).astype(np.float64)

    def bias(self, name, n):
        return self.t(name) if self.g.has(name) else np.zeros(n)


def rel_positions(d, first, rows):
    k = np.arange(d // 2)
    div = np.exp((2 * k) * (-math.log(10000.0) / d))
    p = (first - np.arange(rows))[:, None] * div[None, :]
    out = np.zeros((rows, d))
    out[:, 0::2], out[:, 1::2] = np.sin(p), np.cos(p)
    return out


def rope_table(frames, hd, theta):
    i = np.arange(hd // 2)
    a = np.arange(frames)[:, None] * theta ** (-2.0 * i / hd)[None, :]
    return np.concatenate([np.cos(a), np.sin(a)], axis=1)


def rope(y, table, heads, hd):
    """NEOX split-half rotation inside each head (src/cpu/ops.rs:94-106)."""
    t = y.shape[0]
    half = hd // 2
    cos, sin = table[:t, :half], table[:t, half:]
    out = y.copy()
    for h in range(heads):
        y0, y1 = y[:, h * hd:h * hd + half], y[:, h * hd + half:(h + 1) * hd]
        out[:, h * hd:h * hd + half] = y0 * cos - y1 * sin
        out[:, h * hd + half:(h + 1) * hd] = y1 * cos + y0 * sin
    return out


def block64(W, i, x, cfg, rel, mistake=None):
    """Block::run (src/cpu/conformer.rs:159-200) of block i over x [t][d]."""
    d, heads, K = cfg["d"], cfg["heads"], cfg["kernel"]
    hd, t = d // heads, x.shape[0]
    p = f"enc.blocks.{i}."
    bias = not rel
    lw = lambda n: (W.m(p + n + ".weight"), W.bias(p + n + ".bias", 0) if bias else None)
    nm = lambda n: (W.t(p + n + ".weight"), W.t(p + n + ".bias"))
    half_ff = 1.0 if mistake == "no_half" else 0.5
    x = np.asarray(x, np.float64).copy()
    # ff1
    y = ln(x, *nm("norm_ff1"))
    h = silu(gemm(y, *lw("ff1.linear1")))
    x = x + half_ff * gemm(h, *lw("ff1.linear2"))
    # attention
    if rel:
        y = ln(x, *nm("norm_attn"))
        q, k, v = (gemm(y, W.m(p + f"attn.linear_{n}.weight")) for n in "qkv")
        pos = gemm(rel_positions(d, t + 15, 2 * t + 15), W.m(p + "attn.linear_pos.weight"))
        u, vb = W.t(p + "attn.pos_bias_u").ravel(), W.t(p + "attn.pos_bias_v").ravel()
        if mistake == "swap_uv":
            u, vb = vb, u
        o = np.zeros((t, d))
        idx = np.arange(t)[None, :] - np.arange(t)[:, None] + t + 15  # [i][j] -> row j − i + t + 15
        for hh in range(heads):
            sl = slice(hh * hd, (hh + 1) * hd)
            s = (q[:, sl] + u[sl]) @ k[:, sl].T
            pt = (q[:, sl] + vb[sl]) @ pos[:, sl].T  # [i][row]
            s = s + np.take_along_axis(pt, idx, axis=1)
            o[:, sl] = softmax_rows(s / math.sqrt(hd)) @ v[:, sl]
    else:
        y = ln(x, *nm("norm_attn"))
        table = rope_table(t, hd, 5000.0)
        wq, bq = lw("attn.linear_q")
        wk, bk = lw("attn.linear_k")
        if mistake == "rope_after":
            q, k = rope(gemm(y, wq, bq), table, heads, hd), rope(gemm(y, wk, bk), table, heads, hd)
        else:
            yr = rope(y, table, heads, hd)
            q, k = gemm(yr, wq, bq), gemm(yr, wk, bk)
        v = gemm(y, *lw("attn.linear_v"))
        o = np.zeros((t, d))
        for hh in range(heads):
            sl = slice(hh * hd, (hh + 1) * hd)
            o[:, sl] = softmax_rows(q[:, sl] @ k[:, sl].T / math.sqrt(hd)) @ v[:, sl]
    x = x + gemm(o, *lw("attn.linear_out"))
    # conv module
    y = ln(x, *nm("norm_conv"))
    hh = gemm(y, *lw("conv.pointwise1"))
    glu = hh[:, :d] * sigmoid(hh[:, d:])
    taps = W.t(p + "conv.depthwise.weight").reshape(d, K)  # [d][kernel] in the file
    acc = np.tile(W.t(p + "conv.depthwise.bias") if bias else np.zeros(d), (t, 1))
    for kk in range(K):
        src = np.arange(t) + kk - K // 2
        ok = (src >= 0) & (src < t)
        acc[ok] += glu[src[ok]] * taps[:, kk]
    if rel:
        bw, bb = W.t(p + "conv.bn.weight"), W.t(p + "conv.bn.bias")
        mean, var = W.t(p + "conv.bn.running_mean"), W.t(p + "conv.bn.running_var")
        scale = bw / (var if mistake == "bn_var" else np.sqrt(var + EPS))
        z = acc * scale + (bb - mean * scale)
    else:
        z = ln(acc, *nm("conv.ln"))
    x = x + gemm(silu(z), *lw("conv.pointwise2"))
    # ff2
    y = ln(x, *nm("norm_ff2"))
    h = silu(gemm(y, *lw("ff2.linear1")))
    x = x + half_ff * gemm(h, *lw("ff2.linear2"))
    return x if mistake == "no_norm_out" else ln(x, *nm("norm_out"))


def check(got, want, tol, mistakes):
    err = rel_err(got, want)
    print(f"rel L2 {err:.3g} (tol {tol:.3g})", {k: round(rel_err(got, w), 6) for k, w in mistakes.items()})
    assert err < tol, f"oracle vs restatement rel L2 {err:.3g}"
    for name, wrong in mistakes.items():
        e = rel_err(got, wrong)
        assert e > 20 * tol, f"the check cannot see the mistake {name!r}: rel L2 {e:.3g}"
    return err


@pytest.fixture(scope="module")
def parakeet():
    path = synth.model_path("parakeet", small=True, perturb=True)
    return path, Weights(path), ox.Model(path), synth.SMALL["parakeet"]


@pytest.fixture(scope="module")
def gigaam():
    path = synth.model_path("gigaam", small=True, perturb=True)
    return path, Weights(path), ox.Model(path), synth.SMALL["gigaam"]


@pytest.mark.parametrize("layers", [1, 2])
def test_relative_blocks(parakeet, layers):
    _, W, om, cfg = parakeet
    t = 41
    x = np.random.default_rng(3).normal(0, 1, (t, cfg["d"])).astype(np.float32)
    got = om.blocks(x, layers)
    want = x.astype(np.float64)
    for i in range(layers):
        want = block64(W, i, want, cfg, True)
    wrong = {}
    for m in ("swap_uv", "no_half", "no_norm_out", "bn_var"):
        w = x.astype(np.float64)
        for i in range(layers):
            w = block64(W, i, w, cfg, True, m)
        wrong[m] = w
    check(got, want, 2e-5, wrong)


def test_rotary_block(gigaam):
    _, W, om, cfg = gigaam
    t = 37
    x = np.random.default_rng(4).normal(0, 1, (t, cfg["d"])).astype(np.float32)
    got = om.blocks(x, 1)
    want = block64(W, 0, x, cfg, False)
    wrong = {m: block64(W, 0, x, cfg, False, m) for m in ("rope_after", "no_half", "no_norm_out")}
    check(got, want, 5e-5, wrong)


def half_len(n):
    return (n - 1) // 2 + 1


def parakeet_encode64(W, cfg, mel, mistake=None):
    """Parakeet Encoder::run (src/parakeet/cpu.rs:67-174) with valid = all mel frames."""
    mels, ch, d = cfg["mels"], cfg["ch"], cfg["d"]
    mf = mel.shape[0]
    valid = mf
    t1, f1 = half_len(valid), half_len(mels)
    t2, f2 = half_len(half_len(mf)), half_len(f1)
    t, f = half_len(half_len(half_len(mf - 1))), half_len(f2)
    taps = lambda i: (W.t(f"enc.pre_encode.conv.{i}.weight").reshape(ch, 9), W.t(f"enc.pre_encode.conv.{i}.bias"))
    w0, b0 = taps(0)
    w2, b2 = taps(2)
    w5, b5 = taps(5)
    melp = np.zeros((valid + 2, mels + 2))
    melp[1:valid + 1, 1:mels + 1] = mel[:valid]
    c0 = np.zeros((t1, f1, ch))
    for tap in range(9):
        dt, df = tap // 3, tap % 3
        xs = melp[dt:dt + 2 * t1:2, df:df + 2 * f1:2][:t1, :f1]
        c0 += xs[:, :, None] * w0[:, tap][None, None, :]
    c0 = np.maximum(c0 + b0, 0.0)
    c0p = np.zeros((t1 + 2, f1 + 2, ch))
    c0p[1:t1 + 1, 1:f1 + 1] = c0
    c2 = np.zeros((t2, f2, ch))
    for tap in range(9):
        dt, df = tap // 3, tap % 3
        c2 += c0p[dt:dt + 2 * t2:2, df:df + 2 * f2:2][:t2, :f2] * w2[:, tap]
    c2 += b2
    c2[half_len(t1):] = 0.0  # conv2's rows from ⌈valid/4⌉ on are masked
    c3 = np.maximum(gemm(c2.reshape(-1, ch), W.m("enc.pre_encode.conv.3.weight"),
                         W.t("enc.pre_encode.conv.3.bias")), 0.0).reshape(t2, f2, ch)
    c3p = np.zeros((t2 + 2, f2 + 2, ch))
    c3p[1:t2 + 1, 1:f2 + 1] = c3
    c5 = np.zeros((t, f, ch))
    for tap in range(9):
        dt, df = tap // 3, tap % 3
        c5 += c3p[dt:dt + 2 * t:2, df:df + 2 * f:2][:t, :f] * w5[:, tap]
    c5 += b5
    c6 = np.maximum(gemm(c5.reshape(-1, ch), W.m("enc.pre_encode.conv.6.weight"),
                         W.t("enc.pre_encode.conv.6.bias")), 0.0).reshape(t, f, ch)
    flat = c6.transpose(0, 2, 1).reshape(t, ch * f)  # [t][ch·f]
    if mistake == "flatten_f_major":
        flat = c6.reshape(t, f * ch)
    x = gemm(flat, W.m("enc.pre_encode.out.weight"), W.t("enc.pre_encode.out.bias"))
    for i in range(cfg["layers"]):
        x = block64(W, i, x, cfg, True)
    return gemm(x, W.m("joint.enc.weight"), W.t("joint.enc.bias"))


def test_parakeet_encoder(parakeet):
    _, W, om, cfg = parakeet
    mel = synth.parakeet_mel(synth.audio(3.3, 5))
    got = om.encode(mel)
    want = parakeet_encode64(W, cfg, mel)
    assert got.shape == want.shape
    check(got, want, 5e-4, {"flatten_f_major": parakeet_encode64(W, cfg, mel, "flatten_f_major")})


def gigaam_encode64(W, cfg, mel, mistake=None):
    """GigaAM Encoder::record (src/gigaam/encoder.rs:83-93): two conv1d [5, 2, 2] + ReLU, blocks, head."""
    d = cfg["d"]

    def conv(x, name):
        tt, c = x.shape
        rows = (tt + 4 - 5) // 2 + 1
        xp = np.zeros((tt + 4, c))
        xp[2:tt + 2] = x
        col = np.stack([xp[2 * i:2 * i + 5].T.reshape(-1) for i in range(rows)])  # [c·5 + k]
        if mistake == "im2col_k_major":
            col = np.stack([xp[2 * i:2 * i + 5].reshape(-1) for i in range(rows)])
        return np.maximum(gemm(col, W.m(name + ".weight"), W.t(name + ".bias")), 0.0)

    x = conv(conv(mel.astype(np.float64), "enc.pre_encode.conv.0"), "enc.pre_encode.conv.2")
    for i in range(cfg["layers"]):
        x = block64(W, i, x, cfg, False)
    return gemm(x, W.m("head.ctc.weight"), W.t("head.ctc.bias"))


def test_gigaam_encoder(gigaam):
    _, W, om, cfg = gigaam
    mel = synth.gigaam_mel(synth.audio(2.2, 6))
    got = om.encode(mel)[:, :cfg["classes"]]
    want = gigaam_encode64(W, cfg, mel)
    check(got, want, 5e-4, {"im2col_k_major": gigaam_encode64(W, cfg, mel, "im2col_k_major")})


@pytest.fixture(scope="module")
def whisper():
    path = synth.model_path("whisper", small=True, perturb=True)
    return path, Weights(path), ox.Model(path), synth.SMALL["whisper"]


def whisper_encode64(W, cfg, mel, mistake=None):
    """Whisper's encoder (src/whisper/cpu.rs:40-47, src/cpu/transformer.rs:94-117)."""
    d, heads, t = cfg["d"], cfg["heads"], cfg["frames"]
    hd = d // heads

    def conv(x, name, stride):
        tt, c = x.shape
        rows = (tt + 2 - 3) // stride + 1
        xp = np.zeros((tt + 2, c))
        xp[1:tt + 1] = x
        col = np.stack([xp[stride * i:stride * i + 3].T.reshape(-1) for i in range(rows)])
        return gemm(col, W.m(name + ".weight"), W.t(name + ".bias"))

    h = gelu(conv(mel.astype(np.float64), "enc.conv.0", 1))
    x = W.t("enc.pos_emb.weight") + gelu(conv(h, "enc.conv.1", 2))
    for i in range(cfg["layers"]):
        p = f"enc.blocks.{i}."
        y = ln(x, W.t(p + "norm_attn.weight"), W.t(p + "norm_attn.bias"))
        q = gemm(y, W.m(p + "attn.q.weight"), W.t(p + "attn.q.bias"))
        k = gemm(y, W.m(p + "attn.k.weight"))
        v = gemm(y, W.m(p + "attn.v.weight"), W.t(p + "attn.v.bias"))
        o = np.zeros((t, d))
        for hh in range(heads):
            sl = slice(hh * hd, (hh + 1) * hd)
            o[:, sl] = softmax_rows(q[:, sl] @ k[:, sl].T / math.sqrt(hd)) @ v[:, sl]
        x = x + gemm(o, W.m(p + "attn.out.weight"), W.t(p + "attn.out.bias"))
        nf = "norm_attn" if mistake == "wrong_norm" else "norm_ffn"
        y = ln(x, W.t(p + nf + ".weight"), W.t(p + nf + ".bias"))
        x = x + gemm(gelu(gemm(y, W.m(p + "ffn.fc1.weight"), W.t(p + "ffn.fc1.bias"))),
                     W.m(p + "ffn.fc2.weight"), W.t(p + "ffn.fc2.bias"))
    if mistake == "no_final_norm":
        return x
    return ln(x, W.t("enc.final_norm.weight"), W.t("enc.final_norm.bias"))


def test_whisper_encoder(whisper):
    _, W, om, cfg = whisper
    mel = synth.whisper_mel(synth.audio(2.0, 4), cfg["mels"], 2 * cfg["frames"])
    got = om.encode(mel)
    want = whisper_encode64(W, cfg, mel)
    wrong = {m: whisper_encode64(W, cfg, mel, m) for m in ("wrong_norm", "no_final_norm")}
    check(got, want, 3e-4, wrong)


class Decoder64:
    """Decoder::cache / step (src/cpu/transformer.rs:161-266) in float64, caches rounded to f16 as the
    reference's pack rounds them, queries rounded to f16 as attend rounds them (src/cpu/ops.rs:304-337)."""

    def __init__(self, W, cfg, enc, mistake=None):
        self.W, self.cfg, self.mistake = W, cfg, mistake
        d = cfg["d"]
        self.own = [[] for _ in range(cfg["dec_layers"])]
        self.cross = []
        for i in range(cfg["dec_layers"]):
            p = f"dec.blocks.{i}.cross_attn."
            k = gemm(enc, W.m(p + "k.weight"))
            v = gemm(enc, W.m(p + "v.weight"), W.t(p + "v.bias"))
            self.cross.append((h16(k), h16(v)))
        self.d = d

    def attend(self, q, k, v):
        heads = self.cfg["dec_heads"]
        hd = self.d // heads
        q = h16(q)
        o = np.zeros(self.d)
        for hh in range(heads):
            sl = slice(hh * hd, (hh + 1) * hd)
            s = k[:, sl] @ q[sl] / math.sqrt(hd)
            p = np.exp(s - s.max())
            o[sl] = (p / p.sum()) @ v[:, sl]
        return o

    def step(self, token, pos):
        W, d = self.W, self.d
        x = W.m("dec.token_embd.weight")[token] + W.t("dec.pos_emb.weight")[pos]
        nm = lambda p, n: (W.t(p + n + ".weight"), W.t(p + n + ".bias"))
        for i in range(self.cfg["dec_layers"]):
            p = f"dec.blocks.{i}."
            y = ln(x, *nm(p, "norm_self"))
            q = gemv(y, W.m(p + "self_attn.q.weight"), W.t(p + "self_attn.q.bias"))
            k = gemv(y, W.m(p + "self_attn.k.weight"))
            v = gemv(y, W.m(p + "self_attn.v.weight"), W.t(p + "self_attn.v.bias"))
            self.own[i].append((h16(k), h16(v)))
            ks = np.stack([a for a, _ in self.own[i]])
            vs = np.stack([b for _, b in self.own[i]])
            x = x + gemv(self.attend(q, ks, vs), W.m(p + "self_attn.out.weight"), W.t(p + "self_attn.out.bias"))
            y = ln(x, *nm(p, "norm_cross"))
            q = gemv(y, W.m(p + "cross_attn.q.weight"), W.t(p + "cross_attn.q.bias"))
            kc, vc = self.cross[i]
            if self.mistake == "cross_kv_swapped":
                kc, vc = vc, kc
            x = x + gemv(self.attend(q, kc, vc), W.m(p + "cross_attn.out.weight"), W.t(p + "cross_attn.out.bias"))
            y = ln(x, *nm(p, "norm_ffn"))
            h = gelu(gemv(y, W.m(p + "ffn.fc1.weight"), W.t(p + "ffn.fc1.bias")))
            x = x + gemv(h, W.m(p + "ffn.fc2.weight"), W.t(p + "ffn.fc2.bias"))
        y = ln(x, *nm("", "dec.final_norm")) if self.mistake != "no_final_norm" else x
        return gemv(y, W.m("dec.token_embd.weight"))


def test_whisper_decoder_steps(whisper):
    _, W, om, cfg = whisper
    enc = np.random.default_rng(8).normal(0, 1, (cfg["frames"], cfg["d"])).astype(np.float32)
    om.whisper_begin(enc)
    right = Decoder64(W, cfg, enc)
    wrong = {m: Decoder64(W, cfg, enc, m) for m in ("cross_kv_swapped", "no_final_norm")}
    tokens = np.random.default_rng(9).integers(0, cfg["vocab"], 6)
    for pos, tok in enumerate(tokens):
        got = om.whisper_step(int(tok), pos, cfg["vocab"])
        check(got, right.step(int(tok), pos), 1e-4, {m: w.step(int(tok), pos) for m, w in wrong.items()})


def predict64(W, cfg, token, state, mistake=None):
    """Decoder::predict (src/parakeet/decoder.rs:107-133): LSTM layers (gates i, f, g, o) on the
    embedding of `token` (zeros for None), then the joint's predictor projection."""
    n, layers = cfg["hidden"], cfg["lstm_layers"]
    x = np.zeros(n) if token is None else W.m("pred.embed.weight")[token]
    nxt = np.zeros(2 * layers * n)
    for l in range(layers):
        h, c = state[2 * n * l:2 * n * l + n], state[2 * n * l + n:2 * n * (l + 1)]
        g = gemv(x, W.m(f"pred.lstm.{l}.Wx")) + gemv(h, W.m(f"pred.lstm.{l}.Wh")) + W.t(f"pred.lstm.{l}.bias")
        i_, f_, g_, o_ = g[:n], g[n:2 * n], g[2 * n:3 * n], g[3 * n:]
        if mistake == "gates_ifog_as_fiog":
            i_, f_ = f_, i_
        nc = sigmoid(f_) * c + sigmoid(i_) * np.tanh(g_)
        nh = sigmoid(o_) * np.tanh(nc)
        nxt[2 * n * l:2 * n * l + n], nxt[2 * n * l + n:2 * n * (l + 1)] = nh, nc
        x = nh
    return nxt, gemv(x, W.m("joint.pred.weight"), W.t("joint.pred.bias"))


def joint64(W, enc_row, pred, mistake=None):
    z = np.maximum(np.asarray(enc_row, np.float64) + pred, 0.0)
    if mistake == "no_relu":
        z = np.asarray(enc_row, np.float64) + pred
    return gemv(z, W.m("joint.out.weight"), W.t("joint.out.bias"))


def test_tdt_predictor_and_joint(parakeet):
    _, W, om, cfg = parakeet
    n, layers, j = cfg["hidden"], cfg["lstm_layers"], cfg["joint"]
    outs = cfg["vocab"] + len(cfg["durations"])
    rng = np.random.default_rng(12)
    state = np.zeros(2 * layers * n, np.float32)
    for token in (None, 5, 700, 5):
        if token == 700:  # a state away from the trajectory: large h and c
            state = rng.normal(0, 1, 2 * layers * n).astype(np.float32)
        got_next, got_pred = om.predict(-1 if token is None else token, state, n, j, layers)
        want_next, want_pred = predict64(W, cfg, token, state.astype(np.float64))
        _, wrong_pred = predict64(W, cfg, token, state.astype(np.float64), "gates_ifog_as_fiog")
        wrong_next, _ = predict64(W, cfg, token, state.astype(np.float64), "gates_ifog_as_fiog")
        check(got_next, want_next, 1e-5, {"gates": wrong_next})
        check(got_pred, want_pred, 1e-5, {"gates": wrong_pred})
        enc_row = rng.normal(0, 1, j).astype(np.float32)
        check(om.joint(enc_row, got_pred, outs), joint64(W, enc_row, got_pred.astype(np.float64)), 1e-5,
              {"no_relu": joint64(W, enc_row, got_pred.astype(np.float64), "no_relu")})
        state = got_next


def test_batch_norm_fold_closed_form():
    """src/conformer.rs:130-139: scale = γ/√(var + ε), shift = β − mean·scale."""
    rng = np.random.default_rng(2)
    d = 37
    w, b, mean = (rng.normal(0, 1, d).astype(np.float32) for _ in range(3))
    var = rng.uniform(0.1, 2.0, d).astype(np.float32)
    scale, shift = np.zeros(d, np.float32), np.zeros(d, np.float32)
    f = lambda a: a.ctypes.data_as(ox._fp)
    ox.lib().ox_batch_norm(f(w), f(b), f(mean), f(var), d, f(scale), f(shift))
    s64 = w.astype(np.float64) / np.sqrt(var.astype(np.float64) + 1e-5)
    assert np.allclose(scale, s64, rtol=1e-6)
    assert np.allclose(shift, b - mean.astype(np.float64) * s64, rtol=1e-5, atol=1e-6)
