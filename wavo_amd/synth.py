"""Seeded synthetic models, audio and log-mel features for the benchmark configurations.

Models are GGUF v3 files with the metadata keys and tensor names the reference's family loaders read
(src/gigaam/mod.rs:55-84, src/parakeet/mod.rs:49-122 and decoder.rs:46-89, src/whisper/mod.rs:79-155,
src/conformer.rs:34-61 and :180-229, src/transformer.rs:103-223).  Weights are random-init N(0, 0.02)
and the linear (GEMM) weights are stored in one GGUF type (Q8_0 by default, as the benchmark
configurations state; F16 or Q4_0 on request); norms have gain 1 and bias 0, BatchNorm mean 0, var 1,
gain 1, bias 0; biases N(0, 0.02).  Each tensor draws from its own seed (a hash of the model seed and
its name), so a tensor does not depend on which others exist.

Audio follows the benchmark generator: Gaussian noise σ = 0.05 plus 3 linear chirps (100–4000 Hz,
amplitude 0.1) spanning the clip, 16 kHz mono.  The log-mel frontends compute each family's feature
shape (frame count, bins, normalization) in numpy; they are inputs for both the oracle and the
device path, not a restatement of the reference's FFT frontends (which stay on the host there too).
"""

import hashlib
import os

import numpy as np

from . import gguf

SR = 16000

CONFIGS = {
    # GigaAM-v3 shape, CTC over 256 tokens + blank, 11 s.
    "gigaam": dict(arch="gigaam", layers=16, d=768, heads=16, d_ff=3072, kernel=5, mels=64, classes=257),
    # Parakeet-TDT-0.6B-v3 shape, 60 s.
    "parakeet": dict(arch="parakeet", layers=24, d=1024, heads=8, d_ff=4096, kernel=9, mels=128, ch=256,
                     joint=640, hidden=640, vocab=8193, durations=[0, 1, 2, 3, 4], lstm_layers=1),
    # Whisper-large-v3-turbo shape.
    "whisper": dict(arch="whisper", layers=32, d=1280, heads=20, d_ff=5120, dec_layers=4, dec_heads=20,
                    vocab=51866, mels=128, frames=1500, context=448),
}

# Small shapes of the same families for parity tests that the CPU oracle finishes in seconds.
SMALL = {
    "gigaam": dict(arch="gigaam", layers=2, d=256, heads=4, d_ff=1024, kernel=5, mels=64, classes=257),
    "parakeet": dict(arch="parakeet", layers=2, d=256, heads=2, d_ff=1024, kernel=9, mels=128, ch=64,
                     joint=320, hidden=128, vocab=1025, durations=[0, 1, 2, 3, 4], lstm_layers=2),
    "whisper": dict(arch="whisper", layers=2, d=256, heads=4, d_ff=1024, dec_layers=2, dec_heads=4,
                    vocab=1000, mels=80, frames=100, context=64),
    # A decoder context past one 256-key attend part (long decodes).
    "whisper_ctx": dict(arch="whisper", layers=2, d=256, heads=4, d_ff=1024, dec_layers=2, dec_heads=4,
                        vocab=1000, mels=80, frames=100, context=320),
}


def _rng(seed, name):
    h = hashlib.blake2b(f"{seed}/{name}".encode(), digest_size=8).digest()
    return np.random.default_rng(int.from_bytes(h, "little"))


class _Builder:
    def __init__(self, seed, wtype, perturb=False):
        self.w = gguf.Writer()
        self.seed = seed
        self.wtype = wtype
        # perturb: norms, BatchNorm statistics and position biases away from their identity values
        # (gain 1 + N(0, 0.2), shift N(0, 0.2), BN mean N(0, 0.2) and var U(0.5, 1.5), u/v N(0, 0.3),
        # LSTM gate biases N(0, 1): gates that differ, not all near one half),
        # so that a check of the composition sees which parameter goes where.
        self.perturb = perturb

    def normal(self, name, n, std=0.02):
        return (_rng(self.seed, name).standard_normal(n, dtype=np.float32) * np.float32(std)).astype(np.float32)

    def f32(self, name, dims, values):
        self.w.tensor(name, dims, gguf.F32, np.ascontiguousarray(values, np.float32).tobytes())

    def linear(self, name, dims, bias=True, row_scale=None):
        """A GEMM weight in the model's type (ggml dims, last = outputs), with a N(0, 0.02) bias;
        row_scale (row, factor) multiplies one output row."""
        n = int(np.prod(dims))
        w = self.normal(name + ".weight", n)
        k = int(np.prod(dims[:-1]))
        if row_scale is not None:
            r, f = row_scale
            w[r * k:(r + 1) * k] *= np.float32(f)
        wt = self.wtype if k % 32 == 0 else gguf.F32
        # Quantize in pieces of 16M values to bound the temporary memory.
        step = 1 << 24
        raw = b"".join(gguf.encode(w[i:i + step], wt) for i in range(0, n, step))
        self.w.tensor(name + ".weight", dims, wt, raw)
        if bias:
            self.f32(name + ".bias", [dims[-1]], self.normal(name + ".bias", dims[-1]))

    def norm(self, name, d, bias=True):
        g = 1.0 + self.normal(name + ".weight", d, 0.2) if self.perturb else np.ones(d, np.float32)
        self.f32(name + ".weight", [d], g)
        if bias:
            self.f32(name + ".bias", [d], self.normal(name + ".bias", d, 0.2) if self.perturb else np.zeros(d, np.float32))


def _conformer_blocks(b, c, arch):
    d, f, k, heads = c["d"], c["d_ff"], c["kernel"], c["heads"]
    bias = arch == "gigaam"
    for i in range(c["layers"]):
        p = f"enc.blocks.{i}."
        b.norm(p + "norm_ff1", d)
        b.linear(p + "ff1.linear1", [d, f], bias)
        b.linear(p + "ff1.linear2", [f, d], bias)
        b.norm(p + "norm_attn", d)
        for n in ("q", "k", "v", "out"):
            b.linear(p + f"attn.linear_{n}", [d, d], bias)
        if arch == "parakeet":
            b.linear(p + "attn.linear_pos", [d, d], False)
            for n in ("u", "v"):
                b.f32(p + f"attn.pos_bias_{n}", [d // heads, heads],
                      b.normal(p + f"attn.pos_bias_{n}", d, 0.3 if b.perturb else 0.02))
        b.norm(p + "norm_conv", d)
        b.linear(p + "conv.pointwise1", [1, d, 2 * d], bias)
        b.f32(p + "conv.depthwise.weight", [k, 1, d], b.normal(p + "conv.depthwise.weight", k * d))
        if bias:
            b.f32(p + "conv.depthwise.bias", [d], b.normal(p + "conv.depthwise.bias", d))
        if arch == "gigaam":
            b.norm(p + "conv.ln", d)
        else:
            if b.perturb:
                b.f32(p + "conv.bn.weight", [d], 1.0 + b.normal(p + "conv.bn.weight", d, 0.2))
                b.f32(p + "conv.bn.bias", [d], b.normal(p + "conv.bn.bias", d, 0.2))
                b.f32(p + "conv.bn.running_mean", [d], b.normal(p + "conv.bn.running_mean", d, 0.2))
                b.f32(p + "conv.bn.running_var", [d],
                      _rng(b.seed, p + "conv.bn.running_var").uniform(0.5, 1.5, d).astype(np.float32))
            else:
                b.f32(p + "conv.bn.weight", [d], np.ones(d))
                b.f32(p + "conv.bn.bias", [d], np.zeros(d))
                b.f32(p + "conv.bn.running_mean", [d], np.zeros(d))
                b.f32(p + "conv.bn.running_var", [d], np.ones(d))
        b.linear(p + "conv.pointwise2", [1, d, d], bias)
        b.norm(p + "norm_ff2", d)
        b.linear(p + "ff2.linear1", [d, f], bias)
        b.linear(p + "ff2.linear2", [f, d], bias)
        b.norm(p + "norm_out", d)


def _encoder_keys(w, arch, c, conv_norm):
    e = f"stt.{arch}.encoder."
    w.u32(e + "n_layers", c["layers"])
    w.u32(e + "d_model", c["d"])
    w.u32(e + "n_heads", c["heads"])
    w.u32(e + "d_ff", c["d_ff"])
    w.u32(e + "conv_kernel", c["kernel"])
    w.str(e + "conv_norm_type", conv_norm)


def _vocab(w, n, blank):
    w.str("tokenizer.ggml.model", "bpe")
    w.strs("tokenizer.ggml.tokens", [f"▁t{i}" for i in range(n - 1)] + ["<blank>"] if blank else
           [f"t{i}" for i in range(n)])
    w.i32s("tokenizer.ggml.token_type", [1] * n)


def build_gigaam(c, b):
    w = b.w
    w.str("general.architecture", "gigaam")
    _encoder_keys(w, "gigaam", c, "layer_norm")
    w.str("stt.gigaam.encoder.self_attention_model", "rotary")
    w.u32("stt.gigaam.encoder.subs_kernel_size", 5)
    w.u32("stt.gigaam.encoder.subsampling_factor", 4)
    w.u32("stt.gigaam.encoder.pos_emb_max_len", 5000)
    w.str("stt.gigaam.head_kind", "ctc")
    w.u32("stt.gigaam.head.feat_in", c["d"])
    w.u32("stt.gigaam.head.num_classes", c["classes"])
    w.u32("stt.frontend.sample_rate", SR)
    w.u32("stt.frontend.n_fft", 320)
    w.u32("stt.frontend.win_length", 320)
    w.u32("stt.frontend.hop_length", 160)
    w.u32("stt.frontend.num_mels", c["mels"])
    _vocab(w, c["classes"], True)
    w.u32("tokenizer.ggml.blank_token_id", c["classes"] - 1)
    # The frontend's tables as the converter stores them (src/gigaam/frontend.rs:28-45): periodic Hann
    # of 320 and an HTK filterbank [mels][161].
    b.f32("frontend.window", [320], hann_periodic(320))
    b.f32("frontend.mel_filterbank", [161, c["mels"]], htk_filters(SR, 320, c["mels"]))
    d, m = c["d"], c["mels"]
    b.linear("enc.pre_encode.conv.0", [5, m, d])
    b.linear("enc.pre_encode.conv.2", [5, d, d])
    _conformer_blocks(b, c, "gigaam")
    b.linear("head.ctc", [1, d, c["classes"]])


def build_parakeet(c, b):
    w = b.w
    w.str("general.architecture", "parakeet")
    w.str("stt.parakeet.head_kind", "tdt")
    w.str("stt.parakeet.encoder.att_context_style", "regular")
    _encoder_keys(w, "parakeet", c, "batch_norm")
    for k, v in (("subsampling_factor", 8), ("subsampling_channels", c["ch"])):
        w.u32("stt.parakeet.encoder." + k, v)
    w.bool("stt.parakeet.encoder.use_bias", False)
    w.bool("stt.parakeet.encoder.xscaling", False)
    for k, v in (("att_context_left", -1), ("att_context_right", -1), ("conv_context_left", c["kernel"] // 2),
                 ("conv_context_right", c["kernel"] // 2)):
        w.i32("stt.parakeet.encoder." + k, v)
    w.str("stt.frontend.type", "mel")
    w.str("stt.frontend.window", "hann")
    w.str("stt.frontend.normalize", "per_feature")
    for k, v in (("sample_rate", SR), ("num_mels", c["mels"]), ("n_fft", 512), ("win_length", 400),
                 ("hop_length", 160)):
        w.u32("stt.frontend." + k, v)
    w.f32("stt.frontend.pre_emphasis", 0.97)
    w.f32("stt.frontend.f_min", 0.0)
    w.f32("stt.frontend.f_max", 8000.0)
    vocab, hidden, joint = c["vocab"], c["hidden"], c["joint"]
    w.u32("stt.parakeet.joint.hidden", joint)
    w.str("stt.parakeet.joint.activation", "relu")
    w.u32("stt.parakeet.joint.num_extra_outputs", len(c["durations"]))
    w.u32("stt.parakeet.predictor.hidden", hidden)
    w.u32("stt.parakeet.predictor.n_layers", c["lstm_layers"])
    w.u32("stt.parakeet.predictor.vocab", vocab)
    w.i32s("stt.parakeet.tdt.durations", c["durations"])
    w.u32("stt.parakeet.tdt.max_symbols", c.get("max_symbols", 10))
    if "symbol_budget" in c:
        w.str("stt.parakeet.tdt.symbol_budget", c["symbol_budget"])
    _vocab(w, vocab, True)
    w.u32("tokenizer.ggml.unknown_token_id", 0)
    w.u32("tokenizer.ggml.blank_token_id", vocab - 1)
    d, ch = c["d"], c["ch"]
    for i in (0, 2, 5):
        n = f"enc.pre_encode.conv.{i}"
        b.f32(n + ".weight", [3, 3, 1, ch], b.normal(n + ".weight", 9 * ch))
        b.f32(n + ".bias", [ch], b.normal(n + ".bias", ch))
    b.linear("enc.pre_encode.conv.3", [1, 1, ch, ch])
    b.linear("enc.pre_encode.conv.6", [1, 1, ch, ch])
    f8 = (((c["mels"] - 1) // 2 + 1 - 1) // 2 + 1 - 1) // 2 + 1
    b.linear("enc.pre_encode.out", [ch * f8, d])
    _conformer_blocks(b, c, "parakeet")
    b.linear("joint.enc", [d, joint])
    # TDT decoder (src/parakeet/decoder.rs:66-89).
    b.linear("pred.embed", [hidden, vocab], False)
    for l in range(c["lstm_layers"]):
        # The LSTM matrices carry no `.weight` suffix (src/parakeet/decoder.rs:66-72).
        for n in ("Wx", "Wh"):
            name = f"pred.lstm.{l}.{n}"
            b.w.tensor(name, [hidden, 4 * hidden], b.wtype, gguf.encode(b.normal(name, 4 * hidden * hidden), b.wtype))
        b.f32(f"pred.lstm.{l}.bias", [4 * hidden], b.normal(f"pred.lstm.{l}.bias", 4 * hidden, 1.0 if b.perturb else 0.02))
    b.linear("joint.pred", [hidden, joint])
    # blank_bias: added to the blank's output bias (a decoder that emits blanks often).
    outs = vocab + len(c["durations"])
    b.linear("joint.out", [joint, outs], False)
    ob = b.normal("joint.out.bias", outs)
    ob[vocab - 1] += np.float32(c.get("blank_bias", 0.0))
    b.f32("joint.out.bias", [outs], ob)


def sinusoids(length, channels, max_timescale=10000.0):
    """Whisper's encoder positions: [sin | cos] of log-spaced timescales."""
    inc = np.log(max_timescale) / (channels // 2 - 1)
    inv = np.exp(-inc * np.arange(channels // 2))
    t = np.arange(length)[:, None] * inv[None, :]
    return np.concatenate([np.sin(t), np.cos(t)], axis=1).astype(np.float32)


def build_whisper(c, b):
    w = b.w
    w.str("general.architecture", "whisper")
    for k, v in (("stt.frontend.type", "mel"), ("stt.frontend.window", "hann_periodic"),
                 ("stt.frontend.normalize", "whisper_logmel"), ("stt.frontend.pad_mode", "reflect"),
                 ("stt.whisper.encoder.activation", "gelu"), ("stt.whisper.decoder.activation", "gelu")):
        w.str(k, v)
    frames = c["frames"]
    for k, v in (("stt.frontend.sample_rate", SR), ("stt.frontend.n_fft", 400), ("stt.frontend.win_length", 400),
                 ("stt.frontend.hop_length", 160), ("stt.frontend.n_samples", frames * 320),
                 ("stt.frontend.nb_max_frames", 2 * frames), ("stt.whisper.encoder.max_source_positions", frames)):
        w.u32(k, v)
    w.bool("stt.whisper.decoder.tie_word_embeddings", True)
    w.bool("stt.whisper.decoder.scale_embedding", False)
    d = c["d"]
    for part, layers, heads in (("encoder", c["layers"], c["heads"]), ("decoder", c["dec_layers"], c["dec_heads"])):
        w.u32(f"stt.whisper.{part}.d_model", d)
        w.u32(f"stt.whisper.{part}.n_heads", heads)
        w.u32(f"stt.whisper.{part}.n_layers", layers)
        w.u32(f"stt.whisper.{part}.ffn_dim", c["d_ff"])
    w.u32("stt.whisper.decoder.vocab_size", c["vocab"])
    w.u32("stt.whisper.decoder.max_target_positions", c["context"])
    w.u32("stt.whisper.encoder.num_mel_bins", c["mels"])
    # The frontend's tables (src/whisper/frontend.rs:29-41): periodic Hann of 400 and a Slaney
    # filterbank [mels][201].
    b.f32("frontend.window", [400], hann_periodic(400))
    b.f32("frontend.mel_filterbank", [201, c["mels"]], _mel_filters(SR, 400, c["mels"]).astype(np.float32))
    # Special ids as large-v3's layout: EOT 50257, SOT 50258, …, no-timestamps 50364, <|0.00|> 50365.
    vocab = c["vocab"]
    eot = min(50257, vocab - 110)
    w.u32("tokenizer.ggml.eos_token_id", eot)
    w.u32("stt.whisper.sot_token_id", eot + 1)
    w.u32("stt.whisper.transcribe_token_id", eot + 102)
    w.u32("stt.whisper.no_timestamps_token_id", eot + 107)
    # Suppression lists as large-v3 carries them: ~90 text ids (seeded here), and the begin list
    # [" ", EOT] (src/whisper/mod.rs:131-141 reads both).
    rng = _rng(b.seed, "suppress_tokens")
    w.i32s("stt.whisper.suppress_tokens", sorted(int(x) for x in rng.choice(eot, 88, replace=False)))
    w.i32s("stt.whisper.begin_suppress_tokens", [220 % eot, eot])
    w.bool("stt.capability.lang_detect", False)
    w.strs("tokenizer.ggml.tokens", [f"t{i}" for i in range(vocab)])
    b.linear("enc.conv.0", [3, c["mels"], d])
    b.linear("enc.conv.1", [3, d, d])
    b.f32("enc.pos_emb.weight", [d, frames], sinusoids(frames, d))
    for i in range(c["layers"]):
        p = f"enc.blocks.{i}."
        b.norm(p + "norm_attn", d)
        b.linear(p + "attn.q", [d, d])
        b.linear(p + "attn.k", [d, d], False)
        b.linear(p + "attn.v", [d, d])
        b.linear(p + "attn.out", [d, d])
        b.norm(p + "norm_ffn", d)
        b.linear(p + "ffn.fc1", [d, c["d_ff"]])
        b.linear(p + "ffn.fc2", [c["d_ff"], d])
    b.norm("enc.final_norm", d)
    for i in range(c["dec_layers"]):
        p = f"dec.blocks.{i}."
        b.norm(p + "norm_self", d)
        b.linear(p + "self_attn.q", [d, d])
        b.linear(p + "self_attn.k", [d, d], False)
        b.linear(p + "self_attn.v", [d, d])
        b.linear(p + "self_attn.out", [d, d])
        b.norm(p + "norm_cross", d)
        b.linear(p + "cross_attn.q", [d, d])
        b.linear(p + "cross_attn.k", [d, d], False)
        b.linear(p + "cross_attn.v", [d, d])
        b.linear(p + "cross_attn.out", [d, d])
        b.norm(p + "norm_ffn", d)
        b.linear(p + "ffn.fc1", [d, c["d_ff"]])
        b.linear(p + "ffn.fc2", [c["d_ff"], d])
    b.norm("dec.final_norm", d)
    # eot_scale: EOT's embedding row (the tied head's EOT logit) scaled, so that a window ends on EOT.
    b.linear("dec.token_embd", [d, vocab], False, (eot, c["eot_scale"]) if "eot_scale" in c else None)
    b.f32("dec.pos_emb.weight", [d, c["context"]], b.normal("dec.pos_emb.weight", d * c["context"]))


def write_model(path, config, seed=0, wtype=gguf.Q8_0, perturb=False):
    """Writes a synthetic GGUF for `config` (a CONFIGS/SMALL entry or a dict) and returns the path."""
    c = dict(config)
    b = _Builder(seed, wtype, perturb)
    {"gigaam": build_gigaam, "parakeet": build_parakeet, "whisper": build_whisper}[c["arch"]](c, b)
    tmp = path + ".tmp"
    b.w.write(tmp)
    os.replace(tmp, path)
    return path


def model_path(name, small=False, seed=0, wtype=gguf.Q8_0, directory=None, perturb=False):
    """A cached synthetic model file under `directory` (default /tmp/wavo_models)."""
    directory = directory or os.environ.get("WAVO_MODELS", "/tmp/wavo_models")
    os.makedirs(directory, exist_ok=True)
    # v2: the files carry the frontend's tables (GigaAM, Whisper).
    tag = f"{name}{'-small' if small else ''}-s{seed}-t{wtype}{'-p' if perturb else ''}-v2.gguf"
    path = os.path.join(directory, tag)
    if not os.path.exists(path):
        write_model(path, (SMALL if small else CONFIGS)[name], seed, wtype, perturb)
    return path


# ---------------------------------------------------------------------------------------- audio


def audio(seconds, seed=0, gaps=None):
    """Gaussian σ = 0.05 noise plus 3 linear chirps (f0, f1 ~ U[100, 4000] Hz, amplitude 0.1)."""
    rng = np.random.default_rng(seed)
    n = int(round(seconds * SR))
    t = np.arange(n, dtype=np.float64) / SR
    x = rng.normal(0.0, 0.05, n)
    for _ in range(3):
        f0, f1 = rng.uniform(100, 4000, 2)
        phase = 2 * np.pi * (f0 * t + (f1 - f0) * t * t / (2 * max(seconds, 1e-9)))
        x += 0.1 * np.sin(phase)
    if gaps:
        for start, length in gaps:
            x[int(start * SR):int((start + length) * SR)] = 0.0
    return x.astype(np.float32)


def long_audio(seconds, seed=0):
    """The long-form generator: the same audio with seeded 0.3–1.5 s silences every 5–20 s; returns
    (pcm, gaps) with gaps as (start, length) seconds."""
    rng = np.random.default_rng(seed + 1)
    gaps, at = [], 0.0
    while True:
        at += rng.uniform(5, 20)
        length = rng.uniform(0.3, 1.5)
        if at + length >= seconds:
            break
        gaps.append((at, length))
        at += length
    return audio(seconds, seed, gaps), gaps


def split_at_gaps(seconds, gaps, limit=60.0):
    """Segments (start, end) of at most `limit` s, cut inside the gaps (src/split.rs:42-65 cuts at
    pauses): the last gap that keeps a segment under the limit, else a hard cut."""
    cuts = [g[0] + g[1] / 2 for g in gaps]
    segs, start = [], 0.0
    while seconds - start > limit:
        inside = [c for c in cuts if start < c <= start + limit]
        end = inside[-1] if inside else start + limit
        segs.append((start, end))
        start = end
    segs.append((start, seconds))
    return segs


def hann_periodic(n):
    """0.5 − 0.5·cos(2πi/n), i < n (torch.hann_window(n, periodic=True))."""
    return (0.5 - 0.5 * np.cos(2.0 * np.pi * np.arange(n) / n)).astype(np.float32)


def htk_filters(sr, n_fft, mels, fmin=0.0, fmax=None):
    """HTK-scale triangular filterbank without area normalization [mels][n_fft/2 + 1]
    (torchaudio's melscale_fbanks with mel_scale="htk", norm=None)."""
    fmax = fmax or sr / 2
    freqs = np.linspace(0.0, sr / 2, n_fft // 2 + 1)
    mel = lambda f: 2595.0 * np.log10(1.0 + f / 700.0)
    pts = 700.0 * (10.0 ** (np.linspace(mel(fmin), mel(fmax), mels + 2) / 2595.0) - 1.0)
    diff = pts[1:] - pts[:-1]
    slopes = pts[None, :] - freqs[:, None]
    down = -slopes[:, :-2] / diff[:-1]
    up = slopes[:, 2:] / diff[1:]
    return np.maximum(0.0, np.minimum(down, up)).T.astype(np.float32)


def _mel_filters(sr, n_fft, mels, fmin=0.0, fmax=None):
    """Slaney-style mel filterbank [mels][n_fft/2 + 1] (area-normalized triangles)."""
    fmax = fmax or sr / 2

    def hz_to_mel(f):
        f = np.asarray(f, np.float64)
        lin = f / (200.0 / 3)
        log = 15.0 + np.log(np.maximum(f, 1e-10) / 1000.0) / (np.log(6.4) / 27.0)
        return np.where(f >= 1000.0, log, lin)

    def mel_to_hz(m):
        m = np.asarray(m, np.float64)
        lin = m * (200.0 / 3)
        log = 1000.0 * np.exp((np.log(6.4) / 27.0) * (m - 15.0))
        return np.where(m >= 15.0, log, lin)

    freqs = np.linspace(0, sr / 2, n_fft // 2 + 1)
    pts = mel_to_hz(np.linspace(hz_to_mel(fmin), hz_to_mel(fmax), mels + 2))
    fb = np.zeros((mels, len(freqs)))
    for i in range(mels):
        lo, c, hi = pts[i], pts[i + 1], pts[i + 2]
        fb[i] = np.maximum(0, np.minimum((freqs - lo) / (c - lo), (hi - freqs) / (hi - c)))
        fb[i] *= 2.0 / (hi - lo)
    return fb


def _power(frames, n_fft, window):
    spec = np.fft.rfft(frames * window, n=n_fft)
    return spec.real ** 2 + spec.imag ** 2


def parakeet_mel(pcm, mels=128):
    """[pcm.len()/160 + 1][mels]: pre-emphasis 0.97, 400-sample Hann in a 512 FFT, hop 160, log,
    per-feature normalization over all frames but the last, which is zero (src/parakeet/frontend.rs:52-72)."""
    x = np.concatenate([pcm[:1], pcm[1:] - 0.97 * pcm[:-1]]).astype(np.float64)
    frames = len(x) // 160 + 1
    padded = np.concatenate([np.zeros(256), x, np.zeros(256 + 512)])
    idx = np.arange(frames)[:, None] * 160 + np.arange(512)[None, :]
    win = np.zeros(512)
    win[56:456] = np.hanning(402)[1:-1]
    p = _power(padded[idx], 512, win)
    m = np.log(p @ _mel_filters(SR, 512, mels).T + 2.0 ** -24)
    n = frames - 1
    mean = m[:n].mean(axis=0)
    std = np.sqrt(((m[:n] - mean) ** 2).sum(axis=0) / max(n - 1, 1))
    out = (m - mean) / (std + 1e-5)
    out[n] = 0.0
    return out.astype(np.float32)


def gigaam_mel(pcm, mels=64):
    """[(len − 320)/160 + 1][mels]: full 320-sample frames (center = False), Hann, power spectrum,
    ln(clamp(mel, 1e-9, 1e9)) (src/gigaam/frontend.rs:1-71)."""
    frames = (len(pcm) - 320) // 160 + 1
    idx = np.arange(frames)[:, None] * 160 + np.arange(320)[None, :]
    p = _power(pcm.astype(np.float64)[idx], 320, np.hanning(322)[1:-1])
    m = p @ _mel_filters(SR, 320, mels).T
    return np.log(np.clip(m, 1e-9, 1e9)).astype(np.float32)


def whisper_mel(pcm, mels=128, frames=3000):
    """[frames][mels] of a 30 s window: 400-point periodic Hann, hop 160, log10 clamped to max − 8,
    (x + 4) / 4 (Whisper's log-mel)."""
    n = frames * 160
    x = np.zeros(n)
    x[:min(n, len(pcm))] = pcm[:n]
    padded = np.pad(x, (200, 200), mode="reflect")
    idx = np.arange(frames)[:, None] * 160 + np.arange(400)[None, :]
    win = 0.5 - 0.5 * np.cos(2 * np.pi * np.arange(400) / 400)
    p = _power(padded[idx], 400, win)
    m = np.log10(np.maximum(p @ _mel_filters(SR, 400, mels).T, 1e-10))
    m = np.maximum(m, m.max() - 8.0)
    return ((m + 4.0) / 4.0).astype(np.float32)
