"""End-to-end parity of the family encoders (and Whisper's decoder steps) on the device against the CPU
oracle, on the same synthetic GGUF and the same seeded log-mel input.

Bars: encoder outputs within relative L2 1e-2 — the kernels round GEMM operands
to f16 exactly as the oracle (wavo's CPU backend) does, so the remaining error comes from f32 summation
order (~1e-4 after it moves a few f16 roundings) — and identical greedy token ids: CTC (src/gigaam/decoder.rs:135-151), TDT
(src/parakeet/decoder.rs:158-191), and the argmax of every Whisper step.  Each token mismatch would
be reported with the top-2 gap at its frame.
"""

import os

import numpy as np
import pytest

import oracle as ox
import wavo_amd as wa
from parity import ctc_parity, tdt_device_parity, tdt_parity, top2_gap
from wavo_amd import gguf, synth

pytestmark = pytest.mark.gpu

MODELS = os.environ.get("WAVO_MODELS", "/tmp/wavo_models")


def rel_l2(got, want):
    return float(np.linalg.norm(got - want) / max(np.linalg.norm(want), 1e-30))


# The encoder bar (BASELINE): relative L2 1e-2.  Observed errors are ~1e-4: an f32 summation-order
# difference sometimes moves an activation across an f16 rounding boundary before the next GEMM,
# one f16 ulp (2^-11) on that element, as between the reference's own GPU and CPU backends.
ENCODER_TOL = 1e-2


def check_ctc(m, full, want):
    """The product's CTC on the device output equals the oracle's CTC on the same logits, on the host
    and on the device; against the oracle's encoder output only provable near-tie frames may differ."""
    classes = want.shape[1]
    got = full[:, :classes]
    assert m.greedy(full) == ox.ctc(got, classes - 1)
    fb = m.gpu.upload(np.ascontiguousarray(full))
    assert m.greedy_device(fb, full.shape[0], full.shape[1]) == ox.ctc(got, classes - 1)
    flips = ctc_parity(got, want, classes)
    if not flips:
        assert m.greedy(full) == ox.ctc(want, classes - 1)
    return flips


def check_tdt(m, om, got, want):
    """TDT on the device output: the host decoder equals the oracle's, the device decoder
    (wh_model_greedy_device) too up to f32 near-ties; then the device output against the oracle's."""
    assert m.greedy(got) == om.tdt(got), "the product's TDT decoder differs from the oracle's"
    gb = m.gpu.upload(np.ascontiguousarray(got))
    dev_flip = tdt_device_parity(om, m.greedy_device(gb, got.shape[0], got.shape[1]), got)
    assert dev_flip is None or dev_flip[2] <= dev_flip[3]
    flip, tg, tw = tdt_parity(om, got, want)
    if flip is None:
        assert tg == tw
    return flip


@pytest.mark.parametrize("wtype", [gguf.Q8_0, gguf.F16, gguf.Q4_0])
def test_gigaam_small(gpu, wtype):
    path = synth.model_path("gigaam", small=True, wtype=wtype, directory=MODELS)
    mel = synth.gigaam_mel(synth.audio(11, 1))
    want = ox.Model(path).encode(mel)
    m = wa.Model(gpu, path)
    full = m.encode(mel)
    got = full[:, :want.shape[1]]
    assert rel_l2(got, want) < ENCODER_TOL, rel_l2(got, want)
    check_ctc(m, full, want)


@pytest.mark.parametrize("wtype", [gguf.Q8_0, gguf.F16])
def test_parakeet_small(gpu, wtype):
    path = synth.model_path("parakeet", small=True, wtype=wtype, directory=MODELS)
    mel = synth.parakeet_mel(synth.audio(10, 2))
    om = ox.Model(path)
    want = om.encode(mel)
    m = wa.Model(gpu, path)
    got = m.encode(mel)
    assert got.shape == want.shape
    assert rel_l2(got, want) < ENCODER_TOL, rel_l2(got, want)
    check_tdt(m, om, got, want)


@pytest.mark.parametrize("small,seconds", [(True, 3.0), (False, 60.0), (False, 7.3)])
def test_parakeet_attention_reads_in_place(gpu, small, seconds):
    """One window's attention reads K and the position rows where the projections wrote them, and Vᵀ
    from the qkv projection's epilogue (no packing launch); at full size (256 channels) the
    subsampling's last conv writes its image flattened (no flatten launch), and the conv module's first
    pointwise conv applies the GLU in its epilogue.  The values are the same as after the separate
    launches, so the encoder output equals that path's (wh_tune epilogue_fusion 0) bit for bit.
    Each setting runs eagerly, then recorded, then replayed (a tuning change is not replayed from a
    recording made before it)."""
    m = wa.Model(gpu, synth.model_path("parakeet", small=small, directory=MODELS))
    mel = synth.parakeet_mel(synth.audio(seconds, seed=9))
    direct = m.encode(mel)
    outs = {}
    gpu.tune("epilogue_fusion", 0)
    try:
        outs["separate launches"] = [m.encode(mel) for _ in range(3)]
    finally:
        gpu.tune("epilogue_fusion", 1)
    outs["default"] = [m.encode(mel) for _ in range(3)]
    for key, runs in outs.items():
        for got in runs:
            assert got.shape == direct.shape
            assert np.array_equal(direct, got), (key, float(np.abs(direct - got).max()))


def test_parakeet_kestrel_valid(gpu):
    # The kestrel length masking: the last mel frame is padding (src/parakeet/mod.rs:140-141).
    path = synth.model_path("parakeet", small=True, directory=MODELS)
    mel = synth.parakeet_mel(synth.audio(7.3, 5))
    valid = mel.shape[0] - 1
    want = ox.Model(path).encode(mel, valid)
    got = wa.Model(gpu, path).encode(mel, valid)
    assert rel_l2(got, want) < ENCODER_TOL


def test_conformer_blocks_match_layer_by_layer(gpu):
    path = synth.model_path("parakeet", small=True, directory=MODELS)
    om, m = ox.Model(path), wa.Model(gpu, path)
    t = 57
    x = np.random.default_rng(3).normal(0, 1, (t, om.d)).astype(np.float32)
    for layers in (1, 2):
        want = om.blocks(x, layers)
        xb = gpu.upload(x)
        m.blocks_device(xb, t, layers)
        got = gpu.read(xb, x.shape)
        assert rel_l2(got, want) < ENCODER_TOL, (layers, rel_l2(got, want))


def test_whisper_small(gpu):
    path = synth.model_path("whisper", small=True, directory=MODELS)
    cfg = synth.SMALL["whisper"]
    mel = synth.whisper_mel(synth.audio(2.0, 4), cfg["mels"], 2 * cfg["frames"])
    om, m = ox.Model(path), wa.Model(gpu, path)
    want = om.encode(mel)
    got = m.encode(mel)
    assert rel_l2(got, want) < ENCODER_TOL, rel_l2(got, want)
    # Decoder steps from the oracle's encoder output on both sides: logits and the greedy token.
    vocab = cfg["vocab"]
    vp = vocab if vocab % 32 == 0 else (vocab + 63) // 64 * 64
    eb, lb = gpu.upload(want), gpu.buffer(vp)
    om.whisper_begin(want)
    m.whisper_begin(eb, want.shape[0])
    token = 890 % vocab
    for pos in range(12):
        wl = om.whisper_step(token, pos, vocab)
        m.whisper_step(token, pos, lb)
        gl = gpu.read(lb, (vp,))[:vocab]
        assert rel_l2(gl, wl) < ENCODER_TOL, (pos, rel_l2(gl, wl))
        nxt, gnxt = int(np.argmax(wl)), int(np.argmax(gl))
        assert nxt == gnxt, f"step {pos}: {gnxt} vs {nxt} (top-2 gap {top2_gap(wl):.3g})"
        token = nxt


def test_whisper_long_decode(gpu):
    """300 recorded decoder steps (the step replays one graph, its position read on the device) past
    the first 256-key part of the self-attention cache, each step's logits against the oracle's."""
    path = synth.model_path("whisper_ctx", small=True, directory=MODELS)
    cfg = synth.SMALL["whisper_ctx"]
    om, m = ox.Model(path), wa.Model(gpu, path)
    enc = np.random.default_rng(21).normal(0, 1, (cfg["frames"], cfg["d"])).astype(np.float32)
    vocab = cfg["vocab"]
    vp = vocab if vocab % 32 == 0 else (vocab + 63) // 64 * 64
    eb, lb = gpu.upload(enc), gpu.buffer(vp)
    om.whisper_begin(enc)
    m.whisper_begin(eb, enc.shape[0])
    tokens = np.random.default_rng(22).integers(0, vocab, 300)
    worst = 0.0
    for pos, token in enumerate(tokens):
        wl = om.whisper_step(int(token), pos, vocab)
        m.whisper_step(int(token), pos, lb)
        gl = gpu.read(lb, (vp,))[:vocab]
        worst = max(worst, rel_l2(gl, wl))
        assert rel_l2(gl, wl) < ENCODER_TOL, (pos, rel_l2(gl, wl))
        if int(np.argmax(gl)) != int(np.argmax(wl)):  # only a near tie, within the measured noise
            noise = 4.0 * float(np.abs(gl - wl).max())
            assert top2_gap(wl) < noise, f"step {pos}: argmax {np.argmax(gl)} vs {np.argmax(wl)}"
    print(f"worst step rel L2 {worst:.2e}")


def test_gigaam_full_config(gpu):
    """the GigaAM-v3 shape (16 layers, d 768, 16 heads of 48), 11 s, q8_0."""
    path = synth.model_path("gigaam", directory=MODELS)
    mel = synth.gigaam_mel(synth.audio(11, 1))
    want = ox.Model(path).encode(mel)
    m = wa.Model(gpu, path)
    full = m.encode(mel)
    got = full[:, :want.shape[1]]
    assert want.shape[0] == 275
    err = rel_l2(got, want)
    assert err < ENCODER_TOL, err
    check_ctc(m, full, want)


def test_parakeet_full_config(gpu):
    """the Parakeet-TDT-0.6B-v3 shape (24 layers, d 1024, FFN 4096), 60 s, q8_0 —
    the FFN's k-split residual projections finish inside the following LayerNorm's kernel."""
    path = synth.model_path("parakeet", directory=MODELS)
    mel = synth.parakeet_mel(synth.audio(60, 0))
    om = ox.Model(path)
    want = om.encode(mel)
    m = wa.Model(gpu, path)
    got = m.encode(mel)[:, :want.shape[1]]
    assert want.shape[0] == 750
    err = rel_l2(got, want)
    assert err < ENCODER_TOL, err
    flip = check_tdt(m, om, got, want)
    print(f"parakeet 60 s: rel L2 {err:.2e}, TDT {'identical' if flip is None else f'near-tie flip {flip}'}")


def whisper_decode_parity(om, m, gpu, enc, vocab):
    """Whisper's window search (src/whisper/search.rs:35-71) from the same encoder output on both sides:
    the device decode (wh_whisper_decode: steps on the device, rules on the host) against the oracle's.
    The ids must match; a divergence passes only as a near tie, where the oracle's top-2 margin after
    the rules is below the logit noise measured on the steps before it."""
    eb = gpu.upload(enc)
    got, ns, lp = m.whisper_decode(eb, enc.shape[0])
    ids = om.whisper_ids()
    om.whisper_begin(enc)
    sot = om.whisper_step(ids.sot, 0, vocab)
    want, _, gaps = om.whisper_decode(sot.copy(), 1, False)
    assert ns == pytest.approx(ox.probability(sot, ids.no_timestamps - 1), rel=1e-2, abs=1e-6)
    if got == want:
        return len(want), None
    k = next((i for i in range(min(len(got), len(want))) if got[i] != want[i]), min(len(got), len(want)))
    # Logit noise: the device's logits against the oracle's on the agreed prefix.
    vp = vocab if vocab % 32 == 0 else (vocab + 63) // 64 * 64
    lb = gpu.buffer(vp)
    m.whisper_begin(eb, enc.shape[0])
    om.whisper_begin(enc)
    noise = 0.0
    for pos, tok in enumerate([ids.sot] + want[:k]):
        m.whisper_step(tok, pos, lb)
        gl = gpu.read(lb, (vp,))[:vocab]
        wl = om.whisper_step(tok, pos, vocab)
        noise = max(noise, float(np.abs(gl - wl).max()))
    assert gaps[k] <= 4.0 * noise, f"pick {k}: {got[k:k + 3]} vs {want[k:k + 3]}, margin {gaps[k]:.3g} > 4·noise {noise:.3g}"
    return k, (k, float(gaps[k]), noise)


@pytest.mark.parametrize("wtype", [gguf.Q8_0, gguf.F16])
def test_whisper_full_config(gpu, wtype):
    """the Whisper-large-v3-turbo shape (30 s window → 1500 frames, 32 layers,
    d 1280, 20 heads, FFN 5120; decoder 4 layers, 51866-token head), once in q8_0 and once in f16.
    The encoder against the oracle; 224 forced decoder steps (the oracle's greedy tokens fed to both)
    logit by logit; then the window search under the real rules from the same encoder output."""
    path = synth.model_path("whisper", wtype=wtype, directory=MODELS)
    cfg = synth.CONFIGS["whisper"]
    mel = synth.whisper_mel(synth.audio(30.0, 4), cfg["mels"], 2 * cfg["frames"])
    om, m = ox.Model(path), wa.Model(gpu, path)
    want = om.encode(mel)
    got = m.encode(mel)
    assert want.shape == (1500, 1280)
    err = rel_l2(got, want)
    assert err < ENCODER_TOL, err
    vocab = cfg["vocab"]
    vp = vocab if vocab % 32 == 0 else (vocab + 63) // 64 * 64
    eb, lb = gpu.upload(want), gpu.buffer(vp)
    om.whisper_begin(want)
    m.whisper_begin(eb, want.shape[0])
    token, worst, flips = om.whisper_ids().sot, 0.0, 0
    for pos in range(224):
        wl = om.whisper_step(token, pos, vocab)
        m.whisper_step(token, pos, lb)
        gl = gpu.read(lb, (vp,))[:vocab]
        worst = max(worst, rel_l2(gl, wl))
        assert rel_l2(gl, wl) < ENCODER_TOL, (pos, rel_l2(gl, wl))
        if int(np.argmax(gl)) != int(np.argmax(wl)):
            flips += 1
            assert top2_gap(wl) < 4.0 * float(np.abs(gl - wl).max()), f"step {pos}: argmax flip off a near tie"
        token = int(np.argmax(wl))
    n, flip = whisper_decode_parity(om, m, gpu, want, vocab)
    print(f"whisper type {wtype}: encoder rel L2 {err:.2e}; 224 steps worst logits rel L2 {worst:.2e}, "
          f"{flips} near-tie argmax flips; search: {n} ids agree{'' if flip is None else f', then near tie {flip}'}")


def test_whisper_search_small(gpu):
    """The window search on the small Whisper shape: the device decode's ids equal the oracle's."""
    path = synth.model_path("whisper", small=True, directory=MODELS)
    cfg = synth.SMALL["whisper"]
    mel = synth.whisper_mel(synth.audio(2.0, 4), cfg["mels"], 2 * cfg["frames"])
    om, m = ox.Model(path), wa.Model(gpu, path)
    enc = om.encode(mel)
    n, flip = whisper_decode_parity(om, m, gpu, enc, cfg["vocab"])
    assert n > 0


def test_parakeet_batch16(gpu):
    """long-form audio cut at its pauses into ≤ 60 s segments (src/split.rs:42-65),
    16 of them through the config[1] encoder in one padded batch (wh_model_encode_batch: per-window
    subsampling, key masks and conv-input masks).  Every window's valid frames against the oracle's
    encoder on that segment alone (relative L2), and its TDT tokens."""
    path = synth.model_path("parakeet", directory=MODELS)
    pcm, gaps = synth.long_audio(16 * 55.0, seed=11)
    segs = synth.split_at_gaps(len(pcm) / synth.SR, gaps)[:16]
    assert len(segs) == 16
    mels = [synth.parakeet_mel(pcm[int(a * synth.SR):int(b * synth.SR)]) for a, b in segs]
    mf = max(x.shape[0] for x in mels)
    om, m = ox.Model(path), wa.Model(gpu, path)
    frames, width = m.frames(mf)
    batch = np.zeros((16, mf, mels[0].shape[1]), np.float32)
    for i, x in enumerate(mels):
        batch[i, :x.shape[0]] = x
    mb, ob = gpu.upload(batch), gpu.buffer(16 * frames * width)
    m.encode_batch_device(mb, 16, mf, [x.shape[0] for x in mels], ob)
    out = gpu.read(ob, (16, frames, width))
    worst, flips = 0.0, []
    for i, x in enumerate(mels):
        want = om.encode(x)
        got = out[i, :want.shape[0], :want.shape[1]]
        err = rel_l2(got, want)
        worst = max(worst, err)
        assert err < ENCODER_TOL, (i, err)
        flip = check_tdt(m, om, got, want)
        if flip is not None:
            flips.append((i, flip))
    print(f"16 windows of {[round(b - a, 1) for a, b in segs]} s: worst rel L2 {worst:.2e}, TDT near-tie flips {flips}")


def test_parakeet_batch_ragged(gpu):
    """A batch of 3 windows of different lengths (the remainder batch of configs[3]'s long input, which
    the reference runs piece by piece, src/lib.rs:844-886): each window's valid frames against the
    oracle's encoder on that window alone, and its TDT tokens; then the same three windows in the other
    order, which must give each window the same output bit for bit."""
    path = synth.model_path("parakeet", directory=MODELS)
    clips = [synth.audio(47.3, seed=21), synth.audio(12.3, seed=22), synth.audio(31.1, seed=23)]
    mels = [synth.parakeet_mel(c) for c in clips]
    mf = max(x.shape[0] for x in mels)
    om, m = ox.Model(path), wa.Model(gpu, path)
    frames, width = m.frames(mf)

    def run(order):
        batch = np.zeros((len(order), mf, mels[0].shape[1]), np.float32)
        for j, i in enumerate(order):
            batch[j, :mels[i].shape[0]] = mels[i]
        mb, ob = gpu.upload(batch), gpu.buffer(len(order) * frames * width)
        m.encode_batch_device(mb, len(order), mf, [mels[i].shape[0] for i in order], ob)
        out = gpu.read(ob, (len(order), frames, width))
        return {i: out[j] for j, i in enumerate(order)}

    got = run([0, 1, 2])
    flips = []
    for i, x in enumerate(mels):
        want = om.encode(x)
        g = got[i][:want.shape[0], :want.shape[1]]
        err = rel_l2(g, want)
        assert err < ENCODER_TOL, (i, err)
        flip = check_tdt(m, om, g, want)
        if flip is not None:
            flips.append((i, flip))
    back = run([2, 1, 0])
    for i, x in enumerate(mels):
        rows = m.frames(x.shape[0])[0]  # the window's own encoder frames
        assert np.array_equal(back[i][:rows], got[i][:rows]), f"window {i} differs with its position in the batch"
    print(f"3 windows of {[round(len(c) / synth.SR, 1) for c in clips]} s: TDT near-tie flips {flips}")


@pytest.mark.parametrize("name", ["parakeet", "gigaam", "whisper"])
def test_graph_replays_equal_eager_calls(gpu, name):
    # The second call with the same buffers is recorded into a HIP graph and later ones replay it.
    # Every replay, with the program's own eager work and synchronizations between them, must give
    # the eager call's bytes exactly (the same kernels in the same order).
    path = synth.model_path(name, small=True, directory=MODELS)
    m = wa.Model(gpu, path)
    mel = {"parakeet": synth.parakeet_mel, "gigaam": synth.gigaam_mel}.get(name, None)
    if mel is None:
        mel = synth.whisper_mel(synth.audio(2, 3), mels=80, frames=200)
    else:
        mel = mel(synth.audio(3, 3))
    frames, width = m.frames(mel.shape[0])
    melb, outb = gpu.upload(mel), gpu.buffer(frames * width)
    m.graphs(False)
    m.encode_device(melb, mel.shape[0], outb)
    eager = gpu.read(outb, (frames, width)).copy()
    m.graphs(True)
    other = gpu.buffer(frames * width)
    for call in range(4):  # eager, recorded, replay, replay
        gpu.zero(outb)
        m.encode_device(melb, mel.shape[0], outb)
        got = gpu.read(outb, (frames, width))
        assert np.array_equal(got, eager), f"call {call} differs from the eager result"
        # Eager work of the program's own between the replays.
        gpu.zero(other)
        gpu.sync()


@pytest.mark.parametrize("graphs", [False, True])
def test_position_projection_kept_per_frame_count(gpu, graphs):
    """The Parakeet position projection depends only on the frame count t and the weights, so a call
    at the t whose projection its buffers hold skips that GEMM (a tag on the device, checked by the
    kernel: a recorded pass stays right whatever t a later call leaves there).  Calls alternating
    between two frame counts, one window (packed positions) and a batch of two (plain), eagerly or
    recorded and replayed, with a call over fewer blocks in between: every output is the same bytes
    as from a context that recomputes the projection every call."""
    path = synth.model_path("parakeet", small=True, directory=MODELS)
    mels = [synth.parakeet_mel(synth.audio(s, 5)) for s in (3.0, 2.2)]
    ref_ctx = wa.Gpu(0)
    try:
        ref_ctx.tune("position_cache", 0)
        ref = wa.Model(ref_ctx, path)
        want = [ref.encode(x) for x in mels]
        d = ref.frames(mels[0].shape[0])[1]  # the model width
        x0 = np.random.default_rng(2).normal(0, 1, (30, d)).astype(np.float32)
        xw = ref_ctx.upload(x0)
        ref.blocks_device(xw, 30, 1)
        want_blocks = ref_ctx.read(xw, (30, d)).copy()
        mf = max(x.shape[0] for x in mels)
        batch = np.zeros((2, mf, mels[0].shape[1]), np.float32)
        for i, x in enumerate(mels):
            batch[i, :x.shape[0]] = x
        fb, wb = ref.frames(mf)
        bb, ob = ref_ctx.upload(batch), ref_ctx.buffer(2 * fb * wb)
        ref.encode_batch_device(bb, 2, mf, [x.shape[0] for x in mels], ob)
        want_batch = ref_ctx.read(ob, (2, fb, wb)).copy()
        ref.free()
    finally:
        ref_ctx.close()
    m = wa.Model(gpu, path)
    m.graphs(graphs)
    bufs = []
    for x in mels:
        f, w = m.frames(x.shape[0])
        bufs.append((gpu.upload(x), gpu.buffer(f * w), f, w))
    bb, ob = gpu.upload(batch), gpu.buffer(2 * fb * wb)
    for rnd in range(3):  # eager, recorded, replayed (with graphs)
        for i in (0, 1, 0):
            xb, outb, f, w = bufs[i]
            gpu.zero(outb)
            m.encode_device(xb, mels[i].shape[0], outb)
            assert np.array_equal(gpu.read(outb, (f, w)), want[i]), f"round {rnd} window {i}"
        gpu.zero(ob)
        m.encode_batch_device(bb, 2, mf, [x.shape[0] for x in mels], ob)
        assert np.array_equal(gpu.read(ob, (2, fb, wb)), want_batch), f"round {rnd} batch"
    xw = gpu.upload(x0)
    m.blocks_device(xw, 30, 1)  # packs one block's positions: the tag is cleared
    assert np.array_equal(gpu.read(xw, (30, d)), want_blocks)
    xb, outb, f, w = bufs[0]
    m.encode_device(xb, mels[0].shape[0], outb)
    assert np.array_equal(gpu.read(outb, (f, w)), want[0]), "after a call over fewer blocks"
    m.free()
