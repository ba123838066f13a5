"""Greedy decoding on the device (wh_model_greedy_device) against the oracle's decoders on the same
encoder output: CTC (src/gigaam/decoder.rs:135-151) bit-exact, TDT (src/parakeet/decoder.rs:91-191)
identical up to provable f32 near-ties (tests/parity.py: tdt_device_parity).

The TDT cases feed random encoder outputs straight to the decoder (the encoder has its own tests), on
small Parakeet decoders that exercise each rule of the loop: emissions and blanks, the per-frame
symbol limit, and the global symbol budget that ends the loop before the last frame.  A decode runs
in recorded runs of 32 decisions, so one call covers the eager run, the recording and its replays;
repeated calls and graphs switched off must give the same lists.
"""

import hashlib
import os

import numpy as np
import pytest

import oracle as ox
import wavo_amd as wa
from parity import tdt_device_parity
from wavo_amd import gguf, synth

pytestmark = pytest.mark.gpu

MODELS = os.environ.get("WAVO_MODELS", "/tmp/wavo_models")


def decoder_model(wtype=gguf.Q8_0, **over):
    """A small Parakeet (one encoder block) whose TDT decoder has the given settings."""
    cfg = dict(synth.SMALL["parakeet"], layers=1, **over)
    tag = hashlib.md5(repr(sorted(cfg.items())).encode()).hexdigest()[:10]
    path = os.path.join(MODELS, f"tdt-{tag}-t{wtype}.gguf")
    os.makedirs(MODELS, exist_ok=True)
    if not os.path.exists(path):
        synth.write_model(path, cfg, 0, wtype)
    return path


def random_enc(frames, width, seed, scale=1.0):
    return (np.random.default_rng(seed).standard_normal((frames, width)) * scale).astype(np.float32)


def decode(gpu, m, enc, cap=None):
    eb = gpu.upload(enc)
    return m.greedy_device(eb, enc.shape[0], enc.shape[1], cap)


def check(gpu, m, om, enc):
    got = decode(gpu, m, enc)
    flip = tdt_device_parity(om, got, enc)
    want, trace, _ = om.tdt_trace(enc)
    print(f"frames {enc.shape[0]}: {len(want)} tokens in {len(trace)} decisions, "
          f"{'identical' if flip is None else f'near-tie {flip}'}")
    return got, want, trace


@pytest.mark.parametrize("wtype", [gguf.Q8_0, gguf.F16, gguf.Q4_0])
def test_tdt_two_layers(gpu, wtype):
    """Two LSTM layers ([Wx | Wh] joined per layer), every weight type, three calls of different
    lengths on one model (eager, recorded and replayed runs of decisions)."""
    path = decoder_model(wtype)
    om, m = ox.Model(path), wa.Model(gpu, path)
    for frames, seed in ((400, 1), (97, 2), (400, 3)):
        got, want, trace = check(gpu, m, om, random_enc(frames, 320, seed))
        assert len(trace) > 64  # more than two recorded runs of decisions


def test_tdt_f32_wide(gpu):
    """F32 weights at the C1 decoder's widths (hidden 640, joint 640): a workgroup's weight rows no longer
    fit one 32 KiB staging round (the joint's 16 rows of 2560 bytes, each LSTM gate's 4 rows of 5120
    bytes), so the later rounds of the copy into LDS run, for both LSTM layers."""
    path = decoder_model(gguf.F32, hidden=640, joint=640)
    om, m = ox.Model(path), wa.Model(gpu, path)
    for frames, seed in ((300, 4), (120, 5)):
        check(gpu, m, om, random_enc(frames, 640, seed))


def test_tdt_blanks_and_symbol_limit(gpu):
    """A decoder that emits blanks about half the time (decisions whose predictor launches are switched
    off), with a per-frame limit of two symbols over durations {0, 1, 2}: emissions at duration 0, and
    frames left because the limit was reached."""
    path = decoder_model(blank_bias=1.0, max_symbols=2, durations=[0, 1, 2])
    om, m = ox.Model(path), wa.Model(gpu, path)
    blank = 1024
    for frames, seed in ((600, 4), (600, 5)):
        got, want, trace = check(gpu, m, om, random_enc(frames, 320, seed))
        tokens, durs = trace[:, 1], trace[:, 2]
        assert 0.2 < np.mean(tokens == blank) < 0.8, np.mean(tokens == blank)
        # Two zero-duration emissions in a row at one frame: the limit moves on to the next frame.
        limited = sum(1 for k in range(1, len(trace)) if trace[k][0] == trace[k - 1][0] and durs[k] == 0
                      and durs[k - 1] == 0 and tokens[k] != blank and tokens[k - 1] != blank)
        assert limited > 0


@pytest.mark.parametrize("blank_bias", [1.0, 1.3])
def test_tdt_global_budget(gpu, blank_bias):
    """The global symbol budget (stt.parakeet.tdt.symbol_budget = "global", one symbol per frame):
    max_symbols · frames decisions in all, and a blank advances at least one frame.  Blank bias 1.0:
    emissions at duration 0 spend the budget before the last frame.  1.3: mostly blanks, many of them
    at duration 0 (each moves on one frame), and the loop reaches the last frame."""
    path = decoder_model(symbol_budget="global", max_symbols=1, durations=[0, 1, 2], blank_bias=blank_bias)
    om, m = ox.Model(path), wa.Model(gpu, path)
    frames, blank = 300, 1024
    got, want, trace = check(gpu, m, om, random_enc(frames, 320, 6))
    if blank_bias == 1.0:
        assert len(trace) == frames and trace[-1][0] < frames - 1
    else:
        assert np.sum((trace[:, 1] == blank) & (trace[:, 2] == 0)) > 10 and trace[-1][0] == frames - 1


def test_tdt_graphs_off_and_cap(gpu):
    """Graphs off gives the same list as replayed runs; a cap below the count returns the count and
    the first cap pairs; zero frames decode to nothing."""
    path = decoder_model()
    om, m = ox.Model(path), wa.Model(gpu, path)
    enc = random_enc(250, 320, 7)
    on = decode(gpu, m, enc)
    assert decode(gpu, m, enc) == on
    m.graphs(False)
    assert decode(gpu, m, enc) == on
    m.graphs(True)
    eb = gpu.upload(enc)
    out = np.zeros(2 * 5, np.uint32)
    n = wa.lib().wh_model_greedy_device(m.h, eb.ptr, 250, 320, out.ctypes.data, 5)
    assert n == len(on) and [(int(out[2 * i]), int(out[2 * i + 1])) for i in range(5)] == on[:5]
    assert m.greedy_device(eb, 0, 320) == []


def test_tdt_wide_encoder_rows(gpu):
    """Encoder rows wider than the joint (padded columns past it are not read)."""
    path = decoder_model()
    om, m = ox.Model(path), wa.Model(gpu, path)
    enc = random_enc(200, 384, 8)
    enc[:, 320:] = 1e30
    got = decode(gpu, m, enc)
    tdt_device_parity(om, got, np.ascontiguousarray(enc[:, :320]))


def gigaam_small(gpu):
    path = synth.model_path("gigaam", small=True, directory=MODELS)
    return wa.Model(gpu, path)


@pytest.mark.parametrize("frames", [1, 2, 275, 4097, 70000])
def test_ctc_ties_and_sizes(gpu, frames):
    """Integer logits (many ties: the first maximum wins), blanks and repeats; one frame up to more
    frames than the collapse kernel's threads many times over; padded columns past the classes are
    ignored."""
    m = gigaam_small(gpu)
    classes, width, blank = 257, 320, 256
    rng = np.random.default_rng(frames)
    logits = rng.integers(0, 4, (frames, width)).astype(np.float32)
    logits[rng.random(frames) < 0.3, blank] = 9.0  # runs of blanks
    rep = rng.random(frames) < 0.3
    rep[0] = False
    logits[rep] = logits[np.nonzero(rep)[0] - 1]  # repeats of the previous frame
    logits[:, classes:] = 1e9
    want = ox.ctc(np.ascontiguousarray(logits[:, :classes]), blank)
    assert decode(gpu, m, logits) == want


def test_ctc_cap_and_empty(gpu):
    m = gigaam_small(gpu)
    logits = np.random.default_rng(9).standard_normal((500, 320)).astype(np.float32)
    want = ox.ctc(np.ascontiguousarray(logits[:, :257]), 256)
    eb = gpu.upload(logits)
    out = np.zeros(2 * 3, np.uint32)
    n = wa.lib().wh_model_greedy_device(m.h, eb.ptr, 500, 320, out.ctypes.data, 3)
    assert n == len(want) and [(int(out[2 * i]), int(out[2 * i + 1])) for i in range(3)] == want[:3]
    assert m.greedy_device(eb, 0, 320) == []
    logits[:] = 0.0
    logits[:, 256] = 1.0  # all blank
    assert decode(gpu, m, logits) == []
