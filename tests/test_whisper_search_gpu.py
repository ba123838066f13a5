"""Whisper's window search on the device (wh_whisper_decode: a pick kernel per step, recorded runs of
(step, pick) pairs) against the same loop with every pick on the host (wh_tune "whisper_host":
wh_whisper_pick, src/whisper/search.rs:46-127, whose rules the CPU tests pin against the oracle).

Both sides run the same device steps, so they see identical logits and must pick identical ids; the
average log-probability (forced on with wh_tune "whisper_logprobs", since a random model's no-speech
probability stays below 0.6) differs only in the order of the f64 sums over the vocabulary: within
1e-5 relative.  Cases: the small shape (2 timestamp ids: the pair rules at every step), the context
limit (a 60-id prompt in a 64-position decoder), a cap below the count, windows that end on EOT
(EOT's head row scaled: after one timestamp, after seven ids; also against the oracle's search), and
the full large-v3-turbo shape (1501 timestamp ids, 51866-id vocabulary) on three clips, with and
without a prompt."""

import hashlib
import os

import pytest

import oracle as ox
import wavo_amd as wa
from wavo_amd import gguf, synth

pytestmark = pytest.mark.gpu

MODELS = os.environ.get("WAVO_MODELS", "/tmp/wavo_models")
LP_REL = 1e-5


def both(gpu, m, eb, frames, prompt=(), cap=512):
    """(device search, host-pick search) results, log-probabilities forced on."""
    gpu.tune("whisper_logprobs", 1)
    try:
        dev = m.whisper_decode(eb, frames, prompt, cap)
        gpu.tune("whisper_host", 1)
        try:
            host = m.whisper_decode(eb, frames, prompt, cap)
        finally:
            gpu.tune("whisper_host", 0)
    finally:
        gpu.tune("whisper_logprobs", 0)
    return dev, host


def check(dev, host, what):
    (gd, nd, ld), (gh, nh, lh) = dev, host
    print(f"{what}: {len(gd)} ids, no-speech {nd:.3g}, avg logprob {ld:.6g} / {lh:.6g}")
    assert gd == gh, (what, gd[:20], gh[:20])
    assert nd == nh, what
    assert ld == pytest.approx(lh, rel=LP_REL, abs=1e-7), what


def encoded(gpu, m, name, seconds, seed, small=True):
    cfg = (synth.SMALL if small else synth.CONFIGS)[name]
    mel = synth.whisper_mel(synth.audio(seconds, seed), cfg["mels"], 2 * cfg["frames"])
    enc = m.encode(mel)
    return gpu.upload(enc), enc.shape[0]


@pytest.mark.parametrize("seed", [4, 9, 13])
def test_search_small(gpu, seed):
    m = wa.Model(gpu, synth.model_path("whisper", small=True, directory=MODELS))
    eb, frames = encoded(gpu, m, "whisper", 2.0, seed)
    check(*both(gpu, m, eb, frames), f"small seed {seed}")
    ids = m.whisper_ids()
    check(*both(gpu, m, eb, frames, [ids.sot, ids.sot + 101]), f"small seed {seed}, prompt [sot, transcribe]")
    # Without the log-probabilities the average is 0 on both sides.
    got, _, lp = m.whisper_decode(eb, frames)
    assert lp == 0.0 and got == both(gpu, m, eb, frames)[0][0]


def test_search_context_limit_and_cap(gpu):
    m = wa.Model(gpu, synth.model_path("whisper", small=True, directory=MODELS))
    eb, frames = encoded(gpu, m, "whisper", 2.0, 4)
    ids = m.whisper_ids()
    prompt = [ids.sot] + [(7 * i) % ids.eot for i in range(1, 60)]
    dev, host = both(gpu, m, eb, frames, prompt)
    check(dev, host, "60-id prompt, context 64")
    assert len(dev[0]) <= 64 - 60 + 1
    full = dev[0]
    if len(full) > 1:
        part = m.whisper_decode(eb, frames, prompt, cap=1)[0]
        assert part == full[:1]


def test_search_long_context(gpu):
    """A 320-position decoder: runs well past one recorded run of pairs, up to the 256-id budget."""
    m = wa.Model(gpu, synth.model_path("whisper_ctx", small=True, directory=MODELS))
    eb, frames = encoded(gpu, m, "whisper_ctx", 2.0, 5)
    dev, host = both(gpu, m, eb, frames)
    check(dev, host, "context 320")


@pytest.mark.parametrize("eot_scale", [16.0, -8.0])
def test_search_ends_on_eot(gpu, eot_scale):
    cfg = dict(synth.SMALL["whisper"], eot_scale=eot_scale)
    tag = hashlib.md5(repr(sorted(cfg.items())).encode()).hexdigest()[:10]
    path = os.path.join(MODELS, f"whisper-{tag}.gguf")
    os.makedirs(MODELS, exist_ok=True)
    if not os.path.exists(path):
        synth.write_model(path, cfg, 0)
    om, m = ox.Model(path), wa.Model(gpu, path)
    mel = synth.whisper_mel(synth.audio(2.0, 4), cfg["mels"], 2 * cfg["frames"])
    enc = om.encode(mel)
    dev, host = both(gpu, m, gpu.upload(enc), enc.shape[0])
    check(dev, host, f"EOT row × {eot_scale}")
    assert len(dev[0]) < cfg["context"] - 1
    ids = om.whisper_ids()
    om.whisper_begin(enc)
    want = om.whisper_decode(om.whisper_step(ids.sot, 0, cfg["vocab"]).copy(), 1, False)[0]
    assert dev[0] == want


@pytest.mark.parametrize("seed", [4, 21, 33])
def test_search_full_config(gpu, seed):
    m = wa.Model(gpu, synth.model_path("whisper", wtype=gguf.Q8_0, directory=MODELS))
    eb, frames = encoded(gpu, m, "whisper", 30.0, seed, small=False)
    check(*both(gpu, m, eb, frames), f"large-v3-turbo shape, seed {seed}")
    if seed == 4:
        ids = m.whisper_ids()
        check(*both(gpu, m, eb, frames, [ids.sot, ids.sot + 1, ids.sot + 101]), "large-v3-turbo shape, prompt")
