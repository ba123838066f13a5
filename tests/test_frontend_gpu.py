"""The log-mel frontends on the device (wh_model_mel) against the oracle's (oracle/frontend.c) on the
same seeded audio (BASELINE's synthetic clips: Gaussian noise plus chirps).

The transforms, power spectra and filter sums use the reference's operations in its order and the
same tables, so they agree bit for bit: checked by both sides writing each filter's sum before the
logarithm (wh_tune "mel_raw", ox.mel_raw) and requiring identical arrays.  What may differ after it
is the logarithm (the device's logf / log10 against the C library's, within an ulp) and, for
Parakeet, the order of the f64 sums of the per-bin normalization, which an ulp of the logarithms
moves for every value of the bin.  Bar: max |Δ| ≤ 1e-5 on features of order 1–20 (the share of
bit-identical values is reported).  Then the Parakeet path end to end: device mel → encoder →
device TDT against the oracle's mel → encoder → TDT."""

import os

import numpy as np
import pytest

import oracle as ox
import wavo_amd as wa
from parity import tdt_device_parity, tdt_parity
from wavo_amd import synth

pytestmark = pytest.mark.gpu

MODELS = os.environ.get("WAVO_MODELS", "/tmp/wavo_models")
TOL = 1e-5


def compare(gpu, m, pcm, oracle_fn, what):
    """The features within TOL of the oracle's, and the filter sums before the logarithm bit-identical."""
    got, want = m.mel(pcm), oracle_fn(pcm)
    assert got.shape == want.shape, (what, got.shape, want.shape)
    if got.size == 0:
        return
    d = np.abs(got.astype(np.float64) - want.astype(np.float64))
    same = float(np.mean(got == want))
    gpu.tune("mel_raw", 1)
    ox.mel_raw(True)
    try:
        raw, raw_want = m.mel(pcm), oracle_fn(pcm)
    finally:
        gpu.tune("mel_raw", 0)
        ox.mel_raw(False)
    print(f"{what}: {got.shape}, max |Δ| {d.max():.2e}, bit-identical {same:.4f}; filter sums identical "
          f"{np.array_equal(raw, raw_want)}")
    assert d.max() <= TOL, (what, d.max())
    assert np.array_equal(raw, raw_want), (what, float(np.abs(raw - raw_want).max()))


@pytest.mark.parametrize("seconds", [0.0199, 0.02, 1.0, 60.0])
def test_parakeet_mel(gpu, seconds):
    m = wa.Model(gpu, synth.model_path("parakeet", small=True, directory=MODELS))
    pcm = synth.audio(seconds, seed=4) if seconds >= 1.0 else np.full(int(seconds * 16000), 0.1, np.float32)
    compare(gpu, m, pcm, ox.parakeet_mel, f"parakeet {seconds} s")


@pytest.mark.parametrize("seconds", [0.0199, 0.02, 11.0])
def test_gigaam_mel(gpu, seconds):
    m = wa.Model(gpu, synth.model_path("gigaam", small=True, directory=MODELS))
    pcm = synth.audio(seconds, seed=5) if seconds >= 1.0 else np.full(int(seconds * 16000), 0.1, np.float32)
    tables = synth.hann_periodic(320), synth.htk_filters(16000, 320, m.mels)
    compare(gpu, m, pcm, lambda x: ox.gigaam_mel(x, *tables), f"gigaam {seconds} s")


@pytest.mark.parametrize("seconds", [0.0, 12.0, 31.5])
def test_whisper_mel(gpu, seconds):
    m = wa.Model(gpu, synth.model_path("whisper", small=True, directory=MODELS))
    pcm = synth.audio(seconds, seed=6) if seconds > 0 else np.zeros(0, np.float32)
    tables = synth.hann_periodic(400), synth._mel_filters(16000, 400, m.mels).astype(np.float32)
    compare(gpu, m, pcm, lambda x: ox.whisper_mel(x, *tables), f"whisper {seconds} s")


def test_parakeet_audio_to_tokens(gpu):
    """Audio on the device → mel → encoder → TDT, all on the device, against the oracle's chain."""
    path = synth.model_path("parakeet", small=True, directory=MODELS)
    om, m = ox.Model(path), wa.Model(gpu, path)
    pcm = synth.audio(8.0, seed=7)
    frames = m.mel_frames(len(pcm))
    pb, mb = gpu.upload(pcm), gpu.buffer(frames * m.mels)
    assert m.mel_device(pb, len(pcm), mb) == frames
    enc_frames, width = m.frames(frames)
    ob = gpu.buffer(enc_frames * width)
    m.encode_device(mb, frames, ob)
    tokens = m.greedy_device(ob, enc_frames, width)
    want_mel = ox.parakeet_mel(pcm)
    want = om.encode(want_mel)
    got = gpu.read(ob, (enc_frames, width))[:, :want.shape[1]]
    err = float(np.linalg.norm(got - want) / np.linalg.norm(want))
    assert err < 1e-2, err
    # The device decoder against the oracle's on the device's encoder output, then that output's
    # tokens against the oracle's chain (near ties only).
    dev = tdt_device_parity(om, tokens, np.ascontiguousarray(got))
    flip, tg, tw = tdt_parity(om, got, want)
    print(f"8 s: rel L2 {err:.2e}, {len(tokens)} tokens, device decoder {'identical' if dev is None else dev}, "
          f"encoder {'identical' if flip is None else f'near-tie flip {flip}'}")
