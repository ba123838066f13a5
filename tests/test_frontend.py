"""Pins of the oracle's log-mel frontends (oracle/frontend.c: src/fft.rs and the three family
frontends) on the CPU.

- The reference's own tests: the FFT against a DFT at 320, 360, 400, 512 and 15 points (f32 within
  1e-4, f64 within 1e-10, src/fft.rs:151-175); Parakeet's short inputs and frame ranges
  (src/parakeet/frontend.rs:143-161).
- Float64 restatements written here with numpy's FFT: the Parakeet filterbank (librosa's Slaney
  formula), the three frontends end to end (window, padding, pre-emphasis, power, filterbank, log,
  normalization or Whisper's clamp and scale).  Each also runs with a plausible mistake planted (a
  symmetric window where the reference has a periodic one, no pre-emphasis, the biased variance, a
  window not centred, constant instead of reflect padding, no max − 8 clamp) and requires that
  version to miss the oracle by far more than the tolerance.
"""

import numpy as np
import pytest

import oracle as ox
from wavo_amd import synth

SR = 16000


def dft(x):
    n = len(x)
    k = np.arange(n)[:, None]
    ph = 2 * np.pi * ((k * np.arange(n)[None, :]) % n) / n
    x = np.asarray(x, np.float64)
    return (x[None, :] * np.cos(ph)).sum(1), -(x[None, :] * np.sin(ph)).sum(1)


@pytest.mark.parametrize("n", [320, 360, 400, 512, 15])
def test_fft_matches_dft(n):
    x = np.array([((i * 7919 % 1000) / 500.0 - 1.0) * 0.3 for i in range(n)])
    for f64, tol in ((True, 1e-10), (False, 1e-4)):
        inp = x.astype(np.float64 if f64 else np.float32)
        re, im = ox.fft(inp, f64)
        wr, wi = dft(inp)
        assert np.abs(re - wr).max() < tol and np.abs(im - wi).max() < tol


def test_fft_a_mistake_is_seen():
    """The DFT check sees a transposed output order (bit-reversed bins) and a conjugated spectrum."""
    x = np.random.default_rng(0).standard_normal(512)
    re, im = ox.fft(x, True)
    wr, wi = dft(x)
    assert np.abs(im + wi).max() > 1.0  # a conjugate would fail
    assert np.abs(re[::-1] - wr).max() > 1.0


def test_parakeet_short_input():
    assert ox.parakeet_mel(np.full(319, 0.1, np.float32)).shape == (0, 128)
    m = ox.parakeet_mel(np.full(320, 0.1, np.float32))
    assert m.shape == (3, 128) and np.isfinite(m).all()


def test_parakeet_frame_ranges():
    pcm = (np.sin(np.arange(16000, dtype=np.float32) * np.float32(0.01)) * np.float32(0.5)).astype(np.float32)
    full = ox.parakeet_log_mel(pcm, 0, 101)
    for a, b in [(0, 1), (0, 7), (3, 40), (95, 101), (100, 101)]:
        assert np.array_equal(ox.parakeet_log_mel(pcm, a, b), full[a:b])


def slaney(n_fft, mels, fmax=8000.0):
    """librosa.filters.mel(norm='slaney', htk=False) in float64."""
    def hz_to_mel(f):
        f = np.asarray(f, np.float64)
        return np.where(f >= 1000.0, 15.0 + np.log(np.maximum(f, 1e-10) / 1000.0) / (np.log(6.4) / 27.0), f * 3.0 / 200.0)

    def mel_to_hz(m):
        m = np.asarray(m, np.float64)
        return np.where(m >= 15.0, 1000.0 * np.exp((np.log(6.4) / 27.0) * (m - 15.0)), m * 200.0 / 3.0)

    freqs = np.arange(n_fft // 2 + 1) * SR / n_fft
    pts = mel_to_hz(np.linspace(0.0, hz_to_mel(fmax), mels + 2))
    lo, c, hi = pts[:-2, None], pts[1:-1, None], pts[2:, None]
    fb = np.maximum(0.0, np.minimum((freqs - lo) / (c - lo), (hi - freqs) / (hi - c)))
    return fb * (2.0 / (hi - lo))


def test_parakeet_filterbank_is_slaney():
    got = ox.parakeet_filterbank().astype(np.float64)
    want = slaney(512, 128)
    assert np.abs(got - want).max() <= 1e-6 * np.abs(want).max()
    assert np.abs(got - slaney(512, 128, fmax=7600.0)).max() > 1e-3 * np.abs(want).max()


def parakeet_f64(pcm, periodic=False, pre=0.97, biased=False, centred=True):
    """Float64 restatement of src/parakeet/frontend.rs:52-108: (log-mel, normalized)."""
    pcm = np.asarray(pcm, np.float64)
    x = np.concatenate([pcm[:1], pcm[1:] - np.float64(np.float32(pre)) * pcm[:-1]])
    frames = len(pcm) // 160 + 1
    padded = np.concatenate([np.zeros(256), x, np.zeros(512 + 256)])
    win = np.zeros(512)
    k = np.arange(400)
    hann = 0.5 - 0.5 * np.cos(2 * np.pi * k / (400 if periodic else 399))
    win[(56 if centred else 0):(56 if centred else 0) + 400] = hann
    idx = np.arange(frames)[:, None] * 160 + np.arange(512)[None, :]
    spec = np.fft.rfft(padded[idx] * win, n=512)
    power = (spec.real ** 2 + spec.imag ** 2).astype(np.float32).astype(np.float64)
    fb = ox.parakeet_filterbank().astype(np.float64)
    logm = np.log(power @ fb.T + 2.0 ** -24)
    n = frames - 1
    mean = logm[:n].mean(0)
    var = ((logm[:n] - mean) ** 2).sum(0) / (n if biased else n - 1)
    out = (logm - mean) / (np.sqrt(var) + np.float64(np.float32(1e-5)))
    out[n] = 0.0
    return logm, out


def test_parakeet_mel_float64():
    pcm = synth.audio(10.0, seed=3)
    got_log = ox.parakeet_log_mel(pcm, 0, len(pcm) // 160 + 1).astype(np.float64)
    got = ox.parakeet_mel(pcm).astype(np.float64)
    want_log, want = parakeet_f64(pcm)
    assert np.abs(got_log - want_log).max() < 1e-5
    assert np.abs(got - want).max() < 1e-5
    for bad in (dict(periodic=True), dict(pre=0.0), dict(centred=False)):
        assert np.abs(got_log - parakeet_f64(pcm, **bad)[0]).max() > 1e-2, bad
    assert np.abs(got - parakeet_f64(pcm, biased=True)[1]).max() > 2e-4


def test_gigaam_mel_float64():
    pcm = synth.audio(11.0, seed=1)
    window, filters = synth.hann_periodic(320), synth.htk_filters(SR, 320, 64)
    got = ox.gigaam_mel(pcm, window, filters).astype(np.float64)

    def f64(win):
        frames = (len(pcm) - 320) // 160 + 1
        idx = np.arange(frames)[:, None] * 160 + np.arange(320)[None, :]
        spec = np.fft.rfft(pcm.astype(np.float64)[idx] * win, n=320)
        return np.log(np.clip((spec.real ** 2 + spec.imag ** 2) @ filters.astype(np.float64).T, 1e-9, 1e9))

    want = f64(window.astype(np.float64))
    assert got.shape == want.shape == ((len(pcm) - 320) // 160 + 1, 64)
    assert np.abs(got - want).max() < 5e-4
    symmetric = 0.5 - 0.5 * np.cos(2 * np.pi * np.arange(320) / 319)
    assert np.abs(got - f64(symmetric)).max() > 1e-2
    assert ox.gigaam_mel(pcm[:319], window, filters).shape == (0, 64)


def whisper_f64(pcm, window, filters, reflect=True, clamp=True):
    n = max(len(pcm), 480000)
    x = np.zeros(n)
    x[:len(pcm)] = pcm
    padded = np.pad(x, 200, mode="reflect" if reflect else "constant")
    frames = n // 160
    idx = np.arange(frames)[:, None] * 160 + np.arange(400)[None, :]
    spec = np.fft.rfft(padded[idx] * window.astype(np.float64), n=400)
    m = np.log10(np.maximum((spec.real ** 2 + spec.imag ** 2) @ filters.astype(np.float64).T, 1e-10))
    if clamp:
        m = np.maximum(m, m.max() - 8.0)
    return (m + 4.0) / 4.0


def test_whisper_mel_float64():
    pcm = synth.audio(12.0, seed=2)
    window, filters = synth.hann_periodic(400), synth._mel_filters(SR, 400, 80).astype(np.float32)
    got = ox.whisper_mel(pcm, window, filters).astype(np.float64)
    want = whisper_f64(pcm, window, filters)
    assert got.shape == (3000, 80)
    assert np.abs(got - want).max() < 2e-5
    # Frames past the audio are digital silence: every value the clamp's floor.
    assert np.all(got[-100:] == got[-100:].min())
    assert np.abs(got - whisper_f64(pcm, window, filters, reflect=False)).max() > 1e-2
    assert np.abs(got - whisper_f64(pcm, window, filters, clamp=False)).max() > 1e-2
