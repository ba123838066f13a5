"""The token-parity checks themselves, with flips planted in CPU-side logits: a near-tie flip under
typical noise passes, a flip at a frame whose discrepancy is far above the typical noise fails."""

import numpy as np
import pytest

from parity import ctc_parity, top2_gap


def noisy(w, eps, seed):
    return w + np.random.default_rng(seed).uniform(-eps, eps, w.shape)


def test_identical_logits_have_no_flips():
    w = np.random.default_rng(0).normal(size=(50, 9))
    assert ctc_parity(w, w, 9) == []


def test_a_near_tie_flip_is_accepted():
    w = np.random.default_rng(1).normal(size=(40, 9))
    w[7, 3], w[7, 5] = 4.0, 4.0 - 1e-7
    g = noisy(w, 1e-6, 2)
    g[7, 3], g[7, 5] = 4.0, 4.0 + 1e-7  # the noise moves the second past the first
    flips = ctc_parity(g, w, 9)
    assert [f[0] for f in flips] == [7]


def test_a_flip_far_above_the_noise_fails():
    w = np.random.default_rng(3).normal(size=(40, 9))
    g = noisy(w, 1e-6, 4)
    i = int(np.argmax(w[11]))
    g[11, (i + 1) % 9] = w[11, i] + 0.3  # a planted wrong winner at one frame
    with pytest.raises(AssertionError, match="frame 11"):
        ctc_parity(g, w, 9)


def test_top2_gap():
    assert top2_gap([1.0, 3.0, 2.5]) == pytest.approx(0.5)
