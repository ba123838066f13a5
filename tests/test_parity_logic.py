"""The token-parity checks themselves, with flips planted in CPU-side logits: a near-tie flip under
typical noise passes, a flip at a frame whose discrepancy is far above the typical noise fails; for the
device TDT decoder, a near-tie flip after which the lists agree again passes, one after which they keep
differing fails."""

import numpy as np
import pytest

from parity import ctc_parity, tdt_device_parity, top2_gap


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


class TdtTrace:
    """The oracle's side of tdt_device_parity: its (token, frame) list, its decisions (frame, token) and
    their top-2 gaps, and the joint's Lipschitz bound."""

    def __init__(self, want, trace, gaps, lipschitz=1.0):
        self.want, self.trace, self.gaps, self.lipschitz = want, trace, gaps, lipschitz

    def tdt_trace(self, enc):
        return self.want, self.trace, self.gaps

    def tdt_lipschitz(self):
        return self.lipschitz


WANT = [(5, 0), (7, 2), (9, 4), (3, 10), (4, 60), (6, 70)]
TRACE = [(f, t) for t, f in WANT]


def test_tdt_identical_lists_pass():
    assert tdt_device_parity(TdtTrace(WANT, TRACE, [1.0] * 6), list(WANT), None) is None


def test_tdt_near_tie_then_agreement_passes():
    got = [(5, 0), (7, 2), (8, 4), (3, 10), (4, 60), (6, 70)]
    om = TdtTrace(WANT, TRACE, [1.0, 1.0, 1e-9, 1.0, 1.0, 1.0])
    assert tdt_device_parity(om, got, None)[:2] == (2, 4)


def test_tdt_near_tie_then_lasting_difference_fails():
    got = [(5, 0), (7, 2), (8, 4), (1, 10), (2, 60), (2, 70)]
    om = TdtTrace(WANT, TRACE, [1.0, 1.0, 1e-9, 1.0, 1.0, 1.0])
    with pytest.raises(AssertionError, match="do not agree again"):
        tdt_device_parity(om, got, None)


def test_tdt_flip_without_a_near_tie_fails():
    got = [(5, 0), (7, 2), (8, 4), (3, 10), (4, 60), (6, 70)]
    with pytest.raises(AssertionError, match="smallest gap"):
        tdt_device_parity(TdtTrace(WANT, TRACE, [1.0] * 6), got, None)
