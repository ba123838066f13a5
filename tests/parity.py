"""Token-parity checks shared by the GPU model tests.

A greedy decision can differ between two implementations only at a near-tie.  The noise level is
taken from the whole output, not from the decision itself (which would make any flip look
explained): noise = the median over frames of the largest per-frame discrepancy, times
NOISE_FACTOR.  A flipped decision passes as a near-tie finding only if the oracle's top-2 gap there
is at most twice that noise (for TDT, twice the joint output layer's Lipschitz bound times the
encoder-row noise); any other flip fails.  Without flips the token lists must be identical.
"""

import numpy as np

NOISE_FACTOR = 10.0


def top2_gap(row):
    s = np.sort(np.asarray(row, np.float64))
    return float(s[-1] - s[-2])


def frame_noise(got, want):
    d = np.abs(np.asarray(got, np.float64) - np.asarray(want, np.float64)).max(axis=1)
    return NOISE_FACTOR * float(np.median(d))


def ctc_parity(got, want, classes):
    """Per-frame argmax of the first `classes` columns; returns the near-tie flips [(frame, gap,
    noise)] and asserts that every flip is one."""
    g = np.asarray(got, np.float64)[:, :classes]
    w = np.asarray(want, np.float64)[:, :classes]
    noise = frame_noise(g, w)
    flips = []
    for t in np.nonzero(g.argmax(1) != w.argmax(1))[0]:
        gap = top2_gap(w[t])
        assert gap <= 2 * noise, f"frame {t}: argmax flipped with top-2 gap {gap:.3g} > 2·noise {2 * noise:.3g}"
        flips.append((int(t), gap, noise))
    return flips


def tdt_parity(om, got, want):
    """TDT greedy on the device's encoder output against the oracle's: the paths agree up to the first
    flipped decision, whose gap must be within 2·L·noise (L the joint output layer's max row L1 norm,
    noise of the encoder rows).  Returns (flip or None, tokens on got, tokens on want)."""
    tg, trg, gg = om.tdt_trace(got)
    tw, trw, gw = om.tdt_trace(want)
    if tg == tw:
        return None, tg, tw
    n = min(len(trg), len(trw))
    k = next(i for i in range(n) if tuple(trg[i]) != tuple(trw[i]))
    frame = int(trw[k][0])
    assert int(trg[k][0]) == frame, "the decision paths diverged before a flipped decision"
    bound = 2 * om.tdt_lipschitz() * frame_noise(got, want)
    gap = float(gw[k])
    assert gap <= bound, f"decision {k} (frame {frame}) flipped with gap {gap:.3g} > bound {bound:.3g}"
    return (k, frame, gap, bound), tg, tw
