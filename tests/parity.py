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


# Relative tie bound of the device TDT decoder: both sides compute the joint and the predictor in f32,
# summing in different orders, so their logits differ by about 1e-6 of the output layer's Lipschitz
# bound times |z|; a flipped decision needs an oracle top-2 gap of that order.
TDT_TIE_REL = 1e-4
# After a near-tie flip the two decoders carry different predictor states; the encoder rows bring them
# back to the same decisions within this many frames, from where on every entry must agree again.
TDT_RESYNC_FRAMES = 50


def tdt_device_parity(om, tokens, enc):
    """The device TDT decoder's (token, frame) list against the oracle's on the same encoder output.
    Identical, or else the first flipped decision is a near tie: it lies after the oracle's decision
    that emitted the last shared token (the lists agree up to it) and at a frame no later than either
    list's first differing entry, and some oracle decision in that window has a top-2 gap of at most
    TDT_TIE_REL times the joint output layer's Lipschitz bound; and the lists agree again, entry for
    entry, from some frame within TDT_RESYNC_FRAMES after it (no second divergence goes unchecked).
    Returns None or (index, frame, smallest gap in the window, bound)."""
    want, trace, gaps = om.tdt_trace(enc)
    if tokens == want:
        return None
    n = min(len(tokens), len(want))
    i = next((k for k in range(n) if tokens[k] != want[k]), n)
    frame = min(lst[i][1] for lst in (tokens, want) if i < len(lst))
    # The oracle's decision that emitted want[i - 1]: emissions are the decisions whose (token,
    # frame) is the next list entry (a blank is never in the list).
    start, j = 0, 0
    for k in range(len(trace)):
        if j < i and (int(trace[k][1]), int(trace[k][0])) == want[j]:
            j += 1
            start = k + 1
    window = [k for k in range(start, len(trace)) if trace[k][0] <= frame]
    assert window, f"token {i} (frame {frame}) differs with no oracle decision where it could have flipped"
    gap = float(min(gaps[k] for k in window))
    bound = TDT_TIE_REL * om.tdt_lipschitz()
    assert gap <= bound, f"token {i} (frame {frame}) differs; smallest gap in decisions {start}.. is {gap:.3g} > bound {bound:.3g}"
    later = lambda lst, g: [e for e in lst if e[1] >= g]
    assert any(later(tokens, g) == later(want, g) for g in range(frame + 1, frame + TDT_RESYNC_FRAMES + 1)), (
        f"after the near tie at token {i} (frame {frame}) the lists do not agree again within {TDT_RESYNC_FRAMES} frames")
    return i, frame, gap, bound
