"""Whisper's greedy window search (src/whisper/search.rs): the oracle's restatement (oracle/search.c)
and the product's host code (wh_whisper_pick / wh_whisper_retrieve in libwavo_hip.so, which need no
GPU) against the reference's own unit tests (src/whisper/search.rs:184-244), against each other on
seeded random logits, and against float64 restatements of the rules' closed forms.
"""

import math

import numpy as np
import pytest

import oracle as ox
import wavo_amd as wa

# The reference tests' vocabulary of 20: text 0..10, EOT 10, notimestamps 12, timestamps 13..20
# (src/whisper/search.rs:188-193).
T = 13


def ids_ox(suppress=(11,), begin_suppress=(1, 10)):
    return ox.WhisperIds.make(10, 12, T, suppress, begin_suppress)


def ids_wa(suppress=(11,), begin_suppress=(1, 10)):
    return wa.WhisperIds.make(10, 12, T, suppress, begin_suppress)


def allowed(s):
    return [i in s for i in range(20)]


# src/whisper/search.rs:195-214: (generated, the ids timestamp_rules leaves finite on zero logits).
RULE_CASES = [
    ([], set(range(T, 20))),
    ([T, 3, T + 2], set(range(T + 2, 20))),
    ([T, 3, T + 2, T + 2], set(range(12))),
    ([T + 1, 3], set(range(T + 2, 20))),
]


@pytest.mark.parametrize("gen,want", RULE_CASES)
def test_timestamp_rules_reference_cases_oracle(gen, want):
    got = ox.timestamp_rules(ids_ox(), np.zeros(20, np.float32), gen)
    assert list(np.isfinite(got)) == allowed(want)


@pytest.mark.parametrize("gen,want", RULE_CASES)
def test_timestamp_rules_reference_cases_product(gen, want):
    # With empty suppression lists, pick leaves exactly what timestamp_rules leaves.
    _, _, got = wa.whisper_pick(ids_wa((), ()), np.zeros(20, np.float32), gen)
    assert list(np.isfinite(got)) == allowed(want)


def one_hot(i):
    v = np.zeros(20, np.float32)
    v[i] = 5.0
    return v


def test_decode_stops_at_eot_and_counts_logprobs():
    """src/whisper/search.rs:216-231 with a scripted step: the prompt picks T, then 3, then T + 4,
    then EOT; steps are called with (token, position) from the prompt length on."""
    script = [3, T + 4, 10]
    for pick, ids in ((ox.whisper_pick, ids_ox()), (wa.whisper_pick, ids_wa())):
        calls, gen, lps = [], [], []
        nxt, lp, _ = pick(ids, one_hot(T), gen, True)
        lps.append(lp)
        for pos in range(3, 3 + 256):
            if nxt == 10:
                break
            gen.append(nxt)
            calls.append((nxt, pos))
            nxt, lp, _ = pick(ids, one_hot(script[len(calls) - 1]), gen, True)
            lps.append(lp)
        assert gen == [T, 3, T + 4]
        assert calls == [(T, 3), (3, 4), (T + 4, 5)]
        avg = sum(lps) / len(lps)
        assert -1.0 < avg < 0.0


# src/whisper/search.rs:233-243: (generated, frames) -> (segments, advance).
RETRIEVE_CASES = [
    ([T, 1, 2, T + 3], ([(0, [1, 2])], 3000)),
    ([T, 1, T + 2, T + 2, 3, T + 5], ([(0, [1]), (2, [3])], 3000)),
    ([T, 1, T + 2, T + 3, 4, T + 5, T + 5], ([(0, [1]), (3, [4])], 10)),
    ([T, 1, T + 2, T + 3, 4], ([(0, [1])], 4)),
    ([], ([], 3000)),
]


@pytest.mark.parametrize("gen,want", RETRIEVE_CASES)
def test_retrieve_reference_cases(gen, want):
    assert ox.whisper_retrieve(ids_ox(), gen, 3000) == want
    assert wa.whisper_retrieve(ids_wa(), gen, 3000) == want


def rules64(logits, gen, begin=T, eot=10, no_ts=12, vocab=20, max_initial=50):
    """The timestamp rules restated in float64 numpy from HF's WhisperTimeStampLogitsProcessor, which
    the reference cites (src/whisper/search.rs:73-76): an independent statement of the same rules."""
    l = np.asarray(logits, np.float64).copy()
    ts = lambda i: i >= begin
    l[no_ts] = -np.inf
    n = len(gen)
    if n:
        last_ts = ts(gen[-1])
        pen_ts = n < 2 or ts(gen[-2])
        if last_ts:
            if pen_ts:
                l[begin:] = -np.inf
            else:
                l[:eot] = -np.inf
        stamps = [g for g in gen if ts(g)]
        if stamps:
            low = stamps[-1] if (last_ts and not pen_ts) else stamps[-1] + 1
            l[begin:low] = -np.inf
    else:
        l[:begin] = -np.inf
        l[min(begin + max_initial + 1, vocab):] = -np.inf
    lse = np.logaddexp.reduce(l[begin:]) if np.isfinite(l[begin:]).any() else -np.inf
    if lse > l[:begin].max():
        l[:begin] = -np.inf
    return l


def random_history(rng, n):
    return [int(x) for x in rng.integers(0, 20, n)]


@pytest.mark.parametrize("seed", range(40))
def test_pick_product_equals_oracle_and_float64_rules(seed):
    rng = np.random.default_rng(seed)
    logits = (rng.standard_normal(20) * rng.uniform(0.1, 4.0)).astype(np.float32)
    gen = random_history(rng, int(rng.integers(0, 6)))
    io, lo, ao = ox.whisper_pick(ids_ox(), logits, gen, True)
    iw, lw, aw = wa.whisper_pick(ids_wa(), logits, gen, True)
    assert io == iw and lo == lw
    assert np.array_equal(np.isfinite(ao), np.isfinite(aw))
    # The float64 statement (with the suppression applied first) leaves the same ids, except where the
    # two masses tie to within f32 rounding.
    l = logits.astype(np.float64)
    l[11] = -np.inf
    if not gen:
        l[[1, 10]] = -np.inf
    ref = rules64(l, gen)
    fin = np.isfinite(l[T:])
    lse = np.logaddexp.reduce(l[T:][fin]) if fin.any() else -np.inf
    if not math.isclose(lse, l[:T].max(), rel_tol=1e-5, abs_tol=1e-5):
        assert np.array_equal(np.isfinite(ref), np.isfinite(aw)), (gen, logits)
        assert iw == int(np.argmax(ref))
    # The log-softmax of the pick over the finite logits left.
    left = aw[np.isfinite(aw)].astype(np.float64)
    assert abs(lw - (aw[iw] - np.logaddexp.reduce(left))) < 1e-5


def test_probability():
    rng = np.random.default_rng(7)
    l = rng.standard_normal(100).astype(np.float32)
    l[5] = -np.inf
    p = np.exp(l.astype(np.float64) - l.max())
    p /= p.sum()
    for i in (0, 5, 42):
        assert abs(ox.probability(l, i) - p[i]) < 1e-6
        assert abs(wa.whisper_probability(l, i) - p[i]) < 1e-6


@pytest.mark.parametrize("seed", range(30))
def test_retrieve_product_equals_oracle(seed):
    rng = np.random.default_rng(100 + seed)
    n = int(rng.integers(0, 14))
    # Histories with timestamp runs: mostly timestamps and text ids.
    gen = [int(x) for x in np.where(rng.random(n) < 0.5, rng.integers(T, 20, n), rng.integers(0, 10, n))]
    assert ox.whisper_retrieve(ids_ox(), gen, 3000) == wa.whisper_retrieve(ids_wa(), gen, 3000)


def test_pick_rejects_bad_ids():
    with pytest.raises(wa.WavoError):
        wa.whisper_pick(wa.WhisperIds.make(30, 12, T), np.zeros(20, np.float32), [])
