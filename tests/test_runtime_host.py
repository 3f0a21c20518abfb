"""Host code of the Needle 2 runtime and model facade (no GPU): the sampler
and its xorshift32 generator (model/model.ts:202-240), logSoftmaxAt and
argmax (model/math.ts:140-160), and the online probe pool
(model/runtime.ts:48-105) -- what NeedleRuntime and NeedleModel compute on
the host in the reference too."""

import math

import numpy as np
import pytest
from scipy.special import logsumexp, softmax

from needle_hip.needle2 import ProbeHead
from needle_hip.runtime import (OnlineProbePool, argmax, log_softmax_at, sample, sigmoid,
                                xorshift32)


def test_xorshift32_known_sequence():
    """Marsaglia's xorshift32 (13, 17, 5) from state 1: 270369, 67634689,
    2647435461 (the published first outputs), each divided by 2^32."""
    draw = xorshift32(1)
    assert [round(draw() * 2**32) for _ in range(3)] == [270369, 67634689, 2647435461]
    zero = xorshift32(0)  # a zero seed becomes 1 (model.ts:203)
    assert round(zero() * 2**32) == 270369
    d = xorshift32(0x6D2B79F5)
    vals = [d() for _ in range(1000)]
    assert all(0.0 <= v < 1.0 for v in vals) and 0.45 < np.mean(vals) < 0.55


def test_sample_greedy_topk_and_distribution():
    rng = np.random.default_rng(3)
    logits = rng.normal(size=50).astype(np.float32)
    assert sample(logits, 0.0, 0, xorshift32(1)) == int(np.argmax(logits))
    assert sample(logits, -1.0, 5, xorshift32(1)) == int(np.argmax(logits))
    top = set(np.argsort(-logits)[:3].tolist())
    draw = xorshift32(9)
    seen = [sample(logits, 1.0, 3, draw) for _ in range(300)]
    assert set(seen) <= top
    # Frequencies follow softmax(logits / T) over the top 3 (chi-square-ish bound).
    p = softmax(np.sort(logits)[::-1][:3].astype(np.float64) / 1.0)
    order = np.argsort(-logits)[:3]
    freq = np.array([seen.count(int(i)) for i in order]) / len(seen)
    assert np.all(np.abs(freq - p) < 0.1)
    # A draw of exactly u maps to the first index whose cumulative mass >= u * sum.
    constant = lambda: 0.5  # noqa: E731
    two = np.array([0.0, 0.0], np.float32)
    assert sample(two, 1.0, 0, constant) == 0  # 0.5 * 2 - 1 <= 0


def test_sample_edge_cases_follow_the_reference():
    """model.ts:213-240 evaluated by hand: 0 < topK < 1 gives count 0, an
    empty candidate list and `indices[count - 1] ?? 0` = 0; a NaN logit makes
    Math.max NaN, every probability NaN, no `threshold <= 0` test passes and
    the last candidate (the last id, topK keeping every id) is returned."""
    logits = np.array([0.5, 2.0, -1.0, 0.25], np.float32)
    assert sample(logits, 1.0, 0.5, xorshift32(4)) == 0
    assert sample(logits, 0.7, 0.99, lambda: 0.0) == 0
    nan = logits.copy()
    nan[1] = np.nan
    for draw in (0.0, 0.3, 0.999):
        assert sample(nan, 1.0, 0, lambda: draw) == 3
        assert sample(nan, 2.0, 4, lambda: draw) == 3
    # Without NaN a draw of 0 returns the first candidate with nonzero mass.
    assert sample(logits, 1.0, 0, lambda: 0.0) == 0


def test_log_softmax_and_argmax():
    rng = np.random.default_rng(4)
    logits = (rng.normal(size=8192) * 20).astype(np.float32)
    for t in (0, 17, int(np.argmax(logits))):
        assert math.isclose(log_softmax_at(logits, t),
                            float(logits[t]) - float(logsumexp(logits.astype(np.float64))),
                            rel_tol=1e-12, abs_tol=1e-12)
    tie = np.array([1, 3, 3, 2], np.float32)
    assert argmax(tie) == 1
    assert argmax(np.array([np.nan, 1, 2], np.float32)) == 0  # NaN first is kept
    assert argmax(np.array([0, np.nan, 2], np.float32)) == 2

    def scan(values):  # the reference loop as written: `>` from index 0
        best, best_value = 0, float(values[0])
        for i in range(1, len(values)):
            if float(values[i]) > best_value:
                best, best_value = i, float(values[i])
        return best

    for _ in range(200):
        v = rng.integers(-3, 4, size=int(rng.integers(1, 12))).astype(np.float32)
        v[rng.random(v.size) < 0.2] = np.nan
        v[rng.random(v.size) < 0.1] = -np.inf
        v[rng.random(v.size) < 0.05] = np.inf
        assert argmax(v) == scan(v), v


def test_probe_pool_equals_softmax_pooling():
    """Online pooling equals the closed form: per probe, the softmax over
    cells of score = cell . probe / sqrt(d), weighting the cells."""
    rng = np.random.default_rng(5)
    d, p = 32, 3
    head = ProbeHead(rng.normal(size=(p, d)), rng.normal(size=(1, p * d)) * 0.1,
                     np.array([0.2]))
    pool = OnlineProbePool(head, d)
    cells = rng.normal(size=(9, d)).astype(np.float32)
    for c in cells:
        pool.add(c)
    scores = cells.astype(np.float64) @ head.probes.T.astype(np.float64) / math.sqrt(d)
    weights = softmax(scores, axis=0)
    pooled = (weights.T @ cells.astype(np.float64)).astype(np.float32).reshape(-1)
    want = float(pooled.astype(np.float64) @ head.projection[0].astype(np.float64) + 0.2)
    assert math.isclose(float(pool.output()[0]), want, rel_tol=1e-5, abs_tol=1e-6)
    assert math.isclose(sigmoid(2.0), 1 / (1 + math.exp(-2.0)), rel_tol=1e-15)
