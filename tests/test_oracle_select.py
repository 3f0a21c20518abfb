"""Pins the oracle's token selection (model/runtime.ts:880-899, math.ts:140-160).

Checks: tests/golden/select.json (winners fixed by the strict '>' rule),
brute force over random logits and allowed lists, and the log-probability
against scipy.special.logsumexp in float64.
"""

import json
import math
from pathlib import Path

import numpy as np
import pytest
from scipy.special import logsumexp

import oracle

GOLDEN = Path(__file__).resolve().parent / "golden"


def brute_select(logits, allowed):
    cand = list(range(len(logits))) if allowed is None else list(allowed)
    best_id = cand[0]
    best = float(logits[best_id])
    for c in cand[1:]:
        if float(logits[c]) > best:
            best, best_id = float(logits[c]), c
    return best_id


def test_golden_cases():
    for case in json.loads((GOLDEN / "select.json").read_text()):
        logits = np.array(case["logits"], dtype=np.float32)
        got, lp = oracle.select(logits, case["allowed"])
        assert got == case["id"], case["name"]
        if "log_probability" in case:
            assert abs(lp - case["log_probability"]) < 1e-12


def test_random_against_brute_force(rng):
    for trial in range(200):
        vocab = int(rng.integers(1, 300))
        logits = rng.normal(size=vocab).astype(np.float32)
        if trial % 3 == 0:
            logits = np.round(logits * 2) / 2  # many exact ties
        if trial % 2 == 0:
            count = int(rng.integers(1, vocab + 1))
            allowed = rng.choice(vocab, size=count, replace=False).astype(np.uint32)
            if trial % 4 == 0:
                allowed.sort()
        else:
            allowed = None
        got, lp = oracle.select(logits, allowed)
        assert got == brute_select(logits, allowed)
        ref = float(logits[got]) - logsumexp(logits.astype(np.float64))
        assert abs(lp - ref) <= 1e-12 * max(1.0, abs(ref))


def test_mask_form_equals_ascending_list(rng):
    from needle_hip.synth import pack_bits

    for _ in range(50):
        vocab = int(rng.integers(1, 700))
        logits = np.round(rng.normal(size=vocab) * 3).astype(np.float32)
        bits = rng.random(vocab) < 0.1
        bits[int(rng.integers(vocab))] = True
        mask = pack_bits(bits[None, :])[0]
        allowed = np.flatnonzero(bits).astype(np.uint32)
        assert oracle.select_mask(logits, mask) == oracle.select(logits, allowed)


def test_errors_and_nan_logprob():
    with pytest.raises(oracle.OracleError):
        oracle.select(np.zeros(4, np.float32), [])
    with pytest.raises(oracle.OracleError):
        oracle.select(np.zeros(4, np.float32), [1, 4])
    _, lp = oracle.select(np.array([1, float("nan"), 2], np.float32))
    assert math.isnan(lp)
