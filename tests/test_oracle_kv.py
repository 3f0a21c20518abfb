"""Pins the oracle's int8 KV quantizer (model/runtime.ts:679-717, 901-907).

Checks: Python's round() (round-half-even) on random and tie values, the
known-answer vectors of tests/golden/kv_quant.json (fixed by construction),
and the invariants |code| <= 127, code(absmax) = +-127, |x - code*s| <= s/2
in exact rational arithmetic.  Plus the slot map and window/sink layout.
"""

import json
import struct
from fractions import Fraction
from pathlib import Path

import numpy as np
import pytest

import oracle

GOLDEN = Path(__file__).resolve().parent / "golden"


def f32_bits(x):
    return struct.unpack("<I", struct.pack("<f", x))[0]


def test_round_ties_even_matches_python_round(rng):
    values = list(rng.normal(0, 50, 2000)) + [k + 0.5 for k in range(-130, 130)]
    values += [-0.5, 0.5, -1.5, 1.5, 2.5, -2.5, 0.0, -0.0, 1e-300, -1e-300, 126.5, -126.5]
    for v in values:
        assert oracle.round_ties_even(v) == float(round(v)), v


def test_golden_vectors():
    cases = json.loads((GOLDEN / "kv_quant.json").read_text())
    assert len(cases) >= 10
    for case in cases:
        codes, scale = oracle.kv_quantize(np.array(case["x"], dtype=np.float32))
        assert codes.tolist() == case["codes"], case["name"]
        assert f32_bits(scale) == case["scale_bits"], case["name"]


@pytest.mark.parametrize("sigma", [1e-14, 1e-6, 1.0, 37.0, 1e6])
def test_invariants_exact(rng, sigma):
    for _ in range(40):
        x = (rng.normal(0, sigma, 64)).astype(np.float32)
        codes, scale = oracle.kv_quantize(x)
        m = max(1e-12, float(np.max(np.abs(x.astype(np.float64)))))
        s = m / 127  # float64, as the reference computes it
        assert scale == np.float32(s)
        assert np.all(np.abs(codes.astype(int)) <= 127)
        if m > 1e-12:
            i = int(np.argmax(np.abs(x)))
            assert abs(int(codes[i])) == 127
        sf = Fraction(s)
        for xi, ci in zip(x.tolist(), codes.tolist()):
            # Rounding of the float64 quotient may move the exact error by at
            # most one ulp of x/s beyond s/2.
            err = abs(Fraction(xi) - ci * sf)
            assert err <= sf / 2 + sf * Fraction(2) ** -45, (xi, ci, s)


def test_zero_vector_uses_floor():
    codes, scale = oracle.kv_quantize(np.zeros(64, np.float32))
    assert not codes.any()
    assert scale == np.float32(1e-12 / 127)


def test_slot_map_window_and_sink():
    kv = oracle.KvCache(1, 1, max_length=40, sink=3, window=5)
    assert kv.alloc == 8
    # runtime.ts:659-664
    expect = [p if p < 3 else 3 + (p - 3) % 5 for p in range(40)]
    assert [kv.slot(p) for p in range(40)] == expect
    kv0 = oracle.KvCache(1, 1, max_length=10, sink=0, window=0)
    assert kv0.alloc == 10 and [kv0.slot(p) for p in range(10)] == list(range(10))
    kv_small = oracle.KvCache(1, 1, max_length=6, sink=3, window=5)
    assert kv_small.alloc == 6


def test_store_layout_and_float_mode(rng):
    kv = oracle.KvCache(2, 3, max_length=8)
    k = rng.normal(size=(3, 64)).astype(np.float32)
    v = rng.normal(size=(3, 64)).astype(np.float32)
    kv.store(1, 5, k, v)
    for h in range(3):
        kc, vc, ks, vs = kv.read(1, h)
        ck, sk = oracle.kv_quantize(k[h])
        cv, sv = oracle.kv_quantize(v[h])
        assert kc[5].tolist() == ck.tolist() and vc[5].tolist() == cv.tolist()
        assert ks[5] == np.float32(sk) and vs[5] == np.float32(sv)
        assert not kc[:5].any() and not kc[6:].any()
        kc0, _, _, _ = kv.read(0, h)
        assert not kc0.any()
