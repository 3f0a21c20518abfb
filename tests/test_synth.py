"""Pins the synthetic-data generator (splitmix64 spec in needle_hip.synth)."""

import json
from pathlib import Path

import numpy as np

from needle_hip import synth

GOLDEN = Path(__file__).resolve().parent / "golden"


def test_splitmix64_published_vector():
    g = json.loads((GOLDEN / "splitmix64.json").read_text())
    out = synth.splitmix64(g["seed"], len(g["outputs"]))
    assert [hex(int(v)) for v in out] == [hex(int(h, 16)) for h in g["outputs"]]


def test_streams_are_deterministic_and_in_range():
    a = synth.Stream(7, "w").int8((64, 64))
    b = synth.Stream(7, "w").int8((64, 64))
    assert np.array_equal(a, b)
    assert a.min() >= -127 and a.max() <= 127
    big = synth.Stream(1, "big").int8((1 << 16,))
    assert big.min() == -127 and big.max() == 127
    u = synth.Stream(7, "s").uniform((10000,), 0.001, 0.02)
    assert u.dtype == np.float32 and u.min() >= 0.001 and u.max() < 0.02
    z = synth.Stream(7, "n").normal((20000,))
    assert abs(float(z.mean())) < 0.05 and abs(float(z.std()) - 1) < 0.05
    assert not np.array_equal(synth.Stream(7, "w").int8((8,)), synth.Stream(8, "w").int8((8,)))


def test_mask_pack_roundtrip():
    s = synth.Stream(3, "mask")
    mask = s.bernoulli_mask(5, 1000, 0.02)
    bits = synth.unpack_bits(mask, 1000)
    assert bits.any(axis=1).all()
    assert np.array_equal(synth.pack_bits(bits), mask)
