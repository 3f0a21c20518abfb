"""GPU parity of the one-pass prefill against the oracle's sequential steps.

The oracle prefill is the reference's: one step per prompt token
(model/runtime.ts:227-243).  Bars: KV codes identical except where a value
sits on a rounding boundary (at most one code apart, at most 0.5% of the
codes; layer 0 measures ~1e-5); the last position's logits within 1e-3
relative normwise and the same greedy token; and a prefill split at any
position equals the unsplit one exactly.

Why normwise end to end: a K/V element whose x/s lies within ~1e-5 of a
half-integer rounds to the other code when the GPU's fp32 projection differs
from the oracle's float64 one in the last bits; one such code shifts later
attention outputs by up to ~5e-4 relative (measured), so elementwise
1e-3/1e-4 is the per-kernel bar (matvec, matmul, attention on identical
inputs) and the whole model is held to the relative bar normwise.
"""

import sys

import numpy as np
import pytest

import oracle
from needle_hip import HipKvCache, NeedleError, synth
from needle_hip.models import DecoderGeometry, DecoderWeights, HipDecoder, HipPrefill

pytestmark = pytest.mark.gpu


def say(*args):
    print("[case]", *args, file=sys.stderr, flush=True)


def compare(hip, g, n, seed):
    weights = DecoderWeights(g, seed)
    dec = HipDecoder(hip, weights)
    pre = HipPrefill(dec, n, n)
    cache = HipKvCache(hip, g.layers, g.kv_heads, max_length=n)
    tokens = synth.Stream(seed, "prompt").integers(n, 0, g.vocab - 1)
    logits = pre.run(cache, tokens)
    ref = oracle.SynthDecoder(weights)
    rc = ref.new_cache(n)
    want = None
    for p, t in enumerate(tokens):
        want = ref.step(rc, int(t), p)
    total = differ = 0
    for l in range(g.layers):
        for h in range(g.kv_heads):
            got_k, got_v, got_ks, got_vs = cache.read(l, h)
            ref_k, ref_v, ref_ks, ref_vs = rc.read(l, h)
            for a, b in ((got_k, ref_k), (got_v, ref_v)):
                d = np.abs(a.astype(int) - b.astype(int))
                assert d.max() <= 1, (l, h)
                total += d.size
                differ += int((d != 0).sum())
            np.testing.assert_allclose(got_ks, ref_ks, rtol=1e-3)
            np.testing.assert_allclose(got_vs, ref_vs, rtol=1e-3)
            if l == 0:  # inputs of layer 0 are bit-exact: scales agree to fp32
                np.testing.assert_allclose(got_ks, ref_ks, rtol=1e-6)
    # Layer 0 flips ~1e-5 of its codes; each flip perturbs later layers, whose
    # flip rate measures ~1e-3 (2-layer GQA model: 310 of 204800).
    assert differ <= max(8, total * 5e-3), (differ, total)
    err = np.abs(logits.astype(np.float64) - want)
    assert err.max() <= 1e-3 * np.abs(want).max(), err.max()
    assert int(np.argmax(logits)) == oracle.argmax(want)
    pre.free()
    cache.free()
    dec.free()
    return differ, total


def test_prefill_small_model(hip):
    say("prefill small")
    compare(hip, DecoderGeometry(layers=2, vocab=4096), 300, 5)


def test_prefill_gqa_model(hip):
    say("prefill gqa")
    compare(hip, DecoderGeometry(layers=2, heads=8, kv_heads=4, vocab=2048), 200, 6)


def test_prefill_full_geometry(hip):
    say("prefill full geometry")
    compare(hip, DecoderGeometry(), 512, 2026)


def test_prefill_split_equals_unsplit(hip):
    say("prefill split")
    g = DecoderGeometry(layers=2, vocab=4096)
    dec = HipDecoder(hip, DecoderWeights(g, 8))
    pre = HipPrefill(dec, 400, 400)
    tokens = synth.Stream(8, "prompt").integers(400, 0, g.vocab - 1)
    whole = HipKvCache(hip, g.layers, g.kv_heads, max_length=400)
    parts = HipKvCache(hip, g.layers, g.kv_heads, max_length=400)
    want = pre.run(whole, tokens)
    pre.run(parts, tokens[:123], 0, want_logits=False)
    pre.run(parts, tokens[123:300], 123, want_logits=False)
    got = pre.run(parts, tokens[300:], 300)
    # Layer 0 sees identical inputs either way, so its cache is bit-identical;
    # attention may split its context differently for a different number of
    # query rows (a different fp32 summation order), so later layers agree to
    # fp32 rounding.
    assert np.abs(got - want).max() <= 1e-5 * np.abs(want).max()
    for h in range(g.kv_heads):
        for a, b in zip(whole.read(0, h), parts.read(0, h)):
            assert np.array_equal(a, b)
        for a, b in zip(whole.read(1, h)[:2], parts.read(1, h)[:2]):
            assert np.abs(a.astype(int) - b.astype(int)).max() <= 1
    with pytest.raises(NeedleError) as e:
        pre.run(parts, tokens[:10], 395)
    assert e.value.code == "CONTEXT_OVERFLOW"
    pre.free()
    whole.free()
    parts.free()
    dec.free()
