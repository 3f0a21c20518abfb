"""ResidentExecutionSession at method granularity (nd_needle_begin_token ...
nd_needle_forward) driven by NeedleRuntime's unchanged control flow
(model/runtime.ts:280-583), through the C ABI.

* A token run through the session methods launches the same kernels in the
  same order as the whole-step extension (nd_needle_step), so logits,
  selected ids, log-probabilities and the resident confidence must be
  bit-identical to it, and within the usual bars of the oracle.
* forward_resident_layer one layer at a time, with a read of the lanes in
  the middle of a token, equals forward_resident_token.
* With resident layers off, the runtime runs its own lane mix, engram ring
  and confidence pool on the host and calls forward() per layer ("nextX");
  logits within 1e-3 of the largest, ids identical to the oracle's.
* generate over the runtime: greedy ids identical to the graph-replayed
  generate; temperature / top-k sampling identical to the same sampler over
  the oracle's logits; an abort signal stops it with GENERATION_ABORTED.
"""

import sys

import numpy as np
import pytest

import oracle
from needle_hip import AbortSignal, HipBackend, NeedleError, NeedleModel, synth
from needle_hip.needle2 import Needle2Geometry, Needle2Weights
from needle_hip.runtime import (ResidentLayerRequest, ResidentTokenRequest, argmax,
                                log_softmax_at, sample, xorshift32)

pytestmark = pytest.mark.gpu

SMALL = Needle2Geometry(vocab=512, dim=128, heads=4, kv_heads=2, layers=3, head_dim=64,
                        max_length=48, hadamard=256, lanes=4, engram_slots=64, engram_sub=128,
                        engram_tables=4, engram_taps=4, orders=(2, 3), sites=(0, 2), kv_window=8)


def say(*args):
    print("[case]", *args, file=sys.stderr, flush=True)


def bits(a):
    return np.asarray(a, np.float32).view(np.uint32)


def close(got, want, what):
    err = np.abs(got.astype(np.float64) - want.astype(np.float64))
    assert err.max() <= 1e-3 * np.abs(want).max(), (what, float(err.max()))


@pytest.fixture(scope="module")
def small(hip):
    w = Needle2Weights(SMALL, 31)
    model = NeedleModel(hip, w)
    yield w, model
    model.dispose()


def test_session_token_equals_whole_step(small):
    w, model = small
    say("session token == whole step")
    rt = model.create_runtime()
    rt.reset(SMALL.max_length, 3)
    whole = model.create_resident_runtime()
    whole.reset(SMALL.max_length, 3)
    ref = oracle.Needle2(w).runtime(SMALL.max_length, 3)
    tokens = synth.Stream(5, "sess").integers(30, 0, SMALL.vocab - 1)
    tokens[7:10] = tokens[3:6]  # repeated n-grams hit the same engram rows
    for i, t in enumerate(tokens):
        got = rt.step(int(t))
        assert np.array_equal(bits(got), bits(whole.step(int(t)))), i
        close(got, ref.step(int(t)), i)
        assert rt.position == i + 1
    assert rt.resolve_confidence() == whole.resolve_confidence()
    allowed = np.unique(synth.Stream(7, "sess-allowed").integers(60, 0, SMALL.vocab - 1))
    tok = int(tokens[-1])
    for i in range(6):
        a = allowed if i % 2 else None
        sel = rt.step_selected(tok, a)
        gid, glp = whole.step_selected(tok, a)
        assert (sel.id, sel.log_probability) == (gid, glp), i
        rid, rlp = oracle.select(ref.step(tok), a)
        assert sel.id == rid and abs(sel.log_probability - rlp) <= 1e-3 * max(1.0, abs(rlp))
        tok = sel.id
    # the mirror's prefill is repeated steps (runtime.ts:227-243)
    rt.reset(40, 2)
    ref = oracle.Needle2(w).runtime(40, 2)
    prompt = synth.Stream(6, "sess-prompt").integers(20, 0, SMALL.vocab - 1)
    got = rt.prefill(prompt)
    for t in prompt:
        want = ref.step(int(t))
    close(got, want, "prefill")
    rt.dispose()


def test_session_token_equals_whole_step_cactus_quant(hip):
    """The session methods over a Cactus-Quant model (the shipped archive's
    form): the host-driven step (embedding row through nd_row, engram rows
    gathered from the host's lookups) gives the whole step's logits bit for
    bit, and both agree with the oracle."""
    say("session token == whole step, cactus-quant")
    w = Needle2Weights(SMALL, 61, cq_bits=4)
    model = NeedleModel(hip, w)
    try:
        rt = model.create_runtime()
        rt.reset(SMALL.max_length, 2)
        whole = model.create_resident_runtime()
        whole.reset(SMALL.max_length, 2)
        ref = oracle.Needle2(w).runtime(SMALL.max_length, 2)
        tokens = synth.Stream(8, "sess-cq").integers(16, 0, SMALL.vocab - 1)
        tokens[9:11] = tokens[3:5]
        for i, t in enumerate(tokens):
            got = rt.step(int(t))
            assert np.array_equal(bits(got), bits(whole.step(int(t)))), i
            close(got, ref.step(int(t)), i)
        rt.dispose()
    finally:
        model.dispose()


def test_layer_granularity_and_lane_reads(small):
    """forward_resident_layer per layer, with readResidentLanes between two
    layers, gives the same token as forward_resident_token."""
    w, model = small
    say("session layers")
    model.backend.weights = w
    a = model.backend.create_resident_session()
    b = model.backend.create_resident_session()
    from needle_hip.runtime import ResidentExecutionResetOptions
    for s in (a, b):
        assert s.reset(ResidentExecutionResetOptions(SMALL.max_length, 0))
    emb = synth.Stream(3, "lanes").normal((SMALL.dim,))
    x = np.tile(emb, SMALL.lanes)
    keys = [synth.Stream(4, f"k{i}").normal((SMALL.dim,)) for i in range(len(SMALL.sites))]
    vals = [synth.Stream(5, f"v{i}").normal((SMALL.dim,)) for i in range(len(SMALL.sites))]
    for pos in range(3):
        assert a.begin_resident_token(x) and b.begin_resident_token(x)
        a.forward_resident_token(ResidentTokenRequest(pos, keys, vals))
        for layer in range(SMALL.layers):
            site = SMALL.sites.index(layer) if layer in SMALL.sites else -1
            b.forward_resident_layer(ResidentLayerRequest(
                layer, pos, keys[site] if site >= 0 else None, vals[site] if site >= 0 else None))
            if layer == 1:
                lanes = b.read_resident_lanes()
                assert lanes.shape == (SMALL.lanes * SMALL.dim,) and np.isfinite(lanes).all()
        la, lb = a.finish_resident_token(True), b.finish_resident_token(True)
        assert np.array_equal(bits(la), bits(lb)), pos
    assert a.resident_confidence() == b.resident_confidence()
    a.dispose()
    b.dispose()


def test_session_call_order_and_api_errors(small):
    w, model = small
    say("session errors")
    model.backend.weights = w
    s = model.backend.create_resident_session()
    from needle_hip.runtime import ResidentExecutionResetOptions
    assert s.reset(ResidentExecutionResetOptions(8, 0))
    x = np.zeros(SMALL.lanes * SMALL.dim, np.float32)
    with pytest.raises(NeedleError) as e:
        s.forward_resident_layer(ResidentLayerRequest(0, 0))
    assert e.value.code == "INVALID_CACT"  # before begin
    assert s.begin_resident_token(x)
    assert s.begin_resident_token(x)  # an open token (an aborted step) is dropped
    with pytest.raises(NeedleError) as e:
        s.forward_resident_layer(ResidentLayerRequest(1, 0))
    assert e.value.code == "INVALID_CACT"  # out of order
    with pytest.raises(NeedleError) as e:
        s.forward_resident_layer(ResidentLayerRequest(0, 0))
    assert "engram" in str(e.value)  # layer 0 is an engram site; no engrams given
    with pytest.raises(NeedleError) as e:
        s.finish_resident_token(True)
    assert e.value.code == "INVALID_CACT"  # layers missing
    with pytest.raises(NeedleError) as e:
        s.select_resident_token()
    assert e.value.code == "BACKEND_UNAVAILABLE"  # no logits for selection
    # whole-step calls are refused until the next reset
    with pytest.raises(NeedleError) as e:
        s.resident.step(3)
    assert e.value.code == "INVALID_CACT" and "session" in str(e.value)
    assert s.reset(ResidentExecutionResetOptions(8, 0))
    s.resident.step(3)
    with pytest.raises(NeedleError):
        s.begin_resident_token(x)
    with pytest.raises(NeedleError) as e:
        s.reset(ResidentExecutionResetOptions(SMALL.max_length + 1, 0))
    assert e.value.code == "CONTEXT_OVERFLOW"
    s.dispose()
    assert not s.begin_resident_token(x)  # disposed


def test_forward_fallback_with_resident_layers_off():
    """The runtime's own per-layer path: lane mix, engram ring and confidence
    pool on the host, forward() on the device returning the next lanes."""
    say("session forward fallback")
    w = Needle2Weights(SMALL, 33)
    backend = HipBackend(resident_layers=False)
    model = NeedleModel(backend, w)
    try:
        rt = model.create_runtime()
        rt.reset(SMALL.max_length, 2)
        assert not rt.session.resident_layers_enabled()
        ref = oracle.Needle2(w).runtime(SMALL.max_length, 2)
        tokens = synth.Stream(9, "fallback").integers(14, 0, SMALL.vocab - 1)
        tokens[6:8] = tokens[2:4]
        for i, t in enumerate(tokens):
            close(rt.step(int(t)), ref.step(int(t)), ("fallback", i))
        conf, want = rt.resolve_confidence(), ref.confidence()
        assert abs(conf - want) <= 1e-3 * want
        sel = rt.step_selected(int(tokens[-1]))
        assert sel.id == oracle.select(ref.step(int(tokens[-1])))[0]
        rt.dispose()
    finally:
        model.dispose()
        backend.dispose()


def test_generate_over_runtime(small):
    w, model = small
    say("generate over the runtime")
    prompt = synth.Stream(8, "sess-gen").integers(16, 3, SMALL.vocab - 1)
    greedy = model.generate(prompt, max_new_tokens=20, sink_tokens=1, eos=None)
    fast = model.generate_resident(prompt, max_new_tokens=20, sink_tokens=1, eos=None)
    # (the graph path batches the prompt on int8 MFMA; the runtime steps it)
    assert greedy.token_ids == fast.token_ids and greedy.finish_reason == "length"
    np.testing.assert_allclose(greedy.token_log_probabilities, fast.token_log_probabilities,
                               rtol=1e-3, atol=1e-3)
    # Sampling at temperature 0.8 over the 40 largest logits, seed 7: the
    # same draws over the oracle's logits pick the same tokens.
    got = model.generate(prompt, max_new_tokens=12, temperature=0.8, top_k=40, seed=7, eos=None)
    ref = oracle.Needle2(w).runtime(len(prompt) + 12, 0)
    for t in prompt:
        logits = ref.step(int(t))
    draw = xorshift32(7)
    want = []
    for k in range(12):
        tok = sample(logits, 0.8, 40, draw)
        want.append(tok)
        if k + 1 < 12:
            logits = ref.step(tok)
    assert got.token_ids == want
    # An abort raised from the layer callback of the third prompt token.
    signal = AbortSignal()

    def on_layer(event):
        if event["position"] == 2 and event["layer"] == 1:
            signal.abort("stop")

    rt = model.create_runtime(on_layer=on_layer)
    rt.reset(SMALL.max_length, 0)
    with pytest.raises(NeedleError) as e:
        rt.prefill(prompt, signal)
    assert e.value.code == "GENERATION_ABORTED" and rt.position == 2
    rt.dispose()
    with pytest.raises(NeedleError) as e:
        model.generate(prompt, 4, signal=signal)
    assert e.value.code == "GENERATION_ABORTED"


@pytest.mark.parametrize("cq_bits", [0, 4])
def test_full_geometry_session_equals_whole_steps(hip, cq_bits):
    """The shipped geometry (27 layers, engram sites 2 and 15, window 256),
    int8 and Cactus-Quant (CQ4) matrices: twelve tokens through the session
    methods (one launch each for Wo, mix and projection) equal the whole
    steps (Wo, mix and projection in one launch per layer)."""
    say("session full geometry", cq_bits)
    w = Needle2Weights(Needle2Geometry(), 2026, cq_bits=cq_bits)
    model = NeedleModel(hip, w)
    try:
        rt = model.create_runtime()
        rt.reset(64, 0)
        whole = model.create_resident_runtime()
        whole.reset(64, 0)
        for i, t in enumerate(synth.Stream(2026, "sess-full").integers(12, 0, 8191)):
            assert np.array_equal(bits(rt.step(int(t))), bits(whole.step(int(t)))), i
        assert rt.resolve_confidence() == whole.resolve_confidence()
        rt.dispose()
    finally:
        model.dispose()


def test_float32_kv_cache(small):
    """kvCache "float32" (model/runtime.ts:30-40, 186-204, 686-692): the
    cache keeps the projected K/V values themselves with scale 1, through the
    session methods and through whole steps with a batched prompt; logits
    within 1e-3 of the oracle's float32-cache runtime, and layer 0's rows
    equal to the oracle's values up to fp32 rounding."""
    w, model = small
    say("float32 kv cache")
    rt = model.create_runtime(kv_cache="float32")
    rt.reset(SMALL.max_length, 3)
    ref = oracle.Needle2(w).runtime(SMALL.max_length, 3, kv_cache="float32")
    tokens = synth.Stream(14, "f32kv").integers(20, 0, SMALL.vocab - 1)
    for i, t in enumerate(tokens):
        close(rt.step(int(t)), ref.step(int(t)), ("float32 session", i))
    k, v, ks, vs = rt.session.kv_read(0, 1)
    rk, rv, rks, rvs = ref.kv_read(0, 1)
    assert k.dtype == np.float32 and np.all(ks == 1.0) and np.all(vs == 1.0)
    np.testing.assert_allclose(k, rk, rtol=1e-5, atol=1e-5 * np.abs(rk).max())
    np.testing.assert_allclose(v, rv, rtol=1e-5, atol=1e-5 * np.abs(rv).max())
    rt.dispose()
    whole = model.create_resident_runtime(kv_cache="float32")
    whole.reset(40, 0)
    ref = oracle.Needle2(w).runtime(40, 0, kv_cache="float32")
    prompt = synth.Stream(15, "f32kv-prompt").integers(24, 0, SMALL.vocab - 1)
    got = whole.prefill(prompt)
    for t in prompt:
        want = ref.step(int(t))
    close(got, want, "float32 batched prefill")
    tok = int(np.argmax(got))
    for i in range(4):
        close(whole.step(tok), ref.step(tok), ("float32 step", i))
        tok = (tok * 7 + 3) % SMALL.vocab
    # back to int8 on the next reset: the graphs and kernels follow the mode
    whole = model.create_resident_runtime()
    whole.reset(40, 0)
    ref = oracle.Needle2(w).runtime(40, 0)
    close(whole.prefill(prompt), [ref.step(int(t)) for t in prompt][-1], "int8 after float32")
