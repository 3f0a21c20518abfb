"""GPU parity of the Needle 2 runtime (nd_needle_*) against the oracle's
NeedleRuntime.step restatement, through the C ABI.

Bars: logits within 1e-3 of the largest logit (one K/V code that rounds
the other way at a boundary moves later outputs by ~1e-4 relative); greedy
token sequences and selected ids identical; log-probabilities within 1e-3.
Appended KV codes: in layer 0, whose inputs agree with the oracle's to fp32
rounding, equal to the oracle's or one apart with the oracle's quotient
x / s within 1e-4 of the rounding boundary between them, scales within 1e-5
relative; in deeper layers (inputs that drifted by the model's own fp32
rounding) at most one code apart on at most 1% of a layer's codes, scales
within 1e-3 relative.
"""

import dataclasses
import sys

import numpy as np
import pytest

import oracle
from helpers import assert_codes_or_boundary_flips
from needle_hip import NeedleError, NeedleModel, synth
from needle_hip.needle2 import Needle2Geometry, Needle2Weights

pytestmark = pytest.mark.gpu

# Every engram site, lane, GQA group and a window that wraps; hadamard > dim
# exercises the zero-padded transform.
SMALL = Needle2Geometry(vocab=512, dim=128, heads=4, kv_heads=2, layers=3, head_dim=64,
                        max_length=48, hadamard=256, lanes=4, engram_slots=64, engram_sub=128,
                        engram_tables=4, engram_taps=4, orders=(2, 3), sites=(0, 2), kv_window=8)


def say(*args):
    print("[case]", *args, file=sys.stderr, flush=True)


def close(got, want, what):
    err = np.abs(got.astype(np.float64) - want.astype(np.float64))
    assert err.max() <= 1e-3 * np.abs(want).max(), (what, float(err.max()))


def slot_positions(written, alloc, sink, window):
    """The position whose K/V each cache slot holds once positions [0,
    written) were stored (#kvSlot, model/runtime.ts:659-664); -1 if none."""
    pos = np.full(alloc, -1)
    for p in range(written):
        pos[p if window == 0 or p < sink else sink + (p - sink) % window] = p
    return pos


def check_kv(model, ref, g, written, sink, what):
    """The GPU cache against the oracle's (which captured its vectors before
    quantization from position 0): see the module docstring for the bars."""
    alloc = min(g.max_length, sink + g.kv_window) if g.kv_window else g.max_length
    pos = slot_positions(written, alloc, sink, g.kv_window)
    used = np.flatnonzero(pos >= 0)
    for layer in range(g.layers):
        differ = total = 0
        worst = 0.0
        for h in range(g.kv_heads):
            gk, gv, gks, gvs = model.resident.kv_read(layer, h)
            rk, rv, rks, rvs = ref.kv_read(layer, h)
            assert gk.shape == rk.shape
            if layer == 0:
                raw_k, raw_v = ref.kv_read_raw(0, h, 0, written)
                for got, want, raw in ((gk, rk, raw_k), (gv, rv, raw_v)):
                    assert_codes_or_boundary_flips(got[used], want[used], raw[pos[used]], 1e-4,
                                                   f"{what} layer 0 head {h}")
            else:
                for got, want in ((gk, rk), (gv, rv)):
                    d = np.abs(got[used].astype(int) - want[used].astype(int))
                    assert d.max() <= 1, (what, layer, h)
                    differ += int((d != 0).sum())
                    total += d.size
            tol = 1e-5 if layer == 0 else 1e-3
            for got, want in ((gks, rks), (gvs, rvs)):
                rel = np.abs(got[used].astype(np.float64) / want[used] - 1.0)
                worst = max(worst, float(rel.max())) if layer else worst
                assert rel.max() <= tol, (what, layer, h, float(rel.max()))
        if layer:
            say(f"[measure] {what} layer {layer}: {differ}/{total} codes differ, "
                f"scale rel err max {worst:.2e}")
            assert differ <= 0.01 * total, (what, layer, differ, total)


def close_confidence(got, want, what):
    """The probe head's sigmoid output: within 1e-3 relative of the oracle's
    (the pooled cells carry the whole model's 1e-4-level differences)."""
    assert got is not None and 0.0 < got < 1.0, (what, got)
    assert abs(got - want) <= 1e-3 * want, (what, got, want)


@pytest.fixture(scope="module")
def small(hip):
    w = Needle2Weights(SMALL, 31)
    model = NeedleModel(hip, w)
    yield w, model
    model.dispose()


@pytest.mark.parametrize("sink", [0, 3])
def test_step_logits_and_kv_match_oracle(small, sink):
    w, model = small
    say("needle2 step sink", sink)
    rt = model.create_resident_runtime()
    rt.reset(SMALL.max_length, sink)
    ref = oracle.Needle2(w).runtime(SMALL.max_length, sink)
    ref.capture_kv(0, SMALL.max_length)
    tokens = synth.Stream(5, f"n2tok{sink}").integers(30, 0, SMALL.vocab - 1)
    tokens[7:10] = tokens[3:6]  # repeated n-grams hit the same engram rows
    for i, t in enumerate(tokens):
        want = ref.step(int(t))
        got = rt.step(int(t))
        close(got, want, (sink, i))
        assert rt.position == i + 1
        if i in (0, 9, len(tokens) - 1):
            close_confidence(rt.resolve_confidence(), ref.confidence(), ("confidence", sink, i))
    assert model.resident.kv_read(0, 0)[0].shape == (sink + SMALL.kv_window, 64)
    check_kv(model, ref, SMALL, len(tokens), sink, f"steps sink {sink}")


@pytest.mark.parametrize("heads,kv_heads,window,length", [(2, 2, 8, 48), (4, 2, 0, 600)])
def test_attention_group_sizes_and_chunked_slots(hip, heads, kv_heads, window, length):
    """One query head per KV head, and a 600-slot cache without a window
    whose three chunks are mostly unwritten slots at the first steps (a tile
    with no visible position must leave its wave's softmax state empty, not
    NaN): step logits agree with the oracle's."""
    geo = dataclasses.replace(SMALL, heads=heads, kv_heads=kv_heads, kv_window=window,
                              max_length=max(SMALL.max_length, length))
    say("needle2 attention paths", heads, kv_heads, window, length)
    w = Needle2Weights(geo, 41)
    model = NeedleModel(hip, w)
    try:
        rt = model.create_resident_runtime()
        rt.reset(length, 0)
        ref = oracle.Needle2(w).runtime(length, 0)
        tokens = synth.Stream(6, f"n2paths{heads}{window}").integers(12, 0, geo.vocab - 1)
        for i, t in enumerate(tokens):
            close(rt.step(int(t)), ref.step(int(t)), (heads, window, i))
    finally:
        model.dispose()


def test_step_ignores_stale_nan_slots(small):
    """A step's attention walks every ring slot and masks the ones its position
    cannot see; such slots must add nothing even when they hold NaN (stale or
    never-written memory).  The cache is poisoned with NaN rows (code 0, scale
    NaN) before a fresh reset, and the steps must still match the oracle."""
    import ctypes as C

    from needle_hip import lib as L

    w, model = small
    say("needle2 stale NaN slots")
    rt = model.create_resident_runtime()
    rt.reset(SMALL.max_length, 0)
    sess = model.resident
    kv = sess.lib.nd_needle_kv(sess.handle)
    alloc = C.c_uint32()
    sess._check(sess.lib.nd_kv_info(kv, C.byref(alloc), None, None, None, None), "nd_kv_info")
    poison = np.full((alloc.value, SMALL.kv_heads, 64), np.nan, np.float32)
    for layer in range(SMALL.layers):
        sess._check(sess.lib.nd_kv_store(sess.backend.ctx, kv, layer, 0, alloc.value,
                                         L.ptr(poison), L.ptr(poison)), "nd_kv_store")
    assert np.isnan(sess.kv_read(0, 0)[3]).all()
    rt.reset(SMALL.max_length, 0)
    ref = oracle.Needle2(w).runtime(SMALL.max_length, 0)
    for i, t in enumerate(synth.Stream(6, "n2nan").integers(12, 0, SMALL.vocab - 1)):
        close(rt.step(int(t)), ref.step(int(t)), ("nan slots", i))


def test_prefill_and_step_selected(small):
    w, model = small
    say("needle2 prefill + step_selected")
    rt = model.create_resident_runtime()
    rt.reset(40, 2)
    ref = oracle.Needle2(w).runtime(40, 2)
    prompt = synth.Stream(6, "n2prompt").integers(20, 0, SMALL.vocab - 1)
    got = rt.prefill(prompt)
    for t in prompt:
        want = ref.step(int(t))
    close(got, want, "prefill")
    close_confidence(rt.resolve_confidence(), ref.confidence(), "confidence after prefill")
    allowed = np.unique(synth.Stream(7, "n2allowed").integers(60, 0, SMALL.vocab - 1))
    tok = int(prompt[-1])
    for i in range(6):
        gid, glp = rt.step_selected(tok, allowed if i % 2 else None)
        logits = ref.step(tok)
        rid, rlp = oracle.select(logits, allowed if i % 2 else None)
        assert gid == rid, i
        assert abs(glp - rlp) <= 1e-3 * max(1.0, abs(rlp)), i
        tok = gid
    close_confidence(rt.resolve_confidence(), ref.confidence(), "confidence after selection")
    # reset clears the pool: one token pools that token's cells only
    rt.reset(40, 2)
    ref = oracle.Needle2(w).runtime(40, 2)
    rt.step(int(prompt[0]), want_logits=False)
    ref.step(int(prompt[0]), want_logits=False)
    close_confidence(rt.resolve_confidence(), ref.confidence(), "confidence after reset")


def test_generate_matches_stepwise_oracle(small):
    w, model = small
    say("needle2 generate small")
    prompt = synth.Stream(8, "n2gen").integers(16, 3, SMALL.vocab - 1)
    res = model.generate_resident(prompt, max_new_tokens=20, sink_tokens=1, eos=None)
    ref = oracle.Needle2(w).runtime(len(prompt) + 20, 1)
    for t in prompt:
        logits = ref.step(int(t))
    ids, lps = [], []
    for k in range(20):
        tok = oracle.argmax(logits)
        ids.append(tok)
        lps.append(oracle.log_softmax_at(logits, tok))
        if k + 1 < 20:
            logits = ref.step(tok)
    assert res.token_ids == ids
    np.testing.assert_allclose(res.token_log_probabilities, lps, rtol=1e-3, atol=1e-3)
    assert res.finish_reason == "length" and res.generated_tokens == 20
    # Graph replays and direct launches give the same sequence.
    rt = model.create_resident_runtime()
    rt.reset(len(prompt) + 20, 1)
    logits = rt.prefill(prompt)
    assert int(np.argmax(logits)) == ids[0]
    tok = ids[0]
    for k in range(1, 6):
        tok, _ = rt.step_selected(tok)
        assert tok == ids[k]


def test_generate_stops_before_eos_and_at_limit(small):
    w, model = small
    say("needle2 generate eos/limit")
    prompt = synth.Stream(9, "n2eos").integers(10, 3, SMALL.vocab - 1)
    full = model.generate_resident(prompt, max_new_tokens=12, eos=None)
    stop = full.token_ids[4]
    first = full.token_ids.index(stop)
    cut = model.generate_resident(prompt, max_new_tokens=12, eos=stop)
    assert cut.token_ids == full.token_ids[:first] and cut.finish_reason == "eos"
    # The context limit caps the count: 48 - 40 = 8 tokens.
    long_prompt = synth.Stream(10, "n2lim").integers(40, 3, SMALL.vocab - 1)
    lim = model.generate_resident(long_prompt, max_new_tokens=30, eos=None)
    assert lim.generated_tokens == 8
    with pytest.raises(NeedleError) as e:
        model.generate_resident(synth.Stream(11, "n2over").integers(48, 3, SMALL.vocab - 1), 4, eos=None)
    assert e.value.code == "CONTEXT_OVERFLOW"


def test_runtime_errors(small):
    w, model = small
    say("needle2 errors")
    rt = model.create_resident_runtime()
    with pytest.raises(NeedleError) as e:
        rt.reset(SMALL.max_length + 1)
    assert e.value.code == "CONTEXT_OVERFLOW"
    rt.reset(2)
    with pytest.raises(NeedleError) as e:
        rt.step(SMALL.vocab)
    assert e.value.code == "INVALID_CACT"
    rt.step(1, want_logits=False)
    rt.step(2, want_logits=False)
    with pytest.raises(NeedleError) as e:
        rt.step(3)
    assert e.value.code == "CONTEXT_OVERFLOW"
    with pytest.raises(NeedleError) as e:
        rt.prefill([])
    assert e.value.code == "INVALID_CACT"
    rt.reset(5)
    with pytest.raises(NeedleError) as e:
        rt.step_selected(4, np.array([1, SMALL.vocab], np.uint32))
    assert e.value.code == "INVALID_CACT"


def test_fused_wait_that_runs_out_is_reported_until_reset(small):
    """The fused layer launch's bounded waits, made to run out from the host
    (the test hook has the mix wait for one more output-projection workgroup
    than the launch has, every wait bounded at 64 sleep rounds): step,
    step_selected, a prefill whose slots wrap (stepped positions) and
    generate each return BACKEND_UNAVAILABLE naming the wait, and every
    kernel exits (the calls return).  The status stays set after the hook is
    cleared until reset() clears it; then steps agree with the oracle."""
    w, model = small
    res = model.resident
    rt = model.create_resident_runtime()
    tokens = synth.Stream(8, "n2waits").integers(14, 0, SMALL.vocab - 1)
    say("needle2 fused wait runs out")
    try:
        res.test_waits(1, 64)
        calls = (("step", lambda: rt.step(int(tokens[0]))),
                 ("step_selected", lambda: rt.step_selected(int(tokens[0]))),
                 ("prefill", lambda: rt.prefill([int(t) for t in tokens[:12]])),
                 ("generate", lambda: res.generate([int(t) for t in tokens[:4]], 3)))
        for name, call in calls:
            rt.reset(SMALL.max_length, 0)
            with pytest.raises(NeedleError) as e:
                call()
            assert e.value.code == "BACKEND_UNAVAILABLE", name
            assert "output projection rows" in str(e.value), (name, str(e.value))
        res.test_waits(0, 0)
        with pytest.raises(NeedleError) as e:  # still set: no reset since
            rt.step(int(tokens[1]))
        assert e.value.code == "BACKEND_UNAVAILABLE"
    finally:
        res.test_waits(0, 0)
    rt.reset(SMALL.max_length, 0)
    ref = oracle.Needle2(w).runtime(SMALL.max_length, 0)
    for i, t in enumerate(tokens):
        close(rt.step(int(t)), ref.step(int(t)), ("after reset", i))
    ids, _ = res.generate([int(t) for t in tokens[:4]], 3, eos=None)
    ref = oracle.Needle2(w).runtime(7, 0)
    for t in tokens[:4]:
        logits = ref.step(int(t))
    want = []
    for k in range(3):
        want.append(oracle.argmax(logits))
        if k < 2:
            logits = ref.step(want[-1])
    assert list(ids) == want


def test_generate_full_geometry_greedy_identical(hip):
    """The shipped geometry (27 layers, vocab 8192, window 256): 128 prompt
    tokens, 64 greedy tokens, identical to the oracle's greedy sequence."""
    say("needle2 generate full geometry")
    g = Needle2Geometry()
    w = Needle2Weights(g, 2026)
    model = NeedleModel(hip, w)
    try:
        prompt = synth.Stream(2026, "needle2.prompt").integers(128, 0, g.vocab - 1)
        res = model.generate_resident(prompt, max_new_tokens=64, eos=None)
        ref = oracle.Needle2(w).runtime(128 + 64, 0)
        ref.capture_kv(0, 128 + 64)
        for t in prompt[:-1]:
            ref.step(int(t), want_logits=False)
        logits = ref.step(int(prompt[-1]))
        ids, lps = [], []
        for k in range(64):
            tok = oracle.argmax(logits)
            ids.append(tok)
            lps.append(oracle.log_softmax_at(logits, tok))
            if k + 1 < 64:
                logits = ref.step(tok)
        assert res.token_ids == ids
        np.testing.assert_allclose(res.token_log_probabilities, lps, rtol=1e-3, atol=1e-3)
        # 128 prompt positions and 63 generated ones were stored (the last
        # generated token is never run), over the 256-position window.
        check_kv(model, ref, g, 128 + 63, 0, "generate")
        # the graph-replayed steps pooled every token they ran
        close_confidence(model.resident.confidence(), ref.confidence(), "generate confidence")
        # one launch per layer (Wo, mix, projection and attention together)
        # plus begin, the engram launches, the final mix, lm head, selection
        # and the pool
        assert model.resident.step_launches() == 2 + len(g.sites) + g.layers + 3 + 1
    finally:
        model.dispose()


@pytest.mark.parametrize("cq_bits,sink,group", [(4, 3, 32), (3, 0, 32), (2, 0, 32), (5, 3, 32),
                                                ("mixed", 3, 32), ("mixed", 0, 32), (4, 0, 16),
                                                (3, 3, 8)])
def test_cactus_quant_model_steps_prefill_and_generate(hip, cq_bits, sink, group):
    """The resident runtime over Cactus-Quant matrices, the form every matrix
    of the shipped archive takes (model/cact.ts:398-562, backends/cq.ts:106-295),
    one width for every matrix or each matrix its own width and group
    (mixed: every width on every kind of matrix across the layers): step
    logits, the cache and the confidence against the oracle's cqMatvec /
    dequantizeCqRow restatement, a prompt (one batched pass while its cache
    slots do not wrap, steps after) and a greedy continuation with identical
    ids.  Groups of 8 and 16 put several groups in each 32-code unit."""
    say("needle2 cactus-quant", cq_bits, sink, group)
    w = Needle2Weights(SMALL, 51, cq_bits=cq_bits, cq_group=group)
    model = NeedleModel(hip, w)
    try:
        rt = model.create_resident_runtime()
        rt.reset(SMALL.max_length, sink)
        ref = oracle.Needle2(w).runtime(SMALL.max_length, sink)
        ref.capture_kv(0, SMALL.max_length)
        tokens = synth.Stream(6, f"cq{cq_bits}").integers(14, 0, SMALL.vocab - 1)
        tokens[8:10] = tokens[2:4]  # repeated n-grams hit the same engram rows
        for i, t in enumerate(tokens):
            close(rt.step(int(t)), ref.step(int(t)), ("cq step", cq_bits, i))
        close_confidence(rt.resolve_confidence(), ref.confidence(), ("cq confidence", cq_bits))
        check_kv(model, ref, SMALL, len(tokens), sink, f"cq{cq_bits} steps")
        # A prompt and greedy tokens through the generate path (graph replays).
        prompt = synth.Stream(7, f"cqp{cq_bits}").integers(12, 0, SMALL.vocab - 1)
        res = model.generate_resident(prompt, max_new_tokens=10, eos=None)
        ref2 = oracle.Needle2(w).runtime(12 + 10, 0)
        for t in prompt[:-1]:
            ref2.step(int(t), want_logits=False)
        logits = ref2.step(int(prompt[-1]))
        ids = []
        for k in range(10):
            tok = oracle.argmax(logits)
            ids.append(tok)
            if k + 1 < 10:
                logits = ref2.step(tok)
        assert res.token_ids == ids, (cq_bits, res.token_ids, ids)
    finally:
        model.dispose()


@pytest.mark.parametrize("bits", [4, 5, "mixed"])
def test_cact_archive_through_the_resident_runtime(hip, bits):
    """A .cact archive in the shipped layout (synthetic weights, the
    reference's tensor order) parsed by parse_cact_weights and run as is --
    Cactus-Quant matrices, its geometry, its confidence head: step logits and
    confidence against the oracle on the same archive, then a greedy
    generate."""
    from needle_hip.cact import parse_cact_weights, synthetic_needle2_archive
    from needle_hip.needle2 import weights_from_cact

    say("needle2 cact archive", bits)
    geo = dict(kv_window=8, kv_bits=8, vocabulary_size=512, model_dimension=128,
               number_of_heads=4, number_of_kv_heads=2, number_of_layers=3, head_dimension=64,
               maximum_sequence_length=48, hadamard_dimension=256, mhc_lanes=4,
               engram_slots=64, engram_sub_dimension=128, number_of_engram_tables=4,
               engram_convolution_taps=4, engram_convolution_dilation=1,
               engram_orders=[2, 3], engram_layers=[0, 2], rope_theta=10000.0)
    archive = (synthetic_needle2_archive(geo, 17, mixed=True) if bits == "mixed"
               else synthetic_needle2_archive(geo, 17, bits=bits))
    w = weights_from_cact(parse_cact_weights(archive))
    g = w.geometry
    model = NeedleModel(hip, w)
    try:
        rt = model.create_resident_runtime()
        rt.reset(g.max_length, 2)
        ref = oracle.Needle2(w).runtime(g.max_length, 2)
        tokens = synth.Stream(9, f"cact{bits}").integers(12, 0, g.vocab - 1)
        for i, t in enumerate(tokens):
            close(rt.step(int(t)), ref.step(int(t)), ("archive step", bits, i))
        close_confidence(rt.resolve_confidence(), ref.confidence(), ("archive confidence", bits))
        prompt = synth.Stream(10, f"cactp{bits}").integers(10, 0, g.vocab - 1)
        res = model.generate_resident(prompt, max_new_tokens=8, eos=None)
        ref2 = oracle.Needle2(w).runtime(10 + 8, 0)
        for t in prompt[:-1]:
            ref2.step(int(t), want_logits=False)
        logits = ref2.step(int(prompt[-1]))
        ids = []
        for k in range(8):
            ids.append(oracle.argmax(logits))
            if k + 1 < 8:
                logits = ref2.step(ids[-1])
        assert res.token_ids == ids
    finally:
        model.dispose()


def test_generate_full_geometry_mixed_width_greedy_identical(hip):
    """The shipped geometry with every matrix in its own Cactus-Quant width
    and group (the mixed archive's form): 128 prompt tokens and 64 greedy
    tokens identical to the oracle's, log-probabilities within 1e-3, the
    cache and the confidence within their bars."""
    say("needle2 generate full geometry mixed widths")
    g = Needle2Geometry()
    w = Needle2Weights(g, 2027, cq_bits="mixed")
    model = NeedleModel(hip, w)
    try:
        prompt = synth.Stream(2027, "needle2.prompt").integers(128, 0, g.vocab - 1)
        res = model.generate_resident(prompt, max_new_tokens=64, eos=None)
        ref = oracle.Needle2(w).runtime(128 + 64, 0)
        ref.capture_kv(0, 128 + 64)
        for t in prompt[:-1]:
            ref.step(int(t), want_logits=False)
        logits = ref.step(int(prompt[-1]))
        ids, lps = [], []
        for k in range(64):
            tok = oracle.argmax(logits)
            ids.append(tok)
            lps.append(oracle.log_softmax_at(logits, tok))
            if k + 1 < 64:
                logits = ref.step(tok)
        assert res.token_ids == ids
        np.testing.assert_allclose(res.token_log_probabilities, lps, rtol=1e-3, atol=1e-3)
        check_kv(model, ref, g, 128 + 63, 0, "mixed generate")
        close_confidence(model.resident.confidence(), ref.confidence(), "mixed confidence")
    finally:
        model.dispose()


def test_cactus_quant_model_rejects_mixed_forms(hip):
    """Every matrix of a model takes one form: a Cactus-Quant embedding with
    an int8 projection is refused with the matrix named."""
    w = Needle2Weights(SMALL, 52, cq_bits=4)
    w.wq[1] = Needle2Weights(SMALL, 52).wq[1]
    model = NeedleModel(hip, w)
    try:
        with pytest.raises(NeedleError) as e:
            model.create_resident_runtime()
        assert "wq" in str(e.value) and "Cactus-Quant" in str(e.value)
    finally:
        model.dispose()


def test_confidence_absent_or_disabled(hip):
    say("needle2 confidence disabled")
    w = Needle2Weights(SMALL, 32)
    model = NeedleModel(hip, w, collect_confidence=False)
    try:
        rt = model.create_resident_runtime()
        rt.reset(8)
        rt.step(3)
        assert rt.resolve_confidence() is None
        import ctypes as C
        out = C.c_double()
        st = hip.lib.nd_needle_confidence(hip.ctx, model.resident.handle, C.byref(out))
        assert st != 0 and b"collectConfidence" in hip.lib.nd_last_error(hip.ctx)
    finally:
        model.dispose()


@pytest.mark.parametrize("window,sink,n_prompt,max_length,cq_bits",
                         [(0, 0, 40, 64, 0), (16, 3, 30, 64, 0), (8, 0, 33, 64, 0),
                          (0, 0, 280, 300, 0), (128, 3, 100, 160, 0), (16, 3, 30, 64, 4),
                          (0, 0, 280, 300, 4), (8, 0, 33, 64, 5)])
def test_batched_prefill_then_steps(hip, window, sink, n_prompt, max_length, cq_bits):
    """Prompt positions whose cache slots do not wrap run as one batched pass
    (int8 MFMA projections, or the Cactus-Quant matvec over the batch's rows
    for a CQ model; one mix workgroup per position), the rest as steps;
    logits, every appended KV row and the engram ring handed to the following
    steps must agree with the oracle's sequential steps (the 300-position
    case batches a prompt longer than one attention chunk; the 100-token
    prompt under a 128-position window with 3 sinks runs the query-block
    attention of a windowed cache with sinks)."""
    say("needle2 batched prefill", window, sink, n_prompt, max_length, cq_bits)
    g = Needle2Geometry(**{**SMALL.__dict__, "kv_window": window, "max_length": max_length})
    w = Needle2Weights(g, 41, cq_bits=cq_bits)
    model = NeedleModel(hip, w)
    try:
        rt = model.create_resident_runtime()
        rt.reset(g.max_length, sink)
        ref = oracle.Needle2(w).runtime(g.max_length, sink)
        ref.capture_kv(0, g.max_length)
        prompt = synth.Stream(12, f"n2pf{window}").integers(n_prompt, 0, g.vocab - 1)
        prompt[10:13] = prompt[2:5]
        got = rt.prefill(prompt)
        for t in prompt:
            want = ref.step(int(t))
        close(got, want, "prefill logits")
        close_confidence(rt.resolve_confidence(), ref.confidence(), "batched prefill confidence")
        check_kv(model, ref, g, n_prompt, sink, "batched prefill")
        tok = int(np.argmax(got))
        for i in range(6):  # steps after the batch read its engram ring and cache
            want = ref.step(tok)
            got = rt.step(tok)
            close(got, want, ("step after prefill", i))
            tok = int(np.argmax(want))
        close_confidence(rt.resolve_confidence(), ref.confidence(), "confidence after steps")
    finally:
        model.dispose()
