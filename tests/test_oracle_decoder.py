"""Pins the oracle's synthetic decoder and its seeded generators.

The decoder step is checked against an independent float64 numpy model of
the layer recipe (dense matrices, vectorized norms, complex-number RoPE,
softmax attention over the dequantized cache), which catches wiring mistakes
(a swapped operand, a missing residual, a wrong norm) that re-reading the C
code would not.  The generators are checked against numpy implementations of
the same integer spec, and the batch driver against sequential single steps.
"""

import numpy as np
import pytest

import oracle
from helpers import assert_close
from needle_hip import synth
from needle_hip.models import (MASK_THRESHOLD24, PREFIX_SCALE, ConstrainedWorkload,
                               DecoderGeometry, DecoderWeights)


def np_mask(seed, vocab, thr):
    z = synth.splitmix64(seed, vocab + 1)
    bits = (z[:vocab] >> np.uint64(40)) < np.uint64(thr)
    forced = int((int(z[vocab]) >> 32) * vocab >> 32)
    bits[forced] = True
    return synth.pack_bits(bits[None, :])[0]


def test_generators_match_numpy_spec():
    for seed in (0, 1, 12345678901234567):
        assert oracle.splitmix64_at(seed, 7) == int(synth.splitmix64(seed, 8)[7])
        m = oracle.gen_mask(seed, 3000, MASK_THRESHOLD24)
        assert np.array_equal(m, np_mask(seed, 3000, MASK_THRESHOLD24))
    bits = synth.unpack_bits(oracle.gen_mask(99, 32768, MASK_THRESHOLD24)[None, :], 32768)
    assert 0.015 < bits.mean() < 0.025
    codes, scale = oracle.gen_kv_row(5, 3, 64, 0.005, 0.02)
    z = synth.splitmix64(5, 65, offset=3 * 65)
    expect = (((z[:64] >> np.uint64(32)) * np.uint64(255)) >> np.uint64(32)).astype(np.int64) - 127
    assert codes.tolist() == expect.tolist()
    u = float(int(z[64]) >> 40) * 2.0 ** -24
    lo, hi = float(np.float32(0.005)), float(np.float32(0.02))  # f32 parameters
    assert scale == np.float32(lo + (hi - lo) * u)


def dense(m):
    return m.codes.astype(np.float64) * m.scales.astype(np.float64)


def numpy_step(w, cache_k, cache_v, token, position):
    """Float64 model of one decoder step; cache_* are per-layer lists of
    [positions][kv_heads][64] arrays of dequantized rows (appended here)."""
    g = w.geometry

    def rms(x, s):
        return (1 + s.astype(np.float64)) * x / np.sqrt(np.mean(x * x) + 1e-6)

    def rope(v, heads):
        v = v.reshape(heads, 64)
        j = np.arange(32)
        ang = position * float(np.float32(g.rope_theta)) ** (-(2 * j) / 64)
        z = (v[:, :32] + 1j * v[:, 32:]) * np.exp(1j * ang)
        return np.concatenate([z.real, z.imag], axis=1)

    x = dense(w.embedding)[token] * np.sqrt(g.dim)
    for l in range(g.layers):
        a = rms(x, w.attn_norm[l])
        q = (dense(w.wq[l]) @ a).reshape(g.heads, 64)
        k = (dense(w.wk[l]) @ a).reshape(g.kv_heads, 64)
        v = (dense(w.wv[l]) @ a).reshape(g.kv_heads, 64)
        q = rope(np.stack([rms(h, w.q_norm[l]) for h in q]), g.heads)
        k = rope(np.stack([rms(h, w.k_norm[l]) for h in k]), g.kv_heads)
        kq = [oracle.kv_quantize(k[h].astype(np.float32)) for h in range(g.kv_heads)]
        vq = [oracle.kv_quantize(v[h].astype(np.float32)) for h in range(g.kv_heads)]
        cache_k[l].append(np.stack([c.astype(np.float64) * s for c, s in kq]))
        cache_v[l].append(np.stack([c.astype(np.float64) * s for c, s in vq]))
        K = np.stack(cache_k[l])  # [t][kvh][64]
        V = np.stack(cache_v[l])
        rep = g.heads // g.kv_heads
        o = np.zeros((g.heads, 64))
        for h in range(g.heads):
            sc = K[:, h // rep] @ q[h] / 8.0
            p = np.exp(sc - sc.max())
            o[h] = (p / p.sum()) @ V[:, h // rep]
        x = x + dense(w.wo[l]) @ o.reshape(-1)
        f = rms(x, w.ffn_norm[l])
        u = dense(w.wup[l]) @ f
        x = x + dense(w.wdown[l]) @ (u / (1 + np.exp(-u)))
    return dense(w.embedding) @ rms(x, w.final_norm)


@pytest.mark.parametrize("kv_heads", [4, 2])
def test_step_matches_float64_model(kv_heads):
    g = DecoderGeometry(layers=2, dim=256, heads=4, kv_heads=kv_heads, ffn=512, vocab=1024)
    w = DecoderWeights(g, 3)
    m = oracle.SynthDecoder(w)
    cache = m.new_cache(16)
    ck = [[] for _ in range(g.layers)]
    cv = [[] for _ in range(g.layers)]
    for pos, tok in enumerate([5, 900, 17, 17, 300]):
        got = m.step(cache, tok, pos)
        ref = numpy_step(w, ck, cv, tok, pos)
        # The model rounds to f32 between ops and requantizes K/V from its own
        # f32 values, so the float64 model agrees to ~1e-5 relative.
        assert_close(got, ref, rtol=2e-4, atol=2e-3, what=f"step {pos}")


def test_batch_driver_equals_sequential_steps():
    g = DecoderGeometry(layers=2, dim=256, heads=4, kv_heads=4, ffn=512, vocab=2048)
    w = DecoderWeights(g, 4)
    m = oracle.SynthDecoder(w)
    wl = ConstrainedWorkload(batch=3, steps=4, min_context=2, max_context=20, vocab=g.vocab)
    lengths, starts = wl.lengths, wl.start_tokens

    def caches():
        out = []
        for b in range(wl.batch):
            c = m.new_cache(wl.max_length)
            kseed, vseed = wl.kv_seeds(b)
            oracle.kv_fill_synthetic(c, kseed, vseed, int(lengths[b]), *PREFIX_SCALE)
            out.append(c)
        return out

    ids, lps = m.decode_batch(caches(), starts, lengths, wl.steps, wl.mask_seed,
                              MASK_THRESHOLD24, threads=2)
    ids1, _ = m.decode_batch(caches(), starts, lengths, wl.steps, wl.mask_seed,
                             MASK_THRESHOLD24, threads=1)
    assert np.array_equal(ids, ids1)
    cs = caches()
    for b in range(wl.batch):
        tok = int(starts[b])
        for t in range(wl.steps):
            logits = m.step(cs[b], tok, int(lengths[b]) + t)
            mask = oracle.gen_mask(oracle.splitmix64_at(wl.mask_seed, t * 65536 + b), g.vocab,
                                   MASK_THRESHOLD24)
            tok, lp = oracle.select_mask(logits, mask)
            assert tok == ids[t, b] and lp == lps[t, b]
            assert synth.unpack_bits(mask[None, :], g.vocab)[0, tok]


def _bits(a):
    return a.view(np.uint32) if a.dtype == np.float32 else a.view(np.uint8)


@pytest.mark.parametrize("position0,threads", [(0, 1), (0, 3), (5, 4)])
def test_prefill_is_bit_identical_to_sequential_steps(position0, threads):
    """or_synth_prefill evaluates layer by layer on several threads; it must
    equal the same tokens run through step() one at a time: last logits,
    every K/V code and scale, and every captured pre-quantization vector."""
    g = DecoderGeometry(layers=3, dim=256, heads=4, kv_heads=2, ffn=512, vocab=1024)
    w = DecoderWeights(g, 9)
    m = oracle.SynthDecoder(w)
    toks = synth.Stream(7, "prefill-toks").integers(40, 0, g.vocab - 1)
    lead = synth.Stream(8, "prefill-lead").integers(position0, 0, g.vocab - 1)
    seq, par = m.new_cache(64), m.new_cache(64)
    for c in (seq, par):
        c.capture(0)
        for p, t in enumerate(lead):
            m.step(c, int(t), p)
    for i, t in enumerate(toks):
        want = m.step(seq, int(t), position0 + i)
    got = m.prefill(par, toks, position0, threads=threads)
    assert np.array_equal(_bits(got), _bits(want))
    n = position0 + len(toks)
    for layer in range(g.layers):
        for h in range(g.kv_heads):
            for a, b in zip(par.read(layer, h), seq.read(layer, h)):
                assert np.array_equal(_bits(a), _bits(b))
            for a, b in zip(par.read_raw(layer, h, 0, n), seq.read_raw(layer, h, 0, n)):
                assert np.array_equal(_bits(a), _bits(b))


def test_prefill_rejects_positions_past_the_cache():
    g = DecoderGeometry(layers=1, dim=256, heads=4, kv_heads=4, ffn=512, vocab=512)
    m = oracle.SynthDecoder(DecoderWeights(g, 1))
    with pytest.raises(oracle.OracleError):
        m.prefill(m.new_cache(8), np.arange(9), 0)
    with pytest.raises(oracle.OracleError):
        m.prefill(m.new_cache(8), [600], 0)


def test_captured_vectors_are_the_stored_inputs_and_requantize_to_the_codes():
    cache = oracle.KvCache(2, 3, max_length=20)
    cache.capture(4)
    s = synth.Stream(3, "capture")
    K, V = s.normal((20, 3, 64)), s.normal((20, 3, 64))
    cache.store(1, 0, K, V)
    for h in range(3):
        rk, rv = cache.read_raw(1, h, 4, 16)
        assert np.array_equal(rk, K[4:, h]) and np.array_equal(rv, V[4:, h])
        kc, vc, ks, vs = cache.read(1, h)
        for p in range(4, 20):
            c, sc = oracle.kv_quantize(rk[p - 4])
            assert np.array_equal(c, kc[p]) and sc == ks[p]
    with pytest.raises(oracle.OracleError):
        cache.read_raw(1, 0, 3, 2)  # before the capture start


def test_decode_checkpoint_logits_equal_the_step_logits():
    g = DecoderGeometry(layers=2, dim=256, heads=4, kv_heads=4, ffn=512, vocab=2048)
    w = DecoderWeights(g, 4)
    m = oracle.SynthDecoder(w)
    wl = ConstrainedWorkload(batch=2, steps=3, min_context=2, max_context=20, vocab=g.vocab)
    lengths, starts = wl.lengths, wl.start_tokens

    def caches():
        out = []
        for b in range(wl.batch):
            c = m.new_cache(wl.max_length)
            oracle.kv_fill_synthetic(c, *wl.kv_seeds(b), int(lengths[b]), *PREFIX_SCALE)
            out.append(c)
        return out

    ids, _, chk = m.decode_batch(caches(), starts, lengths, wl.steps, wl.mask_seed,
                                 MASK_THRESHOLD24, threads=2, check_steps=[0, 2])
    cs = caches()
    for b in range(wl.batch):
        tok = int(starts[b])
        for t in range(wl.steps):
            logits = m.step(cs[b], tok, int(lengths[b]) + t)
            if t in (0, 2):
                assert np.array_equal(_bits(chk[[0, 2].index(t), b]), _bits(logits))
            tok = int(ids[t, b])
