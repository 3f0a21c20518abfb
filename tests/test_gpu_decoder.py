"""GPU parity of the int8-MFMA batched matvec and the batched constrained
decoder against the oracle, through the C ABI.

Bars: matmul outputs within 1e-3 relative / 1e-4 absolute elementwise;
selected ids (greedy, masked) identical at every step; synthetic prefix KV
bit-exact; logits within 1e-3 relative both normwise and elementwise against
the step's largest logit; log-probabilities within 0.05 absolute (the
full-size workload measures 0.034 at logits up to ~146).  Appended K/V
codes:

* layer 0, whose inputs are the token's embedding on both sides: equal to the
  oracle's, or one apart with the oracle's quotient x / s within 1e-4 of the
  rounding boundary between them;
* the last layer: equal to the oracle's #storeKV of the GPU's own
  last-layer projections of that step (keys up to boundary flips within
  1e-5, values bit-exact) -- the codes are the correct rounding of what the
  GPU computed;
* every layer: at most one code from the oracle's (deeper layers see
  drifted inputs, see test_gpu_prefill), on at most 1% of a layer's
  appended codes.
"""

import ctypes as C
import os
import sys

import numpy as np
import pytest

import oracle
from helpers import (assert_close, assert_codes_or_boundary_flips, read_device,
                     storekv_of_projections)
from needle_hip import Int8Matrix, NeedleError, synth
from needle_hip import lib as L
from needle_hip.models import (MASK_THRESHOLD24, PREFIX_SCALE, ConstrainedWorkload,
                               DecoderGeometry, DecoderWeights, HipBatch, HipDecoder)

pytestmark = pytest.mark.gpu
RTOL, ATOL = 1e-3, 1e-4
THREADS = min(16, os.cpu_count() or 1)


def say(*args):
    print("[case]", *args, file=sys.stderr, flush=True)


def batch_cache(hip, gpu, g):
    """The whole batch cache in one copy: K, V codes [layers][batch][kv_heads]
    [alloc][64] and scales [layers][batch][kv_heads][alloc]."""
    kv = hip.lib.nd_batch_kv(gpu.handle)
    alloc = C.c_uint32()
    kp, vp, ksp, vsp = C.c_void_p(), C.c_void_p(), C.c_void_p(), C.c_void_p()
    hip._check(hip.lib.nd_kv_info(kv, C.byref(alloc), C.byref(kp), C.byref(vp), C.byref(ksp),
                                  C.byref(vsp)))
    shape = (g.layers, gpu.batch, g.kv_heads, alloc.value)
    return (read_device(kp, shape + (64,), np.int8), read_device(vp, shape + (64,), np.int8),
            read_device(ksp, shape, np.float32), read_device(vsp, shape, np.float32))


def check_logits(got, want, what):
    g64, w64 = got.astype(np.float64), want.astype(np.float64)
    assert np.linalg.norm(g64 - w64) <= 1e-3 * np.linalg.norm(w64), what
    assert np.abs(g64 - w64).max() <= 1e-3 * np.abs(w64).max(), what


def check_last_layer(weights, ref_theta, proj, kc, vc, ks, vs, positions, what):
    """Codes the GPU stored for the last layer at `positions` (one per
    sequence) against the oracle's #storeKV of the GPU's projections."""
    g = weights.geometry
    last = g.layers - 1
    k, _, tk, tks, tv, tvs = storekv_of_projections(proj, g.heads, g.kv_heads,
                                                    weights.k_norm[last], ref_theta, positions)
    for b, p in enumerate(positions):
        assert_codes_or_boundary_flips(kc[last, b, :, p], tk[b], k[b], 1e-5, f"{what} keys b={b}")
        np.testing.assert_allclose(ks[last, b, :, p], tks[b], rtol=1e-6)
        assert np.array_equal(vc[last, b, :, p], tv[b]), f"{what} values b={b}"
        assert np.array_equal(vs[last, b, :, p].view(np.uint32), tvs[b].view(np.uint32))


def check_appended(caches, lengths, steps, kc, vc, ks, vs, g, what):
    """Appended rows [len_b, len_b + steps) of every sequence against the
    oracle's (which captured its pre-quantization vectors)."""
    differ = np.zeros(g.layers, np.int64)
    total = 0
    for b, c in enumerate(caches):
        p0 = int(lengths[b])
        for l in range(g.layers):
            for h in range(g.kv_heads):
                rk, rv, rks, rvs = c.read(l, h)
                raw_k, raw_v = c.read_raw(l, h, p0, steps)
                for got, want, raw in ((kc[l, b, h, p0:p0 + steps], rk[p0:p0 + steps], raw_k),
                                       (vc[l, b, h, p0:p0 + steps], rv[p0:p0 + steps], raw_v)):
                    if l == 0:
                        assert_codes_or_boundary_flips(got, want, raw, 1e-4,
                                                       f"{what} layer 0 b={b} h={h}")
                    else:
                        d = np.abs(got.astype(int) - want.astype(int))
                        assert d.max() <= 1, (what, l, b)
                        differ[l] += int((d != 0).sum())
                    if l == 0:
                        total += got.size
    say(f"[measure] {what}: codes differing per layer {differ.tolist()} of {total}")
    assert (differ <= 0.01 * total).all(), (what, differ.tolist(), total)


def matmul(hip, m, x):
    y = np.empty((x.shape[0], m.output_size), np.float32)
    hip._check(hip.lib.nd_matmul(hip.ctx, hip.upload(m), L.ptr(x), x.shape[0], L.ptr(y)))
    return y


@pytest.mark.parametrize("rows,n,k", [(1, 512, 512), (3, 1536, 512), (64, 2048, 512),
                                      (64, 512, 2048), (64, 32768, 512), (17, 1024, 128),
                                      (100, 512, 512), (2048, 512, 512), (2048, 512, 2048)])
def test_matmul_matches_oracle(hip, rows, n, k):
    say("matmul", rows, n, k)
    w, s = synth.int8_matrix(17, f"mm{n}x{k}", n, k, k)
    m = Int8Matrix(w, s, k)
    x = synth.Stream(3, f"mmx{rows}").normal((rows, k))
    # Outliers of 30x the row's RMS and denormal-scale entries in one row.  (A
    # row whose largest entry dwarfs the rest by ~1e4 defeats fp32 summation
    # as well as the 2^-22-of-row-maximum digit split, so it is not a case
    # the fp32 tolerance can speak to.)
    x[0, :5] = [1e-30, -30.0, 0.0, 7.0, -7.0]
    if rows > 2:
        x[2] = 0.0  # an all-zero row
    ref = oracle.matvec_i8(w, s, k, x)
    assert_close(matmul(hip, m, x), ref, RTOL, ATOL, f"matmul {rows}x{n}x{k}")


def test_matmul_rejects_group_scales(hip):
    w, s = synth.int8_matrix(1, "g32", 64, 512, 32)
    with pytest.raises(NeedleError) as e:
        matmul(hip, Int8Matrix(w, s, 32), np.zeros((2, 512), np.float32))
    assert e.value.code == "INVALID_CACT"


def run_case(hip, geometry, wl, seed):
    """Steps the batch one step at a time against sequential oracle steps."""
    weights = DecoderWeights(geometry, seed)
    dec = HipDecoder(hip, weights)
    gpu = HipBatch(dec, wl.batch, wl.max_length)
    ref = oracle.SynthDecoder(weights)
    theta = ref.struct.rope_theta
    lengths, tokens = wl.lengths, wl.start_tokens
    caches = []
    for b in range(wl.batch):
        ks, vs = wl.kv_seeds(b)
        gpu.fill_synthetic(b, ks, vs, int(lengths[b]), wl.max_length)
        c = ref.new_cache(wl.max_length)
        oracle.kv_fill_synthetic(c, ks, vs, int(lengths[b]), *PREFIX_SCALE)
        c.capture(int(lengths[b]), wl.steps)
        caches.append(c)
    kc, vc, kss, vss = batch_cache(hip, gpu, geometry)
    for b in (0, wl.batch - 1):  # prefix rows are generated bit-exactly on both sides
        n = int(lengths[b])
        rk, rv, rks, rvs = caches[b].read(geometry.layers - 1, 1)
        assert np.array_equal(kc[-1, b, 1, :n], rk[:n]) and np.array_equal(vc[-1, b, 1, :n], rv[:n])
        assert np.array_equal(kss[-1, b, 1, :n], rks[:n]) and np.array_equal(vss[-1, b, 1, :n], rvs[:n])
    gpu.set_state(tokens, lengths, 0)
    cur = tokens.astype(np.int64).copy()
    for t in range(wl.steps):
        gpu.step(int(lengths.max()) + t, mask_seed=wl.mask_seed)
        ids, pos, lps, logits = gpu.read(logits=True)
        proj = gpu.read_projections()
        kc, vc, kss, vss = batch_cache(hip, gpu, geometry)
        check_last_layer(weights, theta, proj, kc, vc, kss, vss, lengths.astype(np.int64) + t,
                         f"step {t}")
        for b in range(wl.batch):
            p = int(lengths[b]) + t
            want_logits = ref.step(caches[b], int(cur[b]), p)
            mask = oracle.gen_mask(oracle.splitmix64_at(wl.mask_seed, t * 65536 + b),
                                   geometry.vocab, MASK_THRESHOLD24)
            want_id, want_lp = oracle.select_mask(want_logits, mask)
            check_logits(logits[b], want_logits, (t, b))
            assert int(ids[b]) == want_id, (t, b)
            assert abs(lps[b] - want_lp) <= 0.05, (t, b, lps[b], want_lp)
            assert int(pos[b]) == p + 1
        cur = ids.astype(np.int64)
    kc, vc, kss, vss = batch_cache(hip, gpu, geometry)
    check_appended(caches, lengths, wl.steps, kc, vc, kss, vss, geometry, "appended")
    gpu.free()
    dec.free()


def test_batch_decode_small_model(hip):
    say("batch decode small")
    g = DecoderGeometry(layers=2, vocab=4096)
    wl = ConstrainedWorkload(batch=3, steps=6, min_context=1, max_context=300, vocab=g.vocab)
    run_case(hip, g, wl, seed=11)


def test_batch_decode_gqa_model(hip):
    say("batch decode gqa")
    g = DecoderGeometry(layers=2, heads=8, kv_heads=4, vocab=2048)
    wl = ConstrainedWorkload(batch=5, steps=4, min_context=30, max_context=700, vocab=g.vocab)
    run_case(hip, g, wl, seed=12)


def test_batch_decode_full_geometry(hip):
    say("batch decode full geometry")
    g = DecoderGeometry()  # 8 layers, d 512, 8x64, FFN 2048, vocab 32768
    wl = ConstrainedWorkload(batch=4, steps=3, min_context=32, max_context=2048, vocab=g.vocab)
    run_case(hip, g, wl, seed=2026)


def test_constrained_decode_full_size(hip):
    """The constrained decode workload at its own size: 64 sequences with
    contexts U{32..2048}, vocab 32768, a ~2% allowed bitmask per sequence per
    step, 128 greedy steps.  The oracle runs the 64 sequences on host
    threads (decode_batch, equal to sequential steps, pinned on the CPU);
    logits are compared at five steps, ids and log-probabilities at all."""
    say("constrained decode 64 x 128")
    g = DecoderGeometry()
    steps = 128
    checks = [0, 1, 15, 63, 127]
    weights = DecoderWeights(g, 2026)
    wl = ConstrainedWorkload(batch=64, steps=steps, min_context=32, max_context=2048,
                             vocab=g.vocab)
    dec = HipDecoder(hip, weights)
    gpu = HipBatch(dec, wl.batch, wl.max_length)
    ref = oracle.SynthDecoder(weights)
    lengths, starts = wl.lengths, wl.start_tokens
    caches = []
    for b in range(wl.batch):
        ks, vs = wl.kv_seeds(b)
        gpu.fill_synthetic(b, ks, vs, int(lengths[b]), wl.max_length)
        c = ref.new_cache(wl.max_length)
        oracle.kv_fill_synthetic(c, ks, vs, int(lengths[b]), *PREFIX_SCALE)
        c.capture(int(lengths[b]), steps)
        caches.append(c)
    gpu.set_state(starts, lengths, 0)
    got_logits = {}
    projections = []
    for t in range(steps):
        gpu.step(int(lengths.max()) + t, mask_seed=wl.mask_seed)
        if t in checks:
            got_logits[t] = gpu.read(logits=True)[3]
        projections.append(gpu.read_projections())
    ids, lps = gpu.history(0, steps)
    kc, vc, kss, vss = batch_cache(hip, gpu, g)
    want_ids, want_lps, want_logits = ref.decode_batch(
        caches, starts, lengths, steps, wl.mask_seed, MASK_THRESHOLD24, threads=THREADS,
        check_steps=checks)
    mism = np.argwhere(ids != want_ids)
    assert mism.size == 0, f"{len(mism)} ids differ, first (step, seq) {mism[:3].tolist()}"
    say(f"[measure] log-probability max |error| {float(np.abs(lps - want_lps).max()):.4f}")
    assert np.abs(lps - want_lps).max() <= 0.05
    for i, t in enumerate(checks):
        for b in range(wl.batch):
            check_logits(got_logits[t][b], want_logits[i, b], (t, b))
    # The last step's last-layer projections survive in the workspace; earlier
    # steps' were read after each step.
    theta = ref.struct.rope_theta
    for t, proj in enumerate(projections):
        check_last_layer(weights, theta, proj, kc, vc, kss, vss, lengths.astype(np.int64) + t,
                         f"step {t}")
    check_appended(caches, lengths, steps, kc, vc, kss, vss, g, "appended")
    gpu.free()
    dec.free()


def test_batch_rejects_bad_state(hip):
    g = DecoderGeometry(layers=1, vocab=1024)
    dec = HipDecoder(hip, DecoderWeights(g, 1))
    b = HipBatch(dec, 2, 16)
    with pytest.raises(NeedleError) as e:
        b.set_state([1, 2], [3, 16])
    assert e.value.code == "CONTEXT_OVERFLOW"
    with pytest.raises(NeedleError) as e:
        b.set_state([1, 5000], [0, 0])
    assert e.value.code == "INVALID_CACT"
    with pytest.raises(NeedleError):
        b.step(16)
    b.free()
    dec.free()
