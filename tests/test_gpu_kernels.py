"""GPU parity of the four hot-path kernels against the oracle, through the C ABI.

Bars: int8 KV codes, scales and selected ids bit-exact; matvec and attention
outputs within 1e-3 relative / 1e-4 absolute (|gpu - ref| <= 1e-4 + 1e-3|ref|);
log-probabilities within 1e-9 relative (float64 on both sides).
"""

import json
import math
import sys
from pathlib import Path

import numpy as np
import pytest

import oracle
from helpers import DeviceArray, assert_close
from needle_hip import HipKvCache, Int8Matrix, MatrixRowRange, MatvecRequest, NeedleError
from needle_hip import synth

pytestmark = pytest.mark.gpu
GOLDEN = Path(__file__).resolve().parent / "golden"
RTOL, ATOL = 1e-3, 1e-4


def say(*args):
    print("[case]", *args, file=sys.stderr, flush=True)


def matrix(seed, n, k, g):
    w, s = synth.int8_matrix(seed, f"w{n}x{k}g{g}", n, k, g)
    return Int8Matrix(w, s, g)


# ------------------------------------------------------------------ matvec

@pytest.mark.parametrize("n,k,g,batch", [
    (4096, 4096, 32, 1), (4096, 4096, 32, 8),      # isolated matvec workload
    (512, 512, 512, 1), (256, 512, 512, 3), (2048, 512, 512, 1), (512, 2048, 2048, 2),
    (8192, 512, 512, 1), (32768, 512, 512, 1), (100, 128, 32, 5), (33, 8192, 64, 4),
    (1, 1024, 1024, 1), (7, 256, 16, 8),
])
def test_matvec_matches_oracle(hip, n, k, g, batch):
    say("matvec", n, k, g, batch)
    m = matrix(11, n, k, g)
    x = synth.Stream(5, f"x{k}b{batch}").normal((batch, k))
    got = hip.matvec(m, x)
    ref = oracle.matvec_i8(m.codes, m.scales, g, x)
    assert_close(got, ref, RTOL, ATOL, f"matvec {n}x{k} g{g} b{batch}")


def test_matvec_batched_magnitudes_ranges_and_chunks(hip):
    """Batches run on MFMA with each input row split around its own largest
    element: rows of very different magnitude, an all-zero row, elements
    spread over six decades, a row range and a batch above eight."""
    say("matvec batched magnitudes")
    m = matrix(13, 600, 1024, 32)
    s = synth.Stream(9, "xmag")
    x = s.normal((12, 1024))
    x[1] *= 1e-6
    x[2] *= 1e4
    x[3] = 0.0
    x[4] *= np.power(10.0, s.uniform((1024,), -3.0, 3.0)).astype(np.float32)
    got = hip.matvec(m, x)
    assert np.all(got[3] == 0.0)
    assert_close(got, oracle.matvec_i8(m.codes, m.scales, 32, x), RTOL, ATOL, "matvec b12")
    part = hip.matvec(m, x[:3], MatrixRowRange(37, 300))
    assert_close(part, oracle.matvec_i8(m.codes, m.scales, 32, x[:3], 37, 300), RTOL, ATOL,
                 "matvec b3 rows 37..336")


def test_matvec_k_slices(hip):
    """Batches at k >= 4096 run as k-slices, each input row split around its
    largest element within the slice, and the slices summed in order: slices
    of very different magnitude, an all-zero row, groups wider than a slice
    and as wide as k, slices of 512 and of 1024, a row range, a batch above
    eight, and a row count whose partial sums take two launch pairs."""
    say("matvec k-slices magnitudes")
    m = matrix(17, 300, 4096, 32)
    s = synth.Stream(19, "xslices")
    x = s.normal((11, 4096))
    x[0, :512] *= 1e4
    x[0, 1024:1536] *= 1e-5
    x[1] = 0.0
    x[2, 512:] = 0.0
    x[5] *= np.power(10.0, s.uniform((4096,), -3.0, 3.0)).astype(np.float32)
    got = hip.matvec(m, x)
    assert np.all(got[1] == 0.0)
    assert_close(got, oracle.matvec_i8(m.codes, m.scales, 32, x), RTOL, ATOL, "slices b11")
    part = hip.matvec(m, x[:3], MatrixRowRange(5, 200))
    assert_close(part, oracle.matvec_i8(m.codes, m.scales, 32, x[:3], 5, 200), RTOL, ATOL,
                 "slices b3 rows 5..204")
    for n, k, g, batch in [(640, 4096, 1024, 3), (96, 8192, 8192, 4), (4100, 4096, 64, 5),
                           (2100, 8192, 128, 8)]:
        say("matvec k-slices", n, k, g, batch)
        mg = matrix(23, n, k, g)
        xg = synth.Stream(29, f"xs{k}").normal((batch, k))
        assert_close(hip.matvec(mg, xg), oracle.matvec_i8(mg.codes, mg.scales, g, xg), RTOL,
                     ATOL, f"slices {n}x{k} g{g} b{batch}")
    say("matvec k-slices two launch pairs")
    w, sc = synth.int8_matrix(31, "w1028x8192", 1028, 8192, 32)  # rows repeat every 1028
    big = Int8Matrix(np.tile(w, (16, 1))[:16448], np.tile(sc, (16, 1))[:16448], 32)
    xb = synth.Stream(37, "xbig").normal((3, 8192))
    got = hip.matvec(big, xb)
    assert_close(got, oracle.matvec_i8(big.codes, big.scales, 32, xb), RTOL, ATOL,
                 "slices 16448x8192 b3")


def test_matvec_ranges_and_batch_requests(hip):
    say("matvec ranges")
    m = matrix(3, 512, 512, 512)
    m2 = matrix(4, 2048, 512, 512)
    x = synth.Stream(2, "xr").normal((512,))
    full = hip.matvec(m, x)
    part = hip.matvec(m, x, MatrixRowRange(100, 37))
    assert np.array_equal(part, full[100:137])
    outs = hip.matvec_batch([MatvecRequest(m, x), MatvecRequest(m, x, MatrixRowRange(1, 1)),
                             MatvecRequest(m2, x, MatrixRowRange(8, 16))])
    assert np.array_equal(outs[0], full)
    assert np.array_equal(outs[1], full[1:2])
    assert_close(outs[2], oracle.matvec_i8(m2.codes, m2.scales, 512, x, 8, 16), RTOL, ATOL)
    with pytest.raises(NeedleError) as e:
        hip.matvec(m, x, MatrixRowRange(500, 20))
    assert e.value.code == "INVALID_CACT"
    with pytest.raises(NeedleError):
        hip.matvec(m, np.zeros(100, np.float32))


def test_row_is_bit_exact(hip):
    say("row")
    m = matrix(8, 300, 512, 32)
    for r in (0, 1, 150, 299):
        assert np.array_equal(hip.row(m, r), oracle.row_i8(m.codes, m.scales, 32, r))
    with pytest.raises(NeedleError):
        hip.row(m, 300)


# -------------------------------------------------------------- KV quantize

def test_kv_golden_vectors_bit_exact(hip):
    say("kv golden")
    cases = json.loads((GOLDEN / "kv_quant.json").read_text())
    kv = HipKvCache(hip, 1, 1, max_length=len(cases))
    for p, case in enumerate(cases):
        x = np.array(case["x"], np.float32)
        kv.store(0, p, x, -x)
    kc, vc, ks, vs = kv.read(0, 0)
    for p, case in enumerate(cases):
        assert kc[p].tolist() == case["codes"], case["name"]
        assert vc[p].tolist() == [-c for c in case["codes"]], case["name"]
        assert int(ks[p].view(np.uint32)) == case["scale_bits"], case["name"]
    kv.free()


@pytest.mark.parametrize("sigma", [1e-14, 1e-3, 1.0, 1e4])
def test_kv_store_bit_exact_random(hip, sigma):
    say("kv random", sigma)
    layers, heads, n = 2, 8, 300
    kv = HipKvCache(hip, layers, heads, max_length=n)
    ref = oracle.KvCache(layers, heads, max_length=n)
    s = synth.Stream(9, f"kv{sigma}")
    K = (s.normal((n, heads, 64)) * np.float32(sigma)).astype(np.float32)
    V = (s.normal((n, heads, 64)) * np.float32(sigma)).astype(np.float32)
    K[5, 3] = 0.0  # zero vector: 1e-12 floor
    kv.store(1, 0, K[:200], V[:200])        # bulk append
    for p in range(200, n):                  # decode appends
        kv.store(1, p, K[p], V[p])
    ref.store(1, 0, K, V)
    for h in range(heads):
        for a, b in zip(kv.read(1, h), ref.read(1, h)):
            assert np.array_equal(a.view(np.uint8) if a.dtype == np.int8 else a.view(np.uint32),
                                  b.view(np.uint8) if b.dtype == np.int8 else b.view(np.uint32))
    kv.free()


def test_kv_ring_window_and_bulk_overwrite(hip):
    say("kv ring")
    sink, window, n = 3, 5, 23
    kv = HipKvCache(hip, 1, 2, max_length=40, sink=sink, window=window)
    ref = oracle.KvCache(1, 2, max_length=40, sink=sink, window=window)
    s = synth.Stream(4, "ring")
    K, V = s.normal((n, 2, 64)), s.normal((n, 2, 64))
    kv.store(0, 0, K, V)  # one call: later positions win their ring slots
    ref.store(0, 0, K, V)
    for h in range(2):
        for a, b in zip(kv.read(0, h), ref.read(0, h)):
            assert np.array_equal(a, b)
    with pytest.raises(NeedleError) as e:
        kv.store(0, 39, np.zeros((2, 2, 64), np.float32), np.zeros((2, 2, 64), np.float32))
    assert e.value.code == "CONTEXT_OVERFLOW"
    kv.free()


# ---------------------------------------------------------------- attention

def _fill(kv, ref, layer, n, heads, seed):
    s = synth.Stream(seed, f"att{n}")
    K, V = s.normal((n, heads, 64)), s.normal((n, heads, 64))
    kv.store(layer, 0, K, V)
    ref.store(layer, 0, K, V)
    return s


@pytest.mark.parametrize("length", [512, 2048, 8192])
def test_attention_int8_mha_contexts(hip, length):
    say("attention mha", length)
    heads = 8
    kv = HipKvCache(hip, 1, heads, max_length=length)
    ref = oracle.KvCache(1, heads, max_length=length)
    s = _fill(kv, ref, 0, length, heads, 21)
    q = s.normal((heads * 64,))
    for pos in (0, 1, 63, 64, length // 2 + 3, length - 1):
        assert_close(kv.attention(0, pos, q), ref.attention(0, pos, q), RTOL, ATOL,
                     f"attention L={length} pos={pos}")
    kv.free()


def test_chunk_merges_repeat_bit_identically(hip):
    """The launches whose workgroups merge partial results through arrival
    counters -- single-row attention with each head's chunks on one XCD (8192
    positions: 32 chunks of 256 per head; 2048: 16 chunks of 128 on two-wave
    workgroups) and the batch-8 matvec's slice sum -- leave every counter at
    zero: 24 launches in a row give the same bits, which match the oracle."""
    heads = 8
    for length in (8192, 2048):
        say("attention repeat", length)
        kv = HipKvCache(hip, 1, heads, max_length=length)
        ref = oracle.KvCache(1, heads, max_length=length)
        s = _fill(kv, ref, 0, length, heads, 31)
        q = s.normal((heads * 64,))
        first = np.asarray(kv.attention(0, length - 1, q), np.float32)
        assert_close(first, ref.attention(0, length - 1, q), RTOL, ATOL, f"attention L={length}")
        for i in range(24):
            again = np.asarray(kv.attention(0, length - 1, q), np.float32)
            assert np.array_equal(again.view(np.uint32), first.view(np.uint32)), (length, i)
        kv.free()
    say("matvec batch 8 repeat")
    m = matrix(33, 4096, 4096, 32)
    x = synth.Stream(6, "repeat-x").normal((8, 4096))
    first = np.asarray(hip.matvec(m, x), np.float32)
    assert_close(first, oracle.matvec_i8(m.codes, m.scales, 32, x), RTOL, ATOL, "matvec b8")
    for i in range(24):
        again = np.asarray(hip.matvec(m, x), np.float32)
        assert np.array_equal(again.view(np.uint32), first.view(np.uint32)), ("matvec", i)


@pytest.mark.parametrize("sink,window,mode", [(0, 256, "int8"), (7, 256, "int8"), (3, 5, "int8"),
                                              (0, 0, "float32"), (4, 16, "float32")])
def test_attention_gqa_window_sink(hip, sink, window, mode):
    say("attention gqa", sink, window, mode)
    n, hkv, hq = 300, 4, 8
    kv = HipKvCache(hip, 2, hkv, max_length=n, sink=sink, window=window, kv_cache=mode)
    ref = oracle.KvCache(2, hkv, max_length=n, sink=sink, window=window, kv_cache=mode)
    s = synth.Stream(8, f"gqa{sink}{window}{mode}")
    for p in range(n):
        k, v = s.normal((hkv, 64)), s.normal((hkv, 64))
        kv.store(1, p, k, v)
        ref.store(1, p, k, v)
        if p in (0, 2, 5, 6, 100, 255, 256, 299):
            q = s.normal((hq * 64,))
            assert_close(kv.attention(1, p, q), ref.attention(1, p, q), RTOL, ATOL,
                         f"gqa pos={p}")
    kv.free()


@pytest.mark.parametrize("hkv,hq,sink,window", [(4, 8, 0, 0), (2, 8, 0, 0), (1, 8, 3, 1024),
                                                (2, 16, 0, 0), (8, 8, 5, 700)])
def test_attention_split_chunks_every_head_ratio(hip, hkv, hq, sink, window):
    """Contexts long enough to split into several chunks per KV head, for 1, 2,
    4 and 8 query heads per KV head: the cross-chunk merge at each grouping."""
    say("attention split", hkv, hq, sink, window)
    n = 1300
    kv = HipKvCache(hip, 1, hkv, max_length=n, sink=sink, window=window)
    ref = oracle.KvCache(1, hkv, max_length=n, sink=sink, window=window)
    s = synth.Stream(31, f"split{hkv}{hq}{sink}{window}")
    K, V = s.normal((n, hkv, 64)), s.normal((n, hkv, 64))
    kv.store(0, 0, K, V)
    ref.store(0, 0, K, V)
    for pos in (511, 512, 777, n - 1):
        q = s.normal((hq * 64,))
        assert_close(kv.attention(0, pos, q), ref.attention(0, pos, q), RTOL, ATOL,
                     f"split hkv={hkv} hq={hq} pos={pos}")
    kv.free()



@pytest.mark.parametrize("hq,sink,window,mode", [(8, 0, 0, "int8"), (1, 5, 40000, "int8"),
                                                 (2, 0, 0, "float32")])
def test_attention_long_context_several_tiles_per_wave(hip, hq, sink, window, mode):
    """One KV head at 50000 positions: 64 chunks of 1024 positions, so that each
    wave walks several 64-position tiles two at a time -- with an odd count in
    the last chunk (one tile of the last pair masked whole) and, with a
    window, the ring wrapping inside a chunk."""
    say("attention long", hq, sink, window, mode)
    n = 50000
    kv = HipKvCache(hip, 1, 1, max_length=n, sink=sink, window=window, kv_cache=mode)
    ref = oracle.KvCache(1, 1, max_length=n, sink=sink, window=window, kv_cache=mode)
    s = synth.Stream(77, f"long{hq}{sink}{window}{mode}")
    K, V = s.normal((n, 1, 64)), s.normal((n, 1, 64))
    kv.store(0, 0, K, V)
    ref.store(0, 0, K, V)
    for pos in (n - 1, 33000, 40100):
        q = s.normal((hq * 64,))
        assert_close(kv.attention(0, pos, q), ref.attention(0, pos, q), RTOL, ATOL,
                     f"long hq={hq} pos={pos}")
    kv.free()

# ---------------------------------------------------------------- selection

@pytest.mark.parametrize("vocab", [32768, 4096, 1000])
def test_select_mask_batch_on_device(hip, vocab):
    """Masked selection over a batch of rows in HBM (nd_select_mask_d): ids
    bit-exact and log-probabilities to 1e-9, with ties (also between the
    parts of a row split over workgroups), NaN logits inside and outside the
    allowed set, a NaN first candidate, an empty mask and half a row at -inf.
    1000 is not a multiple of 32 and takes the general kernel."""
    say("select mask batch", vocab)
    s = synth.Stream(17, f"selmask{vocab}")
    B = 8
    logits = (s.normal((B, vocab)) * 3.0).astype(np.float32)
    words = (vocab + 31) // 32
    allowed = s.uniform01(B * vocab).reshape(B, vocab) < 0.02
    allowed[:, 5] = True  # every row but the empty one has candidates
    allowed[1, 900] = True
    logits[1, [5, 900]] = 50.0  # tie: the earlier id wins
    logits[2, np.flatnonzero(allowed[2])[1]] = np.nan  # NaN candidate never wins
    logits[3, np.flatnonzero(allowed[3])[0]] = np.nan  # NaN first candidate is kept
    allowed[4] = False  # empty mask
    logits[5, np.flatnonzero(~allowed[5])[3]] = np.nan  # NaN outside: log-prob NaN
    far = vocab - 100  # in another workgroup's part of the row when the row is split
    allowed[6, [7, far]] = True
    logits[6, [7, far]] = 60.0  # tie across parts: the earlier id wins
    logits[7, :vocab // 2] = -np.inf  # parts whose maximum is -inf add nothing
    masks = np.zeros((B, words), np.uint32)
    for r in range(B):
        for i in np.flatnonzero(allowed[r]):
            masks[r, i >> 5] |= np.uint32(1 << (int(i) & 31))
    bufs = [DeviceArray(a) for a in (logits, masks, np.zeros(B, np.uint32), np.zeros(B))]
    dl, dm, ids, lps = bufs
    hip._check(hip.lib.nd_select_mask_d(hip.ctx, dl.ptr, B, vocab, dm.ptr, ids.ptr, lps.ptr, None),
               "nd_select_mask_d")
    got_ids, got_lps = ids.read(), lps.read()
    for b in bufs:
        b.free()
    for r in range(B):
        if r == 4:  # empty set: the oracle refuses it, the batch kernel flags the row
            with pytest.raises(oracle.OracleError):
                oracle.select_mask(logits[r], masks[r])
            assert int(got_ids[r]) == 0xFFFFFFFF and math.isnan(got_lps[r])
            continue
        want_id, want_lp = oracle.select_mask(logits[r], masks[r])
        assert int(got_ids[r]) == want_id, (vocab, r)
        if math.isnan(want_lp):
            assert math.isnan(got_lps[r]), (vocab, r)
        else:
            assert abs(got_lps[r] - want_lp) <= 1e-9 * max(1.0, abs(want_lp)), (vocab, r)
    assert int(got_ids[1]) == 5 and int(got_ids[4]) == 0xFFFFFFFF and int(got_ids[6]) == 7


def test_select_golden_cases(hip):
    say("select golden")
    for case in json.loads((GOLDEN / "select.json").read_text()):
        logits = np.array(case["logits"], np.float32)
        allowed = None if case["allowed"] is None else np.array(case["allowed"], np.uint32)
        got, lp = hip.select(logits, allowed)
        assert got == case["id"], case["name"]
        rid, rlp = oracle.select(logits, allowed)
        assert got == rid
        assert (math.isnan(lp) and math.isnan(rlp)) or abs(lp - rlp) <= 1e-9 * max(1, abs(rlp))


@pytest.mark.parametrize("vocab", [8192, 32768])
def test_select_random_bit_exact_ids(hip, vocab):
    say("select random", vocab)
    s = synth.Stream(12, f"sel{vocab}")
    for trial in range(20):
        logits = s.normal((vocab,)) * np.float32(4)
        if trial % 2:
            logits = np.round(logits).astype(np.float32)  # many ties
        if trial % 3 == 0:
            allowed = None
        else:
            bits = s.uniform01(vocab) < 0.02
            allowed = np.flatnonzero(bits).astype(np.uint32)
            if trial % 3 == 2:
                allowed = allowed[::-1].copy()  # list order, not id order
        got, lp = hip.select(logits, allowed)
        rid, rlp = oracle.select(logits, allowed)
        assert got == rid, trial
        assert abs(lp - rlp) <= 1e-9 * max(1, abs(rlp))
    with pytest.raises(NeedleError):
        hip.select(np.zeros(10, np.float32), np.array([10], np.uint32))
    with pytest.raises(NeedleError):
        hip.select(np.zeros(10, np.float32), np.array([], np.uint32))
