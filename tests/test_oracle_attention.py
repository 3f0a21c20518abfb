"""Pins the oracle's decode attention (model/runtime.ts:719-786).

Checks against textbook float64 softmax attention over the dequantized cache
(numpy), the visible set of the sink + window rule written from its
definition, and closed forms: identical keys give the mean of the values,
a single position gives that value row, one dominant score selects its row.
"""

import numpy as np
import pytest

import oracle
from helpers import assert_close


def textbook(q, kdeq, vdeq, reps):
    """q [Hq][64], kdeq/vdeq [Hkv][n][64] -> [Hq][64] in float64."""
    hq = q.shape[0]
    out = np.zeros((hq, 64))
    for h in range(hq):
        kvh = h // reps
        sc = kdeq[kvh] @ q[h].astype(np.float64) / 8.0
        w = np.exp(sc - sc.max())
        w /= w.sum()
        out[h] = w @ vdeq[kvh]
    return out


def visible(position, sink, window):
    prefix = min(sink, position + 1)
    low = max(prefix, position + 1 - window) if window > 0 else prefix
    return list(range(prefix)) + list(range(low, position + 1))


@pytest.mark.parametrize("hq,hkv,n,sink,window", [(8, 8, 37, 0, 0), (8, 4, 300, 0, 256),
                                                  (8, 4, 300, 7, 256), (4, 2, 20, 3, 5)])
def test_against_textbook(rng, hq, hkv, n, sink, window):
    kv = oracle.KvCache(2, hkv, max_length=n + 5, sink=sink, window=window)
    ks, vs = [], []
    for p in range(n):
        k = rng.normal(size=(hkv, 64)).astype(np.float32)
        v = rng.normal(size=(hkv, 64)).astype(np.float32)
        kv.store(1, p, k, v)
        ks.append([oracle.kv_quantize(k[h]) for h in range(hkv)])
        vs.append([oracle.kv_quantize(v[h]) for h in range(hkv)])
    q = rng.normal(size=(hq, 64)).astype(np.float32)
    pos = n - 1
    vis = visible(pos, sink, window)
    kdeq = np.array([[ks[t][h][0].astype(np.float64) * ks[t][h][1] for t in vis] for h in range(hkv)])
    vdeq = np.array([[vs[t][h][0].astype(np.float64) * vs[t][h][1] for t in vis] for h in range(hkv)])
    ref = textbook(q, kdeq, vdeq, hq // hkv)
    got = kv.attention(1, pos, q).reshape(hq, 64)
    assert_close(got, ref, rtol=1e-5, atol=1e-6, what="oracle attention vs textbook")


def test_closed_forms(rng):
    kv = oracle.KvCache(1, 1, max_length=16)
    k = rng.normal(size=64).astype(np.float32)
    vals = []
    for p in range(10):
        v = rng.normal(size=64).astype(np.float32)
        kv.store(0, p, k, v)
        c, s = oracle.kv_quantize(v)
        vals.append(c.astype(np.float64) * s)
    q = rng.normal(size=64).astype(np.float32)
    assert_close(kv.attention(0, 0, q), vals[0], rtol=1e-6, atol=1e-7)
    assert_close(kv.attention(0, 9, q), np.mean(vals, axis=0), rtol=1e-5, atol=1e-6)


def test_float_mode_matches_textbook(rng):
    kv = oracle.KvCache(1, 2, max_length=32, kv_cache="float32")
    K = rng.normal(size=(20, 2, 64)).astype(np.float32)
    V = rng.normal(size=(20, 2, 64)).astype(np.float32)
    kv.store(0, 0, K, V)
    q = rng.normal(size=(4, 64)).astype(np.float32)
    ref = textbook(q, K.transpose(1, 0, 2).astype(np.float64), V.transpose(1, 0, 2).astype(np.float64), 2)
    assert_close(kv.attention(0, 19, q).reshape(4, 64), ref, rtol=1e-5, atol=1e-6)
