"""The allocation-free attention entry point, nd_attention_static_d, through
the C ABI: the same results as nd_attention_d (the kernels are shared and the
chunking is the same, so the outputs are bit-identical) and within the
1e-3 relative / 1e-4 absolute bar of the oracle, on two calls in a row, the
second over a smaller visible range, so that the second reads the fixed
scratch after the first left it.  The sizes beyond the scratch are rejected
on the host before any launch.
"""

import sys

import numpy as np
import pytest

import oracle
from helpers import DeviceArray, assert_close
from needle_hip import HipKvCache, NeedleError, synth

pytestmark = pytest.mark.gpu


def say(*args):
    print("[case]", *args, file=sys.stderr, flush=True)


def _both(hip, kv, layer, pos, q, q_heads):
    """(static, allocating) outputs of one query."""
    dq = DeviceArray(q)
    d_static = DeviceArray(np.full(q.size, np.nan, np.float32))
    d_alloc = DeviceArray(np.full(q.size, np.nan, np.float32))
    try:
        hip._check(hip.lib.nd_attention_static_d(hip.ctx, kv.handle, layer, pos, dq.ptr, q_heads,
                                                 d_static.ptr, None), "nd_attention_static_d")
        hip._check(hip.lib.nd_sync(hip.ctx), "nd_sync")
        hip._check(hip.lib.nd_attention_d(hip.ctx, kv.handle, layer, pos, dq.ptr, q_heads,
                                          d_alloc.ptr, None), "nd_attention_d")
        hip._check(hip.lib.nd_sync(hip.ctx), "nd_sync")
        return d_static.read(), d_alloc.read()
    finally:
        for d in (dq, d_static, d_alloc):
            d.free()


@pytest.mark.parametrize("kv_heads,q_heads,length,positions", [
    (8, 8, 8192, (8191, 700)),      # 32 chunks per head, then 3
    (8, 64, 4096, (4095, 1500)),    # the largest query-head count the scratch holds
    (4, 8, 2048, (2047, 100)),      # grouped query heads; the second call fits one chunk
])
def test_static_scratch_attention_equals_allocating_entry_point(hip, kv_heads, q_heads, length,
                                                                positions):
    say("no-alloc attention", kv_heads, q_heads, length, positions)
    kv = HipKvCache(hip, 2, kv_heads, max_length=length)
    ref = oracle.KvCache(2, kv_heads, max_length=length)
    s = synth.Stream(77, f"noalloc{kv_heads}{q_heads}{length}")
    K, V = s.normal((length, kv_heads, 64)), s.normal((length, kv_heads, 64))
    kv.store(1, 0, K, V)
    ref.store(1, 0, K, V)
    try:
        for pos in positions:
            q = s.normal((q_heads * 64,))
            got, want = _both(hip, kv, 1, pos, q, q_heads)
            assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), (
                f"pos {pos}: static and allocating outputs differ")
            assert_close(got, ref.attention(1, pos, q), 1e-3, 1e-4,
                         f"static attention kv={kv_heads} q={q_heads} pos={pos}")
    finally:
        kv.free()


def test_static_scratch_rejects_more_query_heads_than_it_holds(hip):
    say("no-alloc attention limit")
    kv = HipKvCache(hip, 1, 16, max_length=64)
    try:
        with pytest.raises(NeedleError) as e:
            hip._check(hip.lib.nd_attention_static_d(hip.ctx, kv.handle, 0, 10, None, 128, None,
                                                     None), "nd_attention_static_d")
        assert e.value.code == "INVALID_CACT"
        dq = DeviceArray(np.zeros(128 * 64, np.float32))
        try:
            with pytest.raises(NeedleError) as e:
                hip._check(hip.lib.nd_attention_static_d(hip.ctx, kv.handle, 0, 10, dq.ptr, 128,
                                                         dq.ptr, None), "nd_attention_static_d")
            assert e.value.code == "INVALID_CACT" and "64" in str(e.value)
        finally:
            dq.free()
    finally:
        kv.free()
