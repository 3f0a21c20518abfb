"""Workgroup placement: the probe nd_create runs, and the agent-scope forms
that replace the XCD-local hand-offs where the probe fails.

The attention chunk merge, the batch matvec's k-slice sum, the split-k GEMM
sum and the Needle 2 fused layer launch pass partial results through one
XCD's L2, which needs workgroup L of a launch on the XCD of workgroup L % 8.
On this GPU the probe passes; the test hook then switches every such path to
its agent-scope form (Needle 2 to separate launches), whose outputs must meet
the same bars against the oracle as the XCD-local forms: matvec and attention
within 1e-3 relative / 1e-4 absolute elementwise, repeated launches
bit-identical (the counters return to zero), the batched decoder's ids
identical with its test's logit bars, Needle 2 step logits within 1e-3 of the
largest logit.
"""

import ctypes as C
import sys

import numpy as np
import pytest

import oracle
from helpers import assert_close
from needle_hip import HipKvCache, Int8Matrix, NeedleModel, synth
from needle_hip.models import ConstrainedWorkload, DecoderGeometry
from needle_hip.needle2 import Needle2Weights

pytestmark = pytest.mark.gpu
RTOL, ATOL = 1e-3, 1e-4


def say(*args):
    print("[case]", *args, file=sys.stderr, flush=True)


def xcd_local(hip, enable):
    probed = C.c_uint32(9)
    hip._check(hip.lib.nd_test_xcd_local(hip.ctx, int(enable), C.byref(probed)))
    return probed.value


def test_placement_probe_passes_on_mi355x(hip):
    """Every workgroup of the probe launches ran on the XCD of workgroup
    L % 8, so the XCD-local forms are selected."""
    say("placement probe")
    assert xcd_local(hip, 1) == 1


def test_agent_scope_forms_match_oracle(hip):
    from test_gpu_decoder import run_case
    from test_gpu_needle2 import SMALL, close

    try:
        xcd_local(hip, 0)
        heads = 8
        for length in (8192, 2048):
            say("agent-scope attention", length)
            kv = HipKvCache(hip, 1, heads, max_length=length)
            ref = oracle.KvCache(1, heads, max_length=length)
            st = synth.Stream(41, f"placement-kv{length}")
            K, V = st.normal((length, heads, 64)), st.normal((length, heads, 64))
            kv.store(0, 0, K, V)
            ref.store(0, 0, K, V)
            q = st.normal((heads * 64,))
            first = np.asarray(kv.attention(0, length - 1, q), np.float32)
            assert_close(first, ref.attention(0, length - 1, q), RTOL, ATOL,
                         f"agent-scope attention L={length}")
            for i in range(4):
                again = np.asarray(kv.attention(0, length - 1, q), np.float32)
                assert np.array_equal(again.view(np.uint32), first.view(np.uint32)), (length, i)
            kv.free()
        say("agent-scope matvec batch 8")
        w, s = synth.int8_matrix(43, "placement-w", 4096, 4096, 32)
        m = Int8Matrix(w, s, 32)
        x = synth.Stream(43, "placement-x").normal((8, 4096))
        first = np.asarray(hip.matvec(m, x), np.float32)
        assert_close(first, oracle.matvec_i8(w, s, 32, x), RTOL, ATOL, "agent-scope matvec b8")
        for i in range(4):
            again = np.asarray(hip.matvec(m, x), np.float32)
            assert np.array_equal(again.view(np.uint32), first.view(np.uint32)), ("matvec", i)
        say("agent-scope batched decode (split-k GEMM sum, batched attention)")
        g = DecoderGeometry(layers=2, heads=8, kv_heads=4, vocab=2048)
        wl = ConstrainedWorkload(batch=5, steps=4, min_context=30, max_context=700, vocab=g.vocab)
        run_case(hip, g, wl, seed=12)
        say("agent-scope Needle 2 steps (separate layer launches)")
        nw = Needle2Weights(SMALL, 31)
        model = NeedleModel(hip, nw)
        try:
            rt = model.create_resident_runtime()
            rt.reset(SMALL.max_length, 3)
            ref = oracle.Needle2(nw).runtime(SMALL.max_length, 3)
            for i, t in enumerate(synth.Stream(5, "placement-n2").integers(20, 0, SMALL.vocab - 1)):
                close(rt.step(int(t)), ref.step(int(t)), ("agent-scope needle2", i))
        finally:
            model.dispose()
    finally:
        xcd_local(hip, 1)
