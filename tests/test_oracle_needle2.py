"""Pins the oracle's Needle 2 step (model/runtime.ts:280-583) with an
independent float64 numpy model of the graph on a reduced geometry.

The numpy model is written from the model description (lanes, engram
hashing/gather/convolution, pre-mix, gated GQA with a sliding window and
sinks, post-attention sandwich norm, Hadamard MLP via scipy's Sylvester
matrix, Sinkhorn routing in log space, lane mean and tied logits) with
vectorized float64 algebra, so a wiring mistake in the C restatement -- a
swapped gate, a missing residual, a wrong lane offset or slot -- shows up as
a mismatch.
"""

import numpy as np
import pytest
from scipy.linalg import hadamard
from scipy.special import expit, logsumexp

import oracle
from needle_hip.needle2 import Needle2Geometry, Needle2Weights

SMALL = Needle2Geometry(vocab=256, dim=128, heads=4, kv_heads=2, layers=3, head_dim=64,
                        max_length=40, hadamard=128, lanes=4, engram_slots=64, engram_sub=32,
                        engram_tables=4, engram_taps=4, orders=(2, 3), sites=(0, 2),
                        kv_window=5)


def dense(m):
    """The matrix a step multiplies by, float64: int8 codes times row scales,
    or for a Cactus-Quant matrix (cq.ts:243-295 read as linear algebra) per
    row and group H_g (codebook[code] * norm) / sqrt(g), H_g the Sylvester
    Hadamard matrix -- the rotation cqMatvec applies to the input instead."""
    if getattr(m, "kind", None) != "cq":
        return m.codes.astype(np.float64) * m.scales.astype(np.float64)
    n, kpad, g = m.output_size, m.input_size_padded, m.group_size
    raw = np.unpackbits(m.packed.reshape(n, -1), axis=1, bitorder="little")
    pb = 2 if m.bits == 5 else m.bits
    codes = raw.reshape(n, kpad, pb) @ (1 << np.arange(pb))  # little-endian fields
    if m.bits == 5:  # crumbs 0, 1, 2, 3 -> 0, +c, 0, -c, c = 1.2240064 / sqrt(g)
        c = 1.2240064 / np.sqrt(g)
        values = np.array([0.0, c, 0.0, -c])[codes]
    else:
        values = m.codebooks[m.bits].astype(np.float64)[codes]
    norms = m.norms.view(np.float16).astype(np.float64)  # [n][kpad / g]
    scaled = values * np.repeat(norms, g, axis=1)
    h = hadamard(g).astype(np.float64) / np.sqrt(g)
    rows = (scaled.reshape(n, kpad // g, g) @ h.T).reshape(n, kpad)
    return rows[:, :m.input_size]


class NumpyNeedle2:
    def __init__(self, w, max_length, sink):
        self.w, self.g = w, w.geometry
        g = self.g
        self.sink = min(sink, max_length)
        self.history = []
        self.pos = 0
        self.depth = (g.engram_taps - 1) * max(g.orders) + 1
        self.ring = np.zeros((len(g.sites), self.depth, g.dim))
        self.valid = np.zeros((len(g.sites), self.depth), bool)
        self.eg_pos = 0
        self.K = [[] for _ in range(g.layers)]  # dequantized rows by position
        self.V = [[] for _ in range(g.layers)]
        self.H = hadamard(g.hadamard) / np.sqrt(g.hadamard)
        self.cells = []  # pooled cells: scaled embedding, then each layer's lane mean

    @staticmethod
    def rms(x, s=None):
        y = x / np.sqrt(np.mean(x * x) + 1e-6)
        return y if s is None else (1 + s.astype(np.float64)) * y

    def rope(self, v, heads):
        g = self.g
        v = v.reshape(heads, g.head_dim)
        half = g.head_dim // 2
        j = np.arange(half)
        ang = self.pos * float(np.float32(g.rope_theta)) ** (-(2 * j) / g.head_dim)
        z = (v[:, :half] + 1j * v[:, half:]) * np.exp(1j * ang)
        return np.concatenate([z.real, z.imag], axis=1)

    def lookup(self):
        g = self.g
        hpo = g.engram_tables // len(g.orders)
        idx, val = [], []
        for oi, order in enumerate(g.orders):
            for h in range(hpo):
                hsh = (0x9E3779B9 * (oi * hpo + h + 1)) & 0xFFFFFFFF
                ok = True
                for off in range(order):
                    hi = len(self.history) - 1 - off
                    tok = self.history[hi] if hi >= 0 else 0
                    hsh = ((hsh ^ tok) * 0x01000193) & 0xFFFFFFFF
                    if off == order - 1:
                        ok = hi >= 0
                hsh ^= hsh >> 15
                idx.append(hsh % g.engram_slots)
                val.append(ok)
        return idx, val

    def step(self, token):
        g, w = self.g, self.w
        self.history.append(token)
        x = np.tile(dense(w.embedding)[token] * np.sqrt(g.dim), (g.lanes, 1))
        self.cells.append(x[0].copy())
        keys, vals = [], []
        idx, ok = self.lookup()
        for s in range(len(g.sites)):
            tabs = dense(w.eg_tables[s])
            cat = np.concatenate([tabs[t * g.engram_slots + idx[t]] if ok[t]
                                  else np.zeros(g.engram_sub) for t in range(g.engram_tables)])
            keys.append(dense(w.eg_key[s]) @ cat)
            slot = self.eg_pos % self.depth
            self.ring[s, slot] = dense(w.eg_value[s]) @ cat
            self.valid[s, slot] = True
            mixed = np.zeros(g.dim)
            for tap in range(g.engram_taps):
                prev = self.eg_pos - tap * max(g.orders)
                if prev >= 0 and self.valid[s, prev % self.depth]:
                    mixed += w.eg_taps[s, tap] * self.ring[s, prev % self.depth]
            vals.append(mixed)
        self.eg_pos += 1
        L = g.lanes
        for l in range(g.layers):
            nl = self.rms(x.reshape(-1))
            pp = dense(w.phi_pre)[l * L:(l + 1) * L] @ nl
            po = dense(w.phi_post)[l * L:(l + 1) * L] @ nl
            pr = dense(w.phi_res)[l * L * L:(l + 1) * L * L] @ nl
            own = l % L
            off = np.where(np.arange(L) == own, 4.0, -4.0)
            hpre = expit(w.a_pre[l] * pp + w.b_pre[l * L:(l + 1) * L] + off)
            upd = hpre @ x
            blk = upd
            if l in g.sites:
                s = g.sites.index(l)
                a = expit(self.rms(upd) @ self.rms(keys[s]) / np.sqrt(g.dim))
                blk = upd + a * vals[s]
            ain = self.rms(blk, w.norm_input[l])
            q = dense(w.wq[l]) @ ain
            k = dense(w.wk[l]) @ ain
            v = dense(w.wv[l]) @ ain
            gate = dense(w.wgate[l]) @ ain
            hd = g.head_dim
            q = np.stack([self.rms(h, w.query_norm[l]) for h in q.reshape(g.heads, hd)])
            k = np.stack([self.rms(h, w.key_norm[l]) for h in k.reshape(g.kv_heads, hd)])
            q, k = self.rope(q, g.heads), self.rope(k, g.kv_heads)
            kq = [oracle.kv_quantize(k[h].astype(np.float32)) for h in range(g.kv_heads)]
            vq = [oracle.kv_quantize(v.reshape(g.kv_heads, hd)[h].astype(np.float32))
                  for h in range(g.kv_heads)]
            self.K[l].append(np.stack([c * s for c, s in kq]))
            self.V[l].append(np.stack([c * s for c, s in vq]))
            prefix = min(self.sink, self.pos + 1)
            low = max(prefix, self.pos + 1 - g.kv_window)
            vis = list(range(prefix)) + list(range(low, self.pos + 1))
            K = np.stack([self.K[l][t] for t in vis])
            V = np.stack([self.V[l][t] for t in vis])
            rep = g.heads // g.kv_heads
            att = np.zeros((g.heads, hd))
            for h in range(g.heads):
                sc = K[:, h // rep] @ q[h] / np.sqrt(hd)
                p = np.exp(sc - sc.max())
                att[h] = (p / p.sum()) @ V[:, h // rep]
            att = att.reshape(-1) * expit(gate)
            proj = dense(w.wo[l]) @ att
            after = blk + expit(w.attention_gate[l]) * self.rms(proj, w.post_attn_norm[l])
            pre = self.rms(after, w.pre_hadamard_norm[l])
            z = np.zeros(g.hadamard)
            z[:g.dim] = pre * w.d1[l]
            z = self.H @ z
            z = z * w.d2[l]
            z = z * expit(z)
            mlp = (self.H @ z)[:g.dim] * w.d3[l]
            delta = after + mlp - upd
            offp = np.where(np.arange(L) == own, 0.0, -4.0)
            hpost = 2 * expit(w.a_post[l] * po + w.b_post[l * L:(l + 1) * L] + offp)
            r = (w.a_res[l] * pr + w.b_res[l * L * L:(l + 1) * L * L]).reshape(L, L)
            for _ in range(20):
                r = r - logsumexp(r, axis=1, keepdims=True)
                r = r - logsumexp(r, axis=0, keepdims=True)
            x = np.exp(r) @ x + hpost[:, None] * delta[None, :]
            self.cells.append(x.mean(axis=0))
        self.pos += 1
        return dense(w.embedding) @ self.rms(x.mean(axis=0), w.final_norm)


@pytest.mark.parametrize("sink,cq_bits", [(0, 0), (3, 0), (0, 4), (3, 3), (0, 2), (0, 5),
                                          (3, "mixed")])
def test_step_matches_float64_model(sink, cq_bits):
    """Int8 weights, and the Cactus-Quant widths of the shipped archive (the
    oracle runs cqMatvec / dequantizeCqRow on them), one width for every
    matrix or each matrix its own width and group (mixed)."""
    w = Needle2Weights(SMALL, 9, cq_bits=cq_bits)
    model = oracle.Needle2(w)
    rt = model.runtime(SMALL.max_length, sink)
    ref = NumpyNeedle2(w, SMALL.max_length, sink)
    tokens = [5, 200, 17, 17, 99, 3, 250, 17, 5, 200, 64, 1]  # repeats exercise the hashes
    for t in tokens:
        got = rt.step(t)
        want = ref.step(t)
        err = np.abs(got - want)
        assert err.max() <= 1e-4 * np.abs(want).max(), (t, err.max())


def test_kv_window_ring_slots():
    w = Needle2Weights(SMALL, 10)
    rt = oracle.Needle2(w).runtime(SMALL.max_length, 2)
    for t in range(12):
        rt.step((7 * t) % SMALL.vocab, want_logits=False)
    kc, vc, ks, vs = rt.kv_read(1, 0)
    assert kc.shape[0] == 2 + SMALL.kv_window  # sink + window slots (runtime.ts:166-170)
    assert (ks > 0).all()


def test_overflow_and_bad_token():
    w = Needle2Weights(SMALL, 11)
    rt = oracle.Needle2(w).runtime(3)
    for t in range(3):
        rt.step(t, want_logits=False)
    with pytest.raises(oracle.OracleError):
        rt.step(1)
    with pytest.raises(oracle.OracleError):
        oracle.Needle2(w).runtime(5).step(SMALL.vocab)


def pooled_confidence(head, cells):
    """Closed form of OnlineProbePool over `cells` (runtime.ts:48-105): per
    probe a softmax over the cells' scores (cell . probe / sqrt(d)), the
    softmax-weighted mean cell, the dense projection plus bias, sigmoid of
    output 0 (runtime.ts:641-645)."""
    from scipy.special import softmax

    cells = np.asarray(cells, np.float64)
    probes = head.probes.astype(np.float64)
    scores = cells @ probes.T / np.sqrt(cells.shape[1])       # [cells][probes]
    weights = softmax(scores, axis=0)
    pooled = (weights.T @ cells).reshape(-1)                  # [probes * d]
    out = head.bias.astype(np.float64) + head.projection.astype(np.float64) @ pooled
    return float(expit(out[0]))


@pytest.mark.parametrize("sink", [0, 3])
def test_confidence_pool_matches_closed_form(sink):
    w = Needle2Weights(SMALL, 12)
    rt = oracle.Needle2(w).runtime(SMALL.max_length, sink)
    ref = NumpyNeedle2(w, SMALL.max_length, sink)
    tokens = [5, 200, 17, 17, 99, 3, 250, 17, 5]
    cells = rt.record_cells(len(tokens) * (SMALL.layers + 1))
    for t in tokens:
        rt.step(t, want_logits=False)
        ref.step(t)
    assert rt.recorded_cells() == len(tokens) * (SMALL.layers + 1)
    want = np.asarray(ref.cells)
    for i, (got_c, want_c) in enumerate(zip(cells, want)):
        assert np.abs(got_c - want_c).max() <= 1e-4 * np.abs(want_c).max(), i
    # the online update equals the closed form on the same cells ...
    conf = rt.confidence()
    assert abs(conf - pooled_confidence(w.confidence, cells)) <= 1e-6 * conf
    # ... and the independent model's cells give the same confidence
    assert abs(conf - pooled_confidence(w.confidence, want)) <= 1e-4 * conf
    assert 0.0 < conf < 1.0


def test_confidence_single_cell_is_that_cell():
    # One step: every probe's softmax pools the step's L + 1 cells; with one
    # token the first cell is the scaled embedding row.
    w = Needle2Weights(SMALL, 13)
    rt = oracle.Needle2(w).runtime(SMALL.max_length)
    cells = rt.record_cells(SMALL.layers + 1)
    rt.step(7, want_logits=False)
    emb = oracle.row_i8(w.embedding.codes, w.embedding.scales, SMALL.dim, 7)
    assert np.array_equal(cells[0], (emb.astype(np.float64) * np.sqrt(SMALL.dim)).astype(np.float32))
    assert abs(rt.confidence() - pooled_confidence(w.confidence, cells)) <= 1e-6
