"""Seeded synthetic tensors shared by the GPU path, the tests and the bench.

Generator spec (the same for every consumer, so that a CPU checker and the
GPU receive identical buffers):

* stream: splitmix64.  Output i of a stream with 64-bit seed s is
  mix(s + (i + 1) * 0x9E3779B97F4A7C15) with the standard splitmix64
  finalizer (xor-shift 30/27/31, multipliers 0xBF58476D1CE4E5B9 and
  0x94D049BB133111EB), all modulo 2**64.
* tensor seed: seed(run_seed, name) = mix(run_seed ^ fnv1a64(name)).
* int8 uniform in [-127, 127]: ((z >> 32) * 255 >> 32) - 127.
* uniform float in [lo, hi): u = (z >> 40) * 2**-24 (exact in binary32),
  value = float32(lo + (hi - lo) * u) computed in float64.
* normal N(0, 1): Box-Muller on two consecutive uniforms computed in float64
  on the host once and rounded to float32; the same host buffer is handed to
  every consumer, so no engine's transcendental functions enter the data.
"""

from __future__ import annotations

import numpy as np

_GOLDEN = np.uint64(0x9E3779B97F4A7C15)
_M1 = np.uint64(0xBF58476D1CE4E5B9)
_M2 = np.uint64(0x94D049BB133111EB)


def _mix(z: np.ndarray) -> np.ndarray:
    with np.errstate(over="ignore"):
        z = (z ^ (z >> np.uint64(30))) * _M1
        z = (z ^ (z >> np.uint64(27))) * _M2
        return z ^ (z >> np.uint64(31))


def fnv1a64(text: str) -> int:
    h = 0xCBF29CE484222325
    for byte in text.encode():
        h ^= byte
        h = (h * 0x100000001B3) & 0xFFFFFFFFFFFFFFFF
    return h


def tensor_seed(run_seed: int, name: str) -> int:
    z = np.array([(run_seed ^ fnv1a64(name)) & 0xFFFFFFFFFFFFFFFF], dtype=np.uint64)
    return int(_mix(z)[0])


def splitmix64(seed: int, count: int, offset: int = 0) -> np.ndarray:
    """Outputs offset .. offset+count-1 of the splitmix64 stream for `seed`."""
    idx = np.arange(offset + 1, offset + count + 1, dtype=np.uint64)
    with np.errstate(over="ignore"):
        state = np.uint64(seed & 0xFFFFFFFFFFFFFFFF) + idx * _GOLDEN
    return _mix(state)


class Stream:
    """A named splitmix64 stream drawing consecutive outputs."""

    def __init__(self, run_seed: int, name: str):
        self.seed = tensor_seed(run_seed, name)
        self.offset = 0

    def _take(self, count: int) -> np.ndarray:
        z = splitmix64(self.seed, count, self.offset)
        self.offset += count
        return z

    def int8(self, shape) -> np.ndarray:
        n = int(np.prod(shape))
        z = self._take(n)
        hi = z >> np.uint64(32)
        v = ((hi * np.uint64(255)) >> np.uint64(32)).astype(np.int64) - 127
        return v.astype(np.int8).reshape(shape)

    def uniform01(self, count: int) -> np.ndarray:
        z = self._take(count)
        return (z >> np.uint64(40)).astype(np.float64) * (2.0**-24)

    def uniform(self, shape, lo: float, hi: float) -> np.ndarray:
        n = int(np.prod(shape))
        u = self.uniform01(n)
        return (lo + (hi - lo) * u).astype(np.float32).reshape(shape)

    def normal(self, shape) -> np.ndarray:
        n = int(np.prod(shape))
        m = (n + 1) // 2
        u1 = self.uniform01(m)
        u2 = self.uniform01(m)
        u1 = np.maximum(u1, 2.0**-25)  # keep log finite
        r = np.sqrt(-2.0 * np.log(u1))
        z = np.concatenate([r * np.cos(2 * np.pi * u2), r * np.sin(2 * np.pi * u2)])
        return z[:n].astype(np.float32).reshape(shape)

    def integers(self, count: int, lo: int, hi_inclusive: int) -> np.ndarray:
        span = hi_inclusive - lo + 1
        z = self._take(count) >> np.uint64(32)
        return ((z * np.uint64(span)) >> np.uint64(32)).astype(np.int64) + lo

    def bernoulli_mask(self, rows: int, vocab: int, p: float) -> np.ndarray:
        """Bitmask [rows][ceil(vocab/32)] uint32 with each id set w.p. p and at
        least one id set per row."""
        u = self.uniform01(rows * vocab).reshape(rows, vocab)
        bits = u < p
        forced = self.integers(rows, 0, vocab - 1)
        bits[np.arange(rows), forced] = True
        return pack_bits(bits)


def pack_bits(bits: np.ndarray) -> np.ndarray:
    rows, vocab = bits.shape
    words = (vocab + 31) // 32
    padded = np.zeros((rows, words * 32), dtype=np.uint64)
    padded[:, :vocab] = bits
    weights = (np.uint64(1) << np.arange(32, dtype=np.uint64))
    return (padded.reshape(rows, words, 32) * weights).sum(axis=2).astype(np.uint32)


def unpack_bits(mask: np.ndarray, vocab: int) -> np.ndarray:
    rows, words = mask.shape
    bits = (mask[:, :, None] >> np.arange(32, dtype=np.uint32)) & 1
    return bits.reshape(rows, words * 32)[:, :vocab].astype(bool)


def int8_matrix(run_seed: int, name: str, n: int, k: int, g: int,
                scale_lo: float = 0.001, scale_hi: float = 0.02):
    """W int8 [n][k] uniform in [-127, 127] and scales f32 [n][k/g] ~ U(lo, hi)."""
    s = Stream(run_seed, name)
    w = s.int8((n, k))
    scales = s.uniform((n, k // g), scale_lo, scale_hi)
    return w, scales


def cq_codebook() -> np.ndarray:
    """A 28-entry archive codebook: CQ2 [0, 4), CQ3 [4, 12), CQ4 [12, 28),
    each width's levels symmetric about zero (the shape of Lloyd-Max levels
    for a rotated, unit-variance weight distribution)."""
    cq2 = np.array([-1.51, -0.4528, 0.4528, 1.51])
    cq3 = np.array([-2.152, -1.344, -0.756, -0.245, 0.245, 0.756, 1.344, 2.152])
    cq4 = np.linspace(-2.7326, 2.7326, 16)
    return np.concatenate([cq2, cq3, cq4]).astype(np.float32)


def cq_matrix(run_seed: int, name: str, n: int, k: int, g: int, bits: int,
              norm_lo: float = 0.01, norm_hi: float = 0.05):
    """Packed Cactus-Quant matrix (packed uint8 [n][row_bytes], binary16
    norms uint16 [n][kpad/g]) with uniform codes; the ternary width (5) draws
    crumbs 0, 1 and 3 (zero, +c, -c) and a few reserved 2s (zero)."""
    from .cact import pack_codes

    s = Stream(run_seed, name)
    kpad = -(-k // g) * g
    if bits == 5:
        codes = np.array([0, 1, 3, 0, 1, 3, 0, 1, 3, 2])[s.integers(n * kpad, 0, 9)]
    else:
        codes = s.integers(n * kpad, 0, (1 << bits) - 1)
    packed = pack_codes(codes.reshape(n, kpad), bits)
    norms = s.uniform((n, kpad // g), norm_lo, norm_hi).astype(np.float16).view(np.uint16)
    return packed, norms
