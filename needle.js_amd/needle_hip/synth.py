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


def tool_pieces(run_seed: int, vocab: int, tools) -> tuple:
    """A synthetic tokenizer vocabulary for tool-call decoding: (pieces,
    eligible).  Ids 0-255 are the byte pieces; a few control pieces (not
    eligible) and one empty piece follow; then JSON punctuation runs, the
    literals and their halves, number fragments, the tools' names, property
    names and enum texts (whole, split, quoted), escapes, UTF-8 characters
    and broken sequences, and seeded words and byte strings up to `vocab`
    pieces, no two alike."""
    import json as _json

    s = Stream(run_seed, "tool-pieces")
    pieces = [bytes([b]) for b in range(256)]
    eligible = [True] * 256
    for ctl in (b"<s>", b"</s>", b"<|im_end|>", b"<unk>"):
        pieces.append(ctl)
        eligible.append(False)
    pieces.append(b"")
    eligible.append(True)
    seen = set(pieces)

    def add(p: bytes):
        if p and p not in seen and len(pieces) < vocab:
            seen.add(p)
            pieces.append(p)
            eligible.append(True)

    punct = ['{"', '":"', '","', '"}', '"},', '}]', '},{"', '":', ':', ',"', '[{"name":"',
             '","arguments":{', '"}}', '}}', '}}]', ']', '[', '[]', '{}', '"]', '"],"', '":[',
             '":{', '":["', '":true', '":false', '":null', ',', '"', '],', '}', '{', '"]}',
             '","arguments":', '"arguments":', '[{"', '{"name":"', '"name":"', ',"arguments":{}',
             '":{}', '":[]', '":0', '":1', '":-', ']}', ']}]', '"}]', '"}}]']
    for p in punct:
        add(p.encode())
    for lit in ("true", "false", "null"):
        for i in range(1, len(lit) + 1):
            add(lit[:i].encode())
            add(lit[i:].encode())
    for p in ["0", "1", "12", "123", "-", "-1", "-0", ".", ".5", "0.", "1.", "e", "E", "e5", "E-3",
              "e+", "1e", "1e5", "2.5", "-2.5", "10", "100", "1000", "3,", "7}", "42]", "0.0",
              "9e999", "1.e5", "00", "-.", "5e-1", "1E+2"]:
        add(p.encode())
    names = set()

    def walk(schema):
        if not isinstance(schema, dict):
            return
        for k, v in schema.get("properties", {}).items():
            names.add(k)
            walk(v)
        for key in ("items", "additionalProperties"):
            walk(schema.get(key))
        for key in ("oneOf", "anyOf"):
            for v in schema.get(key, []):
                walk(v)
        for key in ("$defs", "definitions"):
            for v in schema.get(key, {}).values():
                walk(v)
        for v in schema.get("enum", []) + ([schema["const"]] if "const" in schema else []):
            names.add(_json.dumps(v, separators=(",", ":")))

    for t in tools:
        names.add(t["name"])
        walk(t["parameters"])
    for n in sorted(names):
        for p in (n, '"' + n, n + '"', '"' + n + '"', '"' + n + '":', n[: len(n) // 2],
                  n[len(n) // 2:], n[:1], n[1:]):
            add(p.encode())
    for p in ["\\n", '\\"', "\\u", "\\u00", "\\u00e9", "\\", "\\x", "\\\\", "\\t", "\\ud83d",
              "é", "中", "😀", "é\"", "naïve", "\\u00E9\""]:
        add(p.encode())
    for p in [b"\xc3", b"\xa9", b"\xe4\xb8", b"\xad", b"\xff", b"\xed\xa0\x80", b"\xf4\x90\x80\x80",
              b"\xe0\x80\xaf", b"\xc0\xaf", b"\xf0\x9f", b"\x98\x80"]:
        add(p)
    letters = b"abcdefghijklmnopqrstuvwxyz"
    alphabet = b'abcdefghijklmnopqrstuvwxyz0123456789 "{}[]:,.-_eE\\'
    while len(pieces) < vocab:
        n = int(s.integers(1, 1, 8)[0])
        if s.uniform01(1)[0] < 0.6:
            word = bytes(letters[i] for i in s.integers(n, 0, len(letters) - 1))
            add((b" " if s.uniform01(1)[0] < 0.3 else b"") + word)
        else:
            add(bytes(alphabet[i] for i in s.integers(n, 0, len(alphabet) - 1)))
    return pieces, eligible


# The reference's grammar test schema (tests/grammar.test.ts:7-21).
DEMO_PARAMETERS = {
    "type": "object",
    "properties": {
        "enabled": {"type": "boolean"},
        "level": {"type": "integer", "minimum": 0, "maximum": 10},
        "mode": {"type": "string", "enum": ["eco", "boost"]},
        "tags": {"type": "array", "items": {"type": "string", "minLength": 1}, "minItems": 1,
                 "maxItems": 3},
        "location": {"type": "object", "properties": {"lat": {"type": "number"},
                                                      "lon": {"type": "number"}},
                     "required": ["lat", "lon"]},
    },
    "required": ["enabled", "level", "mode", "tags"],
}

# A schema that uses every grammar feature: oneOf/anyOf, const, enums of
# mixed types, $ref, nested arrays and objects, integer and number, bounds,
# pattern, format, uniqueItems and type unions.
DEMO_RICH = {
    "type": "object",
    "$defs": {"point": {"type": "object", "properties": {"x": {"type": "number"},
                                                         "y": {"type": "integer"}},
                        "required": ["x"]}},
    "properties": {
        "kind": {"oneOf": [{"const": "circle"}, {"const": "square"}]},
        "count": {"type": "integer"},
        "ratio": {"type": "number"},
        "bounded": {"type": "integer", "minimum": 1, "maximum": 5},
        "points": {"type": "array", "items": {"$ref": "#/$defs/point"}, "maxItems": 4},
        "label": {"type": "string", "pattern": "^[a-z]+$"},
        "note": {"type": "string"},
        "flag": {"type": ["boolean", "null"]},
        "mixed": {"enum": ["a", 1, True, None]},
        "alt": {"anyOf": [{"type": "string"}, {"type": "number"},
                          {"type": "array", "items": {"type": "integer"}}]},
        "uniq": {"type": "array", "items": {"type": "string"}, "uniqueItems": True},
        "nested": {"type": "object", "properties": {"deep": {"type": "object", "properties": {
            "deeper": {"type": "array", "items": {"type": "array",
                                                  "items": {"type": "boolean"}}}}}}},
        "email": {"type": "string", "format": "email"},
    },
    "required": ["kind"],
}

DEMO_TOOL_OUTPUT = (
    '[{"name":"get_weather","arguments":{"kind":"circle","count":-12,"ratio":2.5e3,'
    '"bounded":3,"points":[{"x":1.5,"y":2},{"x":-0.0}],"label":"abc",'
    '"note":"h\\u00e9llo \\"q\\" \u4e2d","flag":null,"mixed":true,"alt":[1,2],'
    '"uniq":["a","b"],"nested":{"deep":{"deeper":[[true,false],[]]}},"email":"a@b.co"}},'
    '{"name":"get_time","arguments":{"tz":"CET"}}]')


def demo_tools():
    """Three tools with shared name prefixes: get, get_weather (the rich
    schema) and get_time."""
    from .grammar import normalize_tools

    return normalize_tools([
        {"name": "get", "parameters": {"type": "object", "properties": {"q": {"type": "string"}}}},
        {"name": "get_weather", "parameters": DEMO_RICH},
        {"name": "get_time", "parameters": {"type": "object", "properties": {
            "tz": {"enum": ["UTC", "CET"]}}, "required": ["tz"]}},
    ])
