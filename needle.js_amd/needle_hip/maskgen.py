"""Allowed-token masks of the tool-call grammar on the GPU.

The agent's constrained loop (tools/agent.ts:157-210) asks, every step,
which token pieces a clone of the grammar accepts.  `GrammarMasker` answers
on the device: the tool schemas are compiled once into a program
(`GrammarProgram`), each step's grammar state is serialized into a few
hundred bytes (`state_words`), and one HIP thread per piece runs the grammar
over its bytes (nd_grammar_mask, csrc/grammar.hip).  Pieces whose answer
needs a check the device does not make (enum/const and uniqueness of
values, a pattern outside the automaton's reach, numbers outside the exact
fast path) come back undecided, and the host grammar -- which owns the state -- settles exactly
those.  Layouts are documented with nd_grammar_upload / nd_grammar_mask in
include/needle_hip.h.
"""

from __future__ import annotations

import ctypes as C
import math
from typing import Dict, List, Sequence, Tuple

import numpy as np

from . import jsregex
from . import lib as L
from .errors import NeedleError, invariant
from .grammar import (JS_SPACE, ToolCallGrammar, js_stringify, possible_types,
                      resolve_reference, schema_alternatives)

MAGIC = 0x4E444752
NONE = 0xFFFFFFFF
MAX_DEPTH = 24
NODE_WORDS = 28
STATE_HEADER_WORDS = 24
# Value checks of a node (word 12 of its entry): string checks the device
# makes at the closing quote, numeric checks at the end of a number, and the
# ones it leaves to the host (enum/const, a pattern without an automaton,
# non-numeric bounds).
KC_MIN_LENGTH, KC_MAX_LENGTH, KC_EMAIL, KC_UUID, KC_STRING_HOST, KC_PATTERN = 1, 2, 4, 8, 16, 32
KC_MINIMUM, KC_MAXIMUM, KC_EXCLUSIVE_MINIMUM, KC_EXCLUSIVE_MAXIMUM = 256, 512, 1024, 2048
KC_MULTIPLE_OF, KC_NUMBER_HOST = 4096, 8192
_LENGTH_MAX = 0xFFFFFF  # string lengths are counted up to this
_M_CAP = 10 ** 18  # number mantissas take digits while below this
_TYPE_BITS = {"string": 1, "number": 2, "integer": 4, "boolean": 8, "null": 16, "array": 32,
              "object": 64}
_TOOL_PHASES = ["array-open", "call-open", "name-literal", "tool-name", "arguments-literal",
                "arguments", "call-close", "after-call", "done"]
_ARRAY_PHASES = {"open": 0, "first-or-end": 1, "value": 2, "after-value": 3}
_OBJECT_PHASES = {"open": 0, "key-or-end": 1, "key-required": 2, "key": 3, "colon": 4,
                  "value": 5, "after-value": 6}
_KIND = {"value": 1, "string": 2, "number": 3, "literal": 4, "choice": 5, "array": 6,
         "object": 7, "key": 8}


def value_kind(value) -> int:
    """0 string, 1 number, 2 boolean, 3 null, 4 array, 5 object."""
    if value is None:
        return 3
    if isinstance(value, bool):
        return 2
    if isinstance(value, (int, float)):
        return 1
    if isinstance(value, str):
        return 0
    if isinstance(value, list):
        return 4
    return 5


class GrammarProgram:
    """The tools' JSON Schemas as the device program: schema nodes (resolved
    schemas), value-frame descriptors (a frame's schema before resolution:
    its oneOf/anyOf alternatives, or the candidates when all of them are
    const/enum), properties, candidates and tool names.  Entries are keyed by
    (tool, the schema's JSON text), since references resolve against each
    tool's own parameters."""

    def __init__(self, tools: Sequence[dict]):
        invariant(0 < len(tools) <= 32, "UNSUPPORTED_CACT", "the device mask takes 1..32 tools")
        self.tools = list(tools)
        self.nodes: List[list] = []
        self.values: List[list] = []
        self.alts: List[int] = []
        self.props: List[list] = []
        self.cands: List[list] = []
        self.pool = bytearray()
        self.regex: List[int] = []  # pattern automata, one after another
        self._regex_ix: Dict[str, int] = {}
        self.node_dfa: Dict[int, jsregex.Dfa] = {}
        self._node_ix: Dict[Tuple[int, str], int] = {}
        self._value_ix: Dict[Tuple[int, str], int] = {}
        # (tool, id(schema)) -> (schema, entry): the per-step state lookups
        # skip the JSON text when the frame holds a schema object seen before.
        self._node_id: Dict[Tuple[int, int], tuple] = {}
        self._value_id: Dict[Tuple[int, int], tuple] = {}
        self.tool_entries = []
        for ti, tool in enumerate(self.tools):
            name = tool["name"].encode()
            self.tool_entries.append([self._bytes(name), len(name),
                                      self.value_of(ti, tool["parameters"]), 0])

    def _bytes(self, data: bytes) -> int:
        off = len(self.pool)
        self.pool.extend(data)
        return off

    def value_of(self, ti: int, schema: dict) -> int:
        hit = self._value_id.get((ti, id(schema)))
        if hit is not None and hit[0] is schema:
            return hit[1]
        key = (ti, js_stringify(schema))
        if key in self._value_ix:
            self._value_id[(ti, id(schema))] = (schema, self._value_ix[key])
            return self._value_ix[key]
        idx = len(self.values)
        self._value_ix[key] = idx
        self.values.append([0, 0, 0, 0])
        root = self.tools[ti]["parameters"]
        alts = schema_alternatives(schema, root)
        resolved = [resolve_reference(a, root) for a in alts]
        enum_values = []
        for a in resolved:
            if "const" in a:
                enum_values.append(a["const"])
            elif "enum" in a:
                enum_values.extend(a["enum"])
        if enum_values and all(("const" in a) or ("enum" in a) for a in resolved):
            if len(enum_values) > 32:
                self.values[idx] = [2, 0, len(enum_values), 0]
                return idx
            first = len(self.cands)
            for v in enum_values:
                text = js_stringify(v).encode()
                self.cands.append([self._bytes(text), len(text), value_kind(v), 0])
            self.values[idx] = [1, first, len(enum_values), 0]
            return idx
        nodes = [self.node_of(ti, resolve_reference(a, root)) for a in alts]
        first = len(self.alts)
        self.alts.extend(nodes)
        self.values[idx] = [0, first, len(nodes), 0]
        return idx

    def node_of(self, ti: int, s: dict) -> int:
        hit = self._node_id.get((ti, id(s)))
        if hit is not None and hit[0] is s:
            return hit[1]
        key = (ti, js_stringify(s))
        if key in self._node_ix:
            self._node_id[(ti, id(s))] = (s, self._node_ix[key])
            return self._node_ix[key]
        idx = len(self.nodes)
        self._node_ix[key] = idx
        self.nodes.append([0] * NODE_WORDS)
        types = possible_types(s)
        tmask = 0
        for t in types:
            tmask |= _TYPE_BITS.get(t, 0)
        checks = self._checks(s)
        if checks[0] & KC_PATTERN:
            dfa = jsregex.regexp(s["pattern"]).dfa()
            self.node_dfa[idx] = dfa
            if s["pattern"] not in self._regex_ix:
                self._regex_ix[s["pattern"]] = len(self.regex)
                self.regex.extend(dfa.words())
            checks[3] = self._regex_ix[s["pattern"]] + 1
        flags = 0
        if checks[0] & 0xFF:
            flags |= 1
        if checks[0] & 0xFF00:
            flags |= 2
        if "integer" in types and "number" not in types:
            flags |= 4
        if "const" in s or "enum" in s:
            flags |= 8
        if s.get("uniqueItems"):
            flags |= 16
        props = s.get("properties", {})
        if len(props) > 32:
            raise NeedleError("UNSUPPORTED_CACT", "the device mask takes objects of <= 32 properties")
        items_value = self.value_of(ti, s.get("items", {}))
        first = len(self.props)
        self.props.extend([[0, 0, 0, 0] for _ in props])
        required = s.get("required", [])
        rmask = 0
        for i, (name, sub) in enumerate(props.items()):
            nb = name.encode()
            self.props[first + i] = [self._bytes(nb), len(nb), self.value_of(ti, sub), 0]
            if name in required:
                rmask |= 1 << i
        self.nodes[idx] = [tmask, flags, int(s.get("minItems", 0)), int(s.get("maxItems", 32)),
                           items_value, len(props), first, rmask,
                           int(s.get("minProperties", 0)),
                           int(s.get("maxProperties", len(props))), 0, 0] + checks
        return idx

    @staticmethod
    def _checks(s: dict) -> list:
        """Words 12..27 of a node: check flags, minLength, maxLength, the
        pattern automaton's offset + 1 (filled in by node_of), then minimum,
        maximum, exclusiveMinimum, exclusiveMaximum and multipleOf as float64
        (two words each, low first), 0, 0 (grammar.ts:179-222)."""
        w = [0] * 16
        cf = 0

        def length(key, bit, at):
            nonlocal cf
            if key not in s:
                return
            v = s[key]
            if isinstance(v, int) and not isinstance(v, bool) and 0 <= v < _LENGTH_MAX:
                cf |= bit
                w[at] = v
            else:
                cf |= KC_STRING_HOST

        length("minLength", KC_MIN_LENGTH, 1)
        length("maxLength", KC_MAX_LENGTH, 2)
        if "const" in s or "enum" in s:
            cf |= KC_STRING_HOST
        if "pattern" in s:
            # RegExp's SyntaxError, and a pattern the automaton cannot
            # express, are the host grammar's to meet.
            try:
                ok = isinstance(s["pattern"], str) and jsregex.regexp(s["pattern"]).dfa() is not None
            except jsregex.RegexSyntaxError:
                ok = False
            cf |= KC_PATTERN if ok else KC_STRING_HOST
        if s.get("format") == "email":
            cf |= KC_EMAIL
        elif s.get("format") == "uuid":
            cf |= KC_UUID
        for key, bit, at in (("minimum", KC_MINIMUM, 4), ("maximum", KC_MAXIMUM, 6),
                             ("exclusiveMinimum", KC_EXCLUSIVE_MINIMUM, 8),
                             ("exclusiveMaximum", KC_EXCLUSIVE_MAXIMUM, 10),
                             ("multipleOf", KC_MULTIPLE_OF, 12)):
            if key not in s:
                continue
            v = s[key]
            if isinstance(v, (int, float)) and not isinstance(v, bool) and \
                    math.isfinite(float(v)):
                cf |= bit
                lo, hi = np.array([float(v)], np.float64).view(np.uint32)
                w[at], w[at + 1] = int(lo), int(hi)
            else:
                cf |= KC_NUMBER_HOST
        if "const" in s or "enum" in s:
            cf |= KC_NUMBER_HOST
        w[0] = cf
        return w

    def words(self) -> np.ndarray:
        tables = [np.asarray(self.nodes, np.uint32).reshape(-1, NODE_WORDS),
                  np.asarray(self.values, np.uint32).reshape(-1, 4),
                  np.asarray(self.alts, np.uint32).reshape(-1),
                  np.asarray(self.props, np.uint32).reshape(-1, 4),
                  np.asarray(self.cands, np.uint32).reshape(-1, 4),
                  np.asarray(self.tool_entries, np.uint32).reshape(-1, 4)]
        header = np.zeros(16, np.uint32)
        header[0] = MAGIC
        off = 16
        for i, t in enumerate(tables):
            header[1 + 2 * i] = t.shape[0]
            header[2 + 2 * i] = off
            off += t.size
        regex = np.asarray(self.regex, np.uint32)
        header[15] = off if regex.size else 0
        off += regex.size
        pool = bytes(self.pool)
        pool_words = np.frombuffer(pool + b"\0" * (-len(pool) % 4), np.uint32)
        header[13] = off * 4
        header[14] = len(pool)
        return np.concatenate([header] + [t.reshape(-1) for t in tables] +
                              [regex, pool_words]).astype(np.uint32)


def _utf8_step(s: int, b: int) -> int:
    """One byte of the fatal UTF-8 decode as a DFA: 0 boundary, 1-3
    continuation bytes left, 4 after E0, 5 after ED, 6 after F0, 7 after F4,
    8 error (sticky)."""
    if s == 0:
        return (0 if b < 0x80 else 1 if 0xC2 <= b <= 0xDF else 4 if b == 0xE0 else
                5 if b == 0xED else 2 if 0xE1 <= b <= 0xEF else 6 if b == 0xF0 else
                3 if 0xF1 <= b <= 0xF3 else 7 if b == 0xF4 else 8)
    if s == 1:
        return 0 if 0x80 <= b <= 0xBF else 8
    if s == 2:
        return 1 if 0x80 <= b <= 0xBF else 8
    if s == 3:
        return 2 if 0x80 <= b <= 0xBF else 8
    if s == 4:
        return 1 if 0xA0 <= b <= 0xBF else 8
    if s == 5:
        return 1 if 0x80 <= b <= 0x9F else 8
    if s == 6:
        return 2 if 0x90 <= b <= 0xBF else 8
    if s == 7:
        return 2 if 0x80 <= b <= 0x8F else 8
    return 8


def _utf8_state(data) -> int:
    s = 0
    for b in data:
        s = _utf8_step(s, b)
    return s


def _number_step(s: int, ch: str) -> int:
    """One character of the number-prefix DFA (states as number_step in
    csrc/grammar.hip; 9 = not a prefix)."""
    d = ch in "0123456789"
    if s == 0:
        return 1 if ch == "-" else 2 if ch == "0" else 3 if d else 9
    if s == 1:
        return 2 if ch == "0" else 3 if d else 9
    if s == 2:
        return 4 if ch == "." else 6 if ch in "eE" else 9
    if s == 3:
        return 3 if d else 4 if ch == "." else 6 if ch in "eE" else 9
    if s == 4:
        return 5 if d else 10 if ch in "eE" else 9
    if s == 5:
        return 5 if d else 6 if ch in "eE" else 9
    if s == 6:
        return 7 if ch in "+-" else 8 if d else 9
    if s in (7, 8):
        return 8 if d else 9
    if s == 10:
        return 11 if ch in "+-" else 12 if d else 9
    if s in (11, 12):
        return 12 if d else 9
    return 9


def _number_state(text: str):
    """(DFA state, exponent seen, nonzero fraction digit, integer digits)."""
    s, exp, frac, digits = 0, False, False, 0
    for ch in text:
        s = _number_step(s, ch)
        if s in (6, 10):
            exp = True
        if s == 5 and ch != "0":
            frac = True
        if s in (2, 3):
            digits += 1
    return s, exp, frac, min(digits, 1000)


_ESCAPED = {0x22: 0x22, 0x5C: 0x5C, 0x2F: 0x2F, 0x62: 0x08, 0x66: 0x0C, 0x6E: 0x0A, 0x72: 0x0D,
            0x74: 0x09}


def _email_step(state: int, c: int) -> int:
    at = c == 0x40
    other = not at and c not in JS_SPACE
    if state == 0:
        return 1 if other else 6
    if state == 1:
        return 1 if other else (2 if at else 6)
    if state == 2:
        return 3 if other else 6
    if state == 3:
        return (4 if c == 0x2E else 3) if other else 6
    if state in (4, 5):
        return 5 if other else 6
    return 6


def _uuid_step(pos: int, dead: bool, c: int):
    if dead or pos >= 36:
        return pos, True
    if pos in (8, 13, 18, 23):
        ok = c == 0x2D
    elif pos == 14:
        ok = 0x31 <= c <= 0x38
    elif pos == 19:
        ok = c in (0x38, 0x39, 0x61, 0x62, 0x41, 0x42)
    else:
        ok = 0x30 <= c <= 0x39 or 0x61 <= c <= 0x66 or 0x41 <= c <= 0x46
    return (pos + 1, False) if ok else (pos, True)


def string_accumulator(data, dfa=None) -> List[int]:
    """The device's running summary of a string's bytes after its opening
    quote: [code points so far (Array.from's count: an escaped high
    surrogate followed by an escaped low one is one), word 1 = the pending
    \\u value (bits 0-15) | pending escaped high surrogate (16) | email state
    (17-19) | uuid position (20-25) | uuid mismatch (26), the UTF-8 code point
    being assembled, the state of the pattern automaton `dfa` (code units:
    a code point above U+FFFF steps it twice)]."""
    count, hexv, pend, email, upos, udead, cp, u8 = 0, 0, False, 0, 0, False, 0, 0
    escaped, uni, rx = False, 0, 0

    def emit(cu: int, uesc: bool):
        nonlocal count, pend, email, upos, udead, rx
        if dfa is not None:
            if cu > 0xFFFF:
                rx = dfa.step(rx, 0xD800 + ((cu - 0x10000) >> 10))
                rx = dfa.step(rx, 0xDC00 + ((cu - 0x10000) & 0x3FF))
            else:
                rx = dfa.step(rx, cu)
        if pend and uesc and 0xDC00 <= cu <= 0xDFFF:
            pend = False
        else:
            count = min(count + 1, _LENGTH_MAX)
            pend = uesc and 0xD800 <= cu <= 0xDBFF
        email = _email_step(email, cu)
        upos, udead = _uuid_step(upos, udead, cu)

    for b in data[1:]:  # after the opening quote
        prev = u8
        u8 = _utf8_step(prev, b)  # every byte steps the decode, as on the device
        if uni > 0:
            hexv = (hexv << 4 | int(chr(b), 16)) & 0xFFFF
            uni -= 1
            if uni == 0:
                emit(hexv, True)
        elif escaped:
            escaped = False
            if b == 0x75:
                uni, hexv = 4, 0
            else:
                emit(_ESCAPED[b], False)
        elif b == 0x5C:
            escaped = True
        else:
            if prev == 0:
                if b < 0x80:
                    emit(b, False)
                else:
                    cp = b & (0x1F if b < 0xE0 else 0x0F if b < 0xF0 else 0x07)
            else:
                cp = (cp << 6 | (b & 0x3F)) & 0x1FFFFF
                if u8 == 0:
                    emit(cp, False)
    w1 = hexv | (1 << 16 if pend else 0) | email << 17 | upos << 20 | (1 << 26 if udead else 0)
    return [count, w1, cp, rx]


def number_accumulator(text: str) -> List[int]:
    """The device's running value of a number's text: mantissa m (words 0
    and 1) of the significant digits taken while m < 10^18, k (word 2, two's
    complement) with value = m * 10^(k + exponent), and word 3 = exponent
    digits (saturating at 999999) | minus sign (24) | exponent minus (25) |
    a nonzero digit dropped (26)."""
    m, k, e, neg, eneg, ovf, s = 0, 0, 0, False, False, False, 0
    for ch in text:
        n = _number_step(s, ch)
        d = ord(ch) - 0x30
        if n == 1:
            neg = True
        elif n in (2, 3) and s in (0, 1, 3):
            if m < _M_CAP:
                m = m * 10 + d
            else:
                k += 1
                ovf = ovf or d != 0
        elif n == 5:
            if m < _M_CAP:
                m = m * 10 + d
                k -= 1
            else:
                ovf = ovf or d != 0
        elif n in (7, 11):
            eneg = ch == "-"
        elif n in (8, 12):
            e = min(e * 10 + d, 999999)
        s = n
    k = max(-(1 << 20), min(1 << 20, k))
    return [m & 0xFFFFFFFF, m >> 32, k & 0xFFFFFFFF,
            e | (1 << 24 if neg else 0) | (1 << 25 if eneg else 0) | (1 << 26 if ovf else 0)]


def state_words(program: GrammarProgram, g: ToolCallGrammar) -> np.ndarray:
    """The device form of a ToolCallGrammar state (layout in nd_grammar_mask's
    declaration)."""
    name_live = 0
    for c in g.name_candidates:
        name_live |= 1 << c[0]
    name_off = g.name_candidates[0][2] if g.name_candidates else 0
    used = 0
    for t in g.used_tools:
        used |= 1 << t
    args = g.arguments
    frames: List[List[int]] = []
    acc = [0, 0, 0, 0]
    complete, kind = 0, 0
    if args is not None:
        ti = g.current_tool
        complete = 1 if args._complete else 0
        kind = value_kind(args._value) if args._complete else 0
        for i, f in enumerate(args.stack):
            k = f.kind
            if k == "value":
                frames.append([1, program.value_of(ti, f.schema), 0, 0])
            elif k == "string":
                flags = (1 if f.started else 0) | (2 if f.escaped else 0) | (f.unicode << 2) | \
                        (_utf8_state(f.bytes) << 8)
                node = program.node_of(ti, f.schema)
                frames.append([2 | flags << 16, node, 0, 0])
                if f.started:
                    acc = string_accumulator(f.bytes, program.node_dfa.get(node))
            elif k == "number":
                s, exp, frac, digits = _number_state(f.text)
                flags = (1 if exp else 0) | (2 if frac else 0)
                frames.append([3 | s << 8 | flags << 16, program.node_of(ti, f.schema), 0, digits])
                acc = number_accumulator(f.text)
            elif k == "literal":
                lit = {b"true": 0, b"false": 1, b"null": 2}[bytes(f.bytes)]
                frames.append([4, lit, 0, f.offset])
            elif k == "choice":
                live = 0
                for c in f.candidates:
                    live |= 1 << c[3]
                off = f.candidates[0][2] if f.candidates else 0
                frames.append([5, program.value_of(ti, f.schema), live, off])
            elif k == "array":
                # word 2: the items are these (1), pairwise distinct (2)
                texts = [js_stringify(v) for v in f.values]
                items = 1 | (2 if len(set(texts)) == len(texts) else 0)
                frames.append([6 | _ARRAY_PHASES[f.phase] << 8, program.node_of(ti, f.schema),
                               items, len(f.values)])
            elif k == "object":
                props = list(f.schema.get("properties", {}))
                umask = 0
                for name in f.used:
                    umask |= 1 << props.index(name)
                cur = props.index(f.current_key) if f.current_key is not None else NONE
                frames.append([7 | _OBJECT_PHASES[f.phase] << 8, program.node_of(ti, f.schema),
                               umask, cur])
            else:  # key: the object below it owns the property names
                parent = args.stack[i - 1]
                live = 0
                for c in f.candidates:
                    live |= 1 << c[3]
                off = f.candidates[0][2] if f.candidates else 0
                frames.append([8, program.node_of(ti, parent.schema), live, off])
    if len(frames) > MAX_DEPTH:
        raise NeedleError("UNSUPPORTED_CACT", f"grammar stack of {len(frames)} frames")
    head = [_TOOL_PHASES.index(g.phase), g.literal_offset, name_live, name_off,
            g.current_tool if g.current_tool >= 0 else NONE, used, len(g.calls), g.maximum_calls,
            len(g.tools), 1 if args is not None else 0, complete, kind, len(frames), 0, 0, 0]
    head += acc + [0, 0, 0, 0]
    assert len(head) == STATE_HEADER_WORDS
    return np.asarray(head + [w for f in frames for w in f], np.uint32)


class GrammarMasker:
    """Device masks for one tool set over one piece vocabulary."""

    def __init__(self, backend, tools: Sequence[dict], pieces: Sequence[bytes],
                 eligible: Sequence[bool]):
        self.backend = backend
        self.lib = backend.lib
        self.pieces = list(pieces)
        self.eligible = np.asarray(eligible, np.uint8)
        self.vocab = len(self.pieces)
        offsets = np.zeros(self.vocab + 1, np.uint32)
        offsets[1:] = np.cumsum([len(p) for p in self.pieces])
        data = np.frombuffer(b"".join(self.pieces) or b"\0", np.uint8)
        self.program = GrammarProgram(tools)
        words = self.program.words()
        self._pieces = C.c_void_p()
        self._grammar = C.c_void_p()
        backend._check(self.lib.nd_pieces_upload(backend.ctx, L.ptr(offsets), L.ptr(data),
                                                 L.ptr(self.eligible), self.vocab,
                                                 C.byref(self._pieces)), "nd_pieces_upload")
        backend._check(self.lib.nd_grammar_upload(backend.ctx, L.ptr(words), words.size,
                                                  C.byref(self._grammar)), "nd_grammar_upload")
        self.words = (self.vocab + 31) // 32
        self.last_undecided = 0

    def state(self, g: ToolCallGrammar) -> np.ndarray:
        """The device state words of the grammar `g`."""
        return state_words(self.program, g)

    def settle(self, g: ToolCallGrammar, undecided) -> List[int]:
        """The undecided pieces that a clone of `g` accepts (agent.ts:168-172)."""
        return [int(t) for t in undecided if g.clone().feed(self.pieces[int(t)])]

    def device_masks(self, g: ToolCallGrammar, output_bytes: int = 0, limit: int = 65536):
        """(allowed, undecided) bitmasks [ceil(vocab / 32)] from the device."""
        st = state_words(self.program, g)
        allowed = np.zeros(self.words, np.uint32)
        undecided = np.zeros(self.words, np.uint32)
        budget = max(0, limit - output_bytes)
        self.backend._check(self.lib.nd_grammar_mask(self.backend.ctx, self._grammar, L.ptr(st),
                                                     st.size, self._pieces, budget,
                                                     L.ptr(allowed), L.ptr(undecided)),
                            "nd_grammar_mask")
        return allowed, undecided

    def allowed(self, g: ToolCallGrammar, output_bytes: int = 0, limit: int = 65536) -> List[int]:
        """The allowed token ids of the agent loop (agent.ts:164-175), in id
        order: the device mask, with its undecided pieces settled by clones
        of the host grammar."""
        allowed, undecided = self.device_masks(g, output_bytes, limit)
        bits = np.unpackbits(allowed.view(np.uint8), bitorder="little")[: self.vocab]
        und = np.flatnonzero(np.unpackbits(undecided.view(np.uint8),
                                           bitorder="little")[: self.vocab])
        self.last_undecided = len(und)
        bits[und] = 0
        bits[self.settle(g, und)] = 1
        return [int(t) for t in np.flatnonzero(bits)]

    def free(self) -> None:
        if self._grammar:
            self.lib.nd_grammar_free(self.backend.ctx, self._grammar)
            self._grammar = C.c_void_p()
        if self._pieces:
            self.lib.nd_pieces_free(self.backend.ctx, self._pieces)
            self._pieces = C.c_void_p()
