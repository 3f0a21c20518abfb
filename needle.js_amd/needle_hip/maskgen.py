"""Allowed-token masks of the tool-call grammar on the GPU.

The agent's constrained loop (tools/agent.ts:157-210) asks, every step,
which token pieces a clone of the grammar accepts.  `GrammarMasker` answers
on the device: the tool schemas are compiled once into a program
(`GrammarProgram`), each step's grammar state is serialized into a few
hundred bytes (`state_words`), and one HIP thread per piece runs the grammar
over its bytes (nd_grammar_mask, csrc/grammar.hip).  Pieces whose answer
needs a check the device does not make (regular-expression patterns,
string lengths, numeric bounds, enum/const/uniqueness of values) come back
undecided, and the host grammar -- which owns the state -- settles exactly
those.  Layouts are documented with nd_grammar_upload / nd_grammar_mask in
include/needle_hip.h.
"""

from __future__ import annotations

import ctypes as C
from typing import Dict, List, Sequence, Tuple

import numpy as np

from . import lib as L
from .errors import NeedleError, invariant
from .grammar import (ToolCallGrammar, js_stringify, possible_types, resolve_reference,
                      schema_alternatives)

MAGIC = 0x4E444752
NONE = 0xFFFFFFFF
MAX_DEPTH = 24
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
        self._node_ix: Dict[Tuple[int, str], int] = {}
        self._value_ix: Dict[Tuple[int, str], int] = {}
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
        key = (ti, js_stringify(schema))
        if key in self._value_ix:
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
        key = (ti, js_stringify(s))
        if key in self._node_ix:
            return self._node_ix[key]
        idx = len(self.nodes)
        self._node_ix[key] = idx
        self.nodes.append([0] * 12)
        types = possible_types(s)
        tmask = 0
        for t in types:
            tmask |= _TYPE_BITS.get(t, 0)
        flags = 0
        if any(k in s for k in ("minLength", "maxLength", "pattern", "const", "enum")) or \
                s.get("format") in ("email", "uuid"):
            flags |= 1
        if any(k in s for k in ("minimum", "maximum", "exclusiveMinimum", "exclusiveMaximum",
                                "multipleOf", "const", "enum")):
            flags |= 2
        if "integer" in types and "number" not in types:
            flags |= 4
        if "const" in s or "enum" in s or s.get("uniqueItems"):
            flags |= 8
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
                           int(s.get("maxProperties", len(props))), 0, 0]
        return idx

    def words(self) -> np.ndarray:
        tables = [np.asarray(self.nodes, np.uint32).reshape(-1, 12),
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
        pool = bytes(self.pool)
        pool_words = np.frombuffer(pool + b"\0" * (-len(pool) % 4), np.uint32)
        header[13] = off * 4
        header[14] = len(pool)
        return np.concatenate([header] + [t.reshape(-1) for t in tables] + [pool_words]).astype(
            np.uint32)


def _utf8_state(data) -> int:
    s = 0
    for b in data:
        if s == 0:
            s = (0 if b < 0x80 else 1 if 0xC2 <= b <= 0xDF else 4 if b == 0xE0 else
                 5 if b == 0xED else 2 if 0xE1 <= b <= 0xEF else 6 if b == 0xF0 else
                 3 if 0xF1 <= b <= 0xF3 else 7 if b == 0xF4 else 8)
        elif s == 1:
            s = 0 if 0x80 <= b <= 0xBF else 8
        elif s == 2:
            s = 1 if 0x80 <= b <= 0xBF else 8
        elif s == 3:
            s = 2 if 0x80 <= b <= 0xBF else 8
        elif s == 4:
            s = 1 if 0xA0 <= b <= 0xBF else 8
        elif s == 5:
            s = 1 if 0x80 <= b <= 0x9F else 8
        elif s == 6:
            s = 2 if 0x90 <= b <= 0xBF else 8
        elif s == 7:
            s = 2 if 0x80 <= b <= 0x8F else 8
    return s


def _number_state(text: str):
    """(DFA state, exponent seen, nonzero fraction digit, integer digits)."""
    s, exp, frac, digits = 0, False, False, 0
    for ch in text:
        d = ch.isdigit()
        if s == 0:
            s = 1 if ch == "-" else 2 if ch == "0" else 3 if d else 9
        elif s == 1:
            s = 2 if ch == "0" else 3 if d else 9
        elif s == 2:
            s = 4 if ch == "." else 6 if ch in "eE" else 9
        elif s == 3:
            s = 3 if d else 4 if ch == "." else 6 if ch in "eE" else 9
        elif s == 4:
            s = 5 if d else 10 if ch in "eE" else 9
        elif s == 5:
            s = 5 if d else 6 if ch in "eE" else 9
        elif s == 6:
            s = 7 if ch in "+-" else 8 if d else 9
        elif s in (7, 8):
            s = 8 if d else 9
        elif s == 10:
            s = 11 if ch in "+-" else 12 if d else 9
        elif s in (11, 12):
            s = 12 if d else 9
        if s in (6, 10):
            exp = True
        if s == 5 and ch != "0":
            frac = True
        if s in (2, 3):
            digits += 1
    return s, exp, frac, min(digits, 1000)


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
                frames.append([2 | flags << 16, program.node_of(ti, f.schema), 0, 0])
            elif k == "number":
                s, exp, frac, digits = _number_state(f.text)
                flags = (1 if exp else 0) | (2 if frac else 0)
                frames.append([3 | s << 8 | flags << 16, program.node_of(ti, f.schema), 0, digits])
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
                frames.append([6 | _ARRAY_PHASES[f.phase] << 8, program.node_of(ti, f.schema), 0,
                               len(f.values)])
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
        for t in und:
            bits[t] = 1 if g.clone().feed(self.pieces[t]) else 0
        return [int(t) for t in np.flatnonzero(bits)]

    def free(self) -> None:
        if self._grammar:
            self.lib.nd_grammar_free(self.backend.ctx, self._grammar)
            self._grammar = C.c_void_p()
        if self._pieces:
            self.lib.nd_pieces_free(self.backend.ctx, self._pieces)
            self._pieces = C.c_void_p()
