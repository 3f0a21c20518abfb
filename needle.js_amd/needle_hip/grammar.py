"""Schema-constrained tool-call grammar: the host side of constrained decoding.

Mirrors tools/grammar.ts of needle.js (JsonSchemaGrammar, ToolCallGrammar)
and the parts of tools/schema.ts it needs (normalizeTools).  The grammar is
an incremental byte-level pushdown automaton over compact JSON: a stack of
frames (value, string, number, literal, choice, array, object, key) fed one
byte at a time, with JSON Schema checks when a value completes.  Behaviour
follows the reference step for step, including its retry limits (16 and 8
re-dispatches of one byte), its defaults (maxItems 32, maxProperties = the
number of declared properties, an absent schema reads as a string) and
JavaScript's number and JSON conventions (`JSON.stringify` spelling for
enum candidates, `Number()` parsing, `Math.round`).

The agent builds each step's allowed-token list by cloning the grammar for
every token piece and feeding it (tools/agent.ts:164-175); `allowed_pieces`
restates that loop.  On the GPU, `maskgen` compiles the tools and each
grammar state for the HIP mask kernel, which decides the same question for
every piece in parallel.

JavaScript regular expressions keep JavaScript's semantics: a string's
`pattern` runs on `jsregex` (RegExp without flags: Annex B syntax, UTF-16
code units, ECMAScript's \\s and ASCII \\d/\\w), and the email and uuid
`format`s on scanners of their two expressions with the same character
sets and anchors.  The reference's tests hold no schema with `pattern` or
`format`; these are pinned by the specification's own cases and by
cross-checks against an independent matcher where the dialects agree.
"""

from __future__ import annotations

import json
import math
import re
from typing import Any, List, Optional, Sequence

from . import jsregex
from .errors import NeedleError, invariant

_NAME_LITERAL = b'"name":"'  # grammar.ts:674
_ARGUMENTS_LITERAL = b',"arguments":'  # grammar.ts:675
# The code points the \s class of an ECMAScript regular expression matches
# (ECMA-262 WhiteSpace -- TAB, VT, FF, ZWNBSP and the Zs category -- and
# LineTerminator -- LF, CR, LS, PS).  Python's \s differs (it matches
# U+001C..U+001F and U+0085, not U+FEFF), so the format checks below are
# written out with this set instead of using `re`.
JS_SPACE = frozenset([0x09, 0x0A, 0x0B, 0x0C, 0x0D, 0x20, 0xA0, 0x1680, *range(0x2000, 0x200B),
                      0x2028, 0x2029, 0x202F, 0x205F, 0x3000, 0xFEFF])


def js_email(value: str) -> bool:
    r"""/^[^\s@]+@[^\s@]+\.[^\s@]+$/.test(value) (grammar.ts:191), `$` at the
    end of the input only: a local part, '@', then at least three characters
    without whitespace or '@' with a '.' after the first of them and before
    the last.  States: 0 start, 1 local part, 2 after '@', 3 domain, 4 after
    a usable '.', 5 accepting, 6 dead.  Characters step one at a time (a
    UTF-16 surrogate pair steps twice in JavaScript, through the same
    'other' transitions)."""
    state = 0
    for ch in value:
        c = ord(ch)
        at = c == 0x40
        other = not at and c not in JS_SPACE
        if state == 0:
            state = 1 if other else 6
        elif state == 1:
            state = 1 if other else (2 if at else 6)
        elif state == 2:
            state = 3 if other else 6
        elif state == 3:
            state = (4 if c == 0x2E else 3) if other else 6
        elif state in (4, 5):
            state = 5 if other else 6
        else:
            return False
    return state == 5


def js_uuid(value: str) -> bool:
    """/^[0-9a-f]{8}-[0-9a-f]{4}-[1-8][0-9a-f]{3}-[89ab][0-9a-f]{3}-[0-9a-f]{12}$/i
    .test(value) (grammar.ts:192-196): 36 characters, case-insensitive hex
    (no character outside ASCII folds into these classes)."""
    if len(value) != 36:
        return False
    for i, ch in enumerate(value):
        if i in (8, 13, 18, 23):
            ok = ch == "-"
        elif i == 14:
            ok = ch in "12345678"
        elif i == 19:
            ok = ch in "89abAB"
        else:
            ok = ch in "0123456789abcdefABCDEF"
        if not ok:
            return False
    return True


# ------------------------------------------------------------- JS semantics

def js_number_string(x: float) -> str:
    """Number.prototype.toString (radix 10) of a finite double: the shortest
    round-trip digits, exponent form below 1e-6 and from 1e21."""
    if isinstance(x, bool):
        raise TypeError("bool is not a number")
    if isinstance(x, int):
        x = float(x) if abs(x) >= 2**53 else x
        if isinstance(x, int):
            return str(x)
    if x == 0:
        return "0"
    if not math.isfinite(x):
        return "null"  # JSON.stringify spelling
    sign = "-" if x < 0 else ""
    digits, exponent = _shortest_digits(abs(x))
    n = exponent + len(digits)  # decimal point position
    k = len(digits)
    if k <= n <= 21:
        return sign + digits + "0" * (n - k)
    if 0 < n <= 21:
        return sign + digits[:n] + "." + digits[n:]
    if -6 < n <= 0:
        return sign + "0." + "0" * (-n) + digits
    e = n - 1
    mant = digits[0] + ("." + digits[1:] if k > 1 else "")
    return sign + mant + "e" + ("+" if e >= 0 else "-") + str(abs(e))


def _shortest_digits(x: float):
    """(digits, exponent) with x == int(digits) * 10**exponent, digits the
    shortest round-trip string (Python's repr gives the same digits)."""
    r = repr(x)
    if "e" in r or "E" in r:
        mant, exp = r.lower().split("e")
        exp = int(exp)
    else:
        mant, exp = r, 0
    if "." in mant:
        ip, fp = mant.split(".")
    else:
        ip, fp = mant, ""
    if fp == "0":
        fp = ""
    digits = (ip + fp).lstrip("0")
    exponent = exp - len(fp)
    stripped = digits.rstrip("0")
    exponent += len(digits) - len(stripped)
    return stripped or "0", exponent


def _js_string(s: str) -> str:
    out = ['"']
    for ch in s:
        o = ord(ch)
        if ch == '"':
            out.append('\\"')
        elif ch == "\\":
            out.append("\\\\")
        elif ch == "\b":
            out.append("\\b")
        elif ch == "\f":
            out.append("\\f")
        elif ch == "\n":
            out.append("\\n")
        elif ch == "\r":
            out.append("\\r")
        elif ch == "\t":
            out.append("\\t")
        elif o < 0x20 or 0xD800 <= o <= 0xDFFF:
            out.append("\\u%04x" % o)
        else:
            out.append(ch)
    out.append('"')
    return "".join(out)


def js_stringify(value: Any) -> str:
    """JSON.stringify without indentation (key order as inserted)."""
    if value is None:
        return "null"
    if value is True:
        return "true"
    if value is False:
        return "false"
    if isinstance(value, (int, float)):
        return js_number_string(value)
    if isinstance(value, str):
        return _js_string(value)
    if isinstance(value, (list, tuple)):
        return "[" + ",".join(js_stringify(v) for v in value) + "]"
    if isinstance(value, dict):
        return "{" + ",".join(_js_string(str(k)) + ":" + js_stringify(v)
                              for k, v in value.items()) + "}"
    raise TypeError(f"not a JSON value: {value!r}")


def _js_divide(a: float, b: float) -> float:
    """a / b in IEEE arithmetic as JavaScript evaluates it (Python raises on
    a zero divisor instead)."""
    if b == 0:
        if a == 0 or math.isnan(a):
            return math.nan
        return math.copysign(math.inf, a) * math.copysign(1.0, b)
    return a / b


def _js_round(x: float) -> float:
    """Math.round: the nearest integer, ties toward +Infinity; NaN and the
    infinities unchanged."""
    if not math.isfinite(x):
        return x
    r = math.floor(x)
    return r + 1 if x - r >= 0.5 else r


def _deep_equal(a, b) -> bool:
    return js_stringify(a) == js_stringify(b)


def _json_type(value) -> str:
    if value is None:
        return "null"
    if isinstance(value, bool):
        return "boolean"
    if isinstance(value, (int, float)):
        return "number"
    if isinstance(value, str):
        return "string"
    if isinstance(value, list):
        return "array"
    return "object"


# ---------------------------------------------------------------- schemas

def resolve_reference(schema: dict, root: dict) -> dict:
    """grammar.ts:120-143: local `#/...` refs, merged with the local keys."""
    ref = schema.get("$ref")
    if ref is None:
        return schema
    invariant(ref.startswith("#/"), "INVALID_TOOL_SCHEMA",
              f"Only local JSON Schema refs are supported; got {ref}")
    current: Any = root
    for raw in ref[2:].split("/"):
        part = raw.replace("~1", "/").replace("~0", "~")
        invariant(isinstance(current, dict) and part in current, "INVALID_TOOL_SCHEMA",
                  f"Unresolved JSON Schema ref {ref}")
        current = current[part]
    invariant(isinstance(current, dict), "INVALID_TOOL_SCHEMA",
              f"JSON Schema ref {ref} does not point to a schema")
    local = {k: v for k, v in schema.items() if k != "$ref"}
    return {**current, **local}


def schema_alternatives(schema: dict, root: dict) -> List[dict]:
    """grammar.ts:145-150: oneOf/anyOf flattened, refs resolved."""
    resolved = resolve_reference(schema, root)
    choices = resolved.get("oneOf", resolved.get("anyOf"))
    if choices is None:
        return [resolved]
    out: List[dict] = []
    for c in choices:
        out.extend(schema_alternatives(c, root))
    return out


def possible_types(schema: dict) -> List[str]:
    """grammar.ts:152-160."""
    t = schema.get("type")
    if t is not None and not isinstance(t, str):
        return list(t)
    if isinstance(t, str):
        return [t]
    if "properties" in schema:
        return ["object"]
    if "items" in schema:
        return ["array"]
    if "const" in schema:
        return [_json_type(schema["const"])]
    if schema.get("enum"):
        seen: List[str] = []
        for v in schema["enum"]:
            jt = _json_type(v)
            if jt not in seen:
                seen.append(jt)
        return seen
    return ["string"]


def type_starts_with(t: str, byte: int) -> bool:
    """grammar.ts:168-177."""
    if t == "string":
        return byte == 0x22
    if t == "object":
        return byte == 0x7B
    if t == "array":
        return byte == 0x5B
    if t == "boolean":
        return byte in (0x74, 0x66)
    if t == "null":
        return byte == 0x6E
    if t in ("number", "integer"):
        return byte == 0x2D or 0x30 <= byte <= 0x39
    return False


def validate_enum(value, schema: dict) -> bool:
    if "const" in schema and not _deep_equal(value, schema["const"]):
        return False
    if "enum" in schema and not any(_deep_equal(value, c) for c in schema["enum"]):
        return False
    return True


def validate_string(value: str, schema: dict) -> bool:
    """grammar.ts:179-203 (code points counted as Array.from does)."""
    length = len(value)
    if "minLength" in schema and length < schema["minLength"]:
        return False
    if "maxLength" in schema and length > schema["maxLength"]:
        return False
    if "pattern" in schema:
        try:
            if not jsregex.test(schema["pattern"], value):
                return False
        except jsregex.RegexSyntaxError as exc:
            raise NeedleError("INVALID_TOOL_SCHEMA",
                              f"Invalid JSON Schema pattern {schema['pattern']}", exc) from exc
        except RecursionError as exc:
            raise NeedleError("UNSUPPORTED_CACT",
                              f"pattern {schema['pattern']} nests too deeply for this value",
                              exc) from exc
    if schema.get("format") == "email" and not js_email(value):
        return False
    if schema.get("format") == "uuid" and not js_uuid(value):
        return False
    return validate_enum(value, schema)


def validate_number(value: float, schema: dict) -> bool:
    """grammar.ts:205-222."""
    if not math.isfinite(value):
        return False
    types = possible_types(schema)
    if "integer" in types and "number" not in types and not float(value).is_integer():
        return False
    if "minimum" in schema and value < schema["minimum"]:
        return False
    if "maximum" in schema and value > schema["maximum"]:
        return False
    if "exclusiveMinimum" in schema and value <= schema["exclusiveMinimum"]:
        return False
    if "exclusiveMaximum" in schema and value >= schema["exclusiveMaximum"]:
        return False
    if "multipleOf" in schema:
        q = _js_divide(value, schema["multipleOf"])
        if abs(q - _js_round(q)) > 1e-9 * max(1.0, abs(q)):
            return False
    return validate_enum(value, schema)


_NUMBER_PREFIX = re.compile(r"-?(?:0|[1-9][0-9]*)?(?:\.[0-9]*)?(?:[eE][+-]?[0-9]*)?")
_COMPLETE_NUMBER = re.compile(r"-?(?:0|[1-9]\d*)(?:\.\d+)?(?:[eE][+-]?\d+)?")


def is_number_prefix(text: str) -> bool:
    """grammar.ts:229-254, the scan as written (a fraction or exponent may
    follow a sign alone; '0' may not be followed by a digit)."""
    i, n = 0, len(text)
    if i < n and text[i] == "-":
        i += 1
    if i == n:
        return True
    if text[i] == "0":
        i += 1
        if i < n and text[i].isdigit() and text[i] in "0123456789":
            return False
    elif text[i] in "123456789":
        while i < n and text[i] in "0123456789":
            i += 1
    else:
        return False
    if i < n and text[i] == ".":
        i += 1
        while i < n and text[i] in "0123456789":
            i += 1
    if i < n and text[i] in "eE":
        i += 1
        if i < n and text[i] in "+-":
            i += 1
        while i < n and text[i] in "0123456789":
            i += 1
    return i == n


def is_complete_number(text: str) -> bool:
    return _COMPLETE_NUMBER.fullmatch(text) is not None


# ----------------------------------------------------------------- frames

class _Frame:
    __slots__ = ("kind", "schema", "bytes", "started", "escaped", "unicode", "text", "value",
                 "offset", "candidates", "phase", "values", "used", "current_key")

    def __init__(self, kind: str, **kw):
        self.kind = kind
        for k in self.__slots__[1:]:
            setattr(self, k, kw.get(k))

    def clone(self) -> "_Frame":
        """A frame of its own.  The containers this frame fills (bytes,
        candidates, items, properties) are copied; the completed values in
        them are shared, as nothing modifies a value once it is complete."""
        f = _Frame.__new__(_Frame)
        f.kind, f.schema, f.started, f.escaped = self.kind, self.schema, self.started, self.escaped
        f.unicode, f.text, f.offset, f.phase = self.unicode, self.text, self.offset, self.phase
        f.current_key = self.current_key
        f.bytes = None if self.bytes is None else list(self.bytes)
        # [bytes, value_or_name, offset, index]
        f.candidates = None if self.candidates is None else [list(c) for c in self.candidates]
        v = self.value
        f.value = dict(v) if isinstance(v, dict) else (list(v) if isinstance(v, list) else v)
        f.values = None if self.values is None else list(self.values)
        f.used = None if self.used is None else list(self.used)
        return f


class JsonSchemaGrammar:
    """Incremental compact-JSON grammar compiled from a JSON Schema
    (grammar.ts:256-631)."""

    def __init__(self, schema: dict):
        self.root_schema = schema
        self.stack: List[_Frame] = [_Frame("value", schema=schema)]
        self._complete = False
        self._value = None

    @property
    def complete(self) -> bool:
        if self._complete:
            return True
        if len(self.stack) == 1:
            f = self.stack[0]
            if f.kind == "choice" and any(c[2] == len(c[0]) for c in f.candidates):
                return True
        return False

    @property
    def value(self):
        if self._complete:
            return self._value
        f = self.stack[0] if len(self.stack) == 1 else None
        if f is not None and f.kind == "choice":
            for c in f.candidates:
                if c[2] == len(c[0]):
                    return c[1]
        return None

    def clone(self) -> "JsonSchemaGrammar":
        g = JsonSchemaGrammar.__new__(JsonSchemaGrammar)
        g.root_schema = self.root_schema
        g.stack = [f.clone() for f in self.stack]
        g._complete = self._complete
        g._value = self._value  # complete: never modified
        return g

    def feed(self, data: bytes) -> bool:
        for b in data:
            if not self.feed_byte(b):
                return False
        return True

    def feed_byte(self, byte: int) -> bool:
        if self._complete:
            return False
        root = self.root_schema
        for _ in range(16):
            if not self.stack:
                return False
            f = self.stack[-1]
            k = f.kind
            if k == "value":
                alts = schema_alternatives(f.schema, root)
                resolved = [resolve_reference(a, root) for a in alts]
                enum_values = []
                for a in resolved:
                    if "const" in a:
                        enum_values.append(a["const"])
                    elif "enum" in a:
                        enum_values.extend(a["enum"])
                if enum_values and all(("const" in a) or ("enum" in a) for a in resolved):
                    # [JSON bytes, value, offset, index]; the schema is kept
                    # for the device state's value index.
                    self.stack[-1] = _Frame("choice", schema=f.schema, candidates=[
                        [js_stringify(v).encode(), v, 0, i] for i, v in enumerate(enum_values)])
                    continue
                matching = [a for a in alts
                            if any(type_starts_with(t, byte)
                                   for t in possible_types(resolve_reference(a, root)))]
                if not matching:
                    return False
                schema = resolve_reference(matching[0], root)
                selected = next((t for t in possible_types(schema) if type_starts_with(t, byte)),
                                None)
                if selected is None:
                    return False
                if selected == "string":
                    self.stack[-1] = _Frame("string", schema=schema, bytes=[], started=False,
                                            escaped=False, unicode=0)
                elif selected in ("number", "integer"):
                    self.stack[-1] = _Frame("number", schema=schema, text="")
                elif selected == "boolean":
                    v = byte == 0x74
                    self.stack[-1] = _Frame("literal", bytes=b"true" if v else b"false", value=v,
                                            offset=0)
                elif selected == "null":
                    self.stack[-1] = _Frame("literal", bytes=b"null", value=None, offset=0)
                elif selected == "array":
                    self.stack[-1] = _Frame("array", schema=schema, phase="open", values=[])
                elif selected == "object":
                    self.stack[-1] = _Frame("object", schema=schema, phase="open", value={},
                                            used=[])
                else:
                    return False
                continue
            if k == "string":
                if not f.started:
                    if byte != 0x22:
                        return False
                    f.started = True
                    f.bytes.append(byte)
                    return True
                if f.unicode > 0:
                    if not (0x30 <= byte <= 0x39 or 0x41 <= byte <= 0x46 or 0x61 <= byte <= 0x66):
                        return False
                    f.unicode -= 1
                    f.bytes.append(byte)
                    return True
                if f.escaped:
                    if byte not in (0x22, 0x5C, 0x2F, 0x62, 0x66, 0x6E, 0x72, 0x74, 0x75):
                        return False
                    f.escaped = False
                    if byte == 0x75:
                        f.unicode = 4
                    f.bytes.append(byte)
                    return True
                if byte == 0x5C:
                    f.escaped = True
                    f.bytes.append(byte)
                    return True
                if byte < 0x20:
                    return False
                f.bytes.append(byte)
                if byte != 0x22:
                    return True
                try:
                    value = json.loads(bytes(f.bytes).decode("utf-8", errors="strict"))
                except (UnicodeDecodeError, ValueError):
                    return False
                if not isinstance(value, str) or not validate_string(value, f.schema):
                    return False
                self._finish(value)
                return True
            if k == "number":
                ch = chr(byte)
                if ch in "0123456789eE+-.":
                    nxt = f.text + ch
                    if not is_number_prefix(nxt):
                        return False
                    f.text = nxt
                    return True
                if not is_complete_number(f.text):
                    return False
                value = float(f.text)
                if not validate_number(value, f.schema):
                    return False
                self._finish(int(value) if value.is_integer() and abs(value) < 2**53 else value)
                continue
            if k == "literal":
                if byte != f.bytes[f.offset]:
                    return False
                f.offset += 1
                if f.offset == len(f.bytes):
                    self._finish(f.value)
                return True
            if k == "choice":
                cont = [c for c in f.candidates if c[2] < len(c[0]) and c[0][c[2]] == byte]
                if cont:
                    for c in cont:
                        c[2] += 1
                    f.candidates = cont
                    return True
                done = next((c for c in f.candidates if c[2] == len(c[0])), None)
                if done is None:
                    return False
                self._finish(done[1])
                continue
            if k == "array":
                s = f.schema
                if f.phase == "open":
                    if byte != 0x5B:
                        return False
                    f.phase = "first-or-end"
                    return True
                minimum = s.get("minItems", 0)
                maximum = s.get("maxItems", 32)
                if f.phase == "first-or-end":
                    if byte == 0x5D:
                        if len(f.values) < minimum or not validate_enum(f.values, s):
                            return False
                        self._finish(f.values)
                        return True
                    if len(f.values) >= maximum:
                        return False
                    f.phase = "value"
                    self.stack.append(_Frame("value", schema=s.get("items", {})))
                    continue
                if f.phase == "after-value":
                    if byte == 0x2C and len(f.values) < maximum:
                        f.phase = "value"
                        self.stack.append(_Frame("value", schema=s.get("items", {})))
                        return True
                    if byte == 0x5D and len(f.values) >= minimum:
                        if s.get("uniqueItems"):
                            ser = [js_stringify(v) for v in f.values]
                            if len(set(ser)) != len(ser):
                                return False
                        if not validate_enum(f.values, s):
                            return False
                        self._finish(f.values)
                        return True
                    return False
                return False
            if k == "object":
                s = f.schema
                if f.phase == "open":
                    if byte != 0x7B:
                        return False
                    f.phase = "key-or-end"
                    return True
                props = s.get("properties", {})
                required = s.get("required", [])
                minimum = s.get("minProperties", 0)
                maximum = s.get("maxProperties", len(props))
                if f.phase in ("key-or-end", "key-required"):
                    if byte == 0x7D and f.phase == "key-or-end":
                        if len(f.used) < minimum or any(n not in f.used for n in required):
                            return False
                        if not validate_enum(f.value, s):
                            return False
                        self._finish(f.value)
                        return True
                    if byte != 0x22 or len(f.used) >= maximum:
                        return False
                    cands = [[n.encode(), n, 0, i] for i, n in enumerate(props)
                             if n not in f.used]
                    if not cands:
                        return False
                    f.phase = "key"
                    self.stack.append(_Frame("key", candidates=cands))
                    return True
                if f.phase == "colon":
                    if byte != 0x3A or f.current_key is None:
                        return False
                    f.phase = "value"
                    ap = s.get("additionalProperties")
                    sub = props.get(f.current_key, ap if isinstance(ap, dict) else {})
                    self.stack.append(_Frame("value", schema=sub))
                    return True
                if f.phase == "after-value":
                    if byte == 0x2C and len(f.used) < maximum:
                        f.phase = "key-required"
                        return True
                    if (byte == 0x7D and len(f.used) >= minimum
                            and all(n in f.used for n in required)):
                        if not validate_enum(f.value, s):
                            return False
                        self._finish(f.value)
                        return True
                    return False
                return False
            if k == "key":
                if byte == 0x22:
                    done = next((c for c in f.candidates if c[2] == len(c[0])), None)
                    if done is None:
                        return False
                    self.stack.pop()
                    parent = self.stack[-1] if self.stack else None
                    if parent is None or parent.kind != "object":
                        return False
                    parent.current_key = done[1]
                    parent.phase = "colon"
                    return True
                cont = [c for c in f.candidates if c[2] < len(c[0]) and c[0][c[2]] == byte]
                if not cont:
                    return False
                for c in cont:
                    c[2] += 1
                f.candidates = cont
                return True
        return False

    def _finish(self, value) -> None:
        self.stack.pop()
        parent = self.stack[-1] if self.stack else None
        if parent is None:
            self._complete = True
            self._value = value
            return
        if parent.kind == "array" and parent.phase == "value":
            parent.values.append(value)
            parent.phase = "after-value"
            return
        if parent.kind == "object" and parent.phase == "value" and parent.current_key is not None:
            parent.value[parent.current_key] = value
            parent.used.append(parent.current_key)
            parent.current_key = None
            parent.phase = "after-value"
            return
        raise NeedleError("INVALID_TOOL_SCHEMA", "Internal JSON Schema grammar stack is inconsistent")


class ToolCallGrammar:
    """Needle's array-of-tool-calls byte grammar (grammar.ts:677-797)."""

    def __init__(self, tools: Sequence[dict], maximum_calls: int = 4):
        invariant(len(tools) > 0, "INVALID_TOOL_SCHEMA", "Tool-call grammar needs at least one tool")
        self.tools = list(tools)
        self.maximum_calls = max(1, maximum_calls)
        self.phase = "array-open"
        self.literal_offset = 0
        self.name_candidates: List[list] = []  # [index, bytes, offset]
        self.current_tool = -1
        self.used_tools: List[int] = []
        self.arguments: Optional[JsonSchemaGrammar] = None
        self.calls: List[dict] = []

    @property
    def complete(self) -> bool:
        return self.phase == "done"

    def clone(self) -> "ToolCallGrammar":
        g = ToolCallGrammar.__new__(ToolCallGrammar)
        g.tools = self.tools
        g.maximum_calls = self.maximum_calls
        g.phase = self.phase
        g.literal_offset = self.literal_offset
        g.name_candidates = [list(c) for c in self.name_candidates]
        g.current_tool = self.current_tool
        g.used_tools = list(self.used_tools)
        g.arguments = self.arguments.clone() if self.arguments is not None else None
        g.calls = list(self.calls)  # completed calls are never modified
        return g

    def feed(self, data: bytes) -> bool:
        for b in data:
            if not self.feed_byte(b):
                return False
        return True

    def feed_byte(self, byte: int) -> bool:
        for _ in range(8):
            p = self.phase
            if p == "array-open":
                if byte != 0x5B:
                    return False
                self.phase = "call-open"
                return True
            if p == "call-open":
                if byte != 0x7B:
                    return False
                self.phase = "name-literal"
                self.literal_offset = 0
                return True
            if p == "name-literal":
                if byte != _NAME_LITERAL[self.literal_offset]:
                    return False
                self.literal_offset += 1
                if self.literal_offset == len(_NAME_LITERAL):
                    self.phase = "tool-name"
                    self.name_candidates = [[i, t["name"].encode(), 0]
                                            for i, t in enumerate(self.tools)
                                            if i not in self.used_tools]
                return True
            if p == "tool-name":
                if byte == 0x22:
                    c = next((e for e in self.name_candidates if e[2] == len(e[1])), None)
                    if c is None:
                        return False
                    self.current_tool = c[0]
                    self.phase = "arguments-literal"
                    self.literal_offset = 0
                    return True
                cont = [c for c in self.name_candidates if c[2] < len(c[1]) and c[1][c[2]] == byte]
                if not cont:
                    return False
                for c in cont:
                    c[2] += 1
                self.name_candidates = cont
                return True
            if p == "arguments-literal":
                if byte != _ARGUMENTS_LITERAL[self.literal_offset]:
                    return False
                self.literal_offset += 1
                if self.literal_offset == len(_ARGUMENTS_LITERAL):
                    if not (0 <= self.current_tool < len(self.tools)):
                        return False
                    self.arguments = JsonSchemaGrammar(self.tools[self.current_tool]["parameters"])
                    self.phase = "arguments"
                return True
            if p == "arguments":
                g = self.arguments
                if g is None:
                    return False
                if g.complete:
                    self.phase = "call-close"
                    continue
                return g.feed_byte(byte)
            if p == "call-close":
                if byte != 0x7D:
                    return False
                tool = self.tools[self.current_tool] if 0 <= self.current_tool < len(self.tools) \
                    else None
                args = self.arguments.value if self.arguments is not None else None
                if tool is None or not isinstance(args, dict):
                    return False
                self.calls.append({"name": tool["name"], "arguments": args})
                self.used_tools.append(self.current_tool)
                self.phase = "after-call"
                return True
            if p == "after-call":
                if byte == 0x5D:
                    self.phase = "done"
                    return True
                if (byte == 0x2C and len(self.calls) < self.maximum_calls
                        and len(self.used_tools) < len(self.tools)):
                    self.phase = "call-open"
                    return True
                return False
            return False
        return False


def normalize_tools(inputs: Sequence[dict]) -> List[dict]:
    """normalizeTools (tools/schema.ts:138-203) for {name, parameters} or
    OpenAI {function: {...}} dicts."""
    tools, names = [], set()
    for raw in inputs:
        if "function" in raw:
            raw = raw["function"]
        name = raw.get("name")
        invariant(isinstance(name, str) and 0 < len(name) <= 128, "INVALID_TOOL_SCHEMA",
                  "A tool name must contain 1–128 characters")
        invariant(not any(c in '"\\' or ord(c) < 0x20 for c in name), "INVALID_TOOL_SCHEMA",
                  f"Tool name {json.dumps(name)} contains characters that cannot be constrained safely")
        params = raw.get("parameters") or {"type": "object", "properties": {}}
        invariant(params.get("type") in ("object", None), "INVALID_TOOL_SCHEMA",
                  f"Tool {name} parameters must be an object schema")
        props = params.get("properties", {})
        for pname, sch in props.items():
            invariant(len(pname) > 0 and not any(c in '"\\' or ord(c) < 0x20 for c in pname),
                      "INVALID_TOOL_SCHEMA", f"Tool {name} has an invalid parameter name")
            invariant(isinstance(sch, dict), "INVALID_TOOL_SCHEMA",
                      f"Tool {name} parameter {pname} has no schema")
        for req in params.get("required", []):
            invariant(req in props, "INVALID_TOOL_SCHEMA",
                      f"Tool {name} requires unknown parameter {req}")
        invariant(name not in names, "INVALID_TOOL_SCHEMA", f"Duplicate tool name {name}")
        names.add(name)
        tools.append({"name": name, "parameters": {**params, "type": "object", "properties": props}})
    return tools


def allowed_pieces(grammar: ToolCallGrammar, pieces: Sequence[bytes], eligible: Sequence[bool],
                   output_bytes: int = 0, limit: int = 65536) -> List[int]:
    """The candidate loop of tools/agent.ts:164-175: every eligible, non-empty
    piece that fits under the output limit and that a clone of the grammar
    accepts, in id order."""
    out = []
    for tok, data in enumerate(pieces):
        if not eligible[tok] or len(data) == 0 or output_bytes + len(data) > limit:
            continue
        if grammar.clone().feed(data):
            out.append(tok)
    return out
