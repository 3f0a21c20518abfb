"""JavaScript regular expressions as the tool-call grammar evaluates a string
schema's `pattern`: `new RegExp(schema.pattern).test(value)`
(packages/needle.js/src/tools/grammar.ts:184-193).

No flags are given there, so the pattern is parsed by ECMAScript's
non-Unicode grammar with the web-compatibility extensions (Annex B: `]`,
`{` and `}` as literals where they cannot be syntax, legacy octal escapes,
`\\c` without a control letter, identity escapes of any character but `c`
and, where the pattern names a group, `k`), and both the pattern and the
value are sequences of UTF-16 code units: `.` and classes match one code
unit, so a character above U+FFFF is two.  `\\d`, `\\w` and `\\b` are ASCII;
`\\s` is ECMAScript's WhiteSpace and LineTerminator set; `.` excludes the
four line terminators; `^` and `$` match only at the ends of the value.

Two evaluators share the parser:

- `test()` runs the pattern the way the specification's matcher does:
  backtracking over the value from every start position, captures reset at
  each iteration of a quantified group, an iteration that consumes nothing
  rejected once the minimum is reached, a backreference to a group that did
  not take part matching the empty string, lookbehind matching right to
  left.  The host grammar uses it.
- `compile_dfa()` builds, for a pattern without backreferences, lookaround
  or word boundaries, a deterministic automaton over classes of code units
  whose states summarise every match attempt at once: state 0 at the start
  of the value, a state flagged "accepts at end" when the value read so far
  is matched.  The device grammar steps it per code unit of a string.
"""

from __future__ import annotations

from typing import Dict, List, Optional, Sequence, Tuple

MAX_UNIT = 0xFFFF
_INF = None  # an unbounded repeat

# Character sets are sorted tuples of disjoint, non-adjacent (lo, hi)
# intervals of code units.
CharSet = Tuple[Tuple[int, int], ...]


class RegexSyntaxError(ValueError):
    """The pattern is not a JavaScript regular expression (RegExp throws
    SyntaxError)."""


class NotRegular(ValueError):
    """The pattern uses a feature the automaton cannot express."""


def _norm(intervals) -> CharSet:
    out: List[List[int]] = []
    for lo, hi in sorted(intervals):
        if out and lo <= out[-1][1] + 1:
            out[-1][1] = max(out[-1][1], hi)
        else:
            out.append([lo, hi])
    return tuple((a, b) for a, b in out)


def _complement(cs: CharSet) -> CharSet:
    out, at = [], 0
    for lo, hi in cs:
        if lo > at:
            out.append((at, lo - 1))
        at = hi + 1
    if at <= MAX_UNIT:
        out.append((at, MAX_UNIT))
    return tuple(out)


def _contains(cs: CharSet, u: int) -> bool:
    lo, hi = 0, len(cs)
    while lo < hi:
        mid = (lo + hi) // 2
        if cs[mid][1] < u:
            lo = mid + 1
        else:
            hi = mid
    return lo < len(cs) and cs[lo][0] <= u


DIGIT = _norm([(0x30, 0x39)])
WORD = _norm([(0x30, 0x39), (0x41, 0x5A), (0x5F, 0x5F), (0x61, 0x7A)])
# WhiteSpace (TAB, VT, FF, SP, NBSP, ZWNBSP, the Zs category) and
# LineTerminator (LF, CR, LS, PS).
SPACE = _norm([(0x09, 0x0D), (0x20, 0x20), (0xA0, 0xA0), (0x1680, 0x1680), (0x2000, 0x200A),
               (0x2028, 0x2029), (0x202F, 0x202F), (0x205F, 0x205F), (0x3000, 0x3000),
               (0xFEFF, 0xFEFF)])
LINE_TERMINATORS = _norm([(0x0A, 0x0A), (0x0D, 0x0D), (0x2028, 0x2029)])
DOT = _complement(LINE_TERMINATORS)
_CLASS_ESCAPES = {"d": DIGIT, "D": _complement(DIGIT), "s": SPACE, "S": _complement(SPACE),
                  "w": WORD, "W": _complement(WORD)}
_CONTROL = {"f": 0x0C, "n": 0x0A, "r": 0x0D, "t": 0x09, "v": 0x0B}


def utf16_units(text: str) -> List[int]:
    """The UTF-16 code units of a Python string (lone surrogates kept)."""
    data = text.encode("utf-16-le", "surrogatepass")
    return [data[i] | (data[i + 1] << 8) for i in range(0, len(data), 2)]


# ---------------------------------------------------------------- parser
# AST: ("set", CharSet) | ("seq", [..]) | ("alt", [..]) | ("group", index or
# 0, node) | ("repeat", node, min, max or None, greedy, first group, end
# group) | ("bol",) | ("eol",) | ("wordb", negated) | ("look", ahead,
# negated, node) | ("backref", index).


def _is_id_start(u: int) -> bool:
    c = chr(u) if u < 0xD800 or u > 0xDFFF else ""
    return c == "$" or c == "_" or c.isalpha()


def _is_id_part(u: int) -> bool:
    c = chr(u) if u < 0xD800 or u > 0xDFFF else ""
    return c in ("$", "_", "\u200c", "\u200d") or c.isalnum()


class _Parser:
    def __init__(self, pattern: str):
        self.p = utf16_units(pattern)
        self.i = 0
        self.n_groups, self.names = self._scan_groups()
        self.named = bool(self.names)
        self.group_count = 0
        self.seen_names: Dict[str, int] = {}

    # The capture count and group names, known before parsing as the
    # specification's early errors and Annex B's escape rules need them.
    def _scan_groups(self):
        p, i, count, names, in_class = self.p, 0, 0, {}, False
        while i < len(p):
            c = p[i]
            if c == 0x5C:
                i += 2
                continue
            if in_class:
                in_class = c != 0x5D
            elif c == 0x5B:
                in_class = True
            elif c == 0x28:
                if i + 1 < len(p) and p[i + 1] == 0x3F:
                    if i + 2 < len(p) and p[i + 2] == 0x3C and i + 3 < len(p) and \
                            p[i + 3] not in (0x3D, 0x21):
                        count += 1
                        j = i + 3
                        while j < len(p) and p[j] != 0x3E:
                            j += 1
                        names["".join(chr(u) for u in p[i + 3:j])] = count
                else:
                    count += 1
            i += 1
        return count, names

    def peek(self, k: int = 0) -> int:
        j = self.i + k
        return self.p[j] if j < len(self.p) else -1

    def eat(self, u: int) -> bool:
        if self.peek() == u:
            self.i += 1
            return True
        return False

    def fail(self, why: str):
        raise RegexSyntaxError(why)

    def parse(self):
        node = self.disjunction()
        if self.i < len(self.p):
            self.fail("Unmatched ')'")
        return node

    def disjunction(self):
        alts = [self.alternative()]
        while self.eat(0x7C):
            alts.append(self.alternative())
        return alts[0] if len(alts) == 1 else ("alt", alts)

    def alternative(self):
        terms = []
        while self.i < len(self.p) and self.peek() not in (0x7C, 0x29):
            terms.append(self.term())
        return terms[0] if len(terms) == 1 else ("seq", terms)

    def term(self):
        c = self.peek()
        if c == 0x5E:
            self.i += 1
            return ("bol",)
        if c == 0x24:
            self.i += 1
            return ("eol",)
        if c == 0x5C and self.peek(1) in (0x62, 0x42):
            self.i += 2
            return ("wordb", self.p[self.i - 1] == 0x42)
        if c == 0x28 and self.peek(1) == 0x3F:
            kind = self.peek(2)
            if kind in (0x3D, 0x21) or (kind == 0x3C and self.peek(3) in (0x3D, 0x21)):
                behind = kind == 0x3C
                negated = self.peek(3 if behind else 2) == 0x21
                self.i += 4 if behind else 3
                first = self.group_count
                node = self.disjunction()
                if not self.eat(0x29):
                    self.fail("Unterminated group")
                look = ("look", not behind, negated, node)
                if not behind:  # Annex B: a lookahead may be quantified
                    return self.quantified(look, first)
                if self.quantifier_here():
                    self.fail("Invalid quantifier after a lookbehind")
                return look
        first = self.group_count
        return self.quantified(self.atom(), first)

    def quantifier_here(self) -> bool:
        c = self.peek()
        return c in (0x2A, 0x2B, 0x3F) or (c == 0x7B and self.braced(False) is not None)

    def braced(self, consume: bool):
        """{n}, {n,} or {n,m} at the cursor: (n, m or None) or None."""
        j = self.i + 1
        p = self.p

        def digits(j):
            k = j
            while k < len(p) and 0x30 <= p[k] <= 0x39:
                k += 1
            return k

        k = digits(j)
        if k == j:
            return None
        lo = int("".join(chr(u) for u in p[j:k]))
        hi: Optional[int] = lo
        if k < len(p) and p[k] == 0x2C:
            k2 = digits(k + 1)
            hi = int("".join(chr(u) for u in p[k + 1:k2])) if k2 > k + 1 else None
            k = k2
        if k >= len(p) or p[k] != 0x7D:
            return None
        if consume:
            self.i = k + 1
        return lo, hi

    def quantified(self, atom, first_group: int):
        c = self.peek()
        if c == 0x2A:
            lo, hi = 0, None
            self.i += 1
        elif c == 0x2B:
            lo, hi = 1, None
            self.i += 1
        elif c == 0x3F:
            lo, hi = 0, 1
            self.i += 1
        elif c == 0x7B and self.braced(False) is not None:
            lo, hi = self.braced(True)
            if hi is not None and hi < lo:
                self.fail("numbers out of order in {} quantifier")
        else:
            return atom
        greedy = not self.eat(0x3F)
        return ("repeat", atom, lo, hi, greedy, first_group + 1, self.group_count)

    def atom(self):
        c = self.peek()
        if c == 0x2E:
            self.i += 1
            return ("set", DOT)
        if c == 0x28:
            self.i += 1
            index = 0
            if self.peek() == 0x3F:
                if self.peek(1) == 0x3A:
                    self.i += 2
                elif self.peek(1) == 0x3C:
                    self.i += 2
                    name = self.group_name()
                    self.group_count += 1
                    index = self.group_count
                    if name in self.seen_names:
                        self.fail("Duplicate capture group name")
                    self.seen_names[name] = index
                else:
                    self.fail("Invalid group")
            else:
                self.group_count += 1
                index = self.group_count
            node = self.disjunction()
            if not self.eat(0x29):
                self.fail("Unterminated group")
            return ("group", index, node)
        if c == 0x5B:
            return ("set", self.char_class())
        if c == 0x5C:
            return self.atom_escape()
        if c in (0x2A, 0x2B, 0x3F):
            self.fail("Nothing to repeat")
        if c == 0x7B and self.braced(False) is not None:
            self.fail("Nothing to repeat")
        self.i += 1  # a pattern character, `]`, `{` and `}` included
        return ("set", ((c, c),))

    def group_name(self) -> str:
        start = self.i
        if not _is_id_start(self.peek()):
            self.fail("Invalid capture group name")
        self.i += 1
        while _is_id_part(self.peek()):
            self.i += 1
        if not self.eat(0x3E):
            self.fail("Invalid capture group name")
        return "".join(chr(u) for u in self.p[start:self.i - 1])

    def hex_digits(self, count: int) -> Optional[int]:
        ds = self.p[self.i:self.i + count]
        if len(ds) < count or not all(chr(u) in "0123456789abcdefABCDEF" for u in ds):
            return None
        self.i += count
        return int("".join(chr(u) for u in ds), 16)

    def legacy_octal(self) -> int:
        """LegacyOctalEscapeSequence at the cursor (its first digit is 0-7)."""
        p = self.p
        first = p[self.i] - 0x30
        self.i += 1
        value = first
        limit = 2 if first <= 3 else 1
        for _ in range(limit):
            if 0x30 <= self.peek() <= 0x37:
                value = value * 8 + self.p[self.i] - 0x30
                self.i += 1
            else:
                break
        return value

    def character_escape(self, in_class: bool) -> Optional[int]:
        """A CharacterEscape after the backslash (cursor on the letter), or
        None for `\\c` without a control letter (the backslash is then a
        literal and the cursor stays on `c`)."""
        c = self.peek()
        if c in (0x66, 0x6E, 0x72, 0x74, 0x76):
            self.i += 1
            return _CONTROL[chr(c)]
        if c == 0x63:
            nxt = self.peek(1)
            if (0x41 <= nxt <= 0x5A) or (0x61 <= nxt <= 0x7A) or \
                    (in_class and (0x30 <= nxt <= 0x39 or nxt == 0x5F)):
                self.i += 2
                return nxt % 32
            return None
        if c == 0x30 and not (0x30 <= self.peek(1) <= 0x39):
            self.i += 1
            return 0
        if 0x30 <= c <= 0x37:
            return self.legacy_octal()
        if c == 0x78:
            self.i += 1
            v = self.hex_digits(2)
            return 0x78 if v is None else v
        if c == 0x75:
            self.i += 1
            v = self.hex_digits(4)
            return 0x75 if v is None else v
        if c == 0x6B and self.named:
            self.fail("Invalid named reference")
        self.i += 1  # identity escape
        return c

    def atom_escape(self):
        self.i += 1
        c = self.peek()
        if c < 0:
            self.fail("\\ at end of pattern")
        if chr(c) in _CLASS_ESCAPES:
            self.i += 1
            return ("set", _CLASS_ESCAPES[chr(c)])
        if 0x31 <= c <= 0x39:
            j = self.i
            while j < len(self.p) and 0x30 <= self.p[j] <= 0x39:
                j += 1
            n = int("".join(chr(u) for u in self.p[self.i:j]))
            if n <= self.n_groups:
                self.i = j
                return ("backref", n)
            if c >= 0x38:  # \8, \9: identity escapes
                self.i += 1
                return ("set", ((c, c),))
            v = self.legacy_octal()
            return ("set", ((v, v),))
        if c == 0x6B and self.named:
            self.i += 1
            if not self.eat(0x3C):
                self.fail("Invalid named reference")
            name = self.group_name()
            if name not in self.names:
                self.fail("Invalid named capture referenced")
            return ("backref", self.names[name])
        v = self.character_escape(False)
        if v is None:
            return ("set", ((0x5C, 0x5C),))
        return ("set", ((v, v),))

    def class_atom(self):
        """One ClassAtom: (CharSet, is a class escape)."""
        c = self.peek()
        if c < 0:
            self.fail("Unterminated character class")
        if c != 0x5C:
            self.i += 1
            return ((c, c),), False
        self.i += 1
        c = self.peek()
        if c < 0:
            self.fail("\\ at end of pattern")
        if chr(c) in _CLASS_ESCAPES:
            self.i += 1
            return _CLASS_ESCAPES[chr(c)], True
        if c == 0x62:
            self.i += 1
            return ((8, 8),), False
        if c == 0x2D:
            self.i += 1
            return ((0x2D, 0x2D),), False
        if 0x38 <= c <= 0x39:
            self.i += 1
            return ((c, c),), False
        v = self.character_escape(True)
        if v is None:
            return ((0x5C, 0x5C),), False
        return ((v, v),), False

    def char_class(self) -> CharSet:
        self.i += 1
        negated = self.eat(0x5E)
        parts: List[Tuple[int, int]] = []
        while True:
            if self.peek() < 0:
                self.fail("Unterminated character class")
            if self.eat(0x5D):
                break
            left, left_escape = self.class_atom()
            if self.peek() == 0x2D and self.peek(1) not in (0x5D, -1):
                self.i += 1
                right, right_escape = self.class_atom()
                if left_escape or right_escape:  # Annex B: `-` is a literal here
                    parts.extend(left)
                    parts.append((0x2D, 0x2D))
                    parts.extend(right)
                    continue
                lo, hi = left[0][0], right[0][0]
                if lo > hi:
                    self.fail("Range out of order in character class")
                parts.append((lo, hi))
                continue
            parts.extend(left)
        cs = _norm(parts)
        return _complement(cs) if negated else cs


def parse(pattern: str):
    """The pattern's syntax tree and its number of capturing groups;
    RegexSyntaxError where RegExp would throw."""
    p = _Parser(pattern)
    return p.parse(), p.n_groups


# ---------------------------------------------------------------- matcher


def _is_word(s: Sequence[int], i: int) -> bool:
    return 0 <= i < len(s) and _contains(WORD, s[i])


def _compile(node, forward: bool):
    """A matcher m(s, pos, caps, k) -> bool: match `node` at pos (reading
    rightwards when forward, else leftwards), then the continuation
    k(pos, caps)."""
    kind = node[0]
    if kind == "set":
        cs = node[1]
        if forward:
            def m(s, pos, caps, k):
                return pos < len(s) and _contains(cs, s[pos]) and k(pos + 1, caps)
        else:
            def m(s, pos, caps, k):
                return pos > 0 and _contains(cs, s[pos - 1]) and k(pos - 1, caps)
        return m
    if kind == "seq":
        parts = [_compile(t, forward) for t in node[1]]
        if not forward:
            parts.reverse()

        def chain(i):
            if i == len(parts):
                return lambda s, pos, caps, k: k(pos, caps)
            head, rest = parts[i], chain(i + 1)
            return lambda s, pos, caps, k: head(s, pos, caps,
                                                lambda p2, c2: rest(s, p2, c2, k))
        return chain(0)
    if kind == "alt":
        parts = [_compile(t, forward) for t in node[1]]

        def m(s, pos, caps, k):
            return any(part(s, pos, caps, k) for part in parts)
        return m
    if kind == "group":
        index, inner = node[1], _compile(node[2], forward)
        if index == 0:
            return inner

        def m(s, pos, caps, k):
            def done(p2, c2):
                span = (pos, p2) if forward else (p2, pos)
                return k(p2, c2[:index] + (span,) + c2[index + 1:])
            return inner(s, pos, caps, done)
        return m
    if kind == "bol":
        return lambda s, pos, caps, k: pos == 0 and k(pos, caps)
    if kind == "eol":
        return lambda s, pos, caps, k: pos == len(s) and k(pos, caps)
    if kind == "wordb":
        negated = node[1]
        return lambda s, pos, caps, k: ((_is_word(s, pos - 1) != _is_word(s, pos)) != negated
                                        and k(pos, caps))
    if kind == "look":
        ahead, negated, inner = node[1], node[2], _compile(node[3], node[1])

        def m(s, pos, caps, k):
            found = []

            def stop(p2, c2):
                found.append(c2)
                return True
            ok = inner(s, pos, caps, stop)
            if negated:
                return (not ok) and k(pos, caps)
            return ok and k(pos, found[0])
        return m
    if kind == "backref":
        index = node[1]

        def m(s, pos, caps, k):
            span = caps[index]
            if span is None:
                return k(pos, caps)
            sub = s[span[0]:span[1]]
            n = len(sub)
            if forward:
                return pos + n <= len(s) and s[pos:pos + n] == sub and k(pos + n, caps)
            return pos - n >= 0 and s[pos - n:pos] == sub and k(pos - n, caps)
        return m
    if kind == "repeat":
        return _compile_repeat(node, forward)
    raise AssertionError(kind)


def _compile_repeat(node, forward: bool):
    _, atom, lo, hi, greedy, g0, g1 = node
    inner = _compile(atom, forward)
    step = 1 if forward else -1
    if atom[0] == "set":  # one code unit per iteration, no captures inside
        cs = atom[1]

        def m(s, pos, caps, k):
            count, at = 0, pos
            while hi is None or count < hi:
                nxt = at if forward else at - 1
                if not (0 <= nxt < len(s) and _contains(cs, s[nxt])):
                    break
                count += 1
                at += step
            if count < lo:
                return False
            order = range(count, lo - 1, -1) if greedy else range(lo, count + 1)
            return any(k(pos + i * step, caps) for i in order)
        return m

    def rep(s, pos, caps, k, lo_, hi_):
        # RepeatMatcher: captures of the atom's groups reset per iteration;
        # an empty iteration fails once the minimum is met.
        if hi_ == 0:
            return k(pos, caps)

        def after(p2, c2):
            if lo_ == 0 and p2 == pos:
                return False
            return rep(s, p2, c2, k, max(0, lo_ - 1), None if hi_ is None else hi_ - 1)
        cleared = caps if g1 < g0 else caps[:g0] + (None,) * (g1 - g0 + 1) + caps[g1 + 1:]
        if lo_ > 0:
            return inner(s, pos, cleared, after)
        if not greedy:
            return k(pos, caps) or inner(s, pos, cleared, after)
        return inner(s, pos, cleared, after) or k(pos, caps)

    return lambda s, pos, caps, k: rep(s, pos, caps, k, lo, hi)


class JsRegExp:
    """A compiled pattern: test(value) as RegExp.prototype.test without flags."""

    def __init__(self, pattern: str):
        self.pattern = pattern
        self.tree, self.groups = parse(pattern)
        self._match = _compile(self.tree, True)
        self._dfa: Optional[Dfa] = None
        self._dfa_error: Optional[str] = None

    def test_units(self, units: Sequence[int]) -> bool:
        s = list(units)
        caps = (None,) * (self.groups + 1)
        return any(self._match(s, start, caps, lambda p, c: True) for start in range(len(s) + 1))

    def test(self, value: str) -> bool:
        return self.test_units(utf16_units(value))

    def dfa(self) -> Optional["Dfa"]:
        """The automaton, or None when the pattern is not regular or too large."""
        if self._dfa is None and self._dfa_error is None:
            try:
                self._dfa = compile_dfa(self.tree)
            except NotRegular as exc:
                self._dfa_error = str(exc)
        return self._dfa


_CACHE: Dict[str, JsRegExp] = {}


def regexp(pattern: str) -> JsRegExp:
    """new RegExp(pattern), cached; RegexSyntaxError where that throws."""
    r = _CACHE.get(pattern)
    if r is None:
        r = JsRegExp(pattern)
        if len(_CACHE) < 1024:
            _CACHE[pattern] = r
    return r


def test(pattern: str, value: str) -> bool:
    """new RegExp(pattern).test(value)."""
    return regexp(pattern).test(value)


# ---------------------------------------------------------------- automaton

MAX_NFA_STATES = 4096
MAX_DFA_STATES = 1024
MAX_DFA_WORDS = 16384

_CHAR, _SPLIT, _BOL, _EOL, _MATCH = range(5)


class _Nfa:
    def __init__(self):
        self.kind: List[int] = []
        self.arg: List[int] = []   # the set index of a _CHAR state
        self.out: List[List[int]] = []
        self.sets: List[CharSet] = []
        self._set_ix: Dict[CharSet, int] = {}

    def add(self, kind: int, arg: int = -1) -> int:
        if len(self.kind) >= MAX_NFA_STATES:
            raise NotRegular("more than %d automaton states" % MAX_NFA_STATES)
        self.kind.append(kind)
        self.arg.append(arg)
        self.out.append([])
        return len(self.kind) - 1

    def set_index(self, cs: CharSet) -> int:
        if cs not in self._set_ix:
            self._set_ix[cs] = len(self.sets)
            self.sets.append(cs)
        return self._set_ix[cs]

    # Thompson construction: a fragment is (entry state, exit state), both
    # epsilon states linked by out edges.
    def build(self, node) -> Tuple[int, int]:
        kind = node[0]
        if kind == "set":
            a = self.add(_SPLIT)
            c = self.add(_CHAR, self.set_index(node[1]))
            b = self.add(_SPLIT)
            self.out[a].append(c)
            self.out[c].append(b)
            return a, b
        if kind in ("bol", "eol"):
            a = self.add(_BOL if kind == "bol" else _EOL)
            b = self.add(_SPLIT)
            self.out[a].append(b)
            return a, b
        if kind == "seq":
            a = self.add(_SPLIT)
            cur = a
            for t in node[1]:
                x, y = self.build(t)
                self.out[cur].append(x)
                cur = y
            return a, cur
        if kind == "alt":
            a, b = self.add(_SPLIT), self.add(_SPLIT)
            for t in node[1]:
                x, y = self.build(t)
                self.out[a].append(x)
                self.out[y].append(b)
            return a, b
        if kind == "group":
            return self.build(node[2])
        if kind == "repeat":
            _, atom, lo, hi, *_ = node
            a = self.add(_SPLIT)
            cur = a
            for _ in range(lo):
                x, y = self.build(atom)
                self.out[cur].append(x)
                cur = y
            if hi is None:
                x, y = self.build(atom)
                loop = self.add(_SPLIT)
                self.out[cur].append(loop)
                self.out[loop].append(x)
                self.out[y].append(loop)
                return a, loop
            end = self.add(_SPLIT)
            for _ in range(hi - lo):
                x, y = self.build(atom)
                self.out[cur].append(x)
                self.out[cur].append(end)
                cur = y
            self.out[cur].append(end)
            return a, end
        raise NotRegular("the automaton takes no %s" % {
            "wordb": "word boundary", "look": "lookaround",
            "backref": "backreference"}.get(kind, kind))


class Dfa:
    """The automaton as the device reads it: `bounds` [(first code unit,
    class)] sorted by code unit, `accept` per state (the value read so far is
    matched), `next` [state][class]; state 0 is the start of a value."""

    def __init__(self, bounds, accept, table, n_classes):
        self.bounds = bounds
        self.accept = accept
        self.table = table
        self.n_classes = n_classes
        self._starts = [b[0] for b in bounds]

    @property
    def n_states(self) -> int:
        return len(self.accept)

    def unit_class(self, u: int) -> int:
        lo, hi = 0, len(self._starts)
        while hi - lo > 1:
            mid = (lo + hi) // 2
            if self._starts[mid] <= u:
                lo = mid
            else:
                hi = mid
        return self.bounds[lo][1]

    def step(self, state: int, u: int) -> int:
        return self.table[state][self.unit_class(u)]

    def run(self, units: Sequence[int], state: int = 0) -> int:
        for u in units:
            state = self.step(state, u)
        return state

    def matches(self, value: str) -> bool:
        return bool(self.accept[self.run(utf16_units(value))])

    def words(self) -> List[int]:
        """[n_states, n_classes, n_bounds, 0, bounds (first | class << 16),
        accept flags, next states row by row]."""
        out = [self.n_states, self.n_classes, len(self.bounds), 0]
        out += [lo | (k << 16) for lo, k in self.bounds]
        out += [int(a) for a in self.accept]
        for row in self.table:
            out += row
        return out


def compile_dfa(tree) -> Dfa:
    """Subset construction over code-unit classes.  Every position starts a
    new match attempt (test() searches); once an attempt completes the value
    is matched whatever follows, so such a state loops on itself."""
    nfa = _Nfa()
    start, end = nfa.build(tree)
    match = nfa.add(_MATCH)
    nfa.out[end].append(match)

    # Code-unit classes: maximal intervals over which every set's membership
    # is constant, grouped by their membership vector.
    cuts = {0}
    for cs in nfa.sets:
        for lo, hi in cs:
            cuts.add(lo)
            if hi < MAX_UNIT:
                cuts.add(hi + 1)
    cuts = sorted(cuts)
    sig_class: Dict[tuple, int] = {}
    bounds: List[Tuple[int, int]] = []
    reps: List[int] = []
    for lo in cuts:
        sig = tuple(_contains(cs, lo) for cs in nfa.sets)
        if sig not in sig_class:
            sig_class[sig] = len(sig_class)
            reps.append(lo)
        k = sig_class[sig]
        if not bounds or bounds[-1][1] != k:
            bounds.append((lo, k))
    n_classes = len(sig_class)
    class_sets = [[i for i, cs in enumerate(nfa.sets) if _contains(cs, u)] for u in reps]

    def closure(seeds, at_start: bool, at_end: bool) -> frozenset:
        """The states reachable without reading, kept to those that read a
        code unit, wait for the end, or match."""
        seen, stack = set(), list(seeds)
        while stack:
            q = stack.pop()
            if q in seen:
                continue
            seen.add(q)
            k = nfa.kind[q]
            if k == _SPLIT or (k == _BOL and at_start) or (k == _EOL and at_end):
                stack.extend(nfa.out[q])
        return frozenset(q for q in seen if nfa.kind[q] in (_CHAR, _EOL, _MATCH))

    initial = closure([start], True, False)
    if match in initial:  # an empty attempt at the start matches every value
        return Dfa([(0, 0)], [True], [[0]], 1)
    matched_key = ("matched",)
    keys: List = [("initial", initial)]
    sets: List[frozenset] = [initial]
    index: Dict = {keys[0]: 0}
    table: List[List[int]] = []
    accept: List[bool] = []
    i = 0
    while i < len(keys):
        key = keys[i]
        if key == matched_key:
            table.append([i] * n_classes)
            accept.append(True)
            i += 1
            continue
        cur = sets[i]
        accept.append(match in closure(cur, i == 0, True))
        row = []
        for k in range(n_classes):
            live = set(class_sets[k])
            moved = [nfa.out[q][0] for q in cur if nfa.kind[q] == _CHAR and nfa.arg[q] in live]
            nxt = closure(moved + [start], False, False)
            nkey = matched_key if match in nxt else ("state", nxt)
            if nkey not in index:
                if len(keys) >= MAX_DFA_STATES:
                    raise NotRegular("more than %d automaton states" % MAX_DFA_STATES)
                index[nkey] = len(keys)
                keys.append(nkey)
                sets.append(nxt)
            row.append(index[nkey])
        table.append(row)
        i += 1
    if 4 + len(bounds) + len(accept) * (1 + n_classes) > MAX_DFA_WORDS:
        raise NotRegular("automaton larger than %d words" % MAX_DFA_WORDS)
    return Dfa(bounds, accept, table, n_classes)
