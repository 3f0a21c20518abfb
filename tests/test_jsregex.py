"""JavaScript `pattern` semantics (needle_hip.jsregex): the backtracking
matcher the host grammar uses and the automaton the device steps.

Pins: behaviours the ECMAScript specification fixes, as hand vectors (code
units, the \\s and \\d sets, `$` at the end only, Annex B syntax, lookbehind
evaluated right to left, backreferences to groups that did not take part);
RegExp's SyntaxErrors; seeded random patterns over the syntax JavaScript
and Python's `re` share, on ASCII values without line terminators, where
the two must agree (Python's matcher is an independent implementation);
and the automaton against the matcher on random patterns and values drawn
with the code units where JavaScript differs (line terminators, Unicode
spaces, surrogate pairs, lone surrogates).
"""

import re

import numpy as np
import pytest

from needle_hip import jsregex as J

VECTORS = [
    ("^[a-z]+$", "abc", True), ("^[a-z]+$", "ab1", False),
    # one code unit per `.`: a character above U+FFFF is two
    ("^.$", "\U0001F600", False), ("^..$", "\U0001F600", True), ("^\\uD83D", "\U0001F600", True),
    ("^[\U0001F600]$", "\U0001F600", False), ("^[\U0001F600]{2}$", "\U0001F600", True),
    # \s is WhiteSpace + LineTerminator; \d and \w are ASCII
    ("\\s", "\u00a0", True), ("\\s", "\ufeff", True), ("\\s", "\u3000", True),
    ("\\s", "\u0085", False), ("\\s", "\u180e", False), ("\\s", "\u200b", False),
    ("^\\d$", "\u0663", False), ("\\w", "\u00e9", False), ("\\S", "\u00a0", False),
    # `$` only at the end, `.` excludes the four line terminators
    ("a$", "a\n", False), (".", "\r", False), (".", "\u2028", False), (".", "\u0085", True),
    ("[^]", "\n", True), ("[]", "a", False), ("", "", True), ("^$", "", True), ("^$", "a", False),
    ("^a|b$", "cb", True), ("^a|b$", "bc", False),
    # Annex B syntax
    ("]", "]", True), ("a{", "a{", True), ("a{1", "a{1", True), ("{a}", "{a}", True),
    ("\\8", "8", True), ("\\1", "\x01", True), ("\\12", "\x0a", True), ("\\18", "\x018", True),
    ("[\\b]", "\b", True), ("\\cA", "\x01", True), ("\\ca", "\x01", True), ("\\c1", "\\c1", True),
    ("[\\c1]", "\x11", True), ("[\\c_]", "\x1f", True), ("\\k", "k", True), ("\\x4", "x4", True),
    ("\\u12", "u12", True), ("\\0", "\0", True), ("\\07", "\x07", True), ("\\08", "\x008", True),
    ("[\\d-z]", "-", True), ("[\\d-z]", "y", False), ("[--0]", "/", True), ("\\q", "q", True),
    ("(?=a)*b", "b", True), ("\\$\\.", "$.", True),
    # backreferences: to a group that did not take part, the empty string
    ("(a)|\\1b", "b", True), ("^(?:(a)|b)\\1$", "b", True), ("^(a)\\1$", "aa", True),
    ("^(a)\\1$", "ab", False), ("(?<y>\\d)\\k<y>", "11", True), ("(?<y>\\d)\\k<y>", "12", False),
    # lookbehind reads right to left: a backreference left of its group
    # has the capture, one right of it runs first and matches empty
    ("(?<=(o)d\\1)r", "hodor", False), ("(?<=\\1d(o))r", "hodor", True),
    ("(?<=\\$)\\d+", "$42", True), ("(?<!\\$)\\d+", "$4", False), ("(?<!\\$)\\d+", "$42", True),
    # captures reset per iteration; an empty iteration ends the loop
    ("^(?:(a)|b)+\\1$", "abb", True), ("^(?:(a)|b)+\\1$", "aba", False), ("^(a*)*$", "aaa", True),
    ("(a*)*b", "aab", True), ("^(a+)+$", "aaaa", True), ("x*", "", True),
    ("\\bfoo\\b", "a foo b", True), ("\\bfoo\\b", "afoo", False), ("\\Bfoo", "afoo", True),
]


@pytest.mark.parametrize("pattern,value,want", VECTORS)
def test_javascript_semantics(pattern, value, want):
    r = J.regexp(pattern)
    assert r.test(value) is want
    dfa = r.dfa()
    if dfa is not None:
        assert dfa.matches(value) is want


@pytest.mark.parametrize("pattern", ["(", "a**", "[b-a]", "x{2,1}", "*a", "(?<n>a)\\k<m>", "{1}",
                                     ")", "(?<=a)*", "^*", "a\\", "[a", "(?<n>a)(?<n>b)",
                                     "(?<n>a)\\k", "(?<1>a)", "(?x)", "a|*"])
def test_syntax_errors(pattern):
    with pytest.raises(J.RegexSyntaxError):
        J.parse(pattern)


def test_non_regular_features_have_no_automaton():
    for p in ("(a)\\1", "\\bx", "(?=a)b", "(?<!a)b"):
        assert J.regexp(p).dfa() is None
    assert J.regexp("^[a-z]{2}-\\d+$").dfa() is not None


def _random_pattern(rng, depth, lookaround):
    def atom(d):
        r = rng.random()
        if d > 0 and r < 0.2:
            inner = _random_pattern(rng, d - 1, lookaround)
            return rng.choice(["(", "(?:"]) + inner + ")"
        if lookaround and d > 0 and r < 0.26:
            return rng.choice(["(?=", "(?!"]) + _random_pattern(rng, d - 1, lookaround) + ")"
        return str(rng.choice(["a", "b", "c", "1", " ", "[ab]", "[^a]", "[a-c]", "\\d", "\\w",
                               "\\s", ".", "\\D", "[\\d_]", "-"]))

    def term(d):
        r = rng.random()
        if r < 0.06:
            return "^"
        if r < 0.12:
            return "$"
        a = atom(d)
        q = rng.random()
        if q < 0.45:
            return a
        quant = str(rng.choice(["*", "+", "?", "{2}", "{1,}", "{0,2}", "{1,3}"]))
        return a + quant + ("?" if rng.random() < 0.3 else "")

    alts = ["".join(term(depth) for _ in range(int(rng.integers(0, 4))))
            for _ in range(int(rng.integers(1, 3)))]
    return "|".join(alts)


def test_agrees_with_python_re_on_the_shared_syntax():
    """On ASCII values without line terminators, and with the syntax both
    engines read alike, JavaScript's and Python's matchers agree."""
    rng = np.random.default_rng(20261202)
    alphabet = "abc1 _-"
    checked = 0
    for _ in range(400):
        pattern = _random_pattern(rng, 2, lookaround=True)
        py = re.compile(pattern, re.ASCII)
        r = J.regexp(pattern)
        dfa = r.dfa()
        for _ in range(12):
            n = int(rng.integers(0, 7))
            value = "".join(alphabet[int(i)] for i in rng.integers(0, len(alphabet), n))
            want = py.search(value) is not None
            assert r.test(value) is want, (pattern, value)
            if dfa is not None:
                assert dfa.matches(value) is want, (pattern, value)
            checked += 1
    assert checked == 4800


def test_automaton_agrees_with_matcher():
    """The automaton against the backtracking matcher on values with line
    terminators, Unicode spaces, astral characters and lone surrogates."""
    rng = np.random.default_rng(7)
    units = ["a", "b", "1", " ", "\n", "\r", "\u2028", "\u00a0", "\ufeff", "\u00e9",
             "\U0001F600", "\ud83d", "\ude00", "-", "_"]
    extra = ["\\uD83D", "[\\uDC00-\\uDFFF]", "\\n", "[^\\s]", "\u00e9", "[\\u00a0-\\u00ff]", "\\W"]
    for _ in range(300):
        pattern = _random_pattern(rng, 2, lookaround=False)
        if rng.random() < 0.5:
            pattern += str(rng.choice(extra)) + str(rng.choice(["", "*", "+", "?"]))
        r = J.regexp(pattern)
        dfa = r.dfa()
        assert dfa is not None, pattern
        for _ in range(10):
            n = int(rng.integers(0, 6))
            value = "".join(units[int(i)] for i in rng.integers(0, len(units), n))
            assert dfa.matches(value) is r.test(value), (pattern, value)


def test_automaton_words_layout():
    dfa = J.regexp("^[a-z]{2}-\\d+$").dfa()
    w = dfa.words()
    n_states, n_classes, n_bounds = w[0], w[1], w[2]
    assert len(w) == 4 + n_bounds + n_states * (1 + n_classes)
    starts = [x & 0xFFFF for x in w[4:4 + n_bounds]]
    assert starts[0] == 0 and starts == sorted(starts)
    assert all((x >> 16) < n_classes for x in w[4:4 + n_bounds])
    table = w[4 + n_bounds + n_states:]
    assert all(t < n_states for t in table)
