"""The host tool-call grammar (needle_hip.grammar, a mirror of
tools/grammar.ts) on the reference's own test cases (tests/grammar.test.ts),
JavaScript number spelling, and the device program/state compiler (CPU)."""

import numpy as np
import pytest

from needle_hip import NeedleError
from needle_hip.grammar import (JsonSchemaGrammar, ToolCallGrammar, allowed_pieces,
                                js_number_string, js_stringify, normalize_tools)
from needle_hip.maskgen import GrammarProgram, state_words

PARAMETERS = {  # tests/grammar.test.ts:7-21
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


def test_accepts_nested_schema_conforming_json_in_chunks():
    g = JsonSchemaGrammar(PARAMETERS)
    text = '{"mode":"eco","level":3,"enabled":true,"tags":["a","b"],"location":{"lon":2.5,"lat":-1}}'
    for off in range(0, len(text), 7):
        assert g.feed(text[off:off + 7].encode())
    assert g.complete
    assert g.value == {"mode": "eco", "level": 3, "enabled": True, "tags": ["a", "b"],
                       "location": {"lon": 2.5, "lat": -1}}


@pytest.mark.parametrize("text", [
    '{"enabled":true,"level":3,"mode":"eco","tags":["x"],"unknown":1}',
    '{"enabled":true,"level":3,"mode":"eco","mode":"boost","tags":["x"]}',
    '{"enabled":true,"level":3,"mode":"eco"}',
    '{"enabled":true,"level":3,"mode":"invalid","tags":["x"]}',
    '{"enabled":true,"level":11,"mode":"eco","tags":["x"]}',
    '{"enabled":true,"level":3,"mode":"eco","tags":[]}',
    '{"enabled":true,"level":3,"mode":"eco","tags":["x"],}',
])
def test_rejects_schema_violations(text):
    g = JsonSchemaGrammar(PARAMETERS)
    assert not (g.feed(text.encode()) and g.complete)


def test_clones_independently():
    base = JsonSchemaGrammar({"type": "string", "enum": ["alpha", "alpine"]})
    assert base.feed(b'"alp')
    left, right = base.clone(), base.clone()
    assert left.feed(b'ha"') and right.feed(b'ine"')
    assert left.complete and right.complete
    assert (left.value, right.value) == ("alpha", "alpine")


TOOLS = normalize_tools([
    {"name": "configure", "description": "Configure a device", "parameters": PARAMETERS},
    {"name": "ping", "parameters": {"type": "object", "properties": {}}},
])


def test_tool_calls_accept_and_reject():
    g = ToolCallGrammar(TOOLS, 2)
    out = ('[{"name":"configure","arguments":{"enabled":false,"level":5,"mode":"boost",'
           '"tags":["lab"]}},{"name":"ping","arguments":{}}]')
    assert g.feed(out.encode()) and g.complete
    assert g.calls == [{"name": "configure", "arguments": {"enabled": False, "level": 5,
                                                           "mode": "boost", "tags": ["lab"]}},
                       {"name": "ping", "arguments": {}}]
    for bad in ('[{"name":"missing","arguments":{}}]',
                '[{"name":"ping","arguments":{}},{"name":"ping","arguments":{}}]'):
        g = ToolCallGrammar(TOOLS, 3)
        assert not (g.feed(bad.encode()) and g.complete)


def test_normalize_tools_rejects_bad_names_and_duplicates():
    with pytest.raises(NeedleError):
        normalize_tools([{"name": 'a"b'}])
    with pytest.raises(NeedleError):
        normalize_tools([{"name": "a"}, {"name": "a"}])
    with pytest.raises(NeedleError):
        normalize_tools([{"name": "a", "parameters": {"type": "object", "properties": {},
                                                      "required": ["x"]}}])


@pytest.mark.parametrize("value,text", [
    (0.1 + 0.2, "0.30000000000000004"), (1e21, "1e+21"), (1e20, "100000000000000000000"),
    (1e-7, "1e-7"), (1.23e-18, "1.23e-18"), (0.000001, "0.000001"), (-1.5, "-1.5"),
    (2.0 ** 53, "9007199254740992"), (1e300, "1e+300"), (5e-324, "5e-324"), (-0.0, "0"),
    (3, "3"), (2.5e-5, "0.000025"), (123456.789, "123456.789"),
])
def test_js_number_spelling(value, text):
    assert js_number_string(value) == text


def test_js_stringify_escapes():
    assert js_stringify({"a": ["x\n", 1.0, None, True]}) == '{"a":["x\\n",1,null,true]}'
    assert js_stringify("\u0001é") == '"\\u0001é"'


def test_allowed_pieces_follows_the_grammar():
    g = ToolCallGrammar(TOOLS, 2)
    pieces = [b"[", b"[{", b'[{"name":"', b"{", b"", b"x"]
    assert allowed_pieces(g, pieces, [True, True, True, True, True, False]) == [0, 1, 2]
    assert allowed_pieces(g, pieces, [True] * 6, output_bytes=65535) == [0]


def test_device_state_of_a_partial_call():
    prog = GrammarProgram(TOOLS)
    words = prog.words()
    assert words[0] == 0x4E444752 and words.dtype == np.uint32
    g = ToolCallGrammar(TOOLS, 2)
    assert g.feed(b'[{"name":"configure","arguments":{"tags":["ab","c\\u00e9')
    st = state_words(prog, g)
    assert st[0] == 5 and st[9] == 1 and st[12] == 3  # arguments phase, three frames
    frames = st[24:].reshape(-1, 4)
    assert [int(f[0]) & 0xFF for f in frames] == [7, 6, 2]  # object, array, string
    # The string in progress, "c\u00e9" so far: two code points, the last
    # \u value, email state 1 (local part), uuid mismatch at the second.
    acc = st[16:20]
    assert acc[0] == 2 and acc[1] & 0xFFFF == 0xE9 and (acc[1] >> 17) & 7 == 1
    assert (acc[1] >> 20) & 63 == 1 and (acc[1] >> 26) & 1 == 1
    assert frames[0][0] >> 8 & 0xFF == 5 and frames[0][3] == 3  # value of property 3 ("tags")
    assert frames[1][0] >> 8 & 0xFF == 2 and frames[1][3] == 1  # array: one item so far
    assert frames[2][0] >> 16 == 1  # string started, no escape pending, UTF-8 at a boundary


@pytest.mark.parametrize("value,want", [
    ("a@b.co", True), ("a@b.", False), ("a@.b.c", True), ("@b.c", False), ("a@@b.c", False),
    ("a@b..c", True), ("a@..", False), ("a@...", True), ("ab", False), ("a b@c.d", False),
    ("a@b.c\n", False),        # `$` ends the input in JavaScript (Python's `$` would match)
    ("a\ufeff@b.c", False),    # U+FEFF is \s in JavaScript, not in Python
    ("a\x1c@b.c", True),       # U+001C is \s in Python, not in JavaScript
    ("a\x85@b.c", True),       # U+0085 likewise
    ("a\u3000@b.c", False), ("a\u00a0@b.c", False), ("a\u2028@b.c", False),
    ("a\u200b@b.c", True),     # U+200B is not in Zs
    ("\U0001f600@b.c", True),  # a surrogate pair: two 'other' code units
])
def test_email_format_has_javascript_semantics(value, want):
    """format "email" is /^[^\\s@]+@[^\\s@]+\\.[^\\s@]+$/ (grammar.ts:191) with
    ECMAScript's \\s (WhiteSpace + LineTerminator) and `$` at the end only."""
    from needle_hip.grammar import js_email

    assert js_email(value) is want


@pytest.mark.parametrize("value,want", [
    ("123e4567-e89b-12d3-a456-426614174000", True),
    ("123E4567-E89B-12D3-A456-426614174000", True),
    ("123e4567-e89b-92d3-a456-426614174000", False),  # version digit outside [1-8]
    ("123e4567-e89b-12d3-c456-426614174000", False),  # variant outside [89ab]
    ("123e4567-e89b-12d3-a456-426614174000\n", False),
    ("123e4567e89b-12d3-a456-426614174000-", False),
    ("123e4567-e89b-12d3-a456-42661417400", False),
])
def test_uuid_format_has_javascript_semantics(value, want):
    """format "uuid" is the case-insensitive pattern of grammar.ts:192-196,
    anchored at both ends of the input."""
    from needle_hip.grammar import js_uuid

    assert js_uuid(value) is want


def test_device_pattern_automaton_state():
    """A string under `pattern` carries its automaton's state in accumulator
    word 3: the state after the decoded value's UTF-16 code units, whose
    accept flag is RegExp.test of the value so far; a pattern the automaton
    cannot express is left to the host."""
    import json

    from needle_hip import jsregex
    from needle_hip.maskgen import KC_PATTERN, KC_STRING_HOST

    props = {"c": {"type": "string", "pattern": "^[A-Z]{2}-\\d+$"},
             "e": {"type": "string", "pattern": "\\uD83D[^a]|\\s"},
             "r": {"type": "string", "pattern": "(a)\\1"}}
    tools = normalize_tools([{"name": "p", "parameters": {"type": "object", "properties": props}}])
    prog = GrammarProgram(tools)
    words = prog.words()
    assert words[15] > 0 and words[15] * 4 <= words[13]
    schemas = tools[0]["parameters"]["properties"]
    node = {k: prog.node_of(0, schemas[k]) for k in props}
    assert prog.nodes[node["c"]][12] & KC_PATTERN and prog.nodes[node["e"]][12] & KC_PATTERN
    assert prog.nodes[node["r"]][12] & KC_STRING_HOST and prog.nodes[node["r"]][15] == 0
    for key, partial in (("c", "AB-1"), ("c", "AB-"), ("c", "\\u0041B-12"), ("c", ""),
                         ("e", "x\U0001F600"), ("e", "\\ud83d\\ude00"), ("e", "\\ud83da"),
                         ("e", "\\ud83d"), ("e", "a\\tb"), ("e", "　")):
        g = ToolCallGrammar(tools, 1)
        assert g.feed(('[{"name":"p","arguments":{"%s":"%s' % (key, partial)).encode())
        st = state_words(prog, g)
        dfa = prog.node_dfa[node[key]]
        value = json.loads('"%s"' % partial)
        assert st[19] == dfa.run(jsregex.utf16_units(value)), (key, partial)
        assert bool(dfa.accept[st[19]]) == jsregex.test(props[key]["pattern"], value)


def test_clones_keep_their_own_containers():
    """A clone fills its own array items and object properties; the
    original's stay as they were (completed values are shared)."""
    base = ToolCallGrammar(TOOLS, 2)
    assert base.feed(b'[{"name":"configure","arguments":{"enabled":true,"tags":["a"')
    left, right = base.clone(), base.clone()
    assert left.feed(b',"b"],"level":1,"mode":"eco"}}]') and left.complete
    assert right.feed(b'],"level":2,"mode":"boost"}}]') and right.complete
    assert left.calls[0]["arguments"] == {"enabled": True, "tags": ["a", "b"], "level": 1,
                                          "mode": "eco"}
    assert right.calls[0]["arguments"] == {"enabled": True, "tags": ["a"], "level": 2,
                                           "mode": "boost"}
    assert base.feed(b',"c"],"level":3,"mode":"eco"}}]') and base.complete
    assert base.calls[0]["arguments"]["tags"] == ["a", "c"]
