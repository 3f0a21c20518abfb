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
    frames = st[16:].reshape(-1, 4)
    assert [int(f[0]) & 0xFF for f in frames] == [7, 6, 2]  # object, array, string
    assert frames[0][0] >> 8 & 0xFF == 5 and frames[0][3] == 3  # value of property 3 ("tags")
    assert frames[1][0] >> 8 & 0xFF == 2 and frames[1][3] == 1  # array: one item so far
    assert frames[2][0] >> 16 == 1  # string started, no escape pending, UTF-8 at a boundary
