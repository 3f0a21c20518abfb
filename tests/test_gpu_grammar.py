"""Device allowed-token masks of the tool-call grammar (nd_grammar_mask)
against the agent's own loop (tools/agent.ts:164-175: clone the grammar for
every piece and feed it), through the C ABI.

Bar: the allowed id lists are identical at every step -- the device mask
with its undecided pieces settled by the host grammar -- over scripted
complete tool calls (longest-piece tokenization of valid outputs) and
seeded random walks through three tool sets: the reference test's tools, a
schema that uses every grammar feature (oneOf/anyOf, const, enum of mixed
types, $ref, nested arrays and objects, integer and number, bounds,
pattern, format, uniqueItems, type unions), and one made of the value
checks the device decides itself (string lengths counted in code points
over escapes, surrogate pairs and multibyte text, JavaScript patterns by
their automata over UTF-16 code units, the email and uuid formats, numeric
bounds, exclusive bounds, multipleOf, integers written with a fraction or
an exponent) beside a pattern with a backreference, which the host
settles.
"""

import sys

import numpy as np
import pytest

from needle_hip import synth
from needle_hip.grammar import ToolCallGrammar, allowed_pieces, normalize_tools
from needle_hip.maskgen import GrammarMasker

pytestmark = pytest.mark.gpu

TOOLS_A = normalize_tools([
    {"name": "configure", "description": "Configure a device", "parameters": synth.DEMO_PARAMETERS},
    {"name": "ping", "parameters": {"type": "object", "properties": {}}},
])
TOOLS_B = synth.demo_tools()
OUT_A = ('[{"name":"configure","arguments":{"enabled":false,"level":5,"mode":"boost",'
         '"tags":["lab"],"location":{"lat":-1,"lon":2.5}}},{"name":"ping","arguments":{}}]')
OUT_B = synth.DEMO_TOOL_OUTPUT
CHECKS = {
    "type": "object",
    "properties": {
        "name": {"type": "string", "minLength": 2, "maxLength": 5},
        "code": {"type": "string", "format": "uuid"},
        "mail": {"type": "string", "format": "email"},
        "ratio": {"type": "number", "minimum": -1.5, "maximum": 2.5e3},
        "step": {"type": "number", "multipleOf": 0.25, "exclusiveMinimum": 0},
        "count": {"type": "integer", "exclusiveMaximum": 100},
        "big": {"type": "number", "maximum": 1e300},
        "short": {"type": "string", "maxLength": 1},
        "code2": {"type": "string", "pattern": "^[A-Z]{2}-\\d+$"},
        "tag": {"type": "string", "pattern": "\u00e9|\\s|^$|\\uD83D[^a]"},
        "ref": {"type": "string", "pattern": "(a)\\1"},
    },
    "required": ["name"],
}
TOOLS_C = normalize_tools([{"name": "checks", "parameters": CHECKS},
                           {"name": "check", "parameters": {"type": "object", "properties": {
                               "n": {"type": "integer", "minimum": 3}}}}])
OUT_C1 = ('[{"name":"checks","arguments":{"name":"\\ud83d\\ude00\u00e9",'
          '"code":"123e4567-e89b-12d3-a456-426614174000","mail":"a.b@c.de","ratio":2.5e3,'
          '"step":1.75,"count":1.2e1,"big":-1e-5,"short":"\\u00e9","code2":"AB-12",'
          '"tag":"x y","ref":"baab"}},'
          '{"name":"check","arguments":{"n":3.0}}]')
OUT_C2 = ('[{"name":"checks","arguments":{"name":"\u4e2d\u6587\u5b57\\n","mail":"x@y.z",'
          '"count":99,"step":0.5,"ratio":-1.5,"tag":"\U0001F600!","code2":"QZ-0"}}]')


def say(*args):
    print("[case]", *args, file=sys.stderr, flush=True)


@pytest.fixture(scope="module")
def maskers(hip):
    made = {}
    for key, tools, vocab in (("A", TOOLS_A, 8192), ("B", TOOLS_B, 8192), ("B4k", TOOLS_B, 4096),
                              ("C", TOOLS_C, 8192)):
        pieces, eligible = synth.tool_pieces(7, vocab, tools)
        made[key] = (GrammarMasker(hip, tools, pieces, eligible), tools, pieces, eligible)
    yield made
    for m, *_ in made.values():
        m.free()


def check_step(masker, g, pieces, eligible, out_bytes, what):
    want = allowed_pieces(g, pieces, eligible, out_bytes)
    got = masker.allowed(g, out_bytes)
    if got != want:
        extra = sorted(set(got) - set(want))[:5]
        missing = sorted(set(want) - set(got))[:5]
        raise AssertionError(f"{what}: device allowed {len(got)}, host {len(want)}; extra "
                             f"{[pieces[t] for t in extra]} missing {[pieces[t] for t in missing]}")
    return want


@pytest.mark.parametrize("key,out", [("A", OUT_A), ("B", OUT_B), ("C", OUT_C1), ("C", OUT_C2)])
def test_scripted_tool_calls(maskers, key, out):
    masker, tools, pieces, eligible = maskers[key]
    say("grammar scripted", key)
    target = out.encode()
    g = ToolCallGrammar(tools, 4)
    pos, steps, undecided, total = 0, 0, 0, 0
    while pos < len(target):
        allowed = check_step(masker, g, pieces, eligible, pos, (key, pos))
        undecided = max(undecided, masker.last_undecided)
        total += masker.last_undecided
        best = max((t for t in allowed if target.startswith(pieces[t], pos)),
                   key=lambda t: len(pieces[t]), default=None)
        assert best is not None, (key, pos, target[pos:pos + 20])
        assert g.feed(pieces[best])
        pos += len(pieces[best])
        steps += 1
    assert g.complete
    assert check_step(masker, g, pieces, eligible, pos, (key, "done")) == []
    say(f"[measure] grammar scripted {key}: {steps} steps, undecided pieces per state mean "
        f"{total / steps:.2f} max {undecided}")


@pytest.mark.parametrize("seed", range(9))
def test_random_walks(maskers, seed):
    key = "C" if seed >= 6 else ("A" if seed % 2 == 0 else "B4k")
    masker, tools, pieces, eligible = maskers[key]
    say("grammar walk", key, seed)
    rng = np.random.default_rng(seed)
    g = ToolCallGrammar(tools, 2)
    out = 0
    for step in range(36):
        allowed = check_step(masker, g, pieces, eligible, out, (key, seed, step))
        if not allowed:
            break
        # Prefer multi-byte pieces half of the time so walks leave strings.
        long = [t for t in allowed if len(pieces[t]) > 1]
        pool = long if long and rng.random() < 0.5 else allowed
        t = int(pool[rng.integers(len(pool))])
        assert g.feed(pieces[t])
        out += len(pieces[t])


def test_output_budget_and_eligibility(maskers):
    masker, tools, pieces, eligible = maskers["A"]
    say("grammar budget")
    g = ToolCallGrammar(tools, 2)
    for out in (0, 65535, 65536 - 5, 65536):
        check_step(masker, g, pieces, eligible, out, ("budget", out))
    assert masker.allowed(g, 65536) == []
    assert all(eligible[t] for t in masker.allowed(g, 0))


@pytest.mark.parametrize("key", ["A", "C"])
def test_resident_masked_selection(hip, key):
    """The constrained agent loop (tools/agent.ts:157-196) with the allowed
    set kept on the device: nd_needle_grammar_mask into the model's mask
    buffer, the undecided pieces settled by grammar clones, then
    nd_needle_step_select_mask (whole step) and nd_needle_select_token_mask
    (session token).  Bars: both select the same id with the same
    log-probability, bit for bit, as nd_needle_step_select over the host's
    allowed id list on a third copy of the model; the oracle's selection over
    that list picks the same id, log-probability within 1e-3; the allowed
    count plus the settled ids equals the list's length; at a completed call
    the loop raises GRAMMAR_DEAD_END before stepping."""
    import oracle
    from needle_hip import NeedleError, NeedleModel
    from needle_hip.needle2 import Needle2Weights
    from needle_hip.runtime import Needle2Resident
    from test_gpu_needle2 import SMALL

    tools = TOOLS_A if key == "A" else TOOLS_C
    pieces, eligible = synth.tool_pieces(7, SMALL.vocab, tools)
    masker = GrammarMasker(hip, tools, pieces, eligible)
    nw = Needle2Weights(SMALL, 33)
    model = NeedleModel(hip, nw)
    listed = Needle2Resident(hip, nw)
    try:
        whole = model.create_resident_runtime()
        session = model.create_runtime()
        ref = oracle.Needle2(nw).runtime(SMALL.max_length, 2)
        for rt in (whole, session):
            rt.reset(SMALL.max_length, 2)
        listed.reset(SMALL.max_length, 2)
        prompt = [int(t) for t in synth.Stream(9, f"masked-{key}").integers(6, 0, 255)]
        say("resident masked selection", key)
        for t in prompt[:-1]:
            whole.step(t, want_logits=False)
            session.step(t, want_logits=False)
            listed.step(t, want_logits=False)
            ref.step(t, want_logits=False)
        g = ToolCallGrammar(tools, 2)
        tok, out, settled_total = prompt[-1], 0, 0
        while whole.position < SMALL.max_length - 1:
            allowed = allowed_pieces(g, pieces, eligible, out)
            if not allowed:
                break
            count, undecided = whole.resident.grammar_mask(masker, masker.state(g), 65536 - out)
            assert count + len(masker.settle(g, undecided)) == len(allowed), (key, out)
            a = whole.step_constrained(tok, masker, g, out)
            settled_total += masker.last_undecided
            b = session.step_constrained(tok, masker, g, out)
            c = listed.step_selected(tok, np.asarray(allowed, np.uint32))
            rid, rlp = oracle.select(ref.step(tok), np.asarray(allowed, np.uint32))
            what = (key, whole.position, out)
            assert a == c and (b.id, b.log_probability) == c, what
            assert c[0] == rid and abs(c[1] - rlp) <= 1e-3 * max(1.0, abs(rlp)), what
            assert c[0] in allowed
            assert g.feed(pieces[c[0]])
            out += len(pieces[c[0]])
            tok = c[0]
        steps = whole.position - len(prompt) + 1
        say(f"[measure] resident masked selection {key}: {steps} steps, {out} bytes, "
            f"undecided per step {settled_total / max(1, steps):.2f}")
        assert steps >= 10
        # the budget spent: nothing is allowed, and the loop stops before stepping
        position = whole.position
        with pytest.raises(NeedleError) as err:
            whole.step_constrained(tok, masker, g, 65536)
        assert err.value.code == "GRAMMAR_DEAD_END" and whole.position == position
    finally:
        listed.free()
        model.dispose()
        masker.free()


@pytest.mark.parametrize("items", ['"a","b"', '"a","a"', '"a"', '"a","b","b\\u0061"', '',
                                   '"x","\\u0078"', '"a","b","c'])
def test_unique_items_states(maskers, items):
    """Array closes under uniqueItems: decided on the device from the host's
    word for the items it holds (distinct or not), undecided only for pieces
    that complete another item and close in one go; the lists equal the
    clone loop's."""
    masker, tools, pieces, eligible = maskers["B"]
    say("grammar uniqueItems", items)
    prefix = '[{"name":"get_weather","arguments":{"kind":"circle","uniq":[' + items
    g = ToolCallGrammar(tools, 2)
    assert g.feed(prefix.encode())
    check_step(masker, g, pieces, eligible, len(prefix), ("uniq", items))
