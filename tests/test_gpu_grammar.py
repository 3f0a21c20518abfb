"""Device allowed-token masks of the tool-call grammar (nd_grammar_mask)
against the agent's own loop (tools/agent.ts:164-175: clone the grammar for
every piece and feed it), through the C ABI.

Bar: the allowed id lists are identical at every step -- the device mask
with its undecided pieces settled by the host grammar -- over scripted
complete tool calls (longest-piece tokenization of valid outputs) and
seeded random walks through two tool sets: the reference test's tools and a
schema that uses every grammar feature (oneOf/anyOf, const, enum of mixed
types, $ref, nested arrays and objects, integer and number, bounds,
pattern, format, uniqueItems, type unions).
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


def say(*args):
    print("[case]", *args, file=sys.stderr, flush=True)


@pytest.fixture(scope="module")
def maskers(hip):
    made = {}
    for key, tools, vocab in (("A", TOOLS_A, 8192), ("B", TOOLS_B, 8192), ("B4k", TOOLS_B, 4096)):
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


@pytest.mark.parametrize("key,out", [("A", OUT_A), ("B", OUT_B)])
def test_scripted_tool_calls(maskers, key, out):
    masker, tools, pieces, eligible = maskers[key]
    say("grammar scripted", key)
    target = out.encode()
    g = ToolCallGrammar(tools, 4)
    pos, steps, undecided = 0, 0, 0
    while pos < len(target):
        allowed = check_step(masker, g, pieces, eligible, pos, (key, pos))
        undecided = max(undecided, masker.last_undecided)
        best = max((t for t in allowed if target.startswith(pieces[t], pos)),
                   key=lambda t: len(pieces[t]), default=None)
        assert best is not None, (key, pos, target[pos:pos + 20])
        assert g.feed(pieces[best])
        pos += len(pieces[best])
        steps += 1
    assert g.complete
    assert check_step(masker, g, pieces, eligible, pos, (key, "done")) == []
    say("grammar scripted", key, "steps", steps, "max undecided", undecided)


@pytest.mark.parametrize("seed", range(6))
def test_random_walks(maskers, seed):
    key = "A" if seed % 2 == 0 else "B4k"
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
