"""Semantic-unit selection (kv_cache_repair_amd.semantic_units) against the plain
restatement of the reference's algorithm in oracle/semantic_units_ref.py, on
fuzzed inputs: ChatML transcripts with tool elements, JSON values in and out of
qualifying positions and sentence/paragraph breaks (character units); unit
tilings with short units, long units, container runs and gaps (split and merge);
score vectors with ties and budgets from one token to past the suffix
(allocation). The package's implementation was written in a different form (a
backward scan for the JSON lead-in, a decode window per container, a merge scan
that resumes at the merge); these tests hold it to the reference's results."""

from __future__ import annotations

import math
import random

import pytest

from kv_cache_repair_amd import semantic_units as su
from oracle import semantic_units_ref as ref

WORDS = ["the", "cache", "Repair", "token", "KV", "layer", "42", "x", "value", "Query", "<b>", "end", "A1", "ok"]


def sentence(rng: random.Random) -> str:
    words = " ".join(rng.choice(WORDS) for _ in range(rng.randint(1, 9)))
    tail = rng.choice(["", ".", "!", "?", ".\"", "?)", ".]", "...", ". ", "! ", "?\n", ".\t"])
    return words + tail


def json_value(rng: random.Random, depth: int = 0) -> str:
    kind = rng.randint(0, 6 if depth < 2 else 3)
    if kind == 0:
        return str(rng.randint(-5, 500))
    if kind == 1:
        return '"' + rng.choice(WORDS) + '"'
    if kind == 2:
        return rng.choice(["true", "null", "false", "1.5e3"])
    if kind == 3:
        return "[" + ", ".join(json_value(rng, depth + 1) for _ in range(rng.randint(0, 3))) + "]"
    pairs = ", ".join(f'"{rng.choice(WORDS)}": {json_value(rng, depth + 1)}' for _ in range(rng.randint(0, 3)))
    return "{" + pairs + "}"


def json_fragment(rng: random.Random) -> str:
    value = json_value(rng)
    if rng.random() < 0.25:  # broken: truncated or trailing garbage inside
        cut = rng.randint(1, max(1, len(value) - 1))
        value = value[:cut] + rng.choice(["", "}", "]", ",", " oops"])
    lead = rng.choice(["", "args: ", "x = ", "> ", "see ", "\n", "result:\n", "list ", "  "])
    return lead + value


def tool_element(rng: random.Random) -> str:
    tag = rng.choice(["tool_call", "tool_response", "tool_result", "function_call", "function_response", "toolcall"])
    open_tag = "<" + (tag.upper() if rng.random() < 0.2 else tag) + (" id=" + str(rng.randint(0, 9)) if rng.random() < 0.4 else "") + ">"
    body = rng.choice([json_value(rng), sentence(rng), json_fragment(rng) + " " + sentence(rng)])
    close = "</" + tag + ">" if rng.random() < 0.85 else ""
    return open_tag + body + close


def body(rng: random.Random) -> str:
    parts = []
    for _ in range(rng.randint(0, 6)):
        r = rng.random()
        if r < 0.45:
            parts.append(sentence(rng))
        elif r < 0.65:
            parts.append(json_fragment(rng))
        elif r < 0.8:
            parts.append(tool_element(rng))
        else:
            parts.append(rng.choice(["\n\n", "\n \n", "\n", "\t\n\n\n", " "]))
    return rng.choice(["", " ", "\n"]).join(parts)


def transcript(rng: random.Random) -> str:
    pieces = []
    for _ in range(rng.randint(0, 5)):
        r = rng.random()
        if r < 0.55:
            role = rng.choice(["system", "user", "assistant", "tool"])
            end = "<|im_end|>" if rng.random() < 0.9 else ""
            pieces.append(f"<|im_start|>{role}\n{body(rng)}{end}")
        elif r < 0.8:
            pieces.append(body(rng))
        else:
            pieces.append(rng.choice(["\n", "  \n ", "", "\n\n"]))
    return rng.choice(["", "\n"]).join(pieces)


@pytest.mark.parametrize("seed", range(8))
def test_character_units_match_the_reference_restatement(seed):
    rng = random.Random(1000 + seed)
    for _ in range(250):
        text = transcript(rng)
        assert su.semantic_char_units(text) == ref.char_units(text), text


def test_character_units_of_edge_texts():
    for text in ["", " ", "\n\n", "{}", "[1, 2]", "a: {\"k\": [1, {\"z\": null}]} tail.", "<|im_start|><|im_end|>",
                 "<|im_start|>user\n<tool_call>{\"a\": 1}</tool_call><|im_end|>\n\n<|im_start|>x",
                 "x {\"a\": 1}", "line\n  = [1,2] end", "<TOOL_CALL a>b</tool_call>", "Hi.There", "Hi. there",
                 "no break here", "end!)\n\nNext", "\n{\"a\"", "[{]}"]:
        assert su.semantic_char_units(text) == ref.char_units(text), text


def random_units(rng: random.Random) -> list[dict]:
    pos = rng.randint(0, 40)
    units = []
    cid = 0
    for _ in range(rng.randint(1, 30)):
        if rng.random() < 0.3:
            cid += 1
        length = rng.choice([1, 2, 3, 5, 7, 7, 8, 9, 15, 40, 127, 128, 129, 200, 300])
        if rng.random() < 0.08:
            pos += rng.randint(1, 3)  # a gap: the units on either side are not contiguous
        container = cid if rng.random() < 0.8 else f"{cid}:structured:{rng.randint(0, 2)}"
        units.append({"start": pos, "end": pos + length, "container_id": container,
                      "container_kind": rng.choice(["chat_message", "ordinary_text", "json_container"]),
                      "boundary_kind": rng.choice(["generic_sentence_or_paragraph", "tool_container"])})
        pos += length
    return units


@pytest.mark.parametrize("seed", range(6))
def test_split_and_short_unit_merge_match_the_reference_restatement(seed):
    rng = random.Random(2000 + seed)
    for _ in range(400):
        units = random_units(rng)
        split = ref.split_long(units)
        assert [su._chunked(u, u["start"], u["end"]) for u in units] == [ref.with_chunks(u, u["start"], u["end"])
                                                                          for u in units]
        assert su._merge_short(split) == ref.merge_short(split)


def test_balanced_chunks_match_for_every_length_to_1000():
    for n in range(0, 1001):
        assert su._balanced(5, 5 + n) == ref.balanced(5, 5 + n)


def contiguous_units(rng: random.Random) -> list[dict]:
    units = random_units(rng)
    pos = units[0]["start"]
    for u in units:  # close the gaps: allocation needs a tiling of the suffix
        width = u["end"] - u["start"]
        u["start"], u["end"] = pos, pos + width
        pos += width
    return ref.merge_short(ref.split_long(units))


@pytest.mark.parametrize("seed", range(6))
def test_allocation_matches_the_reference_restatement(seed):
    rng = random.Random(3000 + seed)
    for _ in range(150):
        units = contiguous_units(rng)
        end = units[-1]["end"]
        if rng.random() < 0.5:
            scores = [float(rng.randint(0, 3)) for _ in range(end)]  # many ties
        else:
            scores = [rng.gauss(0.0, 2.0) for _ in range(end)]
        span = end - units[0]["start"]
        for budget in {1, rng.randint(1, span), rng.randint(1, span), span, span + 5, 0}:
            got_positions, got_meta = su.select_semantic_unit_support(units=units, token_scores=scores,
                                                                      budget_tokens=budget)
            want_positions, want_meta = ref.select_support(units, scores, budget)
            assert got_positions == want_positions
            for key in ("budget_tokens", "unit_count", "units", "selections"):
                assert got_meta[key] == want_meta[key], key


def test_forward_window_matches_on_tied_and_decaying_scores():
    rng = random.Random(7)
    for _ in range(300):
        n = rng.randint(1, 80)
        scores = [float(rng.choice([0, 0, 1, 5])) if rng.random() < 0.5 else rng.uniform(-3, 3) for _ in range(n)]
        width = rng.randint(1, n)
        assert su.best_forward_causal_window(start=0, end=n, width=width, token_scores=scores) == \
            ref.forward_window(0, n, width, scores)


# ---------------------------------------------------------------------------
# the restatement itself against the reference's known answers
# (the reference's tests/test_semantic_units.py:40-140)
# ---------------------------------------------------------------------------

def oracle_unit(start, end, container=0):
    return {"start": start, "end": end, "container_id": container, "container_kind": "ordinary_text",
            "boundary_kind": "generic_sentence_or_paragraph"}


@pytest.mark.parametrize("peak,expected", [(None, (0, 5)), (2, (2, 7)), (10, (10, 15))])
def test_oracle_partial_window_follows_the_peak(peak, expected):
    scores = [0.0] * 20 if peak is None else [-100.0] * 20
    if peak is not None:
        scores[peak] = 0.0
    window = ref.forward_window(0, 20, 5, scores)
    assert (window["start"], window["end"]) == expected and window["decay_tokens"] == 16.0
    for width in (0, -1, 21):
        with pytest.raises(ValueError, match="partial-window width"):
            ref.forward_window(0, 20, width, [0.0] * 20)


def test_oracle_known_answers_for_units_and_allocation():
    assert ref.balanced(0, 257) == [(0, 86), (86, 172), (172, 257)]
    text = '<tool_result>{"place": "Oslo."}</tool_result>\n\nMetadata: {"count": 2}\n'
    units = ref.char_units(text)
    assert [(u["boundary_kind"], text[u["start"]:u["end"]]) for u in units
            if u["boundary_kind"] != "generic_sentence_or_paragraph"] == [
        ("tool_container", '<tool_result>{"place": "Oslo."}</tool_result>'), ("json_container", '{"count": 2}')]
    assert "".join(text[u["start"]:u["end"]] for u in units) == text
    units = [oracle_unit(0, 8), oracle_unit(8, 16)]
    scores = [4.0] * 4 + [-100.0] * 4 + [3.0] * 8
    assert [u["unit_score"] for u in ref.score_units(units, scores)] == [4.0, 3.0]
    support, meta = ref.select_support(units, scores, 8)
    assert support == list(range(8)) and meta["selections"][0]["selection_kind"] == "complete_unit"
    support, meta = ref.select_support([oracle_unit(4, 12), oracle_unit(12, 20)], [0.0] * 20, 11)
    assert support == list(range(4, 15)) and meta["budget_tokens"] == 11
    assert [e["selection_kind"] for e in meta["selections"]] == ["complete_unit", "partial_forward_causal_window"]
    for bad in (math.inf, -math.inf, math.nan):
        with pytest.raises(RuntimeError, match="invalid semantic unit token scores"):
            ref.score_units([oracle_unit(0, 2)], [1.0, bad])
