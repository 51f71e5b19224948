"""Semantic-unit (SUR) selection on the host: the known answers of the
reference's own tests (tests/test_semantic_units.py), then cases of this build
pinned by hand-worked partitions, brute force and invariants.

The allocator and partitioner are host code (kv_cache_repair_amd.semantic_units);
the GPU scorer that feeds them is covered by test_gpu_scoring.py and the public
selection end to end by test_gpu_api.py.
"""

from __future__ import annotations

import math
import random

import pytest

from kv_cache_repair_amd import semantic_units as su
from kv_cache_repair_amd.semantic_units import (best_forward_causal_window, score_semantic_units,
                                                select_semantic_unit_support, semantic_char_units,
                                                semantic_unit_token_ranges)


class CharTokenizer:
    """One token per character with exact offsets; decoding is refused (units
    come from the canonical text, never from decoded tokens)."""

    def __call__(self, text, *, add_special_tokens=False, return_offsets_mapping=False):
        assert add_special_tokens is False
        out = {"input_ids": [ord(c) for c in text]}
        if return_offsets_mapping:
            out["offset_mapping"] = [(i, i + 1) for i in range(len(text))]
        return out

    def decode(self, ids):
        raise AssertionError("units must come from the canonical text")


def unit(start, end, container=0):
    return {"start": start, "end": end, "container_id": container, "container_kind": "ordinary_text",
            "boundary_kind": "generic_sentence_or_paragraph"}


def spans(units):
    return [(u["start"], u["end"]) for u in units]


def token_units(text, suffix_start=0, token_end=None):
    tok = CharTokenizer()
    return semantic_unit_token_ranges(tokenizer=tok, text=text, expected_token_ids=tok(text)["input_ids"],
                                      suffix_start=suffix_start, token_end=token_end)


# ---------------------------------------------------------------------------
# the reference's known answers (tests/test_semantic_units.py:40-140)
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("peak,expected", [(None, (0, 5)), (2, (2, 7)), (10, (10, 15))])
def test_partial_window_follows_the_peak_without_a_tail_bias(peak, expected):
    scores = [0.0] * 20 if peak is None else [-100.0] * 20
    if peak is not None:
        scores[peak] = 0.0
    window = best_forward_causal_window(start=0, end=20, width=5, token_scores=scores)
    assert (window["start"], window["end"]) == expected
    assert window["decay_tokens"] == 16.0


@pytest.mark.parametrize("width", [0, -1, 21])
def test_partial_window_refuses_a_width_outside_the_unit(width):
    with pytest.raises(ValueError, match="partial-window width"):
        best_forward_causal_window(start=0, end=20, width=width, token_scores=[0.0] * 20)


def test_units_use_canonical_offsets_and_stop_before_a_delayed_query():
    text = "Alpha support sentence.\n\nQuestion: Where?"
    end = text.index("\n\nQuestion:")
    units = token_units(text, 0, end)
    support, _ = select_semantic_unit_support(units=units, token_scores=[float(i) for i in range(end)],
                                              budget_tokens=5)
    assert spans(units) == [(0, end)]
    assert support == list(range(end - 5, end))


def test_units_refuse_a_tokenizer_that_does_not_reproduce_the_ids():
    with pytest.raises(RuntimeError, match="tokenizer identity drift"):
        semantic_unit_token_ranges(tokenizer=CharTokenizer(), text="A sentence.", expected_token_ids=[0],
                                   suffix_start=0)


def test_long_units_become_balanced_chunks():
    assert spans(token_units("A" * 257)) == [(0, 86), (86, 172), (172, 257)]


def test_tool_and_json_containers_stay_whole():
    text = '<tool_result>{"place": "Oslo."}</tool_result>\n\nMetadata: {"count": 2}\n'
    units = semantic_char_units(text)
    structured = [(u["boundary_kind"], text[u["start"]:u["end"]]) for u in units
                  if u["boundary_kind"] != "generic_sentence_or_paragraph"]
    assert structured == [("tool_container", '<tool_result>{"place": "Oslo."}</tool_result>'),
                          ("json_container", '{"count": 2}')]
    assert "".join(text[u["start"]:u["end"]] for u in units) == text


def test_units_rank_by_their_top_four_not_the_mean_of_all():
    units = [unit(0, 8), unit(8, 16)]
    scores = [4.0] * 4 + [-100.0] * 4 + [3.0] * 8
    ranked = score_semantic_units(units=units, token_scores=scores)
    support, meta = select_semantic_unit_support(units=units, token_scores=scores, budget_tokens=8)
    assert [u["unit_score"] for u in ranked] == [4.0, 3.0]
    assert support == list(range(8))
    assert meta["selections"][0]["selection_kind"] == "complete_unit"
    assert meta["kv_probe_token_calls"] == meta["planning_expansion_token_calls"] == 0


def test_ties_take_the_earlier_unit_and_fill_the_last_window():
    support, meta = select_semantic_unit_support(units=[unit(4, 12), unit(12, 20)], token_scores=[0.0] * 20,
                                                 budget_tokens=11)
    assert support == list(range(4, 15))
    assert [e["selection_kind"] for e in meta["selections"]] == ["complete_unit", "partial_forward_causal_window"]
    assert meta["budget_tokens"] == 11


@pytest.mark.parametrize("bad", [math.inf, -math.inf, math.nan])
def test_unit_scores_refuse_non_finite_values(bad):
    with pytest.raises(RuntimeError, match="invalid semantic unit token scores"):
        score_semantic_units(units=[unit(0, 2)], token_scores=[1.0, bad])


# ---------------------------------------------------------------------------
# character units, worked by hand
# ---------------------------------------------------------------------------

def test_sentence_and_paragraph_breaks():
    text = 'One. Two!Three? "Four." 5th\n \n\nSix.Seven'
    got = [text[u["start"]:u["end"]] for u in semantic_char_units(text)]
    # ". " ends One; "!" before a capital ends Two (zero-width lookahead); '? ' ends
    # Three; '." ' (closing quote, space) ends "Four."; the blank lines end 5th;
    # ".S" ends Six (capital lookahead)
    assert got == ["One. ", "Two!", "Three? ", '"Four." ', "5th\n \n\n", "Six.", "Seven"]
    assert {u["boundary_kind"] for u in semantic_char_units(text)} == {"generic_sentence_or_paragraph"}


def test_chat_messages_are_containers_and_whitespace_joins_the_one_before():
    a = "<|im_start|>user\nHi. There<|im_end|>"
    b = "<|im_start|>assistant\nOk<|im_end|>"
    text = "  " + a + "\n\n" + b + " tail."
    units = semantic_char_units(text)
    assert "".join(text[u["start"]:u["end"]] for u in units) == text
    kinds = [(u["container_id"], u["container_kind"], text[u["start"]:u["end"]]) for u in units]
    # leading whitespace with no container before it is ordinary text (id 0); the
    # blank gap joins message 1; " tail." is ordinary text 3
    assert kinds == [(0, "ordinary_text", "  "),
                     (1, "chat_message", "<|im_start|>user\nHi. "),
                     (1, "chat_message", "There<|im_end|>\n\n"),
                     (2, "chat_message", b),
                     (3, "ordinary_text", " tail.")]


def test_json_needs_a_line_start_or_a_lead_in():
    accepted = semantic_char_units('x = [1, 2]\n{"a": 1}\nsee [3]')
    got = [(u["boundary_kind"], u["container_id"]) for u in accepted if u["boundary_kind"] == "json_container"]
    # "x = [1, 2]" (after '='), '{"a": 1}' (opens its line); "see [3]" is prose
    assert got == [("json_container", "0:structured:0"), ("json_container", "0:structured:1")]


def test_json_line_start_without_a_newline_is_the_start_of_the_text():
    """A container with no newline before the bracket takes its line from the
    start of the whole text (the reference's rfind(...) + 1 with no match)."""
    lead_tag = "<|im_start|>x<|im_end|>" + '{"a": 1}'
    lead_word = "<|im_start|>x<|im_end|>" + 'abc {"a": 1}'
    assert any(u["boundary_kind"] == "json_container" for u in semantic_char_units(lead_tag))
    assert not any(u["boundary_kind"] == "json_container" for u in semantic_char_units(lead_word))


def test_overlapping_structures_keep_the_earliest_then_the_longest():
    text = '<tool_call>{"f": [1]}</tool_call>'
    units = semantic_char_units(text)
    assert [(u["boundary_kind"], u["start"], u["end"]) for u in units] == [("tool_container", 0, len(text))]


def test_empty_text_has_no_units():
    assert semantic_char_units("") == []
    with pytest.raises(ValueError, match="suffix start out of range"):
        token_units("")


# ---------------------------------------------------------------------------
# token units
# ---------------------------------------------------------------------------

def test_short_sentences_merge_with_the_shorter_neighbour():
    text = "Ab. Cdefghijklm. Nopqrstuvwxyzab. "
    # sentences of 4, 13 and 17 characters (one token each): the 4-token one
    # merges with its only neighbour, the 13-token one
    assert spans(token_units(text)) == [(0, 17), (17, 34)]
    assert token_units(text)[0]["boundary_kind"] == "short_unit_merged_within_container"


def test_short_units_do_not_merge_across_containers():
    text = "<|im_start|>a<|im_end|>Tiny."
    units = token_units(text)
    assert spans(units) == [(0, 23), (23, 28)]


def test_suffix_start_and_end_bound_the_partition():
    text = "First sentence here. Second sentence here. Third one."
    units = token_units(text, 5, 40)
    assert units[0]["start"] == 5 and units[-1]["end"] == 40
    with pytest.raises(ValueError, match="suffix start out of range"):
        token_units(text, 40, 40)


def merge_restarting_from_the_first_unit(units):
    """The merge rule as stated: after every merge, rescan from the first unit."""
    out = list(units)
    while True:
        found = None
        for i, u in enumerate(out):
            if u["end"] - u["start"] >= su.SEMANTIC_UNIT_MIN_TOKENS:
                continue
            options = []
            if i and out[i - 1]["container_id"] == u["container_id"] and out[i - 1]["end"] == u["start"]:
                options.append((out[i - 1]["end"] - out[i - 1]["start"], 0, i - 1))
            if i + 1 < len(out) and out[i + 1]["container_id"] == u["container_id"] and u["end"] == out[i + 1]["start"]:
                options.append((out[i + 1]["end"] - out[i + 1]["start"], 1, i + 1))
            if options:
                found = (i, min(options)[2])
                break
        if found is None:
            return out
        lo, hi = min(found), max(found)
        merged = {**out[lo], "start": out[lo]["start"], "end": out[hi]["end"],
                  "boundary_kind": "short_unit_merged_within_container"}
        out[lo:hi + 1] = su._chunked(merged, merged["start"], merged["end"])


@pytest.mark.parametrize("seed", range(40))
def test_merge_resuming_at_the_merge_equals_rescanning(seed):
    rng = random.Random(seed)
    units, at, container = [], 0, 0
    for _ in range(rng.randint(1, 40)):
        width = rng.choice([1, 2, 3, 5, 7, 8, 9, 20, 60, 127, 128])
        if rng.random() < 0.2:
            container += 1
        if rng.random() < 0.1:
            at += 1  # a gap: not contiguous
        units += su._chunked(unit(at, at + width, container), at, at + width)
        at += width
    assert su._merge_short(units) == merge_restarting_from_the_first_unit(units)


def test_token_units_tile_a_mixed_document():
    text = ("<|im_start|>system\nYou answer briefly.<|im_end|>\n"
            "<|im_start|>user\nConfig: {\"k\": [1, 2, 3], \"name\": \"x\"}. What is k? " + "Word " * 60 +
            "end.<|im_end|>\n<tool_response>result: 42</tool_response> Done.")
    units = token_units(text, 10)
    assert units[0]["start"] == 10 and units[-1]["end"] == len(text)
    assert all(a["end"] == b["start"] for a, b in zip(units, units[1:]))
    assert all(0 < u["end"] - u["start"] <= 128 for u in units)
    for i, u in enumerate(units):  # a short unit survives only without a contiguous same-container neighbour
        if u["end"] - u["start"] < 8:
            for j in (i - 1, i + 1):
                if 0 <= j < len(units):
                    assert units[j]["container_id"] != u["container_id"]


# ---------------------------------------------------------------------------
# allocation
# ---------------------------------------------------------------------------

def test_window_matches_brute_force_on_random_scores():
    rng = random.Random(7)
    decay = math.exp(-1.0 / 16.0)
    for _ in range(200):
        n = rng.randint(1, 60)
        width = rng.randint(1, n)
        scores = [rng.uniform(-3, 3) for _ in range(n + 5)]
        start = rng.randint(0, 5)
        vals = scores[start:start + n]
        peak = max(vals)
        util, run = [], 0.0
        for v in vals:
            run = max(math.exp(v - peak), decay * run)
            util.append(run)
        sums = [math.fsum(util[i:i + width]) for i in range(n - width + 1)]
        best = max(range(len(sums)), key=lambda i: (sums[i], -i))
        got = best_forward_causal_window(start=start, end=start + n, width=width, token_scores=scores)
        assert got["start"] - start == best
        assert got["end"] - got["start"] == width
        assert math.isclose(got["utility"], sums[best], rel_tol=1e-12)


def test_window_carries_a_peak_forward_with_the_decay():
    scores = [-50.0] * 10
    scores[3] = 0.0
    window = best_forward_causal_window(start=0, end=10, width=3, token_scores=scores)
    # utility 1 at the peak, decayed by exp(-1/16) per token after it, ~0 before
    assert (window["start"], window["end"]) == (3, 6)
    d = math.exp(-1 / 16)
    assert math.isclose(window["utility"], 1 + d + d * d, rel_tol=1e-12)


@pytest.mark.parametrize("seed", range(30))
def test_allocation_invariants(seed):
    rng = random.Random(100 + seed)
    first = rng.randint(0, 50)
    units, at = [], first
    for _ in range(rng.randint(1, 12)):
        w = rng.randint(1, 128)
        units.append(unit(at, at + w, rng.randint(0, 2)))
        at += w
    scores = [rng.choice([rng.uniform(-1, 1), 0.5]) for _ in range(at)]
    budget = rng.randint(0, at - first + 5)
    support, meta = select_semantic_unit_support(units=units, token_scores=scores, budget_tokens=budget)
    want = min(max(1, budget), at - first)
    assert len(support) == len(set(support)) == want == meta["budget_tokens"]
    assert support == sorted(support) and all(first <= p < at for p in support)
    ranked = sorted(score_semantic_units(units=units, token_scores=scores),
                    key=lambda u: (-u["unit_score"], u["start"]))
    taken = set(support)
    for entry in meta["selections"]:
        assert ranked[entry["rank"]]["unit_index"] == entry["unit_index"]
        got = set(range(entry["selected_start"], entry["selected_end"]))
        assert got <= taken and len(got) == entry["selected_tokens"]
        if entry["selection_kind"] == "complete_unit":
            assert (entry["selected_start"], entry["selected_end"]) == (entry["unit_start"], entry["unit_end"])
    assert meta["unit_count"] == len(units) and meta["revision"] == "SEMANTIC_UNIT_REFRESH_V1"


def test_allocation_refuses_no_units():
    with pytest.raises(ValueError, match="requires units"):
        select_semantic_unit_support(units=[], token_scores=[], budget_tokens=1)
