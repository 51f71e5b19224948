"""Semantic-unit support selection (SUR V1): the host half of ``select_support``.

Reference: src/kv_cache_repair/semantic_units.py (the whole module), called from
api.py:86-97 for every budget strictly between empty and the whole suffix. The
token scores come from the GPU scorer (``scoring.dense_query_relevance_scores``);
everything here is host text and list work on a few hundred units.

Selection, in three steps:

1. Character units. The text is cut into containers (ChatML messages
   ``<|im_start|> .. <|im_end|>`` and the ordinary text between them; a gap
   of only whitespace joins the container before it), each container into
   structured pieces (tool/function call or response elements, JSON objects or
   arrays that open a line or follow ``:``, ``=`` or ``>``; overlapping
   candidates resolved earliest-first, longer first) and the rest into
   sentences or paragraphs.
2. Token units. Each suffix token joins the character unit holding its centre
   (from the tokenizer's offset mapping); runs of tokens in one character unit
   form a unit, units longer than 128 tokens are cut into balanced chunks, and
   units shorter than 8 tokens merge with the shorter contiguous neighbour of
   the same container (the earlier one on a tie), re-chunked when the merge
   exceeds 128.
3. Allocation. A unit scores the mean of its top min(4, n) token scores; units
   are taken whole, best first (earlier on ties), until the next one does not
   fit, which then contributes the contiguous window of the remaining width
   with the largest utility under a forward causal decay of 16 tokens.

The constants, the boundary patterns, the error messages and the dictionary
keys and strings of the units and the allocator metadata are the reference's:
they are the selection's observable contract (positions and metadata), so a
caller switching over sees the same ones.
"""

from __future__ import annotations

import json
import math
import re
from typing import Any, Iterable

SEMANTIC_UNIT_MIN_TOKENS = 8
SEMANTIC_UNIT_MAX_TOKENS = 128
SEMANTIC_UNIT_SCORE_TOP_K = 4
FORWARD_CAUSAL_DECAY_TOKENS = 16.0

# ChatML message (reference semantic_units.py:16-19)
_CHAT_MESSAGE = re.compile(r"<\|im_start\|>.*?<\|im_end\|>", re.DOTALL)
# tool / function call and response elements, same tag closing (:20-24)
_TOOL_TAGS = ("tool_call", "tool_response", "tool_result", "function_call", "function_response")
_TOOL_ELEMENT = re.compile(
    r"<(?P<tag>" + "|".join(_TOOL_TAGS) + r")(?:\s[^>]*)?>.*?</(?P=tag)>", re.DOTALL | re.IGNORECASE)
# sentence / paragraph ends (:25): a blank line, or terminal punctuation with
# any closing quotes or brackets followed by whitespace or, directly, by a
# capital, a digit or a tag
_BREAK = re.compile(r"""
    \n[ \t]*\n+
  | [.!?]["')\]]* (?: [ \t\r\n]+ | (?=[A-Z0-9<]) )
""", re.VERBOSE)
_JSON_OPEN = re.compile(r"[\[{]")
_JSON_LEADS = (":", "=", ">")

_SENTENCE = "generic_sentence_or_paragraph"
_GENERIC = "generic_text"
_MERGED = "short_unit_merged_within_container"


# ---------------------------------------------------------------------------
# 1. character units
# ---------------------------------------------------------------------------

def _containers(text: str) -> list[tuple[int, int, Any, str]]:
    """(start, end, container id, kind): ChatML messages and the text between
    them, ids numbered in text order (reference semantic_units.py:60-111)."""
    out: list[list[Any]] = []
    next_id = 0

    def text_gap(start: int, end: int) -> None:
        nonlocal next_id
        if out and not text[start:end].strip():
            out[-1][1] = end  # whitespace only: the previous container absorbs it
        else:
            out.append([start, end, next_id, "ordinary_text"])
            next_id += 1

    cursor = 0
    for m in _CHAT_MESSAGE.finditer(text):
        if cursor < m.start():
            text_gap(cursor, m.start())
        out.append([m.start(), m.end(), next_id, "chat_message"])
        next_id += 1
        cursor = m.end()
    if cursor < len(text):
        text_gap(cursor, len(text))
    return [(s, e, cid, kind) for s, e, cid, kind in out if e > s]


def _json_spans(text: str, start: int, end: int) -> Iterable[tuple[int, int]]:
    """JSON objects/arrays in [start, end) that open a line or follow ':', '='
    or '>' on it (reference semantic_units.py:28-57). The line's start is the
    last newline in [start, bracket) plus one, or the start of the whole text
    when the container has no newline before the bracket (as the reference
    computes it)."""
    decoder = json.JSONDecoder()
    window = text[start:end]  # decoding stops at the container's end
    cursor = start
    while cursor < end:
        m = _JSON_OPEN.search(text, cursor, end)
        if m is None:
            return
        open_at = m.start()
        # the last non-space character of the line before the bracket, if any
        line_start = text.rfind("\n", start, open_at) + 1
        j = open_at - 1
        while j >= line_start and text[j].isspace():
            j -= 1
        if j >= line_start and text[j] not in _JSON_LEADS:
            cursor = open_at + 1
            continue
        try:
            value, close_rel = decoder.raw_decode(window, open_at - start)
        except json.JSONDecodeError:
            cursor = open_at + 1
            continue
        if not isinstance(value, (dict, list)):
            cursor = open_at + 1
            continue
        yield open_at, start + close_rel
        cursor = start + close_rel


def _pieces(text: str, start: int, end: int, cid: Any, kind: str) -> list[tuple[int, int, Any, str, str]]:
    """(start, end, container id, container kind, boundary kind) of one container:
    structured elements and the generic text around them (reference
    semantic_units.py:114-200)."""
    found = [(m.start(), m.end(), "tool_container") for m in _TOOL_ELEMENT.finditer(text, start, end)]
    found += [(s, e, "json_container") for s, e in _json_spans(text, start, end)]
    kept: list[tuple[int, int, str]] = []
    for cand in sorted(found, key=lambda c: (c[0], c[0] - c[1])):
        if all(cand[1] <= s or e <= cand[0] for s, e, _ in kept):
            kept.append(cand)
    kept.sort(key=lambda c: c[0])

    out = []
    cursor = start
    for child, (s, e, ckind) in enumerate(kept):
        if cursor < s:
            out.append((cursor, s, cid, kind, _GENERIC))
        out.append((s, e, f"{cid}:structured:{child}", ckind, ckind))
        cursor = e
    if cursor < end:
        out.append((cursor, end, cid, kind, _GENERIC))
    return [p for p in out if p[1] > p[0]]


def _sentence_spans(text: str, start: int, end: int) -> list[tuple[int, int]]:
    """Consecutive spans of [start, end) ending at each sentence/paragraph break
    (reference semantic_units.py:203-218)."""
    cuts = [m.end() for m in _BREAK.finditer(text, start, end)]
    spans = [(a, b) for a, b in zip([start] + cuts, cuts) if b > a]
    last = cuts[-1] if cuts else start
    if last < end:
        spans.append((last, end))
    return spans or [(start, end)]


def semantic_char_units(text: str) -> list[dict[str, Any]]:
    """Character units of ``text`` in order; they tile the text (reference
    semantic_units.py:221-250)."""
    units = []
    for c_start, c_end, cid, ckind in _containers(text):
        for start, end, pid, pkind, boundary in _pieces(text, c_start, c_end, cid, ckind):
            if boundary == _GENERIC:
                spans, boundary = _sentence_spans(text, start, end), _SENTENCE
            else:
                spans = [(start, end)]
            units += [{"start": s, "end": e, "container_id": pid, "container_kind": pkind, "boundary_kind": boundary}
                      for s, e in spans if e > s]
    return units


# ---------------------------------------------------------------------------
# 2. token units
# ---------------------------------------------------------------------------

def _balanced(start: int, end: int) -> list[tuple[int, int]]:
    """[start, end) in ceil(n / 128) chunks whose widths differ by at most one,
    the wider ones first (reference semantic_units.py:253-269)."""
    n = end - start
    if n <= 0:
        return []
    count = -(-n // SEMANTIC_UNIT_MAX_TOKENS)
    base, wide = divmod(n, count)
    bounds = [start]
    for i in range(count):
        bounds.append(bounds[-1] + base + (i < wide))
    return list(zip(bounds, bounds[1:]))


def _chunked(unit: dict[str, Any], start: int, end: int) -> list[dict[str, Any]]:
    chunks = _balanced(start, end)
    return [{**unit, "start": s, "end": e, "fixed_chunk_index": i, "fixed_chunk_count": len(chunks)}
            for i, (s, e) in enumerate(chunks)]


def _merge_short(units: list[dict[str, Any]]) -> list[dict[str, Any]]:
    """Merge every unit shorter than 8 tokens that has a contiguous neighbour in
    its container with the shorter such neighbour (the earlier on a tie), the
    lowest such unit first, and re-chunk the merge (reference
    semantic_units.py:290-360).

    A merge keeps the left unit's container and start, so units before it gain
    no merge partner from it: the scan resumes at the merge instead of at the
    first unit, with the same result."""
    out = list(units)

    def partner(i: int) -> int | None:
        unit = out[i]
        options = []
        if i > 0:
            prev = out[i - 1]
            if prev["container_id"] == unit["container_id"] and prev["end"] == unit["start"]:
                options.append((prev["end"] - prev["start"], 0, i - 1))
        if i + 1 < len(out):
            nxt = out[i + 1]
            if nxt["container_id"] == unit["container_id"] and unit["end"] == nxt["start"]:
                options.append((nxt["end"] - nxt["start"], 1, i + 1))
        return min(options)[2] if options else None

    i = 0
    while i < len(out):
        other = partner(i) if out[i]["end"] - out[i]["start"] < SEMANTIC_UNIT_MIN_TOKENS else None
        if other is None:
            i += 1
            continue
        left, right = min(i, other), max(i, other)
        merged = {**out[left], "start": out[left]["start"], "end": out[right]["end"], "boundary_kind": _MERGED}
        out[left:right + 1] = _chunked(merged, merged["start"], merged["end"])
        i = left
    return out


def semantic_unit_token_ranges(*, tokenizer: Any, text: str, expected_token_ids: list[int], suffix_start: int,
                               token_end: int | None = None) -> list[dict[str, Any]]:
    """Token units tiling [suffix_start, token_end) (reference
    semantic_units.py:363-423). The tokenizer must reproduce
    ``expected_token_ids`` and give exact character offsets."""
    encoded = tokenizer(text, add_special_tokens=False, return_offsets_mapping=True)
    ids = [int(v) for v in encoded["input_ids"]]
    if ids != [int(v) for v in expected_token_ids]:
        raise RuntimeError("semantic unit tokenizer identity drift")
    stop = len(ids) if token_end is None else int(token_end)
    if not 0 <= int(suffix_start) < stop <= len(ids):
        raise ValueError("semantic unit suffix start out of range")
    offsets = [(int(a), int(b)) for a, b in encoded["offset_mapping"]]
    chars = semantic_char_units(text)
    if not chars:
        raise RuntimeError("semantic unit construction produced no units")

    runs: list[dict[str, Any]] = []
    at = 0
    key = None
    for tok in range(int(suffix_start), stop):
        a, b = offsets[tok]
        centre = a if b <= a else (a + b - 1) / 2.0
        while at + 1 < len(chars) and centre >= chars[at]["end"]:
            at += 1
        unit = chars[at]
        unit_key = (unit["container_id"], unit["start"], unit["end"])
        if unit_key == key:
            runs[-1]["end"] = tok + 1
        else:
            runs.append({"start": tok, "end": tok + 1, "container_id": unit["container_id"],
                         "container_kind": unit["container_kind"], "boundary_kind": unit["boundary_kind"]})
            key = unit_key

    units = _merge_short([chunk for run in runs for chunk in _chunked(run, run["start"], run["end"])])
    if (not units or units[0]["start"] != int(suffix_start) or units[-1]["end"] != stop
            or any(l["end"] != r["start"] for l, r in zip(units, units[1:]))
            or any(u["end"] - u["start"] > SEMANTIC_UNIT_MAX_TOKENS for u in units)):
        raise RuntimeError("semantic unit token partition drift")
    return units


# ---------------------------------------------------------------------------
# 3. allocation
# ---------------------------------------------------------------------------

def score_semantic_units(*, units: list[dict[str, Any]], token_scores: list[float]) -> list[dict[str, Any]]:
    """Each unit with its index, token count and score: the mean of its top
    min(4, n) token scores (reference semantic_units.py:426-448)."""
    scored = []
    for index, unit in enumerate(units):
        start, end = int(unit["start"]), int(unit["end"])
        values = [float(v) for v in token_scores[start:end]]
        if not values or not all(math.isfinite(v) for v in values):
            raise RuntimeError("invalid semantic unit token scores")
        k = min(SEMANTIC_UNIT_SCORE_TOP_K, len(values))
        top = sorted(values, reverse=True)[:k]
        scored.append({**unit, "unit_index": index, "token_count": end - start, "unit_score": sum(top) / k,
                       "score_top_k": k})
    return scored


def best_forward_causal_window(*, start: int, end: int, width: int, token_scores: list[float]) -> dict[str, Any]:
    """The window of ``width`` tokens in [start, end) with the largest utility,
    the earliest on ties. A token's utility is the larger of its own
    exp(score - max) and 16-token-decayed utility carried from the token before
    (reference semantic_units.py:451-484); the window sum slides by adding the
    entering token's utility minus the leaving one's."""
    width = int(width)
    n = int(end) - int(start)
    if not 0 < width <= n:
        raise ValueError("invalid semantic unit partial-window width")
    values = [float(v) for v in token_scores[start:end]]
    peak = max(values)
    decay = math.exp(-1.0 / FORWARD_CAUSAL_DECAY_TOKENS)
    utility = []
    carried = 0.0
    for v in values:
        carried = max(math.exp(v - peak), decay * carried)
        utility.append(carried)
    total = sum(utility[:width])
    best, best_total = 0, total
    for first in range(1, n - width + 1):
        total += utility[first + width - 1] - utility[first - 1]
        if total > best_total:
            best, best_total = first, total
    return {"start": int(start) + best, "end": int(start) + best + width, "utility": best_total,
            "decay_tokens": FORWARD_CAUSAL_DECAY_TOKENS}


def select_semantic_unit_support(*, units: list[dict[str, Any]], token_scores: list[float],
                                 budget_tokens: int) -> tuple[list[int], dict[str, Any]]:
    """Exactly ``budget_tokens`` suffix positions (at least 1, at most the
    suffix), sorted, and the allocator's metadata (reference
    semantic_units.py:487-576)."""
    if not units:
        raise ValueError("semantic unit refresh requires units")
    first, last = int(units[0]["start"]), int(units[-1]["end"])
    budget = min(max(1, int(budget_tokens)), last - first)
    scored = score_semantic_units(units=units, token_scores=token_scores)
    order = sorted(scored, key=lambda u: (-float(u["unit_score"]), int(u["start"])))

    support: list[int] = []
    picks = []
    for rank, unit in enumerate(order):
        left = budget - len(support)
        if left <= 0:
            break
        start, end = int(unit["start"]), int(unit["end"])
        window = None
        if end - start <= left:
            taken, kind = range(start, end), "complete_unit"
        else:
            window = best_forward_causal_window(start=start, end=end, width=left, token_scores=token_scores)
            taken, kind = range(window["start"], window["end"]), "partial_forward_causal_window"
        support += taken
        picks.append({"rank": rank, "unit_index": int(unit["unit_index"]), "unit_start": start, "unit_end": end,
                      "unit_score": float(unit["unit_score"]), "selection_kind": kind,
                      "selected_start": taken[0], "selected_end": taken[-1] + 1, "selected_tokens": len(taken),
                      "partial_window": window})
    if len(support) != budget or len(set(support)) != budget:
        raise RuntimeError("semantic unit refresh support budget drift")
    return sorted(support), {
        "revision": "SEMANTIC_UNIT_REFRESH_V1",
        "information_scope": "current query, edited prompt tokens, and deployable generic container/sentence "
                             "boundaries only",
        "kv_probe_token_calls": 0,
        "planning_expansion_token_calls": 0,
        "budget_tokens": budget,
        "unit_count": len(scored),
        "unit_score_rule": "mean of top min(4, unit_token_count) token scores",
        "long_unit_rule": "balanced fixed chunks with maximum 128 tokens",
        "short_unit_rule": "units shorter than 8 tokens merge with an adjacent unit in the same container when "
                           "one exists",
        "partial_unit_rule": "maximum-utility contiguous remaining-budget window under forward exponential causal "
                             "decay with 16-token scale",
        "units": scored,
        "selections": picks,
    }
