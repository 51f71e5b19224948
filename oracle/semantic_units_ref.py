"""Test infrastructure only: a plain restatement of the reference's semantic-unit
selection (src/kv_cache_repair/semantic_units.py), the checker for the
package's kv_cache_repair_amd.semantic_units in tests/test_semantic_units_diff.py.
Nothing in the package imports it.

Written for transparency, not speed: every step follows the reference's order
literally (the short-unit merge rescans from the first unit after every merge,
JSON candidates are found by a character scan and decoded from a substring,
window utilities are summed incrementally as the reference sums them). The
boundary patterns, constants and strings are the reference's observable
contract and are repeated as data.

Pinned by: the reference's own known answers (its tests/test_semantic_units.py:40-140:
window peaks and width refusals, balanced chunks, whole tool/JSON containers,
top-four ranking, tie order, non-finite refusal), restated against this module in
tests/test_semantic_units_diff.py, and, on fuzzed ChatML / tool / JSON
transcripts, unit lists and score vectors, equality with the package's
implementation, which was written independently in a different form (mutations
of the lead-in set, the merge tie-break, the window tie rule, the whitespace
absorption and the chunk widths planted here each fail those tests).
"""

from __future__ import annotations

import json
import math
import re

MIN_TOKENS = 8          # reference semantic_units.py:11
MAX_TOKENS = 128        # :12
TOP_K = 4               # :13
DECAY_TOKENS = 16.0     # :14

CHAT = re.compile(r"<\|im_start\|>.*?<\|im_end\|>", flags=re.DOTALL)  # :16-19
TOOL = re.compile(  # :20-24
    r"<(?P<tag>tool_call|tool_response|tool_result|function_call|"
    r"function_response)(?:\s[^>]*)?>.*?</(?P=tag)>",
    flags=re.DOTALL | re.IGNORECASE,
)
BREAK = re.compile(r"\n[ \t]*\n+|[.!?][\"')\]]*(?:[ \t\r\n]+|(?=[A-Z0-9<]))")  # :25


def json_blocks(text: str, start: int, end: int) -> list[tuple[int, int]]:
    """reference semantic_units.py:28-58: scan [start, end) for '[' or '{'; a
    bracket qualifies when the stripped text from its line's start (the char
    after the last newline in [start, bracket), else index 0) is empty or ends
    in ':', '=' or '>', and the JSON value decoded from the bracket up to `end`
    is an object or array; the scan then continues after the value."""
    found = []
    p = start
    while p < end:
        if text[p] not in "[{":
            p += 1
            continue
        newline = text.rfind("\n", start, p)
        lead = text[newline + 1:p].strip()
        if lead and lead[-1] not in ":=>":
            p += 1
            continue
        try:
            value, length = json.JSONDecoder().raw_decode(text[p:end])
        except json.JSONDecodeError:
            p += 1
            continue
        if isinstance(value, (dict, list)):
            found.append((p, p + length))
            p += length
        else:
            p += 1
    return found


def containers(text: str) -> list[list]:
    """reference :61-111 as [start, end, container_id, kind] lists."""
    out = []
    ident = 0
    pos = 0

    def gap(a: int, b: int) -> None:
        nonlocal ident
        if out and text[a:b].strip() == "":
            out[-1][1] = b
        else:
            out.append([a, b, ident, "ordinary_text"])
            ident += 1

    for m in CHAT.finditer(text):
        if pos < m.start():
            gap(pos, m.start())
        out.append([m.start(), m.end(), ident, "chat_message"])
        ident += 1
        pos = m.end()
    if pos < len(text):
        gap(pos, len(text))
    elif not out:
        out.append([0, len(text), ident, "ordinary_text"])
    return [c for c in out if c[1] > c[0]]


def structured(text: str, c: list) -> list[dict]:
    """reference :114-193: tool elements and JSON blocks of one container, the
    non-overlapping ones taken by (start, longer first), and generic text
    around them."""
    start, end, cid, kind = c
    cands = [(m.start(), m.end(), "tool_container") for m in TOOL.finditer(text, start, end)]
    cands += [(a, b, "json_container") for a, b in json_blocks(text, start, end)]
    cands.sort(key=lambda t: (t[0], t[0] - t[1]))
    taken = []
    for a, b, k in cands:
        if any(a < tb and ta < b for ta, tb, _ in taken):
            continue
        taken.append((a, b, k))
    taken.sort(key=lambda t: t[0])
    pieces = []
    pos = start
    for i, (a, b, k) in enumerate(taken):
        if pos < a:
            pieces.append(dict(start=pos, end=a, container_id=cid, container_kind=kind, boundary_kind="generic_text"))
        pieces.append(dict(start=a, end=b, container_id=f"{cid}:structured:{i}", container_kind=k, boundary_kind=k))
        pos = b
    if pos < end:
        pieces.append(dict(start=pos, end=end, container_id=cid, container_kind=kind, boundary_kind="generic_text"))
    return [p for p in pieces if p["end"] > p["start"]]


def sentences(text: str, start: int, end: int) -> list[tuple[int, int]]:
    """reference :196-211."""
    spans = []
    pos = start
    for m in BREAK.finditer(text, start, end):
        if m.end() > pos:
            spans.append((pos, m.end()))
        pos = m.end()
    if pos < end:
        spans.append((pos, end))
    return spans if spans else [(start, end)]


def char_units(text: str) -> list[dict]:
    """reference semantic_char_units, :214-244."""
    units = []
    for c in containers(text):
        for piece in structured(text, c):
            if piece["boundary_kind"] == "generic_text":
                spans = sentences(text, piece["start"], piece["end"])
                boundary = "generic_sentence_or_paragraph"
            else:
                spans = [(piece["start"], piece["end"])]
                boundary = piece["boundary_kind"]
            for a, b in spans:
                if b > a:
                    units.append(dict(start=a, end=b, container_id=piece["container_id"],
                                      container_kind=piece["container_kind"], boundary_kind=boundary))
    return units


def balanced(start: int, end: int) -> list[tuple[int, int]]:
    """reference :247-263: ceil(n / 128) chunks, the first n mod count one wider."""
    n = end - start
    if n <= 0:
        return []
    count = math.ceil(n / MAX_TOKENS)
    widths = [n // count + (1 if i < n % count else 0) for i in range(count)]
    out, pos = [], start
    for w in widths:
        out.append((pos, pos + w))
        pos += w
    return out


def with_chunks(unit: dict, start: int, end: int) -> list[dict]:
    chunks = balanced(start, end)
    return [dict(unit, start=a, end=b, fixed_chunk_index=i, fixed_chunk_count=len(chunks))
            for i, (a, b) in enumerate(chunks)]


def split_long(units: list[dict]) -> list[dict]:
    """reference :266-285."""
    out = []
    for u in units:
        out += with_chunks(u, u["start"], u["end"])
    return out


def merge_short(units: list[dict]) -> list[dict]:
    """reference :288-357: repeat { the first unit shorter than 8 with a
    contiguous same-container neighbour merges with the neighbour minimising
    (length, previous-before-next); the merge is re-chunked } until none."""
    units = list(units)
    while True:
        choice = None
        for i, u in enumerate(units):
            if u["end"] - u["start"] >= MIN_TOKENS:
                continue
            options = []
            if i > 0:
                v = units[i - 1]
                if v["container_id"] == u["container_id"] and v["end"] == u["start"]:
                    options.append((v["end"] - v["start"], 0, i - 1))
            if i + 1 < len(units):
                v = units[i + 1]
                if v["container_id"] == u["container_id"] and u["end"] == v["start"]:
                    options.append((v["end"] - v["start"], 1, i + 1))
            if options:
                choice = (i, min(options)[2])
                break
        if choice is None:
            return units
        lo, hi = min(choice), max(choice)
        merged = dict(units[lo], start=units[lo]["start"], end=units[hi]["end"],
                      boundary_kind="short_unit_merged_within_container")
        units[lo:hi + 1] = with_chunks(merged, merged["start"], merged["end"])


def score_units(units: list[dict], token_scores: list[float]) -> list[dict]:
    """reference :424-447: the mean of a unit's top min(4, n) token scores."""
    out = []
    for index, u in enumerate(units):
        scores = [float(s) for s in token_scores[u["start"]:u["end"]]]
        if not scores or not all(math.isfinite(s) for s in scores):
            raise RuntimeError("invalid semantic unit token scores")
        k = min(TOP_K, len(scores))
        out.append(dict(u, unit_index=index, token_count=u["end"] - u["start"],
                        unit_score=sum(sorted(scores, reverse=True)[:k]) / k, score_top_k=k))
    return out


def forward_window(start: int, end: int, width: int, token_scores: list[float]) -> dict:
    """reference :450-485: utility u_i = max(exp(s_i - max s), decay * u_{i-1});
    the width-token window with the largest sum (first on ties), its sum updated
    incrementally as the window slides."""
    n = end - start
    if not 0 < width <= n:
        raise ValueError("invalid semantic unit partial-window width")
    scores = [float(s) for s in token_scores[start:end]]
    top = max(scores)
    decay = math.exp(-1.0 / DECAY_TOKENS)
    util, run = [], 0.0
    for s in scores:
        run = max(math.exp(s - top), decay * run)
        util.append(run)
    total = sum(util[:width])
    best, best_total = 0, total
    for a in range(1, n - width + 1):
        total += util[a + width - 1] - util[a - 1]
        if total > best_total:
            best, best_total = a, total
    return {"start": start + best, "end": start + best + width, "utility": best_total,
            "decay_tokens": DECAY_TOKENS}


def select_support(units: list[dict], token_scores: list[float], budget_tokens: int):
    """reference select_semantic_unit_support, :488-576: (sorted positions,
    metadata). Units by score (earlier first on ties), whole while they fit;
    the first that does not contributes its best forward-causal window."""
    if not units:
        raise ValueError("semantic unit refresh requires units")
    first, last = units[0]["start"], units[-1]["end"]
    budget = min(max(1, int(budget_tokens)), last - first)
    scored = score_units(units, token_scores)
    order = sorted(scored, key=lambda u: (-u["unit_score"], u["start"]))
    support, picks = [], []
    for rank, u in enumerate(order):
        left = budget - len(support)
        if left <= 0:
            break
        if u["end"] - u["start"] <= left:
            positions, kind, window = list(range(u["start"], u["end"])), "complete_unit", None
        else:
            window = forward_window(u["start"], u["end"], left, token_scores)
            positions, kind = list(range(window["start"], window["end"])), "partial_forward_causal_window"
        support += positions
        picks.append({"rank": rank, "unit_index": u["unit_index"], "unit_start": u["start"], "unit_end": u["end"],
                      "unit_score": u["unit_score"], "selection_kind": kind, "selected_start": min(positions),
                      "selected_end": max(positions) + 1, "selected_tokens": len(positions),
                      "partial_window": window})
    if len(support) != budget or len(set(support)) != budget:
        raise RuntimeError("semantic unit refresh support budget drift")
    return sorted(support), {"budget_tokens": budget, "unit_count": len(scored), "units": scored,
                             "selections": picks}
