"""Join and filter admission against the reference's literal known answers.

tests/golden/admission_cases.json holds the cases as data: constructor
arguments and operation sequences with their expected results (groups,
settle events, freed documents, page and token counts, constructor errors).
This module builds each scheduler and interprets the operations.
"""

import json
import os

import numpy as np
import pytest

from quail_amd.pack import FilterAdmission, JoinAdmission, pages_for
from quail_amd.tokens import PrefixTree

HERE = os.path.dirname(os.path.abspath(__file__))
TABLE = json.load(open(os.path.join(HERE, "golden", "admission_cases.json")))
CASES = TABLE["cases"]
ERRORS = {"ValueError": ValueError, "KeyError": KeyError}


def _options(spec):
    """Constructor keyword arguments from a case's JSON options."""
    out = {}
    for name, value in spec.items():
        if name in ("prefix", "docs", "stages", "budget", "arena_pages", "page_tokens"):
            continue
        if name in ("resident", "anchor_partners"):
            value = {int(k): v for k, v in value.items()}
        elif name == "tree":
            value = PrefixTree(value["order"], value["parent"], value["shared"])
        elif name == "answer_dtype":
            value = np.dtype(value).type
        elif name == "can_borrow":
            assert value is False, "only a refusing borrow rule is expressible"
            value = (lambda doc, parent, same_chunk: False)
        out[name] = value
    return out


def _build(case):
    spec = case["new"]
    opts = _options(spec)
    if case["kind"] == "join":
        return JoinAdmission(spec["prefix"], spec["stages"], spec["budget"],
                             spec["arena_pages"], spec["page_tokens"], **opts)
    return FilterAdmission(spec["docs"], spec["stages"], spec["budget"], spec["arena_pages"],
                           spec["page_tokens"], **opts)


def _listed(x):
    """Tuples and numpy values as nested lists and plain numbers, for JSON."""
    if isinstance(x, (tuple, list)):
        return [_listed(v) for v in x]
    if isinstance(x, np.ndarray):
        return x.tolist()
    if isinstance(x, np.generic):
        return x.item()
    return x


def _filter_drive(sched, truth_bit, arena_pages):
    """Admit and report until done, each chunk's answers delivered before the
    next chunk is asked for; every document answers truth_bit at every
    stage. A page ledger (None: no page bin) charges a fresh document its
    own tokens plus the kept extra and credits the documents each report
    frees. Returns the chunks."""
    held = {}
    chunks = []
    while not sched.done():
        free = None if arena_pages is None else arena_pages - sum(held.values())
        groups = sched.next_chunk(free)
        assert groups, "nothing admissible with every answer in"
        chunks.append(groups)
        for doc, _, fresh in groups:
            if fresh:
                held[doc] = pages_for(sched.own_tokens(doc) + sched.kept_extra, 16)
        for doc, stage, _ in groups:
            for gone in sched.report(doc, stage, bool(truth_bit)):
                held.pop(gone)
    return chunks


def _join_op(s, op, args):
    if op == "next_chunk":
        return _listed(s.next_chunk(args[0]))
    if op == "next_chunk_first":
        return _listed(s.next_chunk(args[0])[0])
    if op == "anchors":
        return [g[0] for g in s.next_chunk(args[0])]
    if op == "report":
        a, j, start, end, bits = args
        return _listed(s.report(a, j, start, end, bits))
    if op == "take_settled":
        return _listed(s.take_settled())
    if op == "admit":
        tokens, resident_pages = args
        if resident_pages is None:
            return s.admit(tokens)
        return s.admit(tokens, resident_pages=resident_pages)
    if op == "buildable_tokens":
        return s.buildable_tokens()
    if op == "blocked_pages":
        return s.blocked_pages
    if op == "shared":
        return s.borrowing.shared(args[0])
    if op == "done":
        return s.done()
    if op == "answers":
        j, a = args
        return _listed(s.answers[j][a])
    if op == "drive_scores":
        # every group reports its partners' slice of the given scores
        free, scores = args
        values = np.asarray(scores, dtype=np.float32)
        while not s.done():
            groups = s.next_chunk(free)
            assert groups
            for a, j, start, end, _ in groups:
                s.report(a, j, start, end, values[start:end])
        assert s.answers[0][0].dtype == np.float32
        return None
    raise AssertionError(f"unknown join op {op}")


def _filter_op(s, op, args):
    if op == "next_chunk":
        return _listed(s.next_chunk(args[0]) if args[0] is not None else s.next_chunk())
    if op == "report":
        doc, stage, passed, release = args
        return _listed(s.report(doc, stage, passed, release=release))
    if op == "resident":
        return args[0] in s.resident
    if op == "resident_count":
        return len(s.resident)
    if op == "drain_ready":
        return _listed(s.drain_ready())
    if op == "own_tokens":
        return s.own_tokens(args[0])
    if op == "shared":
        return s.borrowing.shared(args[0])
    if op == "blocked_pages":
        return s.blocked_pages
    if op == "done":
        return s.done()
    if op == "drive":
        chunks = _filter_drive(s, args[0], args[1])
        return {"survivors": len(s.survivors()), "groups": sum(map(len, chunks))}
    raise AssertionError(f"unknown filter op {op}")


def _matches(got, want):
    if isinstance(want, dict) and "first" in want:
        return bool(got) and got[0] == want["first"] and all(g in got for g in want["has"])
    if isinstance(want, dict) and "survivors_at_least" in want:
        return (got["survivors"] >= want["survivors_at_least"]
                and got["groups"] < want["groups_below"])
    return got == want


@pytest.mark.parametrize("case", CASES, ids=[c["name"] for c in CASES])
def test_admission_known_answers(case):
    if "raises" in case:
        with pytest.raises(ERRORS[case["raises"]], match=case["match"]):
            _build(case)
        return
    sched = _build(case)
    run = _join_op if case["kind"] == "join" else _filter_op
    for step, entry in enumerate(case["ops"]):
        op, args, want = entry[0], entry[1:-1], entry[-1]
        if isinstance(want, str) and want in ERRORS:
            with pytest.raises(ERRORS[want]):
                run(sched, op, args)
            continue
        got = run(sched, op, args)
        if want is None and got is None:
            continue
        assert _matches(got, want), f"{case['name']} step {step} {op}{args}: {got} != {want}"


def test_the_table_fails_on_a_changed_answer():
    """A one-value change to a case's expectation fails it."""
    case = json.loads(json.dumps(next(c for c in CASES if c["name"]
                                      == "join_resident_anchor_packs_while_a_fresh_one_waits")))
    case["ops"][1][-1] = 9
    with pytest.raises(AssertionError):
        test_admission_known_answers(case)
