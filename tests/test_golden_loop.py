"""quail_amd's loop against the reference's own, chunk by chunk.

tests/golden/make_loop_golden.py ran the reference's run_filter /
run_join / pack_chunk / prefix_tree (quail/backends/quail/executor/
loop.py, pack.py, arena.py; quail/execution/tokens.py) on seeded corpora
with a stand-in model that answers from each final row's token and
position, and saved every chunk it packed. The same scenarios run here
through quail_amd with the same stand-in; every chunk's token ids,
positions, final rows, causal segments, KV scatter maps, block tables
(physical page ids, so the free-list order too), temporaries, tail
copies and reads must be bit-identical, and so must the answers, the
fresh-token count and the borrowed-token count.
"""

import json
import os
import sys

import numpy as np
import pytest
import torch

HERE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
sys.path.insert(0, HERE)
import scenarios  # noqa: E402
from replay import Passthrough, Recorder, arena, compare  # noqa: E402

from quail_amd import loop  # noqa: E402
from quail_amd.tokens import prefix_tree  # noqa: E402


@pytest.mark.parametrize("sc", scenarios.FILTERS, ids=[s["name"] for s in scenarios.FILTERS])
def test_filter_chunks_match_the_reference(sc):
    docs, questions, budget, pages = scenarios.filter_inputs(sc["seed"])
    rec, stats = Recorder(), {}
    answers, _, total = loop.run_filter(
        torch, arena(pages), rec, Passthrough(), docs, questions, budget, arena_writes=True,
        arena_keys=[("d", i) for i in range(len(docs))], attention_mode=sc["path"],
        prefix_tree=prefix_tree(docs, 16), stats=stats)
    want = compare(sc["name"], rec)
    assert {str(k): v for k, v in answers.items()} == want["answers"]
    assert total == want["tokens"] and stats["borrowed_tokens"] == want["borrowed"]


@pytest.mark.parametrize("sc", scenarios.JOINS, ids=[s["name"] for s in scenarios.JOINS])
def test_join_chunks_match_the_reference(sc):
    anchors, frames, suffixes, budget, pages = scenarios.join_inputs(sc["seed"])
    rec, stats = Recorder(), {}
    answers, _, total = loop.run_join(
        torch, arena(pages), rec, Passthrough(), anchors, suffixes, budget,
        stage_frames=frames, anchor_keys=[("a", i) for i in range(len(anchors))],
        attention_mode=sc["path"], prefix_tree=prefix_tree(anchors, 16), stats=stats)
    want = compare(sc["name"], rec)
    assert [{str(k): v for k, v in s.items()} for s in answers] == want["answers"]
    assert total == want["tokens"] and stats["borrowed_tokens"] == want["borrowed"]


@pytest.mark.parametrize("sc", scenarios.TREES, ids=[s["name"] for s in scenarios.TREES])
def test_prefix_tree_matches_the_reference(sc):
    with open(os.path.join(HERE, "prefix_trees.json")) as f:
        want = json.load(f)[sc["name"]]
    t = prefix_tree(scenarios.tree_inputs(sc["seed"]), 16)
    assert (list(t.order), list(t.parent), list(t.shared)) == \
        (want["order"], want["parent"], want["shared"])
