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

from quail_amd import loop  # noqa: E402
from quail_amd.arena import KVArena  # noqa: E402
from quail_amd.tokens import prefix_tree  # noqa: E402


class _Recorder:
    canvas_ids = ()
    needs_pages = False
    tree_attention = True

    def __init__(self):
        self.chunks = []

    def forward_chunk(self, chunk):
        h = chunk.host
        self.chunks.append((h, chunk.attention_mode, chunk.tokens, int(chunk.meta["max_a"])))
        ids, pos = h["input_ids"], h["positions"]
        return [scenarios.answer_bit(ids[f], pos[f]) for f in h["finals"]]


class _Passthrough:
    dtype = None

    def submit(self, v):
        return v

    def result(self, v):
        return v


def _arena(pages):
    return KVArena(n_layers=1, n_pages=pages, page_tokens=16, n_kv=1, d_head=1,
                   dtype=torch.float32, device="cpu", allocate=False)


def _compare(name, rec):
    with open(os.path.join(HERE, f"{name}.json")) as f:
        want = json.load(f)
    arrays = np.load(os.path.join(HERE, f"{name}.npz"))
    assert len(rec.chunks) == len(want["chunks"]), f"{name}: chunk count"
    for i, ((host, mode, tokens, max_a), w) in enumerate(zip(rec.chunks, want["chunks"])):
        assert (mode, tokens, max_a) == (w["mode"], w["tokens"], w["max_a"]), f"{name} chunk {i}"
        for key in w["keys"]:
            assert key in host, f"{name} chunk {i}: {key} missing"
            got, ref = np.asarray(host[key]), arrays[f"c{i}_{key}"]
            assert got.shape == ref.shape and np.array_equal(got, ref), f"{name} chunk {i}: {key}"
        extra = [k for k in ("kv_src", "reads_rows", "unified_src", "tail_src")
                 if k in host and k not in w["keys"]]
        assert not extra, f"{name} chunk {i}: arrays the reference did not build: {extra}"
    return want


@pytest.mark.parametrize("sc", scenarios.FILTERS, ids=[s["name"] for s in scenarios.FILTERS])
def test_filter_chunks_match_the_reference(sc):
    docs, questions, budget, pages = scenarios.filter_inputs(sc["seed"])
    rec, stats = _Recorder(), {}
    answers, _, total = loop.run_filter(
        torch, _arena(pages), rec, _Passthrough(), docs, questions, budget, arena_writes=True,
        arena_keys=[("d", i) for i in range(len(docs))], attention_mode=sc["path"],
        prefix_tree=prefix_tree(docs, 16), stats=stats)
    want = _compare(sc["name"], rec)
    assert {str(k): v for k, v in answers.items()} == want["answers"]
    assert total == want["tokens"] and stats["borrowed_tokens"] == want["borrowed"]


@pytest.mark.parametrize("sc", scenarios.JOINS, ids=[s["name"] for s in scenarios.JOINS])
def test_join_chunks_match_the_reference(sc):
    anchors, frames, suffixes, budget, pages = scenarios.join_inputs(sc["seed"])
    rec, stats = _Recorder(), {}
    answers, _, total = loop.run_join(
        torch, _arena(pages), rec, _Passthrough(), anchors, suffixes, budget,
        stage_frames=frames, anchor_keys=[("a", i) for i in range(len(anchors))],
        attention_mode=sc["path"], prefix_tree=prefix_tree(anchors, 16), stats=stats)
    want = _compare(sc["name"], rec)
    assert [{str(k): v for k, v in s.items()} for s in answers] == want["answers"]
    assert total == want["tokens"] and stats["borrowed_tokens"] == want["borrowed"]


@pytest.mark.parametrize("sc", scenarios.TREES, ids=[s["name"] for s in scenarios.TREES])
def test_prefix_tree_matches_the_reference(sc):
    with open(os.path.join(HERE, "prefix_trees.json")) as f:
        want = json.load(f)[sc["name"]]
    t = prefix_tree(scenarios.tree_inputs(sc["seed"]), 16)
    assert (list(t.order), list(t.parent), list(t.shared)) == \
        (want["order"], want["parent"], want["shared"])
