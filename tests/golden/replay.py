"""Replay helpers shared by the golden-loop tests: a stand-in model that
records every chunk the loop packs and answers from each final row's token
and position (scenarios.answer_bit), and the chunk-by-chunk comparison
against the reference's saved chunks."""

import json
import os

import numpy as np
import torch

import scenarios
from quail_amd.arena import KVArena

HERE = os.path.dirname(os.path.abspath(__file__))


class Recorder:
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


class Passthrough:
    dtype = None

    def submit(self, v):
        return v

    def result(self, v):
        return v


def arena(pages):
    return KVArena(n_layers=1, n_pages=pages, page_tokens=16, n_kv=1, d_head=1,
                   dtype=torch.float32, device="cpu", allocate=False)


def compare(name, rec):
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
