"""A stand-in model that checks every KV read the packer lays out.

Restates the reference's HashModel idea (tests/kv_checker.py:1-10,
49-277): each packed row gets mix(previous hash, token), where the previous
hash is whatever its attention reads at the position before it, and every
KV write stores (token, position, hash) in a shadow pool indexed by arena
row. A query row that reads a wrong page, a wrong position, or a borrowed
page that was overwritten gets a hash no request has, and its planted
answer is missing. Runs the product's loop (quail_amd.loop.run_filter) on a
tensor-free CPU arena.
"""

import numpy as np
import torch

from quail_amd import loop
from quail_amd.arena import KVArena
from quail_amd.tokens import prefix_tree

MASK = (1 << 61) - 1


def mix(previous, token):
    return (previous * 1_000_003 + int(token) + 1) & MASK


def chain(tokens):
    h = 0
    for t in tokens:
        h = mix(h, t)
    return h


def answer(h):
    return (h >> 7) & 1


class HashModel:
    def __init__(self, arena, answers):
        self.page = arena.page_tokens
        rows = arena.n_pages * self.page
        self.token = np.full(rows, -1, dtype=np.int64)
        self.position = np.full(rows, -1, dtype=np.int64)
        self.hash = np.full(rows, -1, dtype=np.int64)
        self.answers = answers
        self.reads_checked = 0

    def forward_chunk(self, chunk):
        h = chunk.host
        ids = h["input_ids"].tolist()
        positions = h["positions"].tolist()
        hashes = [None] * len(ids)
        if chunk.attention_mode == "unified":
            self._unified(h, ids, positions, hashes)
        else:
            self._tree(h, ids, positions, hashes)
        out = []
        for row in h["finals"].tolist():
            assert hashes[row] in self.answers, (
                f"row {row} at position {positions[row]} read KV no request has")
            out.append(self.answers[hashes[row]])
        return out

    def _phys(self, table, i, view):
        return int(table[i][view // self.page]) * self.page + view % self.page

    def _stored(self, phys):
        return int(self.token[phys]), int(self.position[phys]), int(self.hash[phys])

    def _chain_ok(self, read, rows):
        previous = 0
        for v in range(rows):
            token, pos, hv = read(v)
            assert pos == v, f"resident row {v} holds position {pos}"
            assert hv == mix(previous, token), f"resident row {v} was overwritten"
            previous = hv
            self.reads_checked += 1

    def _unified(self, h, ids, positions, hashes):
        if "unified_cu_q" not in h:
            # unpaged: each causal segment reads only itself
            cu = h["cu_a"].tolist()
            for s in range(len(cu) - 1):
                prev = 0
                for row in range(cu[s], cu[s + 1]):
                    assert positions[row] == row - cu[s]
                    prev = hashes[row] = mix(prev, ids[row])
            return
        cu = h["unified_cu_q"].tolist()
        used = h["unified_used"].tolist()
        table = h["unified_table"]
        written = dict(zip(h["unified_dst"].tolist(), h["unified_src"].tolist()))
        copied = {}
        if "tail_src" in h:
            copied = dict(zip(h["tail_dst"].tolist(), h["tail_src"].tolist()))
        seq_of = {}
        for i in range(len(cu) - 1):
            for row in range(cu[i], cu[i + 1]):
                seq_of[row] = i

        def value(phys):
            if phys in written:
                src = written[phys]
                return ids[src], positions[src], row_hash(src)
            if phys in copied:
                # the tail copy runs after the scatter: it copies this
                # chunk's writes where they land on the copied rows
                return value(copied[phys])
            return self._stored(phys)

        def row_hash(row):
            if hashes[row] is not None:
                return hashes[row]
            i = seq_of[row]
            count = cu[i + 1] - cu[i]
            view = used[i] - count + row - cu[i]
            assert view == positions[row], "a query row's KV index is off"
            assert written.get(self._phys(table, i, view)) == row, \
                "a query row is not written where it reads itself"
            previous = 0
            if view:
                _, pos, previous = value(self._phys(table, i, view - 1))
                assert pos == positions[row] - 1
            hashes[row] = mix(previous, ids[row])
            return hashes[row]

        for row in range(len(ids)):
            row_hash(row)
        for i in range(len(cu) - 1):
            count = cu[i + 1] - cu[i]
            self._chain_ok(lambda v, i=i: value(self._phys(table, i, v)), used[i] - count)
        copies = {dst: value(src) for dst, src in copied.items()}
        for dst, src in written.items():
            self.token[dst], self.position[dst], self.hash[dst] = ids[src], positions[src], hashes[src]
        for dst, stored in copies.items():
            self.token[dst], self.position[dst], self.hash[dst] = stored

    def _tree(self, h, ids, positions, hashes):
        cu_a = h["cu_a"].tolist()
        first = set(cu_a[:-1])
        written = {}
        if "kv_src" in h:
            written = dict(zip(h["kv_dst"].tolist(), h["kv_src"].tolist()))
        read_of, table, read_used = {}, None, []
        if "reads_rows" in h:
            cu_q = h["reads_cu_q"].tolist()
            rows = h["reads_rows"].tolist()
            table = h["reads_table"]
            read_used = h["reads_used"].tolist()
            for i in range(len(cu_q) - 1):
                for row in rows[cu_q[i]:cu_q[i + 1]]:
                    read_of[row] = i
            source = h["reads_source"].tolist()
            for k, row in enumerate(rows):
                assert source[row] == k

        def value(phys):
            if phys in written:
                src = written[phys]
                return ids[src], positions[src], row_hash(src)
            return self._stored(phys)

        def row_hash(row):
            if hashes[row] is not None:
                return hashes[row]
            position = positions[row]
            if row not in first:
                assert positions[row - 1] == position - 1, "a causal segment skips a position"
                previous = row_hash(row - 1)
            elif row in read_of:
                i = read_of[row]
                assert read_used[i] == position, f"row at {position} reads {read_used[i]} rows"
                _, pos, previous = value(self._phys(table, i, position - 1))
                assert pos == position - 1
            else:
                assert position == 0, f"row at {position} starts a segment and reads nothing"
                previous = 0
            hashes[row] = mix(previous, ids[row])
            return hashes[row]

        for row in range(len(ids)):
            row_hash(row)
        for i in range(len(read_used)):
            self._chain_ok(lambda v, i=i: value(self._phys(table, i, v)), read_used[i])
        for dst, src in written.items():
            self.token[dst], self.position[dst], self.hash[dst] = ids[src], positions[src], hashes[src]


class _Pipeline:
    canvas_ids = ()
    needs_pages = False
    tree_attention = True

    def __init__(self, model):
        self.forward_chunk = model.forward_chunk


class _Passthrough:
    dtype = None

    def submit(self, value):
        return value

    def result(self, value):
        return value


def check_filter(docs, questions, *, path, pages=400, budget=600):
    """Run a filter over docs with the product loop; check answers and KV reads."""
    answers = {}
    for doc in docs:
        for q in questions:
            hv = chain(list(doc) + list(q))
            answers[hv] = answer(hv)
    arena = KVArena(n_layers=1, n_pages=pages, page_tokens=16, n_kv=1, d_head=1,
                    dtype=torch.float32, device="cpu", allocate=False)
    model = HashModel(arena, answers)
    got, _, tokens = loop.run_filter(
        torch, arena, _Pipeline(model), _Passthrough(), docs, questions, budget,
        arena_writes=True, arena_keys=[("d", i) for i in range(len(docs))],
        attention_mode=path, prefix_tree=prefix_tree(docs, 16))
    for d, doc in enumerate(docs):
        want = []
        for q in questions:
            want.append(answers[chain(list(doc) + list(q))])
            if not want[-1]:
                break
        assert got[d] == want, f"document {d}"
    assert not arena.accounting.owned, "the filter left pages resident"
    assert arena.free_pages == pages
    return model, tokens


def _arena(pages):
    return KVArena(n_layers=1, n_pages=pages, page_tokens=16, n_kv=1, d_head=1,
                   dtype=torch.float32, device="cpu", allocate=False)


def join_answers(anchors, frame, partners):
    """Planted answers of every (anchor, partner) chain, and of each frame entry."""
    answers = {}
    for anchor in anchors:
        answers[chain(list(anchor) + list(frame))] = 0     # frame entry: discarded
        for partner in partners:
            hv = chain(list(anchor) + list(frame) + list(partner))
            answers[hv] = answer(hv)
    return answers


def check_join(anchors, frame, partners, *, path, pages=400, budget=600, retain=False):
    """Run a join with the product loop; check every pair's answer and KV read.

    With retain, finished anchors stay in the arena as evictable KV that
    later fresh anchors evict for pages (the reference's
    tests/kv_checker.py:364-395).
    """
    answers = join_answers(anchors, frame, partners)
    arena = _arena(pages)
    model = HashModel(arena, answers)
    keys = [("a", i) for i in range(len(anchors))]
    if retain:
        arena.retention_cap_pages = pages
    rows = {}

    def anchor_done(a, row):
        rows[a] = list(row)
        if retain:
            arena.retain(keys[a], len(anchors[a]))
        else:
            arena.free_key(keys[a])

    stats = {}
    _, _, tokens = loop.run_join(
        torch, arena, _Pipeline(model), _Passthrough(), anchors, [partners], budget,
        stage_frames=[frame], anchor_keys=keys, anchor_done=anchor_done,
        attention_mode=path, prefix_tree=prefix_tree(anchors, 16), stats=stats)
    for a, anchor in enumerate(anchors):
        want = [answers[chain(list(anchor) + list(frame) + list(p))] for p in partners]
        assert rows[a] == want, f"anchor {a}"
    arena.evict_retained(pages)
    assert not arena.accounting.owned, "the join left pages resident"
    assert arena.free_pages == pages
    return model, tokens, stats


def check_feed(docs, question, frame, partners, *, path, pages=400, budget=600):
    """A filter whose held survivors feed a join as resident anchors
    (the reference's tests/kv_checker.py:398-424)."""
    answers = join_answers(docs, frame, partners)
    for doc in docs:
        hv = chain(list(doc) + list(question))
        answers[hv] = answer(hv >> 3)
    arena = _arena(pages)
    model = HashModel(arena, answers)
    source = loop.FilterStream(
        torch, arena, _Pipeline(model), _Passthrough(), docs, [question], budget,
        arena_writes=True, arena_keys=[("d", i) for i in range(len(docs))],
        hold_survivors=True, hold_extra_tokens=len(frame),
        prefix_tree=prefix_tree(docs, 16), attention_mode=path)
    keys = []
    out, _, _ = loop.run_join(
        torch, arena, _Pipeline(model), _Passthrough(), [], [partners], budget,
        stage_frames=[frame], anchor_keys=keys, anchor_source=source, attention_mode=path)
    survivors = {d for d, doc in enumerate(docs)
                 if answers[chain(list(doc) + list(question))]}
    assert {key[1] for key in keys} == survivors
    for a, key in enumerate(keys):
        doc = docs[key[1]]
        want = [answers[chain(list(doc) + list(frame) + list(p))] for p in partners]
        assert out[0][a] == want, f"anchor {key[1]}"
    assert not arena.accounting.owned
    return model
