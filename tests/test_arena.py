"""The native page arena against the reference's known answers, and its invariants.

tests/golden/arena_cases.json holds the reference's PageArena known answers
(its tests/test_arena.py:10-188) as operation sequences with literal page
ids; test_known_answers interprets them. The randomized test checks the
accounting invariants over long mixed sequences (allocations with borrowed
prefixes, frees, grows, rewinds), and the KVArena test the row maps, block tables,
deferred frees of held keys and retained-KV eviction.
"""

import json
import os
import random

import pytest

from quail_amd.arena import KVArena, PageArena

HERE = os.path.dirname(os.path.abspath(__file__))
CASES = json.load(open(os.path.join(HERE, "golden", "arena_cases.json")))["cases"]
ERRORS = {"KeyError": KeyError, "ValueError": ValueError}


def _runs(rows):
    """Row list -> [start, stop) runs of consecutive rows."""
    out = []
    for r in rows:
        if out and out[-1][1] == r:
            out[-1][1] = r + 1
        else:
            out.append([r, r + 1])
    return out


def _key(k):
    """JSON keys: a string, or an [alias, document] pair (a tuple key)."""
    return tuple(k) if isinstance(k, list) else k


def _plain(v):
    """Tuple keys back to lists, to compare with JSON."""
    if isinstance(v, (tuple, list)):
        return [_plain(x) for x in v]
    return v


class _Policy:
    """A retention policy of the reference's shape (cost/retention.py:19-25)
    with seconds = tokens: (probability * tokens / pages, -next_use,
    -document), uses = {alias: (probability, next_use)}."""

    def __init__(self, uses):
        self.uses = uses

    def priority(self, key, tokens, pages):
        alias, document = key
        probability, next_use = self.uses.get(alias, (0.0, 0))
        return (probability * tokens / pages, -next_use, -document)


def _apply(a, op, args):
    args = [_key(args[0])] + list(args[1:]) if args and op != "configure" else args
    if op == "configure":
        uses, cap = args
        return a.configure_retention(_Policy({k: tuple(v) for k, v in uses.items()}), cap)
    if op == "retain" and len(args) == 2:
        return a.retain(args[0], tuple(args[1]))
    if op == "alloc":
        key, tokens, capacity, borrow = args
        borrowed = a.shared_pages(_key(borrow[0]), *borrow[1:]) if borrow else ()
        return a.alloc(key, tokens, capacity, borrowed=borrowed)
    if op == "shared_pages":
        return a.shared_pages(*args)
    if op in ("free_key", "pin", "retain", "table_pages", "borrowed_tokens"):
        return getattr(a, op)(*args)
    if op in ("grow", "rewind", "drop_leading"):
        return getattr(a, op)(*args)
    if op == "table":
        return a.table_pages(*args)
    if op in ("owned", "borrowed", "tokens"):
        return getattr(a, op)[args[0]]
    if op == "rows":
        return _runs(a.row_indices(*args))
    if op == "pop_victim":
        v = a.pop_retained_victim()
        return None if v is None else _plain(v)
    raise AssertionError(f"unknown op {op}")


def _state(a, want):
    got = {"free_pages": a.free_pages, "resident_tokens": a.resident_tokens,
           "retained_pages": a.retained_pages,
           "retained_prefix_tokens": a.retained_prefix_tokens, "free": a.free,
           "pinned": sorted(a.pinned), "retained": dict(a.retained)}
    return {k: got[k] for k in want}


@pytest.mark.parametrize("case", CASES, ids=[c["name"] for c in CASES])
def test_known_answers(case):
    a = PageArena(case["n_pages"], case["page_tokens"])
    for step, entry in enumerate(case["ops"]):
        op = entry[0]
        if op == "state":
            assert _state(a, entry[1]) == entry[1], f"{case['name']} step {step}"
            continue
        if op in ("pin", "retain", "configure"):
            _apply(a, op, entry[1:])
            continue
        args, want = entry[1:-1], entry[-1]
        if isinstance(want, str) and want in ERRORS:
            with pytest.raises(ERRORS[want]):
                _apply(a, op, args)
            continue
        assert _apply(a, op, args) == want, f"{case['name']} step {step}: {entry}"


def test_accounting_invariants_under_random_operations():
    """Every page is either free or held by exactly the keys whose tables
    list it; nothing leaks or is handed out twice, over mixed operations."""
    rng = random.Random(11)
    n = 96
    a = PageArena(n_pages=n, page_tokens=16)
    live = {}
    for step in range(3000):
        r = rng.random()
        if live and r < 0.35:
            key = rng.choice(sorted(live))
            a.free_key(key)
            del live[key]
        elif live and r < 0.45:
            key = rng.choice(sorted(live))
            borrowed = a.borrowed_tokens(key)
            tokens = a.tokens[key]
            a.rewind(key, rng.randint(borrowed, max(borrowed, tokens)))
        elif live and r < 0.55:
            key = rng.choice(sorted(live))
            a.grow(key, a.tokens[key] + rng.randrange(0, 64))
        else:
            key = f"k{step}"
            tokens = rng.randrange(1, 300)
            borrowed = ()
            if live and rng.random() < 0.5:
                parent = rng.choice(sorted(live))
                shared = min(a.tokens[parent], tokens) // 16 * 16
                borrowed = a.shared_pages(parent, shared)
            if a.alloc(key, tokens, borrowed=borrowed) is not None:
                live[key] = True
        holders = {}
        for key in live:
            for p in a.table_pages(key):
                holders[p] = holders.get(p, 0) + 1
        free = a.free
        assert len(free) == len(set(free)), "page freed twice"
        assert not set(free) & set(holders), "page both free and held"
        assert len(free) + len(holders) == n, "page leaked"
        for key in live:
            own = a.owned[key]
            assert all(holders[p] == 1 for p in own) or any(
                a.borrowed[k] and set(a.borrowed[k]) & set(own) for k in live), "own page shared"
    for key in list(live):
        a.free_key(key)
    assert sorted(a.free) == list(range(n))


def test_kv_arena_rows_tables_holds_and_eviction():
    arena = KVArena(n_layers=1, n_pages=64, page_tokens=16, n_kv=1, d_head=1,
                    device="cpu", allocate=False)
    arena.activate(("d", 0), 100, capacity_tokens=110)
    arena.activate(("d", 1), 94, capacity_tokens=104, borrow=(("d", 0), 64))
    assert arena.owned_pages(("d", 1))[:4] == arena.owned_pages(("d", 0))[:4]
    rows0 = arena.capacity_rows(("d", 0)).tolist()
    assert rows0 == [p * 16 + i for p in arena.owned_pages(("d", 0)) for i in range(16)]
    table, used = arena.block_table([("d", 0), ("d", 1)])
    assert table.shape == (2, 7) and used.tolist() == [100, 94]
    assert table[1].tolist()[:4] == table[0].tolist()[:4]
    assert table[0].tolist()[-1] == arena.owned_pages(("d", 0))[-1]
    # a held parent freed early waits for its borrower's release
    arena.hold(("d", 0), 1)
    assert arena.free_key(("d", 0)) == 0 and arena.is_resident(("d", 0))
    arena.release(("d", 0))
    assert not arena.is_resident(("d", 0))
    arena.free_key(("d", 1))
    assert arena.free_pages == 64
    # retained keys are evicted lowest priority first when pages run short
    events = []
    from quail_amd import arena as arena_module
    arena_module.set_answer_sink(events.append)
    try:
        arena.activate(("d", 2), 160)
        arena.retain(("d", 2), 160)
        assert arena.retained_keys() == [("d", 2)]
        got = arena.activate(("d", 3), 60 * 16)
        assert got is not None and arena.evicted_keys == 1
        assert events == [{"kind": "evict", "alias": "d", "document": 2, "tokens": 160}]
    finally:
        arena_module.set_answer_sink(None)
    with pytest.raises(ValueError):
        KVArena(1, 8, 16, 1, 1, device="cpu", allocate=False, sliding_window=64,
                n_sliding_pages=4, sliding_layers=(0,))


def test_held_keys_are_never_evicted_and_drop_holds_frees_in_hold_order():
    arena = KVArena(n_layers=1, n_pages=8, page_tokens=16, n_kv=1, d_head=1,
                    device="cpu", allocate=False)
    for d in range(3):
        arena.activate(("a", d), 32)
        arena.retain(("a", d), 32)
    arena.hold(("a", 1), 2)
    evicted = arena.evict_retained(8)
    assert ("a", 1) not in evicted and len(evicted) == 2
    arena.free_key(("a", 1))           # deferred: the key is held
    assert arena.is_resident(("a", 1))
    assert arena.drop_holds() and not arena.is_resident(("a", 1))
    assert not arena.drop_holds()



def test_finished_streams_leave_no_handles_behind():
    """A long session runs many filters over one arena: once a stream ends,
    the handle table holds only the keys the arena still holds (here the
    survivors retained for a later operator), and no handle number is
    handed out twice."""
    import torch

    from kv_checker import HashModel, _Passthrough, _Pipeline, answer, chain
    from quail_amd import loop

    arena = KVArena(n_layers=1, n_pages=256, page_tokens=16, n_kv=1, d_head=1,
                    dtype=torch.float32, device="cpu", allocate=False)
    seen = set()
    for round_ in range(3):
        docs = [[7 + round_, 100 + d, 200 + d] * (1 + d % 3) for d in range(20)]
        question = [5, 6]
        answers = {}
        for doc in docs:
            hv = chain(list(doc) + question)
            answers[hv] = answer(hv)
        keys = [("q%d" % round_, d) for d in range(20)]
        got, _, _ = loop.run_filter(torch, arena, _Pipeline(HashModel(arena, answers)),
                                    _Passthrough(), docs, [question], 64, arena_writes=True,
                                    arena_keys=keys, retain_survivors={0, 1, 2, 3})
        kept = {keys[d] for d in range(4) if got[d][-1]}
        assert kept <= set(arena.resident_keys())
        handles = {arena.handle(k) for k in kept}
        assert not handles & seen, "a handle number was handed out twice"
        seen |= handles
        assert len(arena.accounting._keys) == len(arena.resident_keys())
