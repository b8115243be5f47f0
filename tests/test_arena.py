"""PageArena / KVArena accounting against the reference's known answers.

Literal expectations are those of the reference's tests/test_arena.py:10-139
(page counts, LIFO reuse, borrowing, rewind/grow, retention priority).
"""

import random

import pytest

from quail_amd.arena import KVArena, PageArena


def test_fresh_arena_hands_out_pages_in_order_and_reuses_lifo():
    a = PageArena(n_pages=8, page_tokens=16)
    assert a.alloc("x", 40) == [0, 1, 2]
    assert a.alloc("y", 16) == [3]
    a.free_key("x")                      # pushes 0, 1, 2 back
    assert a.free == [7, 6, 5, 4, 0, 1, 2]
    assert a.alloc("z", 17) == [2, 1]    # last freed first
    assert a.row_indices("z") == list(range(32, 48)) + [16]


def test_allocation_retention_rewind_and_pinning():
    a = PageArena(n_pages=10, page_tokens=16)
    pages = a.alloc("d0", 40)
    assert len(pages) == 3 and a.free_pages == 7 and a.resident_tokens == 40
    assert a.free_key("d0") == 3 and a.free_pages == 10 and a.resident_tokens == 0
    assert a.alloc("big", 200) is None
    assert a.alloc("d", 5, capacity_tokens=10) is not None
    assert len(a.row_indices("d")) == 5 and len(a.row_indices("d", 10)) == 10
    with pytest.raises(KeyError):
        a.alloc("d", 5)

    rng = random.Random(5)
    a = PageArena(n_pages=64, page_tokens=16)
    live = {}
    for step in range(500):
        if live and rng.random() < 0.45:
            key = rng.choice(sorted(live))
            a.free_key(key)
            del live[key]
        else:
            key = f"d{step}"
            got = a.alloc(key, rng.randrange(1, 200))
            if got is not None:
                live[key] = got
        held = [p for pages in live.values() for p in pages]
        assert len(held) == len(set(held)), "page double-owned"
        assert len(held) + a.free_pages == 64, "pages leaked"

    a = PageArena(n_pages=3, page_tokens=4)
    a.alloc("doc", 4)
    assert a.grow("doc", 12) == 2
    assert a.grow("doc", 16) is None

    a = PageArena(n_pages=10, page_tokens=4)
    a.alloc("doc", 7, capacity_tokens=11)
    assert len(a.owned["doc"]) == 3
    a.pin("doc")
    assert "doc" in a.pinned
    a.retain("doc")
    assert "doc" not in a.pinned and a.retained["doc"] == 7
    assert a.retained_prefix_tokens == 7
    assert a.rewind("doc", 4) == 2
    assert len(a.owned["doc"]) == 1 and a.tokens["doc"] == 4
    a.free_key("doc")
    assert not a.pinned and not a.retained

    a = PageArena(n_pages=4, page_tokens=16)
    a.alloc("one-page", 16)
    a.alloc("two-pages", 17)
    a.retain("one-page")
    a.retain("two-pages")
    assert a.pop_retained_victim() == ("two-pages", 2, 17)   # 8.5 tokens/page < 16

    a = PageArena(n_pages=2, page_tokens=16)
    a.alloc("doc", 16)
    a.retain("doc")
    a.pin("doc")
    assert a.pop_retained_victim() is None


def test_borrowed_pages_are_shared_until_the_last_holder_frees_them():
    a = PageArena(n_pages=10, page_tokens=16)
    parent = a.alloc("p", 40)
    child = a.alloc("c", 50, borrowed=a.shared_pages("p", 32))
    assert len(child) == 2 and a.free_pages == 5
    assert a.table_pages("c") == parent[:2] + child
    assert a.borrowed_tokens("c") == 32
    assert a.row_indices("c")[:32] == a.row_indices("p")[:32]
    assert a.free_key("p") == 1 and a.free_pages == 6
    assert a.table_pages("c") == parent[:2] + child
    assert a.free_key("c") == 4 and a.free_pages == 10

    a.alloc("p", 40)
    a.alloc("c", 50, borrowed=a.shared_pages("p", 32))
    a.alloc("g", 60, borrowed=a.shared_pages("c", 48))
    assert a.table_pages("g")[:2] == a.table_pages("p")[:2]
    assert a.table_pages("g")[2] == a.owned["c"][0]
    for key in ("p", "c", "g"):
        a.free_key(key)
    assert a.free_pages == 10

    a.alloc("p", 40)
    a.alloc("c", 50, borrowed=a.shared_pages("p", 32))
    assert a.rewind("c", 33) == 1
    assert a.tokens["c"] == 33 and len(a.owned["c"]) == 1
    with pytest.raises(ValueError):
        a.rewind("c", 16)
    assert a.grow("c", 64) == 1
    assert len(a.table_pages("c")) == 4
    assert a.retained_pages == 0
    a.retain("c")
    assert a.retained_pages == 2
    a.free_key("p")
    a.retain("c")
    assert a.retained_pages == 4
    a.alloc("p", 40)
    with pytest.raises(ValueError):
        a.shared_pages("p", 20)
    with pytest.raises(ValueError):
        a.alloc("x", 16, borrowed=a.shared_pages("p", 32))
    with pytest.raises(KeyError):
        a.shared_pages("nobody", 16)
    with pytest.raises(ValueError):
        a.shared_pages("p", 48)
    a.alloc("s", 48, borrowed=a.shared_pages("p", 32, 16))
    assert a.table_pages("s")[:1] == a.table_pages("p")[1:2]
    assert a.drop_leading("s", 2) == 1
    assert a.borrowed["s"] == [] and len(a.owned["s"]) == 1


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
    # widest row pads the other with zeros
    assert table[0].tolist()[-1] == arena.owned_pages(("d", 0))[-1]
    # a held parent freed early waits for its borrower's release
    arena.hold(("d", 0), 1)
    assert arena.free_key(("d", 0)) == 0 and arena.is_resident(("d", 0))
    arena.release(("d", 0))
    assert not arena.is_resident(("d", 0))
    arena.free_key(("d", 1))
    assert arena.free_pages == 64
    # retained keys are evicted lowest priority first when pages run short
    arena.activate(("d", 2), 160)
    arena.retain(("d", 2), 160)
    assert arena.retained_keys() == [("d", 2)]
    got = arena.activate(("d", 3), 60 * 16)
    assert got is not None and arena.evicted_keys == 1
    with pytest.raises(ValueError):
        KVArena(1, 8, 16, 1, 1, device="cpu", allocate=False, sliding_window=64,
                n_sliding_pages=4, sliding_layers=(0,))
