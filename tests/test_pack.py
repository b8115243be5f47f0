"""pack_chunk against the reference's known answers.

pack_chunk literals: the plain-arena cases of the reference's
tests/test_sliding_kv.py:216-297 (borrowing child under unified attention;
siblings stacked under tree attention: cu_a == [0, 100, 101, 112, 119],
reads cu_q == [0, 1, 19], used == [100, 64], max_q == 18). Filter
admission's literal cases are data (tests/golden/admission_cases.json)
and its invariants properties (test_admission_properties.py).
"""

import pytest
import torch

from quail_amd import loop
from quail_amd.arena import KVArena


def plain_arena(pages=64):
    return KVArena(n_layers=1, n_pages=pages, page_tokens=16, n_kv=1, d_head=2,
                   dtype=torch.float32, device="cpu", allocate=False)


def pack(arena, groups, mode):
    return loop.pack_chunk(torch, arena, groups, attention_mode=mode)


def test_unified_single_suffix_writes_the_whole_row_in_place():
    arena = plain_arena()
    key = ("d", 0)
    doc = list(range(100))
    arena.activate(key, 100, capacity_tokens=120)
    chunk = pack(arena, [dict(key=key, prefix=doc, f=100, suffixes=[[500, 501]])],
                 "unified")
    u = chunk.meta["unified"]
    assert chunk.fresh_keys == (key,)
    assert u["src"].tolist() == list(range(102))
    assert u["dst"].tolist() == arena.capacity_rows(key)[:102].tolist()
    assert u["used"].tolist() == [102] and tuple(u["table"].shape) == (1, 8)
    assert u["cu_q"].tolist() == [0, 102] and u["max_q"] == 102
    assert chunk.positions.tolist() == list(range(102))
    assert chunk.final_indices.tolist() == [101]
    # a later stage reads the kept rows; its suffix lands after row 100
    chunk = pack(arena, [dict(key=key, prefix=None, f=100, suffixes=[[600]])], "unified")
    u = chunk.meta["unified"]
    assert u["used"].tolist() == [101]
    assert u["dst"].tolist() == arena.capacity_rows(key)[100:101].tolist()
    # two suffixes take temporaries after a copy of the kept partial page
    chunk = pack(arena, [dict(key=key, prefix=None, f=100, suffixes=[[600], [601, 602]])],
                 "unified")
    u = chunk.meta["unified"]
    assert len(chunk.temporary_keys) == 2
    assert u["used"].tolist() == [101, 102]
    assert u["tail_src"].numel() == 2 * (100 % 16)
    anchor = arena.owned_pages(key)[100 // 16] * 16
    assert u["tail_src"].tolist()[:4] == list(range(anchor, anchor + 4))
    t0 = chunk.temporary_keys[0]
    assert u["tail_dst"].tolist()[:4] == arena.capacity_rows(t0)[:4].tolist()
    assert u["table"][0].tolist()[:6] == arena.owned_pages(key)[:6]
    for temp in chunk.temporary_keys:
        arena.free_key(temp)
    arena.free_key(key)
    assert arena.free_pages == 64


def test_unified_child_reads_borrowed_pages_and_tree_reads_its_own():
    arena = plain_arena()
    doc = list(range(100))
    tail = [500]
    parent, child = ("d", 0), ("d", 1)
    arena.activate(parent, 100, capacity_tokens=110)
    arena.activate(child, 94, capacity_tokens=104, borrow=(parent, 64))
    assert arena.owned_pages(child)[:4] == arena.owned_pages(parent)[:4]
    chunk = pack(arena, [dict(key=parent, prefix=doc, f=100, suffixes=[tail]),
                         dict(key=child, prefix=doc[64:94], start=64, f=94,
                              suffixes=[tail])], "unified")
    assert chunk.fresh_keys == (parent, child)
    assert chunk.tokens == 101 + 31
    pos = chunk.positions.tolist()
    assert pos[:101] == list(range(101)) and pos[101:] == list(range(64, 95))
    u = chunk.meta["unified"]
    assert u["used"].tolist() == [101, 95]
    table = u["table"].tolist()
    assert table[1][:4] == table[0][:4]
    assert u["dst"].tolist()[101:] == arena.capacity_rows(child)[64:95].tolist()
    assert arena.capacity_rows(child)[:64].tolist() == arena.capacity_rows(parent)[:64].tolist()
    # tree attention without a read_key: the fresh rows read the child's own
    # first 64 rows (the borrowed pages), each suffix reads all 94
    chunk = pack(arena, [dict(key=child, prefix=doc[64:94], start=64, f=94,
                              suffixes=[tail, [501]])], "tree")
    reads = chunk.meta["reads"]
    assert reads["used"].tolist() == [64, 94]
    assert reads["cu_q"].tolist() == [0, 30, 32]
    assert chunk.meta["cu_a"].tolist() == [0, 30, 31, 32]
    arena.free_key(parent)
    arena.free_key(child)
    assert arena.free_pages == 64


def test_tree_siblings_stack_one_read_of_their_parent():
    arena = plain_arena()
    doc = list(range(100))
    tail = [500]
    parent, a, b = ("d", 0), ("d", 1), ("d", 2)
    arena.activate(parent, 100, capacity_tokens=110)
    arena.activate(a, 74, capacity_tokens=84, borrow=(parent, 64))
    arena.activate(b, 70, capacity_tokens=80, borrow=(parent, 64))
    chunk = pack(arena, [
        dict(key=parent, prefix=doc, f=100, suffixes=[tail]),
        dict(key=a, prefix=doc[64:74], start=64, read_key=parent, f=74, suffixes=[tail],
             write_suffix_tokens=1),
        dict(key=b, prefix=doc[64:70], start=64, read_key=parent, f=70, suffixes=[tail],
             write_suffix_tokens=1)], "tree")
    assert chunk.fresh_keys == (parent, a, b)
    assert chunk.meta["cu_a"].tolist() == [0, 100, 101, 112, 119]
    reads = chunk.meta["reads"]
    assert reads["cu_q"].tolist() == [0, 1, 19]
    assert reads["used"].tolist() == [100, 64]
    assert reads["max_q"] == 18
    assert reads["rows"].tolist() == [100] + list(range(101, 119))
    table = reads["table"].tolist()
    assert table[1][:4] == table[0][:4]
    src = reads["source"].tolist()
    assert src[100] == 0 and src[101:119] == list(range(1, 19)) and src[0] == -1
    dst = chunk.meta["kv_dst"].tolist()
    assert dst[100:110] == arena.capacity_rows(a)[64:74].tolist()
    assert dst[110:111] == arena.capacity_rows(a)[74:75].tolist()
    assert dst[111:117] == arena.capacity_rows(b)[64:70].tolist()
    assert dst[117:118] == arena.capacity_rows(b)[70:71].tolist()
    for key in (parent, a, b):
        arena.free_key(key)
    assert arena.free_pages == 64


def test_pack_refuses_malformed_groups():
    arena = plain_arena()
    with pytest.raises(ValueError, match="attention_mode"):
        pack(arena, [], "other")
    with pytest.raises(ValueError, match="one suffix"):
        pack(arena, [dict(key="u", prefix=[1, 2], f=2, suffixes=[[3], [4]])], "unified")
    with pytest.raises(ValueError, match="borrowed prefix"):
        pack(arena, [dict(key="u", prefix=[1, 2], start=16, f=18, suffixes=[[3]])], "tree")
    # an unpaged fresh group is one causal segment with no scatter
    chunk = pack(arena, [dict(key="u", prefix=[1, 2, 3], f=3, suffixes=[[4, 5]])], "unified")
    assert chunk.meta["unified"] is None and chunk.meta["cu_a"].tolist() == [0, 5]


def test_arena_full_error_frees_the_temporaries_it_took():
    arena = plain_arena(pages=8)
    key = ("d", 0)
    arena.activate(key, 100, capacity_tokens=100)    # 7 pages, 1 left
    with pytest.raises(loop.ArenaFullError):
        pack(arena, [dict(key=key, prefix=None, f=100, suffixes=[[1] * 10, [2] * 30])],
             "unified")
    assert arena.free_pages == 1
