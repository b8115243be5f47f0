"""Join admission and the join loop (host-only, integer).

Known answers restate the reference's literal join cases
(tests/test_pack.py:252-336 and :405-418); the random-shape driver checks
the invariants the reference checks in tests/test_pack.py:21-108 (every
partner streamed exactly once per stage reached, chunks within budget,
pages never over-claimed or leaked, gating events as the truth implies).
The HashModel checker then runs the real run_join loop and checks every
KV read it lays out (tests/test_kv_reads.py:101-148 in the reference).
"""

import itertools
import random

import numpy as np
import pytest

from kv_checker import check_feed, check_join
from quail_amd.pack import (JoinAdmission, assemble, gate, matches, pages_for,
                            partner_pages)
from quail_amd.tokens import PrefixTree


# ---------------------------------------------------------------- known answers


def test_cut_stream_leads_the_next_chunk_ahead_of_a_fresh_anchor():
    sched = JoinAdmission([100, 50], [[400, 50]], 520, arena_pages=100, page_tokens=16)
    assert sched.next_chunk(100) == [(0, 0, 0, 1, True)]
    assert sched.next_chunk(100) == [(0, 0, 1, 2, False), (1, 0, 0, 1, True)]


def test_resident_anchor_packs_while_a_fresh_one_waits_for_pages():
    sched = JoinAdmission([160, 160], [[10]], 400, arena_pages=10, page_tokens=16,
                          resident={1: 10})
    assert sched.next_chunk(0) == [(1, 0, 0, 1, False)]
    assert sched.blocked_pages == 10
    assert sched.report(1, 0, 0, 1, [1]) == [("finished", 1)]
    assert sched.next_chunk(10) == [(0, 0, 0, 1, True)]


@pytest.mark.parametrize("args, kwargs, message", [
    (([100], [], 400, 100, 16), {}, "at least one stage"),
    (([100], [[10]], 400, 100, 16), {"anchor_partners": {0: [[1]]}}, "out of range"),
    (([100], [[10]], 400, 100, 16), {"anchor_partners": {0: [[0], None]}},
     "partner lists for 2 stages"),
    (([100], [[1050]], 1000, 100, 16), {}, "suffixes are atomic"),
    (([950], [[100]], 1000, 100, 16), {}, "no room for a partner"),
    (([33], [[10]], 1000, 2, 16), {}, "anchor 0 needs 3 KV pages"),
    (([33], [[10]], 1000, 2, 16), {"frame_tokens": [1, 2]}, "frame_tokens must match"),
])
def test_bad_joins_raise(args, kwargs, message):
    with pytest.raises(ValueError, match=message):
        JoinAdmission(*args, **kwargs)


def test_resident_anchor_may_exceed_the_free_arena():
    JoinAdmission([33], [[10]], 1000, arena_pages=2, page_tokens=16, resident={0: 3})


def test_streamed_admission_and_buildable_tokens():
    sched = JoinAdmission([], [[10, 10, 10]], 100, 50, 16, frame_tokens=[5])
    assert sched.done()
    assert sched.buildable_tokens() == 0
    assert sched.admit(40, resident_pages=3) == 0
    assert sched.buildable_tokens() == 5 + 30
    assert sched.admit(80) == 1
    assert sched.buildable_tokens() == 100
    groups = sched.next_chunk(free_pages=50)
    assert groups[0] == (0, 0, 0, 3, False)
    assert sched.report(0, 0, 0, 3, [0, 1, 0]) == [("finished", 0)]
    assert sched.buildable_tokens() == 100
    with pytest.raises(ValueError):
        sched.admit(5000)


def test_temporary_suffix_pages_are_priced():
    sched = JoinAdmission([31, 31], [[1, 1, 1, 1]], 256, 8, 16, temporary_suffix_pages=True)
    groups = sched.next_chunk(8)
    prefix_pages = sum(2 for *_, carried in groups if carried)
    suffix_pages = sum(end - start for _, _, start, end, _ in groups)
    assert prefix_pages + suffix_pages <= 8
    assert suffix_pages < 8
    # one partner's temporary rows follow the anchor's partial last page
    cost = lambda t, b=None: pages_for(t, 16)   # noqa: E731
    assert partner_pages(cost, 16, 31, 0, 1) == 1     # 15 kept rows + 1
    assert partner_pages(cost, 16, 31, 0, 2) == 2     # 15 kept rows + 2
    assert partner_pages(cost, 16, 31, 1, 2) == 1     # the frame fills the page


def test_score_rows_fill_a_typed_answer_array():
    sched = JoinAdmission([16], [[16, 16, 16, 16]], 48, 20, 16, answer_dtype=np.float32)
    expected = np.array([0.0, 0.125, 0.5, 1.0], dtype=np.float32)
    while not sched.done():
        groups = sched.next_chunk(19)
        assert groups
        for a, j, start, end, _ in groups:
            sched.report(a, j, start, end, expected[start:end])
    assert sched.answers[0][0].dtype == np.float32
    np.testing.assert_array_equal(sched.answers[0][0], expected)


def test_join_admission_borrows_through_the_prefix_tree():
    # anchor 0 has no partner, so it settles without a chunk; its child
    # cannot wait for it and packs whole
    tree = PrefixTree(order=[0, 1], parent=[None, 0], shared=[0, 16])
    sched = JoinAdmission([40, 40], [[10]], 512, 64, 16,
                          anchor_partners={0: [[]], 1: [[0]]}, tree=tree)
    assert sched.take_settled() == [("finished", 0)]
    assert sched.next_chunk(free_pages=64) == [(1, 0, 0, 1, True)]
    assert sched.borrowing.shared(1) == 0
    assert sched.report(1, 0, 0, 1, [1]) == [("finished", 1)]
    assert sched.done()

    # anchor 1 shares 80 of 100 tokens: after anchor 0 packs 100 + 10, the
    # 40 left of the 150 budget hold anchor 1's own 20 + 10
    tree = PrefixTree(order=[0, 1], parent=[None, 0], shared=[0, 80])
    sched = JoinAdmission([100, 100], [[10]], 150, 64, 16, tree=tree)
    groups = sched.next_chunk(free_pages=64)
    assert [g[0] for g in groups] == [0, 1]
    assert sched.borrowing.shared(1) == 80


def test_two_stage_gating_moves_an_anchor_on_at_its_first_true():
    # stage 0 has 3 partners; the anchor advances once its whole stage-0
    # stream is launched and one answer is TRUE
    sched = JoinAdmission([20, 20], [[10, 10, 10], [10, 10]], 1000, 64, 16)
    groups = sched.next_chunk(64)
    assert groups == [(0, 0, 0, 3, True), (1, 0, 0, 3, True)]
    assert sched.report(0, 0, 0, 3, [0, 1, 0]) == []
    assert sched.report(1, 0, 0, 3, [0, 0, 0]) == [("dropped", 1)]
    assert sched.next_chunk(64) == [(0, 1, 0, 2, False)]
    assert sched.report(0, 1, 0, 2, [1, 1]) == [("finished", 0)]
    assert sched.done()
    assert sched.answers == [{0: [0, 1, 0], 1: [0, 0, 0]}, {0: [1, 1]}]


def test_gate_matches_and_assemble_against_brute_force():
    rng = random.Random(5)
    for _ in range(50):
        n_a, n_b, n_c = rng.randrange(1, 6), rng.randrange(1, 6), rng.randrange(1, 6)
        ans1 = {b: [rng.randrange(2) for _ in range(n_a)] for b in range(n_b)}
        survivors = gate(ans1)
        assert survivors == sorted(b for b, row in ans1.items() if 1 in row)
        ans2 = {b: [rng.randrange(2) for _ in range(n_c)] for b in survivors}
        brute = sorted((a, b, c) for b in survivors for a in range(n_a) for c in range(n_c)
                       if ans1[b][a] and ans2[b][c])
        assert assemble(ans1, ans2) == brute
        assert matches({0: [0, 1, 1]}) == {0: [1, 2]}


# ---------------------------------------------------------------- random shapes


def _drive(sched, truth, arena_pages, resident, rng):
    """Run the scheduler with a page ledger; answers arrive one chunk late
    or at once, at random."""
    extra = max(sched.frames)
    held = dict(resident)
    free = arena_pages - sum(held.values())
    chunks, outstanding, events = [], [], []
    idle = 0

    def settle(a):
        nonlocal free
        free += held.pop(a, 0)

    while not sched.done():
        for kind, anchor in sched.take_settled():
            events.append((kind, anchor))
            settle(anchor)
        groups = sched.next_chunk(free)
        if groups:
            for a, j, start, end, carried in groups:
                if j == 0 and start == 0:
                    need = pages_for(sched.prefix[a] + extra, sched.page_tokens)
                    free -= need - held.get(a, 0)
                    assert free >= 0, "admitted past the free list"
                    held[a] = need
                    assert carried == (a not in resident)
            chunks.append(groups)
            outstanding.append(groups)
            idle = 0
        else:
            idle += 1
            assert outstanding, "nothing buildable and nothing in flight"
            assert idle < 3, "the scheduler stopped making progress"
        lag = rng.choice((0, 1)) if groups else 0
        while len(outstanding) > lag:
            for a, j, start, end, _ in outstanding.pop(0):
                for kind, anchor in sched.report(a, j, start, end, truth[a][j][start:end]):
                    events.append((kind, anchor))
                    settle(anchor)
    assert free == arena_pages, "pages leaked or freed twice"
    return chunks, events


def _random_join(rng):
    k = rng.randrange(1, 4)
    budget = rng.randrange(2_000, 20_000)
    frames = [rng.choice((0, 0, rng.randrange(1, 40))) for _ in range(k)]
    stages = [[rng.randrange(10, max(11, budget // 4)) for _ in range(rng.randrange(1, 80))]
              for _ in range(k)]
    top = budget - max(frames) - max(max(s) for s in stages)
    n = rng.randrange(1, 40)
    prefix = [rng.randrange(20, max(21, top)) for _ in range(n)]
    lists = []
    for _ in range(n):
        row = []
        for lens in stages:
            roll = rng.random()
            if roll < 0.5:
                row.append(None)
            elif roll < 0.6:
                row.append([])
            else:
                row.append(sorted(rng.sample(range(len(lens)), rng.randrange(1, len(lens) + 1))))
        lists.append(row)
    truth = [[[int(rng.random() < 0.5) for _ in (lens if lst is None else lst)]
              for lens, lst in zip(stages, row)] for row in lists]
    return prefix, stages, frames, budget, truth, lists


@pytest.mark.parametrize("seed", range(4))
def test_admission_invariants_over_random_shapes(seed):
    rng = random.Random(17 + seed)
    for _ in range(20):
        prefix, stages, frames, budget, truth, lists = _random_join(rng)
        need = [pages_for(p + max(frames), 16) for p in prefix]
        arena_pages = max(max(need), rng.randrange(4, 400))
        resident = {a: rng.randrange(1, need[a] + 1)
                    for a in range(len(prefix)) if rng.random() < 0.3}
        while sum(need[a] for a in resident) > arena_pages:
            resident.popitem()
        sched = JoinAdmission(prefix, stages, budget, arena_pages, 16, frame_tokens=frames,
                              resident=resident,
                              anchor_partners={a: lists[a] for a in range(len(prefix))})
        chunks, events = _drive(sched, truth, arena_pages, resident, rng)
        k = len(stages)

        def indices(a, j):
            lst = lists[a][j]
            return list(range(len(stages[j]))) if lst is None else list(lst)

        covered = {(a, j): [] for a in range(len(prefix)) for j in range(k)}
        carried = [0] * len(prefix)
        for groups in chunks:
            tokens = 0
            assert len({g[0] for g in groups}) == len(groups), "one anchor twice in a chunk"
            for a, j, start, end, is_carried in groups:
                assert end > start
                partners = sched.partner_indices(a, j, start, end)
                assert partners == indices(a, j)[start:end]
                tokens += ((prefix[a] if is_carried else 0) + (frames[j] if start == 0 else 0)
                           + sum(stages[j][i] for i in partners))
                covered[(a, j)].extend(range(start, end))
                carried[a] += is_carried
            assert tokens <= budget, "over-budget chunk"
        for a in range(len(prefix)):
            ran, expected = 0, ["finished"]
            for j in range(k):
                ran = j + 1 if indices(a, j) else j
                if not any(truth[a][j]):
                    expected = ["finished"] if j == k - 1 else ["dropped"]
                    break
            for j in range(k):
                if j < ran:
                    assert covered[(a, j)] == list(range(len(indices(a, j))))
                    assert sched.answers[j][a] == truth[a][j]
                else:
                    assert covered[(a, j)] == [] and a not in sched.answers[j]
            assert carried[a] == (0 if a in resident or not ran else 1)
            assert [kind for kind, anchor in events if anchor == a] == expected


# ---------------------------------------------------------------- the join loop


def _corpus(rng, n, vocab=50):
    """Anchors repeating one another's starts, so the prefix tree borrows."""
    header = [rng.randrange(vocab) for _ in range(rng.choice((0, 5, 16, 20)))]
    docs = []
    while len(docs) < n:
        trace = list(header)
        for _ in range(rng.randrange(1, 4)):
            trace = trace + [rng.randrange(vocab) for _ in range(rng.choice((1, 7, 16, 30)))]
            docs.append(trace)
            if rng.random() < 0.2:
                docs.append(list(trace))
    docs = docs[:n]
    rng.shuffle(docs)
    return docs


def _parts(n_partners=3):
    return [95, 96], [[97, 60 + p, 98] for p in range(n_partners)]


@pytest.mark.parametrize("path", ["unified", "tree"])
@pytest.mark.parametrize("seed", range(4))
def test_join_reads_over_random_corpora(path, seed):
    for retain in (False, True):
        rng = random.Random(100 + seed)
        anchors = _corpus(rng, 25)
        frame, partners = _parts(rng.randrange(1, 6))
        budget = max(map(len, anchors)) + rng.choice((8, 60, 600))
        pages = rng.choice((60, 400))
        model, _, _ = check_join(anchors, frame, partners, path=path, pages=pages,
                                 budget=budget, retain=retain)
        assert model.reads_checked > 0


@pytest.mark.parametrize("path", ["unified", "tree"])
def test_join_anchors_borrow_their_shared_root(path):
    # the AI join shape: every anchor = one shared instruction + its document
    rng = random.Random(3)
    root = [rng.randrange(1000) for _ in range(48)]
    anchors = [root + [rng.randrange(1000) for _ in range(rng.randrange(1, 60))]
               for _ in range(12)]
    frame, partners = [900, 901, 902], [[rng.randrange(1000) for _ in range(rng.randrange(2, 9))]
                                        for _ in range(7)]
    _, tokens, stats = check_join(anchors, frame, partners, path=path, pages=300, budget=400)
    assert stats["borrowed_tokens"] == 48 * 11 - 16 * 0   # 3 whole pages per child
    fresh_prefix = sum(map(len, anchors)) - stats["borrowed_tokens"]
    assert tokens == fresh_prefix + len(anchors) * (len(frame) + sum(map(len, partners)))


@pytest.mark.parametrize("path", ["unified", "tree"])
@pytest.mark.parametrize("seed", range(3))
def test_filter_survivors_feed_a_join(path, seed):
    rng = random.Random(200 + seed)
    docs = _corpus(rng, 30)
    frame, partners = _parts()
    check_feed(docs, [90, 91, 92], frame, partners, path=path, pages=rng.choice((80, 400)),
               budget=max(map(len, docs)) + rng.choice((8, 60, 600)))


@pytest.mark.parametrize("path", ["unified", "tree"])
def test_join_reads_every_pair_of_small_anchors(path):
    alphabet = [[1] * 17, [1] * 16 + [2], [1] * 33, [3], [1] * 16 + [2] * 17]
    frame, partners = _parts(2)
    for a, b in itertools.product(alphabet, repeat=2):
        check_join([a, b], frame, partners, path=path, pages=12,
                   budget=max(len(a), len(b)) + 8)
