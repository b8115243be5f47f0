"""Join admission details and the join loop (host-only, integer).

The reference's literal admission cases are data
(tests/golden/admission_cases.json, test_admission_cases.py) and the
admission invariants are properties over generated shapes
(test_admission_properties.py). Here: temporary-page pricing, two-stage
gating, the gate/assemble helpers against brute force, and the HashModel
checker over the real run_join loop, which checks every KV read it lays
out (tests/test_kv_reads.py:101-148 in the reference).
"""

import itertools
import random

import pytest

from kv_checker import check_feed, check_join
from quail_amd.pack import (JoinAdmission, assemble, gate, matches, pages_for,
                            partner_pages)


# ---------------------------------------------------------------- admission details


def test_temporary_suffix_pages_are_priced():
    """Unified joins give each partner temporary rows after a copy of the
    anchor's partial last page: admission charges them, so two 31-token
    anchors (2 pages each) and four 1-token partners cannot all fit 8 pages."""
    sched = JoinAdmission([31, 31], [[1, 1, 1, 1]], 256, 8, 16, temporary_suffix_pages=True)
    groups = sched.next_chunk(8)
    anchors_taken = {a for a, _, _, _, carried in groups if carried}
    partner_rows = [end - start for _, _, start, end, _ in groups]
    # here each streamed partner's temporaries (a copy of its anchor's 15
    # kept rows plus its 1 row) fill exactly one page beside the anchor's two
    assert 2 * len(anchors_taken) + sum(partner_rows) <= 8
    assert sum(partner_rows) < 2 * 4
    # one partner's temporary rows follow the anchor's partial last page
    cost = lambda t, b=None: pages_for(t, 16)   # noqa: E731
    assert partner_pages(cost, 16, 31, 0, 1) == 1     # 15 kept rows + 1
    assert partner_pages(cost, 16, 31, 0, 2) == 2     # 15 kept rows + 2
    assert partner_pages(cost, 16, 31, 1, 2) == 1     # the frame fills the page


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


@pytest.mark.parametrize("retain", [False, True])
@pytest.mark.parametrize("path", ["unified", "tree"])
def test_a_chunk_the_arena_cannot_hold_is_split_in_order(path, retain, monkeypatch):
    """The packer claims a chunk's temporary pages a page at a time, so an
    admitted chunk can still meet a full arena (loop.py:862-885 of the
    reference). Forced here: any chunk of more than two groups raises
    ArenaFullError. With no retained KV to evict, each such chunk is split
    in halves, run depth-first in order, and every pair is still answered
    from the right KV. With finished anchors retained as evictable KV, a
    refused chunk first evicts retained KV and is retried whole, and is
    split only once nothing is left to evict."""
    from quail_amd import loop

    launched, refused = [], []
    real = loop._Join.run_one

    def run_one(self, part):
        if len(part) > 2:
            refused.append(list(part))
            raise loop.ArenaFullError("forced: too many groups")
        launched.append(list(part))
        return real(self, part)

    monkeypatch.setattr(loop._Join, "run_one", run_one)
    rng = random.Random(7)
    anchors = _corpus(rng, 12)
    frame, partners = _parts(3)
    _, _, stats = check_join(anchors, frame, partners, path=path, pages=400,
                             budget=max(map(len, anchors)) + 600, retain=retain)
    assert refused and all(len(p) <= 2 for p in launched)
    if retain:
        # some refused chunk was retried whole after an eviction
        assert any(refused[i] == refused[i + 1] for i in range(len(refused) - 1))
    # the halves of every refused chunk ran in its order, back to back
    flat = [g for part in launched for g in part]
    for part in refused:
        first = flat.index(part[0])
        assert flat[first:first + len(part)] == part
    assert stats["chunks"] == len(launched)
