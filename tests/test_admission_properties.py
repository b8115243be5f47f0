"""Admission properties over generated shapes (hypothesis, derandomized).

A simulator stands in for the arena and the answer channel around a
FilterAdmission or JoinAdmission: it charges the pages each admitted
document or anchor takes, holds answers back for a chosen number of chunks
before reporting them, credits pages whenever the scheduler frees or
settles one, and records what every chunk held. The properties are the
admission contract of the reference (pack.py:212-836): chunks within the
token budget, pages never claimed past the arena and all returned at the
end, every document answered up to its first FALSE, every anchor's partner
stream covered exactly once per stage it reaches, in order, and one
settle event per anchor (finished, or dropped at the first stage with no
TRUE).
"""

from hypothesis import given, settings
from hypothesis import strategies as st

from quail_amd.pack import FilterAdmission, JoinAdmission, pages_for

PAGE = 16
SETTINGS = settings(max_examples=150, deadline=None, derandomize=True)


class Simulator:
    """Page ledger + delayed answers around one scheduler.

    `charge(groups)` returns {key: pages} for what a chunk newly holds;
    `deliver(groups)` reports a chunk's answers and returns the keys whose
    pages come back. Both are given by the scheduler kind below."""

    def __init__(self, sched, arena_pages, lag, charge, deliver, held=None):
        self.sched = sched
        self.arena_pages = arena_pages
        self.lag = lag
        self.charge = charge
        self.deliver = deliver
        self.held = dict(held or {})
        self.chunks = []

    def free(self):
        if self.arena_pages is None:
            return None
        return self.arena_pages - sum(self.held.values())

    def settle(self, keys):
        for key in keys:
            self.held.pop(key, None)

    def run(self, before=None):
        waiting = []
        quiet = 0
        while True:
            # settle events can end the run without a chunk (an anchor
            # with no partners at all)
            if before is not None:
                self.settle(before())
            if self.sched.done():
                break
            groups = self.sched.next_chunk(self.free())
            if groups:
                quiet = 0
                for key, pages in self.charge(groups).items():
                    self.held[key] = self.held.get(key, 0) + pages
                if self.arena_pages is not None:
                    assert sum(self.held.values()) <= self.arena_pages, "pages over the arena"
                self.chunks.append(groups)
                waiting.append(groups)
            else:
                quiet += 1
                assert waiting and quiet < 3, "no chunk buildable and nothing in flight"
            keep = self.lag if groups else 0
            while len(waiting) > keep:
                self.settle(self.deliver(waiting.pop(0)))
        return self.chunks


# ---------------------------------------------------------------- filters

@st.composite
def filter_shapes(draw):
    n_docs = draw(st.integers(1, 40))
    n_stages = draw(st.integers(1, 4))
    docs = draw(st.lists(st.integers(1, 700), min_size=n_docs, max_size=n_docs))
    stages = draw(st.lists(st.integers(1, 60), min_size=n_stages, max_size=n_stages))
    budget = max(docs) + max(stages) + draw(st.integers(0, 1500))
    paged = draw(st.booleans())
    arena = (max(pages_for(max(docs), PAGE), draw(st.integers(1, 150))) if paged else None)
    truth = draw(st.lists(st.lists(st.integers(0, 1), min_size=n_stages, max_size=n_stages),
                          min_size=n_docs, max_size=n_docs))
    lag = draw(st.integers(0, 2))
    return docs, stages, budget, arena, truth, lag


@SETTINGS
@given(filter_shapes())
def test_filter_admission_properties(shape):
    docs, stages, budget, arena, truth, lag = shape
    sched = FilterAdmission(docs, stages, budget, arena, PAGE)

    def charge(groups):
        if arena is None:
            return {}
        return {d: pages_for(sched.own_tokens(d) + sched.kept_extra, PAGE)
                for d, _, fresh in groups if fresh}

    def deliver(groups):
        freed = []
        for d, s, _ in groups:
            freed.extend(sched.report(d, s, bool(truth[d][s])))
        return freed

    sim = Simulator(sched, arena, lag, charge, deliver)
    chunks = sim.run()
    entered = []
    for groups in chunks:
        assert len({d for d, _, _ in groups}) == len(groups), "a document twice in a chunk"
        used = sum(stages[s] + (docs[d] if fresh else 0) for d, s, fresh in groups)
        assert used <= budget, "over-budget chunk"
        assert all(s == 0 for _, s, fresh in groups if fresh), "fresh past stage 0"
        entered += [d for d, _, fresh in groups if fresh]
    assert sorted(entered) == list(range(len(docs))), "a document entered twice or never"
    for d, row in enumerate(truth):
        cut = row.index(0) + 1 if 0 in row else len(row)
        assert sched.answers[d] == row[:cut], f"document {d} gated wrongly"
    assert sched.survivors() == [d for d, row in enumerate(truth) if all(row)]
    assert not sched.resident and not sim.held, "pages left held"


# ---------------------------------------------------------------- joins

@st.composite
def join_shapes(draw):
    k = draw(st.integers(1, 3))
    budget = draw(st.integers(400, 6000))
    frames = [draw(st.sampled_from([0, 0, 3, 17, 39])) for _ in range(k)]
    stages = [draw(st.lists(st.integers(5, max(6, budget // 4)), min_size=1, max_size=30))
              for _ in range(k)]
    room = budget - max(frames) - max(max(s) for s in stages)
    n = draw(st.integers(1, 25))
    prefix = draw(st.lists(st.integers(1, max(1, room)), min_size=n, max_size=n))
    lists = []
    for _ in range(n):
        row = []
        for lens in stages:
            kind = draw(st.sampled_from(["all", "all", "none", "some"]))
            if kind == "all":
                row.append(None)
            elif kind == "none":
                row.append([])
            else:
                row.append(sorted(draw(st.sets(st.integers(0, len(lens) - 1), min_size=1))))
        lists.append(row)
    truth = [[[draw(st.integers(0, 1)) for _ in (lens if lst is None else lst)]
              for lens, lst in zip(stages, row)] for row in lists]
    need = [pages_for(p + max(frames), PAGE) for p in prefix]
    arena = max(max(need), draw(st.integers(1, 300)))
    # resident anchors hold part of their pages already; their full spans
    # together must fit the arena, or growing them could never finish
    resident = {}
    for a in range(n):
        if draw(st.integers(0, 3)) == 0 and sum(need[r] for r in resident) + need[a] <= arena:
            resident[a] = draw(st.integers(1, need[a]))
    lag = draw(st.integers(0, 2))
    return prefix, stages, frames, budget, truth, lists, arena, resident, lag


@SETTINGS
@given(join_shapes())
def test_join_admission_properties(shape):
    prefix, stages, frames, budget, truth, lists, arena, resident, lag = shape
    n, k = len(prefix), len(stages)
    sched = JoinAdmission(prefix, stages, budget, arena, PAGE, frame_tokens=frames,
                          resident=resident,
                          anchor_partners={a: lists[a] for a in range(n)})
    extra = max(frames)
    events = []

    def charge(groups):
        out = {}
        for a, j, start, _, carried in groups:
            assert carried == (j == 0 and start == 0 and a not in resident), \
                f"anchor {a} carried its prefix at stage {j} from partner {start}"
            if carried:
                out[a] = pages_for(prefix[a] + extra, PAGE)
            elif j == 0 and start == 0:
                # a resident anchor grows to its full span
                out[a] = pages_for(prefix[a] + extra, PAGE) - resident[a]
        return out

    def settled(pairs):
        events.extend(pairs)
        return [a for _, a in pairs]

    def deliver(groups):
        gone = []
        for a, j, start, end, _ in groups:
            gone += settled(sched.report(a, j, start, end, truth[a][j][start:end]))
        return gone

    sim = Simulator(sched, arena, lag, charge, deliver, held=resident)
    chunks = sim.run(before=lambda: settled(sched.take_settled()))

    def partners(a, j):
        return list(range(len(stages[j]))) if lists[a][j] is None else list(lists[a][j])

    streamed = {}
    for groups in chunks:
        assert len({g[0] for g in groups}) == len(groups), "an anchor twice in a chunk"
        used = 0
        for a, j, start, end, carried in groups:
            assert end > start
            got = sched.partner_indices(a, j, start, end)
            assert got == partners(a, j)[start:end]
            used += (prefix[a] if carried else 0) + (frames[j] if start == 0 else 0)
            used += sum(stages[j][i] for i in got)
            streamed.setdefault((a, j), []).extend(range(start, end))
        assert used <= budget, "over-budget chunk"
    for a in range(n):
        # the stages anchor a reaches: up to the first one it answers all FALSE
        reached, outcome = k, "finished"
        for j in range(k):
            if partners(a, j) and not any(truth[a][j]):
                reached, outcome = j + 1, ("finished" if j == k - 1 else "dropped")
                break
            if not partners(a, j) and j < k - 1:
                reached, outcome = j, "dropped"
                break
        for j in range(k):
            if j < reached and partners(a, j):
                assert streamed.get((a, j)) == list(range(len(partners(a, j)))), (a, j)
                assert sched.answers[j][a] == truth[a][j]
            else:
                assert (a, j) not in streamed and a not in sched.answers[j], (a, j)
        assert [kind for kind, who in events if who == a] == [outcome], (a, events)
    assert not sim.held, "pages left held"
