"""Chunk admission for filters and joins: which rows enter each forward pass.

Host-only integer logic (no torch). The admission order decides which
pages every document gets, so it restates the reference's rules exactly
(quail/backends/quail/executor/pack.py:76-209, :647-836):
  - survivors' next-stage suffixes pack first, oldest first, and stop at
    the first one that does not fit the chunk room;
  - fresh documents are then taken in queue order (prefix-tree order when a
    tree is given); a document whose pages do not fit stops page claiming
    (it goes back to the head of the queue), one whose tokens do not fit
    the remaining chunk room is skipped and retried next chunk, one whose
    parent is still queued waits (skipped);
  - skipped documents return to the head of the queue in their order.
Lengths are tokens; suffixes are atomic.
"""

from array import array
from bisect import bisect_right
from collections import deque

import numpy as np


def pages_for(tokens: int, page_tokens: int) -> int:
    """Pages for `tokens` rows."""
    return -(-tokens // page_tokens)


class _CompactQueue:
    """Document positions in order, held as ranges and int arrays (pack.py:76-108)."""

    def __init__(self, count: int):
        self._pieces = deque()
        self._length = 0
        if count:
            self._pieces.append([range(count), 0])
            self._length = count

    def __bool__(self):
        return self._length > 0

    def __len__(self):
        return self._length

    def popleft(self) -> int:
        if not self._pieces:
            raise IndexError("pop from an empty document queue")
        piece = self._pieces[0]
        values, position = piece
        value = values[position]
        position += 1
        self._length -= 1
        if position == len(values):
            self._pieces.popleft()
        else:
            piece[1] = position
        return value

    def appendleft(self, value: int) -> None:
        self.prepend(array("I", [value]))

    def prepend(self, values) -> None:
        if len(values):
            self._pieces.appendleft([values, 0])
            self._length += len(values)


class Borrowing:
    """Which parent each admitted document borrows its KV prefix from (pack.py:131-209).

    decide() answers WAIT while the parent is queued, None to pack the
    whole document (no parent, parent skipped, or the arena refuses the
    borrow), else (parent, shared tokens).
    """

    WAIT = "wait"

    def __init__(self, n, tree=None, can_borrow=None):
        self.tree_parent = [None] * n if tree is None else list(tree.parent)
        self.tree_shared = [0] * n if tree is None else list(tree.shared)
        self.can_borrow = can_borrow
        self.admitted = set()
        self.skipped = set()
        self.chosen = {}
        self.borrowed_tokens = 0

    def add(self):
        self.tree_parent.append(None)
        self.tree_shared.append(0)
        return len(self.tree_parent) - 1

    def detach(self, doc):
        self.tree_parent[doc] = None
        self.tree_shared[doc] = 0

    def skip(self, doc):
        self.skipped.add(doc)

    def borrowers(self):
        counts = [0] * len(self.tree_parent)
        for parent in self.tree_parent:
            if parent is not None:
                counts[parent] += 1
        return counts

    def decide(self, doc, chunk):
        parent = self.tree_parent[doc]
        if parent is None or parent in self.skipped:
            return None
        if parent not in self.admitted:
            return self.WAIT
        if self.can_borrow is not None and not self.can_borrow(doc, parent, parent in chunk):
            return None
        return parent, self.tree_shared[doc]

    def record(self, doc, choice):
        self.admitted.add(doc)
        if choice is not None:
            self.chosen[doc] = choice
            self.borrowed_tokens += choice[1]

    def parent(self, doc):
        return self.chosen.get(doc, (None, 0))[0]

    def shared(self, doc):
        return self.chosen.get(doc, (None, 0))[1]


class FilterAdmission:
    """Filter-chain scheduler: chunk groups in admission order (pack.py:647-836).

    Args:
        doc_tokens: tokens per document.
        stage_tokens: question suffix tokens per stage.
        chunk_budget: tokens per forward pass.
        arena_pages: pages in the arena, or None when nothing is written to it.
        page_tokens: tokens per page.
        kept_extra_tokens: extra rows per document its pages must cover.
        limit: stop after this many survivors.
        page_cost: callable(tokens, base_tokens) -> pages; None prices
            whole pages of page_tokens.
        tree: a PrefixTree over the documents, or None.
        can_borrow: as Borrowing takes it.
    """

    def __init__(self, doc_tokens, stage_tokens, chunk_budget, arena_pages,
                 page_tokens, kept_extra_tokens=0, limit=None, page_cost=None,
                 tree=None, can_borrow=None):
        self.page_cost = page_cost or (
            lambda tokens, base_tokens=None: pages_for(tokens, page_tokens))
        self.doc_tokens = doc_tokens
        n = len(doc_tokens)
        self.borrowing = Borrowing(n, tree, can_borrow)
        self.stage_tokens = list(stage_tokens)
        self.chunk_budget = chunk_budget
        self.page_tokens = page_tokens
        self.pages = arena_pages is not None
        self.blocked_pages = 0
        self.limit = limit
        self._survivor_count = 0
        self.kept_extra = kept_extra_tokens
        if tree is not None and arena_pages is None:
            raise ValueError("a prefix tree needs page accounting")
        widest_stage = max(stage_tokens)
        for d, t in enumerate(doc_tokens):
            need = t + widest_stage
            if need > chunk_budget:
                raise ValueError(f"document {d} + question needs {need} "
                                 f"tokens > chunk budget {chunk_budget}")
            if arena_pages is not None and self.page_cost(t + kept_extra_tokens) > arena_pages:
                raise ValueError(f"document {d} needs more pages than the arena holds")
        if tree is None or list(tree.order) == list(range(n)):
            self.pending = _CompactQueue(n)
        else:
            self.pending = _CompactQueue(0)
            self.pending.prepend(array("I", tree.order))
        self.ready = deque()     # (doc, stage) gated TRUE, next suffix
        self.in_flight = set()
        self.resident = set()
        self.answers = {}

    def own_tokens(self, doc) -> int:
        return self.doc_tokens[doc] - self.borrowing.shared(doc)

    def next_chunk(self, free_pages=None):
        """Groups of the next chunk, [(doc, stage, fresh)]; [] when nothing fits."""
        if self._limit_reached():
            return []
        self.blocked_pages = 0
        room = self.chunk_budget
        groups = []
        admitted = set()
        # survivors first: FIFO, stop at the first that does not fit
        for _ in range(len(self.ready)):
            doc, stage = self.ready[0]
            cost = self.stage_tokens[stage]
            if cost > room:
                break
            self.ready.popleft()
            groups.append((doc, stage, False))
            self.in_flight.add(doc)
            room -= cost
        # fresh documents: pages in queue order, chunk room may skip
        skipped = array("I")
        while self.pending:
            doc = self.pending.popleft()
            choice = self.borrowing.decide(doc, admitted)
            if choice == Borrowing.WAIT:
                skipped.append(doc)
                continue
            own = self.doc_tokens[doc] - (choice[1] if choice else 0)
            need_pages = 0
            if free_pages is not None:
                need_pages = self.page_cost(own + self.kept_extra)
                if need_pages > free_pages:
                    self.pending.appendleft(doc)
                    self.blocked_pages = need_pages - free_pages
                    break
            cost = self.stage_tokens[0] + own
            if cost > room:
                skipped.append(doc)
                continue
            if free_pages is not None:
                free_pages -= need_pages
            self.borrowing.record(doc, choice)
            self.resident.add(doc)
            groups.append((doc, 0, True))
            self.in_flight.add(doc)
            admitted.add(doc)
            room -= cost
        self.pending.prepend(skipped)
        return groups

    def report(self, doc, stage, passed, release=True):
        """Record one answer; returns the docs the caller frees."""
        self.in_flight.discard(doc)
        self.answers.setdefault(doc, []).append(1 if passed else 0)
        last = stage == len(self.stage_tokens) - 1
        if passed and last:
            self._survivor_count += 1
        if passed and not last:
            self.ready.append((doc, stage + 1))
            return ()
        self.resident.discard(doc)
        if not self.pages or not release:
            return ()
        return (doc,)

    def _limit_reached(self):
        return self.limit is not None and self._survivor_count >= self.limit

    def done(self):
        if self._limit_reached():
            return not self.in_flight
        return not self.pending and not self.ready and not self.in_flight

    def drain_ready(self):
        out = []
        while self.ready:
            doc, _ = self.ready.popleft()
            self.resident.discard(doc)
            if self.pages:
                out.append(doc)
        return out

    def survivors(self):
        n = len(self.stage_tokens)
        return sorted(d for d, row in self.answers.items() if len(row) == n and all(row))


# ------------------------------------------------------------------ joins
#
# A join scores every (anchor, partner) pair. The anchor's document is
# written into the arena once; every partner is a suffix that reads it.
# Stages chain joins on one anchor: an anchor moves to stage j+1 once its
# whole stage-j stream is launched and one partner answered TRUE, and
# drops out when every partner answered FALSE.


def gate(answer_rows):
    """Anchors with any TRUE answer in their row, sorted (pack.py:31-37)."""
    return sorted(a for a, row in answer_rows.items() if any(row))


def matches(answer_rows):
    """anchor -> sorted partner positions answered TRUE (pack.py:40-43)."""
    return {a: [i for i, v in enumerate(row) if v] for a, row in answer_rows.items()}


def assemble(ans1_rows, ans2_rows):
    """(a, b, c) triples from two join stages sharing the anchor b (pack.py:46-59)."""
    first, second = matches(ans1_rows), matches(ans2_rows)
    return sorted((a, b, c) for b in ans2_rows for a in first.get(b, ()) for c in second[b])


def partner_pages(page_cost, page_tokens, prefix_tokens, frame_tokens, suffix_rows):
    """Temporary pages one partner takes on the unified path (pack.py:120-128).

    The partner's rows follow the anchor's partial last page, whose kept
    rows are copied in ahead of them.
    """
    return page_cost((prefix_tokens + frame_tokens) % page_tokens + suffix_rows, 0)


_SETTLED = -2     # the anchor's last stage answered, or a gate dropped it


class _Anchor:
    """One anchor's costs and progress through the join's stages."""

    __slots__ = ("prefix", "lists", "cums", "pages", "carried", "first", "stage",
                 "next", "true")

    def __init__(self, prefix, lists, cums, pages, carried, n_stages):
        self.prefix = prefix          # prefix tokens (document + preamble)
        self.lists = lists            # per stage: partner indices, or None for all
        self.cums = cums              # per stage: cumulative suffix rows of the list
        self.pages = pages            # pages its admission claims
        self.carried = carried        # prefix tokens it packs (0 when resident)
        self.first = 0                # rows of its first group's first partner
        self.stage = -1               # -1 queued; >= 0 running; _SETTLED
        self.next = 0                 # next partner position at the stage
        self.true = [False] * n_stages


class JoinAdmission:
    """Join scheduler: continuous anchor admission (pack.py:212-644).

    Args:
        prefix_tokens: per-anchor prefix token counts.
        stage_suffixes: per stage, the suffix token count of every partner.
        chunk_budget: tokens per forward pass.
        arena_pages: pages in the KV arena.
        page_tokens: tokens per page.
        frame_tokens: per stage, tokens of the join framing written into an
            anchor's KV ahead of its first partner at that stage.
        resident: anchor -> pages it already holds; such an anchor packs no
            prefix tokens.
        anchor_partners: anchor -> per stage, a list of partner indices or
            None for every partner.
        temporary_suffix_pages: price the unified path's per-partner
            temporary pages against the free list.
        answer_dtype: None for 0/1 answer lists; a numpy dtype for scores.
        canvas_tokens: rows a diffusion model adds after every suffix and
            frame (chunk and page room only, never kept).
        page_cost: callable(tokens, base_tokens) -> pages.
        tree: a PrefixTree over the anchors, or None.
        can_borrow: as Borrowing takes it.

    next_chunk() fills a chunk in priority order: partner streams cut by the
    previous chunk and anchors starting their next stage (FIFO, stopping at
    the first that does not fit), then fresh anchors whose pages fit the
    free list (page-blocked ones stop claiming unless zero-cost anchors
    remain, room-blocked ones are retried next chunk).
    """

    def __init__(self, prefix_tokens, stage_suffixes, chunk_budget, arena_pages,
                 page_tokens, frame_tokens=None, resident=None, anchor_partners=None,
                 temporary_suffix_pages=False, answer_dtype=None, canvas_tokens=0,
                 page_cost=None, tree=None, can_borrow=None):
        self.answer_dtype = answer_dtype
        self.borrowing = Borrowing(len(prefix_tokens), tree, can_borrow)
        self.page_cost = page_cost or (
            lambda tokens, base_tokens=None: pages_for(tokens, page_tokens))
        self.temporary_suffix_pages = temporary_suffix_pages
        self.stages = [[t + canvas_tokens for t in lens] for lens in stage_suffixes]
        self.frames = list(frame_tokens) if frame_tokens else [0] * len(self.stages)
        if len(self.frames) != len(self.stages):
            raise ValueError("frame_tokens must match stage_suffixes")
        # rows a frame entry packs (canvas included); frames are the rows kept
        self.frame_rows = [f + canvas_tokens if f else 0 for f in self.frames]
        if not self.stages:
            raise ValueError("a join needs at least one stage")
        self.chunk_budget = chunk_budget
        self.arena_pages = arena_pages
        self.page_tokens = page_tokens
        self._stage_cum = []
        for j, lens in enumerate(self.stages):
            self._stage_cum.append(_cumulative(lens))
            if lens and self.frame_rows[j] + max(lens) > chunk_budget:
                raise ValueError(
                    f"stage {j}: a {self.frame_rows[j] + max(lens)}-token partner exceeds "
                    f"the {chunk_budget}-token chunk budget (suffixes are atomic)")
        self._extra = max(self.frame_rows)
        self.anchors = []
        self.prefix = []              # per anchor, prefix tokens (public, as the reference)
        self._page_cum_cache = {}
        self._page_reserve = 0
        self._min_fresh = float("inf")
        self._zero_cost = 0
        self._settled = []
        self._answer_counts = [{} for _ in self.stages]
        self.answers = [dict() for _ in self.stages]
        self.pending = deque()
        self.ready = deque()
        self.in_flight = 0
        self.blocked_pages = 0
        resident = dict(resident or {})
        partners = dict(anchor_partners or {})
        for a, tokens in enumerate(prefix_tokens):
            self._register(tokens, resident.get(a), partners.get(a))
        # resident anchors first: they claim few or no pages, so they never
        # wait behind a page-blocked fresh anchor
        order = range(len(self.anchors)) if tree is None else tree.order
        self.pending.extend(a for a in range(len(self.anchors))
                            if a in resident and self.anchors[a].stage == -1)
        self.pending.extend(a for a in order
                            if a not in resident and self.anchors[a].stage == -1)
        for a in resident:
            self.borrowing.detach(a)

    # ---- per-anchor bookkeeping ------------------------------------------

    def _count(self, a, j):
        lst = self.anchors[a].lists[j]
        return len(self.stages[j]) if lst is None else len(lst)

    def _cum(self, a, j):
        anchor = self.anchors[a]
        return self._stage_cum[j] if anchor.lists[j] is None else anchor.cums[j]

    def _suffix(self, a, j, i):
        lst = self.anchors[a].lists[j]
        return self.stages[j][i if lst is None else lst[i]]

    def partner_indices(self, a, j, start, end):
        """Stage-j partner indices of the group [start, end) of anchor a."""
        lst = self.anchors[a].lists[j]
        return list(range(start, end)) if lst is None else list(lst[start:end])

    def _register(self, prefix, resident_pages, partners):
        a = len(self.anchors)
        k = len(self.stages)
        if partners is None:
            lists, cums = [None] * k, [None] * k
        else:
            if len(partners) != k:
                raise ValueError(f"anchor {a}: partner lists for {len(partners)} stages, "
                                 f"the join has {k}")
            lists, cums = [], []
            for j, lst in enumerate(partners):
                if lst is None:
                    lists.append(None)
                    cums.append(None)
                    continue
                lst = list(lst)
                for i in lst:
                    if not 0 <= i < len(self.stages[j]):
                        raise ValueError(f"anchor {a} stage {j}: partner {i} is out of range")
                lists.append(lst)
                cums.append(_cumulative([self.stages[j][i] for i in lst]))
        pages = self.page_cost(prefix + self._extra)
        if resident_pages is not None:
            pages = max(0, pages - resident_pages)
        elif pages > self.arena_pages:
            raise ValueError(f"anchor {a} needs {pages} KV pages; the arena holds "
                             f"{self.arena_pages}")
        anchor = _Anchor(prefix, lists, cums, pages,
                         0 if resident_pages is not None else prefix, k)
        self.anchors.append(anchor)
        self.prefix.append(prefix)
        if self._count(a, 0) == 0:
            # no partner at the first stage: settles without a chunk
            anchor.stage = _SETTLED
            self._settled.append(("finished" if k == 1 else "dropped", a))
            self.borrowing.skip(a)
            return a
        anchor.first = self.frame_rows[0] + self._suffix(a, 0, 0)
        if resident_pages is None and prefix + anchor.first > self.chunk_budget:
            raise ValueError(f"anchor {a}: prefix {prefix} tokens leaves no room for a "
                             f"partner in a {self.chunk_budget}-token chunk")
        if self.temporary_suffix_pages:
            largest = max((self._suffix_page_cost(a, j, i)
                           for j in range(k) for i in range(self._count(a, j))), default=0)
            if self.page_cost(prefix + self._extra) + largest > self.arena_pages:
                raise ValueError("anchor and one suffix exceed the KV arena")
            self._page_reserve = max(self._page_reserve, largest)
        shared = self.borrowing.tree_shared
        borrowable = shared[a] if a < len(shared) else 0
        self._min_fresh = min(self._min_fresh,
                              max(0, anchor.carried - borrowable) + anchor.first)
        if not pages:
            self._zero_cost += 1
        return a

    def admit(self, prefix_tokens, resident_pages=None, partners=None):
        """Queue one more anchor behind the pending ones; returns its index."""
        a = self._register(prefix_tokens, resident_pages, partners)
        self.borrowing.add()
        if self.anchors[a].stage == -1:
            self.pending.append(a)
        return a

    def take_settled(self):
        """("finished"|"dropped", anchor) events of anchors that never ran a chunk."""
        events, self._settled = self._settled, []
        return events

    def buildable_tokens(self):
        """Tokens the next chunk could pack, capped at the budget (page room ignored)."""
        total = 0
        for a in self.ready:
            anchor = self.anchors[a]
            j, i = anchor.stage, anchor.next
            cum = self._cum(a, j)
            total += (self.frame_rows[j] if i == 0 else 0) + cum[-1] - cum[i]
            if total >= self.chunk_budget:
                return self.chunk_budget
        for a in self.pending:
            anchor = self.anchors[a]
            total += anchor.carried + self.frame_rows[0] + self._cum(a, 0)[-1]
            if total >= self.chunk_budget:
                return self.chunk_budget
        return total

    # ---- chunk building ----------------------------------------------------

    def _first_cost(self, a, j, i):
        return self._suffix(a, j, i) + (self.frame_rows[j] if i == 0 else 0)

    def _suffix_page_cost(self, a, j, i):
        return partner_pages(self.page_cost, self.page_tokens, self.anchors[a].prefix,
                             self.frames[j], self._suffix(a, j, i))

    def _page_cum(self, a, j):
        key = (a, j)
        costs = self._page_cum_cache.get(key)
        if costs is None:
            costs = _cumulative([self._suffix_page_cost(a, j, i)
                                 for i in range(self._count(a, j))])
            self._page_cum_cache[key] = costs
        return costs

    def _take(self, a, j, i, room, page_room):
        """(end, tokens, temporary pages) of the longest partner run from i that fits."""
        cum = self._cum(a, j)
        frame = self.frame_rows[j] if i == 0 else 0
        end = bisect_right(cum, cum[i] + room - frame) - 1
        pages = 0
        if self.temporary_suffix_pages:
            costs = self._page_cum(a, j)
            end = min(end, bisect_right(costs, costs[i] + page_room) - 1)
            pages = costs[end] - costs[i]
        return end, frame + cum[end] - cum[i], pages

    def _launch(self, a, j, end):
        self.anchors[a].next = end
        self.in_flight += 1
        return end < self._count(a, j)

    def next_chunk(self, free_pages):
        """Groups of the next chunk, [(anchor, stage, start, end, carried)].

        start/end index the anchor's own partner list at the stage
        (partner_indices maps them); carried says the anchor's prefix is
        packed in this chunk. [] when nothing is buildable.
        """
        self.blocked_pages = 0
        room = self.chunk_budget
        groups, continued = [], []
        temporary = 0
        # 1) placed anchors: cut streams and next-stage starts, FIFO
        for _ in range(len(self.ready)):
            a = self.ready.popleft()
            anchor = self.anchors[a]
            j, i = anchor.stage, anchor.next
            if self._first_cost(a, j, i) > room:
                self.ready.appendleft(a)
                break
            end, tokens, pages = self._take(a, j, i, room, free_pages)
            if end == i:
                self.blocked_pages = self._suffix_page_cost(a, j, i) - free_pages
                self.ready.appendleft(a)
                break
            free_pages -= pages
            temporary += pages
            groups.append((a, j, i, end, False))
            room -= tokens
            if self._launch(a, j, end):
                continued.append(a)
        # 2) fresh anchors: pages in queue order, chunk room may skip one
        held = []
        blocked = False
        admitted = set()
        while self.pending and room >= self._min_fresh:
            a = self.pending.popleft()
            anchor = self.anchors[a]
            borrow = self.borrowing.decide(a, admitted)
            if borrow == Borrowing.WAIT:
                held.append(a)
                continue
            need = (anchor.pages if borrow is None
                    else self.page_cost(anchor.prefix - borrow[1] + self._extra))
            if blocked and need:
                held.append(a)
                if not self._zero_cost:
                    break
                continue
            required = need + max(0, self._page_reserve - temporary)
            if required > free_pages:
                blocked = True
                self.blocked_pages = required - free_pages
                held.append(a)
                if not self._zero_cost:
                    break
                continue
            carried = anchor.carried if borrow is None else anchor.prefix - borrow[1]
            if carried + anchor.first > room:
                held.append(a)
                continue
            end, tokens, pages = self._take(a, 0, 0, room - carried, free_pages - need)
            if end == 0:
                held.append(a)
                self.blocked_pages = need + self._suffix_page_cost(a, 0, 0) - free_pages
                break
            temporary += pages
            groups.append((a, 0, 0, end, carried > 0))
            room -= carried + tokens
            free_pages -= need + pages
            if not anchor.pages:
                self._zero_cost -= 1
            anchor.stage = 0
            admitted.add(a)
            self.borrowing.record(a, borrow)
            if self._launch(a, 0, end):
                continued.append(a)
        self.pending.extendleft(reversed(held))
        self.ready.extendleft(reversed(continued))
        return groups

    # ---- gating ------------------------------------------------------------

    def report(self, a, j, start, end, bits):
        """Record one group's answers; returns ("dropped"|"finished", a) events."""
        if self.answer_dtype is None:
            row = self.answers[j].setdefault(a, [])
            received = len(row)
        else:
            if a not in self.answers[j]:
                self.answers[j][a] = np.empty(self._count(a, j), dtype=self.answer_dtype)
            row = self.answers[j][a]
            received = self._answer_counts[j].get(a, 0)
        if received != start or len(bits) != end - start:
            raise AssertionError(f"anchor {a} stage {j}: answers for partners "
                                 f"{start}:{end} arrived with {received} recorded")
        if self.answer_dtype is None:
            row.extend(bits)
        else:
            row[start:end] = bits
            self._answer_counts[j][a] = end
        self.in_flight -= 1
        anchor = self.anchors[a]
        if np.any(np.asarray(bits)):
            anchor.true[j] = True
        k = len(self.stages)
        n_j = self._count(a, j)
        complete = end == n_j
        events = []
        if j == anchor.stage and j + 1 < k:
            if anchor.true[j] and anchor.next == n_j:
                # the whole stream is launched: the next stage's frame write
                # is queued behind every read of this stage
                anchor.stage, anchor.next = j + 1, 0
                if self._count(a, j + 1):
                    self.ready.append(a)
                else:
                    anchor.stage = _SETTLED
                    events.append(("finished" if j + 2 == k else "dropped", a))
            elif complete and not anchor.true[j]:
                anchor.stage = _SETTLED
                events.append(("dropped", a))
        if j == k - 1 and complete:
            anchor.stage = _SETTLED
            events.append(("finished", a))
        return events

    def done(self):
        return not self.pending and not self.ready and not self.in_flight \
            and not self._settled


def _cumulative(lens):
    out = [0]
    for t in lens:
        out.append(out[-1] + t)
    return out
