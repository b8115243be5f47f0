"""Chunk admission for filters: which documents enter each forward pass.

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
from collections import deque


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
