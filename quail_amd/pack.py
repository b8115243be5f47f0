"""Chunk admission for filters and joins: which rows enter each forward pass.

The admission itself runs in libquail_host.so (quail_amd/host/filter.cpp,
join.cpp); these classes keep the reference's surface (quail/backends/
quail/executor/pack.py:131-836) and hold the answers the caller reports.
The rules, which decide every page id and so follow the reference exactly:
  - filter: survivors' next-stage questions first, oldest first, stopping
    at the first that does not fit the chunk room; then fresh documents in
    queue order (prefix-tree order with a tree): a document whose pages do
    not fit stops admission and stays at the head of the queue; one whose
    tokens do not fit, or whose tree parent is still queued, is skipped for
    this chunk;
  - join: placed anchors' partner streams first, FIFO; then fresh anchors
    whose pages fit, each taking the longest partner run that fits; an
    anchor moves to its next stage once a stream is launched whole and a
    partner answered TRUE, and drops when every partner answered FALSE.
Lengths are tokens; suffixes are atomic.
"""

import numpy as np

from quail_amd import _host


def pages_for(tokens: int, page_tokens: int) -> int:
    """Pages for `tokens` rows."""
    return -(-int(tokens) // int(page_tokens))


def partner_pages(page_cost, page_tokens, prefix_tokens, frame_tokens, suffix_rows):
    """Temporary pages one partner takes on the unified path (pack.py:120-128):
    its rows follow the anchor's partial last page, whose kept rows are
    copied in ahead of them."""
    return page_cost((prefix_tokens + frame_tokens) % page_tokens + suffix_rows, 0)


def gate(answer_rows):
    """Anchors with any TRUE answer in their row, sorted (pack.py:30-36)."""
    return sorted(a for a in answer_rows if np.any(np.asarray(answer_rows[a])))


def matches(answer_rows):
    """anchor -> sorted partner positions answered TRUE (pack.py:39-42)."""
    return {a: [int(i) for i in np.flatnonzero(np.asarray(row))]
            for a, row in answer_rows.items()}


def assemble(ans1_rows, ans2_rows):
    """(a, b, c) triples of two join stages sharing the anchor b (pack.py:45-58)."""
    first, second = matches(ans1_rows), matches(ans2_rows)
    return sorted((a, b, c) for b in ans2_rows for a in first.get(b, ()) for c in second[b])


def _whole_pages(page_cost, page_tokens):
    """The library prices pages as ceil(tokens / page_tokens); a caller's
    page_cost must agree (it does for every arena without a sliding pool)."""
    if page_cost is None:
        return
    for t in (0, 1, page_tokens - 1, page_tokens, page_tokens + 1, 7 * page_tokens + 3, 4097):
        if page_cost(t, None) != pages_for(t, page_tokens):
            raise ValueError("page_cost must price whole pages of page_tokens "
                             "(quail_amd has no sliding-window pricing)")


def _tree_arrays(tree, n):
    if tree is None:
        return None, None, None
    order = _host.i32(list(tree.order))
    parent = _host.i32([-1 if p is None else p for p in tree.parent])
    shared = _host.i64(list(tree.shared))
    if order.size != n or parent.size != n or shared.size != n:
        raise ValueError(f"prefix tree over {order.size} documents, {n} given")
    return order, parent, shared


class Borrowing:
    """Which parent each admitted document borrows its KV prefix from
    (pack.py:131-209), read from the native plan. decide() is the plan's;
    assigning can_borrow installs a caller's check (doc, parent,
    parent_admitted_in_this_chunk) -> bool."""

    WAIT = "wait"

    def __init__(self, plan, kind):
        self._plan = plan
        self._kind = kind
        self._check = None

    def _row(self, doc):
        out = np.empty(5, dtype=np.int64)
        _host.call(f"qp_{self._kind}_borrow", self._plan.ptr, int(doc), out.ctypes.data)
        return out

    def _size(self):
        return int(_host.call(f"qp_{self._kind}_borrowers", self._plan.ptr, None, 0))

    @property
    def tree_parent(self):
        return [None if p < 0 else int(p)
                for p in (self._row(d)[0] for d in range(self._size()))]

    @property
    def tree_shared(self):
        return [int(self._row(d)[1]) for d in range(self._size())]

    def parent(self, doc):
        p = int(self._row(doc)[2])
        return None if p < 0 else p

    def shared(self, doc):
        return int(self._row(doc)[3])

    def borrowers(self):
        n = self._size()
        out = np.empty(n, dtype=np.int32)
        _host.call(f"qp_{self._kind}_borrowers", self._plan.ptr, out.ctypes.data, n)
        return out.tolist()

    @property
    def borrowed_tokens(self):
        state = np.empty(8, dtype=np.int64)
        _host.call(f"qp_{self._kind}_state", self._plan.ptr, state.ctypes.data)
        return int(state[5] if self._kind == "filter" else state[4])

    @property
    def can_borrow(self):
        return self._check

    @can_borrow.setter
    def can_borrow(self, check):
        self._check = check
        if check is None:
            _host.call(f"qp_{self._kind}_set_borrow_check", self._plan.ptr,
                       _host.BORROW_CHECK(), None)
            return

        def trampoline(doc, parent, same_chunk, _ctx):
            try:
                return 1 if check(int(doc), int(parent), bool(same_chunk)) else 0
            except Exception:   # a raising check refuses the borrow
                return 0

        self._trampoline = _host.BORROW_CHECK(trampoline)
        _host.call(f"qp_{self._kind}_set_borrow_check", self._plan.ptr, self._trampoline, None)


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
        page_cost: callable(tokens, base_tokens) -> pages; must price whole
            pages (None: whole pages).
        tree: a PrefixTree over the documents, or None.
        can_borrow: as Borrowing takes it.
    """

    def __init__(self, doc_tokens, stage_tokens, chunk_budget, arena_pages,
                 page_tokens, kept_extra_tokens=0, limit=None, page_cost=None,
                 tree=None, can_borrow=None):
        _whole_pages(page_cost, page_tokens)
        self.doc_tokens = _host.i64(list(doc_tokens))
        self.stage_tokens = list(stage_tokens)
        self.chunk_budget = int(chunk_budget)
        self.page_tokens = int(page_tokens)
        self.kept_extra = int(kept_extra_tokens)
        self.limit = limit
        self.pages = arena_pages is not None
        n = int(self.doc_tokens.size)
        order, parent, shared = _tree_arrays(tree, n)
        st = _host.i64(self.stage_tokens)
        ptr = _host.fn("qp_filter_new")(
            _host.ptr(self.doc_tokens), n, _host.ptr(st), int(st.size), self.chunk_budget,
            -1 if arena_pages is None else int(arena_pages), self.page_tokens, self.kept_extra,
            -1 if limit is None else int(limit), _host.ptr(order), _host.ptr(parent),
            _host.ptr(shared))
        self._plan = _host.Handle(ptr, "qp_filter_delete")
        self.borrowing = Borrowing(self._plan, "filter")
        if can_borrow is not None:
            self.borrowing.can_borrow = can_borrow
        self.answers = {}
        cap = max(n, 1)
        self._docs = np.empty(cap, dtype=np.int32)
        self._stages = np.empty(cap, dtype=np.int32)
        self._fresh = np.empty(cap, dtype=np.uint8)
        self._state = np.empty(8, dtype=np.int64)
        self._free = np.empty(1, dtype=np.int32)

    @property
    def native(self):
        return self._plan.ptr

    def bind_arena(self, arena, keys):
        """Borrow checks against the arena's resident keys (loop.py:1168-1182);
        keys[doc] is each document's arena key."""
        handles = _host.i64([arena.handle(k) for k in keys])
        self._keys = handles
        _host.call("qp_filter_bind_arena", self._plan.ptr, arena.native, _host.ptr(handles),
                   int(handles.size))

    def _groups(self, n):
        return [(int(d), int(s), bool(f))
                for d, s, f in zip(self._docs[:n], self._stages[:n], self._fresh[:n])]

    def next_chunk(self, free_pages=None):
        """Groups of the next chunk, [(doc, stage, fresh)]; [] when nothing fits."""
        n = _host.call("qp_filter_next_chunk", self._plan.ptr,
                       -1 if free_pages is None else int(free_pages), self._docs.ctypes.data,
                       self._stages.ctypes.data, self._fresh.ctypes.data, self._docs.size)
        return self._groups(n)

    def chunk_groups(self):
        """The groups of the last chunk, in packed order."""
        n = _host.call("qp_filter_groups", self._plan.ptr, self._docs.ctypes.data,
                       self._stages.ctypes.data, self._fresh.ctypes.data, self._docs.size)
        return self._groups(n)

    def report(self, doc, stage, passed, release=True):
        """Record one answer; returns the docs the caller frees."""
        self.answers.setdefault(doc, []).append(1 if passed else 0)
        _host.call("qp_filter_report", self._plan.ptr, int(doc), int(stage), int(bool(passed)),
                   int(bool(release)), self._free.ctypes.data)
        return () if self._free[0] < 0 else (int(self._free[0]),)

    def _read_state(self):
        _host.call("qp_filter_state", self._plan.ptr, self._state.ctypes.data)
        return self._state

    @property
    def blocked_pages(self):
        return int(self._read_state()[4])

    def done(self):
        return bool(self._read_state()[6])

    def drain_ready(self):
        out = np.empty(max(int(self._read_state()[1]), 1), dtype=np.int32)
        n = _host.call("qp_filter_drain_ready", self._plan.ptr, out.ctypes.data, out.size)
        return out[:n].tolist()

    def own_tokens(self, doc) -> int:
        return int(self.doc_tokens[doc]) - self.borrowing.shared(doc)

    @property
    def resident(self):
        return {d for d in range(self.doc_tokens.size) if self.borrowing._row(d)[4]}

    def survivors(self):
        n = len(self.stage_tokens)
        return sorted(d for d, row in self.answers.items() if len(row) == n and all(row))


def _lists_arrays(partners, k):
    """Per-stage partner index lists as (pointer array, size array, keepalive)."""
    if partners is None:
        return None, None, ()
    if len(partners) != k:
        raise ValueError(f"partner lists for {len(partners)} stages, the join has {k}")
    keep = [None if lst is None else _host.i32(list(lst)) for lst in partners]
    ptrs = np.array([0 if a is None else a.ctypes.data for a in keep], dtype=np.uint64)
    sizes = _host.i32([0 if a is None else a.size for a in keep])
    return ptrs, sizes, keep


class JoinAdmission:
    """Join scheduler: continuous anchor admission (pack.py:212-644).

    Args follow the reference: prefix_tokens per anchor; stage_suffixes[j]
    the suffix tokens of every stage-j partner; chunk_budget; arena_pages;
    page_tokens; frame_tokens per stage (rows written into the anchor's KV
    ahead of its first partner); resident: anchor -> pages it already
    holds (such an anchor packs no prefix tokens); anchor_partners:
    anchor -> per stage a partner index list or None; temporary_suffix_pages
    prices the unified path's per-partner temporaries; answer_dtype None
    for 0/1 answer lists, else a numpy dtype for scores; canvas_tokens rows
    a diffusion model adds per suffix and frame; page_cost must price whole
    pages; tree a PrefixTree over the anchors.
    """

    def __init__(self, prefix_tokens, stage_suffixes, chunk_budget, arena_pages,
                 page_tokens, frame_tokens=None, resident=None, anchor_partners=None,
                 temporary_suffix_pages=False, answer_dtype=None, canvas_tokens=0,
                 page_cost=None, tree=None, can_borrow=None):
        _whole_pages(page_cost, page_tokens)
        self.answer_dtype = answer_dtype
        self.page_tokens = int(page_tokens)
        self.chunk_budget = int(chunk_budget)
        k = len(stage_suffixes)
        if k == 0:
            raise ValueError("a join needs at least one stage")
        self.frames = list(frame_tokens) if frame_tokens else [0] * k
        if len(self.frames) != k:
            raise ValueError("frame_tokens must match stage_suffixes")
        self._stage_arrays = [_host.i64(list(lens)) for lens in stage_suffixes]
        self._stage_sizes = [int(a.size) for a in self._stage_arrays]
        ptrs = np.array([a.ctypes.data for a in self._stage_arrays], dtype=np.uint64)
        sizes = _host.i32(self._stage_sizes)
        frames = _host.i64(self.frames)
        n = len(prefix_tokens)
        order, parent, shared = _tree_arrays(tree, n)
        ptr = _host.fn("qp_join_new")(
            k, ptrs.ctypes.data, sizes.ctypes.data, frames.ctypes.data, self.chunk_budget,
            int(arena_pages), self.page_tokens, int(bool(temporary_suffix_pages)),
            int(canvas_tokens), n, _host.ptr(parent), _host.ptr(shared))
        self._plan = _host.Handle(ptr, "qp_join_delete")
        self.borrowing = Borrowing(self._plan, "join")
        if can_borrow is not None:
            self.borrowing.can_borrow = can_borrow
        self.prefix = []
        self.answers = [dict() for _ in range(k)]
        self._received = [dict() for _ in range(k)]
        self._lists = []
        resident = dict(resident or {})
        partners = dict(anchor_partners or {})
        for a, tokens in enumerate(prefix_tokens):
            self._register("qp_join_register", tokens, resident.get(a), partners.get(a))
        _host.call("qp_join_seed", self._plan.ptr, _host.ptr(order), 0 if order is None else n)
        self._cap = 0
        self._grow(max(n, 16))
        self._state = np.empty(8, dtype=np.int64)

    @property
    def native(self):
        return self._plan.ptr

    def _grow(self, cap):
        if cap <= self._cap:
            return
        self._cap = cap
        self._a = np.empty(cap, dtype=np.int32)
        self._j = np.empty(cap, dtype=np.int32)
        self._s = np.empty(cap, dtype=np.int64)
        self._e = np.empty(cap, dtype=np.int64)
        self._c = np.empty(cap, dtype=np.uint8)

    def _register(self, name, tokens, resident_pages, partners):
        ptrs, sizes, keep = _lists_arrays(partners, len(self._stage_arrays))
        a = _host.call(name, self._plan.ptr, int(tokens),
                       -1 if resident_pages is None else int(resident_pages),
                       _host.ptr(ptrs), _host.ptr(sizes))
        self.prefix.append(int(tokens))
        self._lists.append(keep)
        return int(a)

    def bind_arena(self, arena, keys):
        """Borrow checks against the arena (loop.py:1168-1182); keys[a] is each
        anchor's arena key (set_key for anchors admitted later)."""
        _host.call("qp_join_bind_arena", self._plan.ptr, arena.native)
        for a, key in enumerate(keys):
            self.set_key(a, arena.handle(key))

    def set_key(self, anchor, handle):
        _host.call("qp_join_set_key", self._plan.ptr, int(anchor), int(handle))

    def admit(self, prefix_tokens, resident_pages=None, partners=None):
        """Queue one more anchor behind the pending ones; returns its index."""
        a = self._register("qp_join_admit", prefix_tokens, resident_pages, partners)
        self._grow(len(self.prefix) + 16)
        return a

    def _events(self, settled):
        kinds = np.empty(64, dtype=np.int32)
        anchors = np.empty(64, dtype=np.int32)
        out = []
        while True:
            n = _host.call("qp_join_events", self._plan.ptr, int(settled), kinds.ctypes.data,
                           anchors.ctypes.data, 64)
            out.extend(("finished" if k else "dropped", int(a))
                       for k, a in zip(kinds[:n], anchors[:n]))
            if n < 64:
                return out

    def take_settled(self):
        """("finished"|"dropped", anchor) events of anchors that never ran a chunk."""
        return self._events(1)

    def _read_state(self):
        _host.call("qp_join_state", self._plan.ptr, self._state.ctypes.data)
        return self._state

    def buildable_tokens(self):
        """Tokens the next chunk could pack, capped at the budget (page room ignored)."""
        return int(self._read_state()[7])

    @property
    def blocked_pages(self):
        return int(self._read_state()[3])

    @property
    def in_flight(self):
        return int(self._read_state()[2])

    def done(self):
        return bool(self._read_state()[5])

    def partner_indices(self, a, j, start, end):
        """Stage-j partner indices of the group [start, end) of anchor a."""
        out = np.empty(max(end - start, 1), dtype=np.int32)
        n = _host.call("qp_join_partners", self._plan.ptr, int(a), int(j), int(start),
                       int(end), out.ctypes.data)
        return out[:n].tolist()

    def next_chunk(self, free_pages):
        """Groups of the next chunk, [(anchor, stage, start, end, carried)]."""
        self._grow(len(self.prefix) + 16)
        n = _host.call("qp_join_next_chunk", self._plan.ptr, int(free_pages),
                       self._a.ctypes.data, self._j.ctypes.data, self._s.ctypes.data,
                       self._e.ctypes.data, self._c.ctypes.data, self._cap)
        return [(int(self._a[i]), int(self._j[i]), int(self._s[i]), int(self._e[i]),
                 bool(self._c[i])) for i in range(n)]

    def report(self, a, j, start, end, bits):
        """Record one group's answers; returns ("dropped"|"finished", a) events."""
        received = self._received[j].get(a, 0)
        if received != start or len(bits) != end - start:
            raise AssertionError(f"anchor {a} stage {j}: answers for partners "
                                 f"{start}:{end} arrived with {received} recorded")
        if self.answer_dtype is None:
            self.answers[j].setdefault(a, []).extend(bits)
        else:
            row = self.answers[j].get(a)
            if row is None:
                row = np.empty(self._partner_count(a, j), dtype=self.answer_dtype)
                self.answers[j][a] = row
            row[start:end] = bits
        self._received[j][a] = end
        flags = (np.asarray(bits) != 0).astype(np.uint8)
        _host.call("qp_join_report", self._plan.ptr, int(a), int(j), int(start), int(end),
                   _host.ptr(flags), int(flags.size))
        return self._events(0)

    def _partner_count(self, a, j):
        lists = self._lists[a]
        if lists and lists[j] is not None:
            return int(lists[j].size)
        return self._stage_sizes[j]
