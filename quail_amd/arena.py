"""Paged KV arena: page accounting (PageArena) and its device pools (KVArena).

The accounting lives in libquail_host.so (quail_amd/host/arena.cpp); these
classes keep the reference's method surface (quail/backends/quail/executor/
arena.py:8-24) and map the caller's keys - any hashable: document ids,
(alias, document) pairs - to the library's integer handles. Temporaries are
TemporaryKey objects that carry the library's own (negative) handle.

Page ids reach the kernels through block tables and scatter maps, so the
library reproduces the reference's page order bit for bit (see arena.cpp):
a fresh arena hands out pages 0, 1, 2, ...; freed pages are reused last in,
first out; a key's table is its borrowed pages, then its own; arena row of
(page, slot) is page * page_tokens + slot (arena.py:519-523); block tables
are zero-padded to the widest row (arena.py:874-887).

The device pools use the MI355X layout of quail_amd.layout (K pages
[n_kv, page, d], V pages transposed [n_kv, d, page]) with the same row
numbering. Sliding-window pools (DiffusionGemma) are not part of this
build: an arena asked for one raises.
"""

from collections.abc import Mapping, Set

import numpy as np

from quail_amd import _host, layout

_answer_sink = None


def set_answer_sink(sink):
    """Install the callable evict events go to (quail/progress.py:70-86)."""
    global _answer_sink
    _answer_sink = sink


def answer_sink():
    return _answer_sink


def evict_event(key, prefix_tokens):
    """The answer-sink entry for an evicted (alias, document) key, or None for
    any other key (the event format of arena.py:279-294)."""
    if not (isinstance(key, tuple) and len(key) == 2 and isinstance(key[0], str)):
        return None
    try:
        document = int(key[1])
    except (TypeError, ValueError):
        return None
    return {"kind": "evict", "alias": key[0], "document": document,
            "tokens": int(prefix_tokens)}


class TemporaryKey:
    """A temporary page set's key; the library chose its handle."""

    __slots__ = ("handle",)

    def __init__(self, handle):
        self.handle = int(handle)

    def __hash__(self):
        return hash(("temporary", self.handle))

    def __eq__(self, other):
        return isinstance(other, TemporaryKey) and other.handle == self.handle

    def __repr__(self):
        return f"TemporaryKey({self.handle})"


class _Keys:
    """Caller keys <-> library handles (positive; temporaries are negative).

    Handles are numbered from 1 and never reused, so a handle the library
    still mentions can never name another key; a key's entry is dropped by
    forget() once the library holds nothing under it."""

    def __init__(self):
        self._handles = {}
        self._keys = {}
        self._next = 1

    def handle(self, key):
        if isinstance(key, TemporaryKey):
            return key.handle
        h = self._handles.get(key)
        if h is None:
            h = self._next
            self._next += 1
            self._handles[key] = h
            self._keys[h] = key
        return h

    def forget(self, key):
        h = self._handles.pop(key, None)
        if h is not None:
            del self._keys[h]

    def __len__(self):
        return len(self._handles)

    def known(self, key):
        """The handle of a key seen before, else None."""
        if isinstance(key, TemporaryKey):
            return key.handle
        return self._handles.get(key)

    def key(self, handle):
        handle = int(handle)
        return TemporaryKey(handle) if handle < 0 else self._keys[handle]

    def handles(self, keys):
        return _host.i64([h for h in (self.known(k) for k in keys) if h is not None])


class _KeyView(Mapping):
    """Read-only mapping over the resident keys, one field each."""

    def __init__(self, arena, field):
        self._arena = arena
        self._field = field

    def __getitem__(self, key):
        if not self._arena._resident(key):
            raise KeyError(key)
        return self._field(key)

    def __iter__(self):
        return iter(self._arena._resident_keys())

    def __len__(self):
        return int(self._arena._stats()[6])

    def __contains__(self, key):
        return self._arena._resident(key)


class _FlagSet(Set):
    """Read-only set of resident keys whose info flag is set."""

    def __init__(self, arena, slot):
        self._arena = arena
        self._slot = slot

    def __contains__(self, key):
        return self._arena._resident(key) and bool(self._arena._info(key)[self._slot])

    def __iter__(self):
        return (k for k in self._arena._resident_keys() if self._arena._info(k)[self._slot])

    def __len__(self):
        return sum(1 for _ in self)


class PageArena:
    """Page accounting: a free-page stack and per-key page lists.

    A key may borrow the leading pages of a resident key's prefix; it reads
    them and never writes them (arena.py:34-40).
    """

    def __init__(self, n_pages: int, page_tokens: int):
        self._native = _host.Handle(_host.fn("qp_arena_new")(int(n_pages), int(page_tokens)),
                                    "qp_arena_delete")
        self._keys = _Keys()
        self.n_pages = int(n_pages)
        self.page_tokens = int(page_tokens)
        self.retention_policy = None
        self._retention_cap = None
        self._buf = np.empty(16, dtype=np.int64)

    # ---- native plumbing -------------------------------------------------

    def _call(self, name, *args):
        return _host.check(name, _host.fn(name)(self._native.ptr, *args))

    def _stats(self):
        self._call("qp_arena_stats", self._buf.ctypes.data)
        return self._buf

    def _resident(self, key):
        h = self._keys.known(key)
        return h is not None and bool(self._call("qp_arena_is_resident", h))

    def _info(self, key):
        out = np.empty(8, dtype=np.int64)
        self._call("qp_arena_key_info", self._require(key), out.ctypes.data)
        return out

    def _require(self, key):
        h = self._keys.known(key)
        if h is None or not self._call("qp_arena_is_resident", h):
            raise KeyError(key)
        return h

    def _list(self, name, *args, dtype=np.int32):
        """A variable-length list call: size it, then fill it."""
        f = _host.fn(name)
        n = _host.check(name, f(self._native.ptr, *args, None, 0))
        out = np.empty(n, dtype=dtype)
        if n:
            _host.check(name, f(self._native.ptr, *args, out.ctypes.data, n))
        return out

    def _resident_keys(self):
        return [self._keys.key(h) for h in self._list("qp_arena_resident_keys", dtype=np.int64)]

    # ---- the reference's accounting surface ----------------------------------

    def pages_needed(self, tokens: int) -> int:
        return -(-int(tokens) // self.page_tokens)

    def alloc(self, key, tokens: int, capacity_tokens=None, borrowed=()):
        """Own pages for a fresh key, or None when the free stack is short."""
        if self._resident(key):
            raise KeyError(f"{key!r} already resident")
        capacity = tokens if capacity_tokens is None else capacity_tokens
        b = _host.i32(list(borrowed))
        status = self._call("qp_arena_alloc", self._keys.handle(key), int(tokens), int(capacity),
                            _host.ptr(b), int(b.size))
        if status == _host.QP_NONE:
            return None
        return self.table_pages(key)[b.size:]

    def shared_pages(self, parent, shared: int, start: int = 0) -> list:
        """The parent's pages for its tokens [start, shared), whole pages."""
        h = self._keys.known(parent)
        if h is None:
            raise KeyError(f"borrow parent {parent!r} is not resident")
        return self._list("qp_arena_shared_pages", h, int(shared), int(start)).tolist()

    def drop_leading(self, key, pages: int) -> int:
        """Drop a key's first pages, borrowed ones first; returns pages freed."""
        return self._call("qp_arena_drop_leading", self._require(key), int(pages))

    def table_pages(self, key) -> list:
        """Pages a key's block table reads: borrowed first, then its own."""
        return self._list("qp_arena_table", self._require(key)).tolist()

    def table_pages_np(self, key):
        return self._list("qp_arena_table", self._require(key))

    def borrowed_tokens(self, key) -> int:
        return int(self._info(key)[1]) * self.page_tokens

    def release_pages(self, pages) -> int:
        p = _host.i32(list(pages))
        return self._call("qp_arena_release_pages", _host.ptr(p), int(p.size))

    def free_key(self, key) -> int:
        return self._call("qp_arena_free_now", self._require(key))

    def pin(self, key) -> None:
        self._call("qp_arena_pin", self._require(key))

    def forget(self, keys) -> None:
        """Drop the handles of `keys` that are no longer resident (freed or
        evicted): a finished stream calls this for its keys, so a long
        session's handle table holds only what the arena still holds."""
        for key in keys:
            if not isinstance(key, TemporaryKey) and not self._resident(key):
                self._keys.forget(key)

    def retain(self, key, priority=None) -> None:
        """Make a resident key evictable after its current use (arena.py:153-179).
        Priority: the given tuple, the policy's, or tokens per page the key
        alone holds."""
        h = self._require(key)
        if priority is None and self.retention_policy is not None:
            sole = self._call("qp_arena_sole_pages", h)
            priority = self.retention_policy.priority(key, int(self._info(key)[0]),
                                                      max(1, sole))
        if priority is None:
            self._call("qp_arena_retain", h, None, 0)
            return
        values = tuple(priority) if isinstance(priority, (tuple, list)) else (priority,)
        p = np.zeros(max(1, len(values)), dtype=np.float64)
        p[:len(values)] = values
        self._call("qp_arena_retain", h, p.ctypes.data, len(values))

    def configure_retention(self, policy, cap_pages: int) -> None:
        if not 0 <= cap_pages <= self.n_pages:
            raise ValueError("retention capacity must fit inside the arena")
        self.retention_policy = policy
        self.retention_cap_pages = cap_pages
        keys = [self._keys.key(h) for h in self._list("qp_arena_retained_keys", dtype=np.int64)]
        self._call("qp_arena_clear_retention")
        for key in keys:
            self.retain(key)

    def pop_retained_victim(self, keep=frozenset()):
        """Remove the retained key with the lowest priority, skipping `keep`."""
        k = self._keys.handles(keep)
        out = np.empty(3, dtype=np.int64)
        status = self._call("qp_arena_pop_victim", _host.ptr(k), int(k.size), out.ctypes.data)
        if status == _host.QP_NONE:
            return None
        return self._keys.key(out[0]), int(out[1]), int(out[2])

    def rewind(self, key, tokens: int) -> int:
        """Keep the first `tokens` and free the trailing own pages; a retained
        key is retained again at its new size."""
        was_retained = bool(self._info(key)[4])
        freed = self._call("qp_arena_rewind", self._require(key), int(tokens))
        if was_retained:
            self.retain(key)
        return freed

    def grow(self, key, capacity_tokens: int):
        """Own pages up to capacity_tokens; None when the free stack is short."""
        added = np.zeros(1, dtype=np.int64)
        status = self._call("qp_arena_grow", self._require(key), int(capacity_tokens),
                            added.ctypes.data)
        return None if status == _host.QP_NONE else int(added[0])

    def row_indices(self, key, tokens=None):
        """Arena rows of the key's first `tokens` tokens (all by default)."""
        n = int(self._info(key)[0]) if tokens is None else int(tokens)
        pages = self.table_pages_np(key).astype(np.int64)
        rows = (pages[:, None] * self.page_tokens
                + np.arange(self.page_tokens, dtype=np.int64)).reshape(-1)
        return rows[:n].tolist()

    # ---- views ------------------------------------------------------------------

    @property
    def free(self) -> list:
        """The free stack, bottom to top (pop() gives the next page)."""
        return self._list("qp_arena_free_list").tolist()

    @property
    def owned(self):
        return _KeyView(self, lambda k: self.table_pages(k)[int(self._info(k)[1]):])

    @property
    def borrowed(self):
        return _KeyView(self, lambda k: self.table_pages(k)[:int(self._info(k)[1])])

    @property
    def tokens(self):
        return _KeyView(self, lambda k: int(self._info(k)[0]))

    @property
    def pinned(self):
        return _FlagSet(self, 3)

    @property
    def retained(self):
        flags = _FlagSet(self, 4)
        return {k: int(self._info(k)[5]) for k in flags}

    @property
    def retention_cap_pages(self):
        return self._retention_cap

    @retention_cap_pages.setter
    def retention_cap_pages(self, pages):
        self._retention_cap = None if pages is None else int(pages)
        self._call("qp_arena_set_retention_cap", -1 if pages is None else int(pages))

    @property
    def free_pages(self) -> int:
        return int(self._stats()[2])

    @property
    def resident_tokens(self) -> int:
        return int(self._stats()[4])

    @property
    def retained_pages(self) -> int:
        return int(self._stats()[3])

    @property
    def retained_prefix_tokens(self) -> int:
        return int(self._stats()[5])


class KVArena:
    """Device K/V pools per layer plus the page accounting.

    The method surface is the reference's (arena.py:8-24) minus the sliding
    window, which only DiffusionGemma uses. `allocate=False` builds the
    accounting and row maps only (host-side tests and planning).
    """

    def __init__(self, n_layers: int, n_pages: int, page_tokens: int,
                 n_kv: int, d_head: int, dtype=None, device="cuda",
                 layer_kv=None, sliding_layers=(), sliding_window=0,
                 n_sliding_pages=0, allocate=True):
        import torch
        self.torch = torch
        if sliding_window or n_sliding_pages or tuple(sliding_layers):
            raise ValueError("quail_amd has no sliding-window pools")
        self.dtype = dtype or torch.bfloat16
        self.device = device
        shapes = ([(n_kv, d_head)] * n_layers if layer_kv is None
                  else [tuple(s) for s in layer_kv])
        if len(shapes) != n_layers:
            raise ValueError(f"layer_kv names {len(shapes)} layers, the arena "
                             f"has {n_layers}")
        self.shapes = shapes
        self.sliding_layers = frozenset()
        self.window = 0
        self.sliding = None
        self._allocate = allocate
        self._build(n_pages, page_tokens)
        self.reset_stats()

    def _build(self, n_pages, page_tokens):
        torch = self.torch
        self.accounting = PageArena(n_pages, page_tokens)
        self.k, self.v = [], []
        if self._allocate:
            for heads, dim in self.shapes:
                self.k.append(torch.empty(layout.k_pool_shape(n_pages, heads, dim, page_tokens),
                                          dtype=self.dtype, device=self.device))
                self.v.append(torch.empty(layout.v_pool_shape(n_pages, heads, dim, page_tokens),
                                          dtype=self.dtype, device=self.device))

    @property
    def native(self):
        """The library's arena object (for the native admission and packer)."""
        return self.accounting._native.ptr

    def handle(self, key):
        return self.accounting._keys.handle(key)

    def key_of(self, handle):
        return self.accounting._keys.key(handle)

    def _call(self, name, *args):
        return self.accounting._call(name, *args)

    def resize(self, n_pages: int, n_sliding_pages: int = 0, *,
               free_resident: bool = False) -> None:
        if n_sliding_pages:
            raise ValueError("quail_amd has no sliding-window pools")
        if free_resident:
            self.drop_holds()
            for key in self.resident_keys():
                self.free_key(key)
        if self.accounting._stats()[6]:
            raise RuntimeError("the arena holds keys; free them before resizing")
        if n_pages == self.n_pages:
            return
        page_tokens = self.page_tokens
        self.k = self.v = None
        self._build(n_pages, page_tokens)

    def reset_stats(self):
        self.evicted_keys = 0
        self.evicted_pages = 0
        self.evicted_prefix_tokens = 0

    def drain_evictions(self):
        """Account and report the evictions the library made since the last
        drain: stats, then one answer-sink event per (alias, document) key."""
        keys, tokens, pages = (np.empty(64, dtype=np.int64) for _ in range(3))
        evicted = []
        while True:
            n = self._call("qp_arena_drain_evictions", keys.ctypes.data, tokens.ctypes.data,
                           pages.ctypes.data, 64)
            for i in range(n):
                key = self.key_of(keys[i])
                evicted.append(key)
                self.evicted_keys += 1
                self.evicted_pages += int(pages[i])
                self.evicted_prefix_tokens += int(tokens[i])
                sink = answer_sink()
                event = evict_event(key, int(tokens[i])) if sink is not None else None
                if event is not None:
                    sink(event)
            if n < 64:
                return tuple(evicted)

    # ---- window API (no sliding layers in quail_amd) ----------------

    @property
    def has_sliding(self) -> bool:
        return False

    def origin(self, base_tokens: int) -> int:
        return 0

    def sliding_start(self, key) -> int:
        return 0

    def keep_window(self, key, shared: int) -> None:
        return None

    def trim_window(self, key) -> int:
        return 0

    # ---- allocation ---------------------------------------------------

    def alloc(self, key, tokens: int, capacity_tokens=None, base_tokens=None,
              sliding_tokens=None, borrow=None):
        borrowed = () if borrow is None else self.accounting.shared_pages(*borrow)
        return self.accounting.alloc(key, tokens, capacity_tokens, borrowed=borrowed)

    def can_borrow(self, parent, shared: int) -> bool:
        h = self.accounting._keys.known(parent)
        return (h is not None and bool(self._call("qp_arena_is_resident", h))
                and shared <= int(self.accounting._info(parent)[0]))

    def pin(self, key):
        self.accounting.pin(key)

    def retain(self, key, tokens: int, priority=None):
        """Rewind a prefix and keep it evictable for a later operator
        (arena.py:541-564); evicts down to the retention cap."""
        if not (isinstance(key, tuple) and len(key) == 2):
            raise TypeError(f"retained keys are (alias, document) pairs, got {key!r}")
        self.accounting.rewind(key, tokens)
        self.accounting.retain(key, priority)
        cap = self.accounting.retention_cap_pages
        before = self.free_pages
        if cap is not None:
            self.evict_retained(max(0, self.accounting.retained_pages - cap))
        return self.free_pages - before

    def evict_retained(self, pages_needed: int) -> tuple:
        self._call("qp_arena_evict_retained", int(pages_needed))
        return self.drain_evictions()

    def evict_key(self, key):
        pages = self._call("qp_arena_evict_key", self.accounting._require(key))
        self.drain_evictions()
        return pages

    def activate(self, key, tokens: int, capacity_tokens=None, base_tokens=None,
                 borrow=None):
        """Make a prefix active, evicting retained KV when required (arena.py:617-658).
        Returns the key's pages, or None when they do not fit."""
        capacity = tokens if capacity_tokens is None else capacity_tokens
        parent, shared = (0, 0)
        if borrow is not None and borrow[1]:
            parent = self.accounting._keys.known(borrow[0])
            if parent is None:
                raise KeyError(f"borrow parent {borrow[0]!r} is not resident")
            shared = int(borrow[1])
        status = self._call("qp_arena_activate", self.handle(key), int(tokens), int(capacity),
                            parent, shared)
        self.drain_evictions()
        if status == _host.QP_NONE:
            return None
        return self.accounting.table_pages(key)

    def alloc_temporary(self, tokens: int, sliding_tokens=None):
        out = np.zeros(1, dtype=np.int64)
        status = self._call("qp_arena_alloc_temporary", int(tokens), out.ctypes.data)
        if status == _host.QP_NONE:
            return None
        key = TemporaryKey(out[0])
        return key, self.accounting.table_pages(key)

    # ---- holds ----------------------------------------------------------

    def hold(self, key, borrowers: int) -> None:
        if borrowers:
            self._call("qp_arena_hold", self.accounting._require(key), int(borrowers))

    def release(self, key) -> None:
        h = self.accounting._keys.known(key)
        if h is not None:
            self._call("qp_arena_release", h)

    def drop_holds(self, keys=None) -> bool:
        if keys is None:
            return bool(self._call("qp_arena_drop_holds", None, 0, 1))
        k = self.accounting._keys.handles(keys)
        return bool(self._call("qp_arena_drop_holds", _host.ptr(k), int(k.size), 0))

    def free_key(self, key):
        """Free a key's pages now, or once its last hold is released."""
        return self._call("qp_arena_free_key", self.accounting._require(key))

    def forget(self, keys) -> None:
        """Drop the key handles of `keys` the arena no longer holds."""
        self.accounting.forget(keys)

    # ---- residency --------------------------------------------------------

    @property
    def page_tokens(self) -> int:
        return self.accounting.page_tokens

    @property
    def n_pages(self) -> int:
        return self.accounting.n_pages

    @property
    def n_sliding_pages(self) -> int:
        return 0

    @property
    def free_pages(self) -> int:
        return self.accounting.free_pages

    def page_cost(self, tokens: int, base_tokens=None) -> int:
        return self.accounting.pages_needed(tokens)

    def held_cost(self, key) -> int:
        info = self.accounting._info(key)
        return int(info[2] - info[1])

    def growth_cost(self, key, capacity_tokens: int) -> int:
        return max(0, self.accounting.pages_needed(capacity_tokens)
                   - int(self.accounting._info(key)[2]))

    @property
    def retained_pages(self) -> int:
        return self.accounting.retained_pages

    @property
    def retained_prefix_tokens(self) -> int:
        return self.accounting.retained_prefix_tokens

    @property
    def retention_cap_pages(self):
        return self.accounting.retention_cap_pages

    @retention_cap_pages.setter
    def retention_cap_pages(self, pages) -> None:
        self.accounting.retention_cap_pages = pages

    def pages_needed(self, tokens: int) -> int:
        return self.accounting.pages_needed(tokens)

    def configure_retention(self, policy, cap_pages: int) -> None:
        self.accounting.configure_retention(policy, cap_pages)

    def is_resident(self, key) -> bool:
        return self.accounting._resident(key)

    def resident_keys(self) -> list:
        return self.accounting._resident_keys()

    def retained_keys(self) -> list:
        return list(self.accounting.retained)

    def owned_pages(self, key) -> list:
        return self.accounting.table_pages(key)

    def capacity_rows_np(self, key):
        """int64 numpy rows of every page in the key's table (host)."""
        pages = self.accounting.table_pages_np(key).astype(np.int64)
        return (pages[:, None] * self.page_tokens
                + np.arange(self.page_tokens, dtype=np.int64)).reshape(-1)

    def capacity_rows(self, key):
        """Row index tensor (CPU) over every row in the key's pages."""
        return self.torch.from_numpy(self.capacity_rows_np(key))

    # ---- tensors for the kernels -----------------------------------------

    def page_pools(self, layer: int):
        """K and V pools of one layer in the MI355X page layout: K [P, n_kv,
        16, d], V [P, n_kv, d, 16]. The kernels take these."""
        return self.k[layer], self.v[layer]

    def layer_kv(self, layer: int):
        """K and V of one layer addressed by the reference's flat arena rows
        (arena.py:851-855): row page * 16 + slot holds [n_kv, d]. No flat
        view of the MI355X pools exists, so these are row-indexed pools
        (layout.RowPool): indexing reads rows, assignment writes them into
        the pages. The kernels take page_pools()."""
        k, v = self.paged_kv(layer)
        return layout.RowPool(k), layout.RowPool(v)

    def paged_kv(self, layer: int):
        """K and V as the reference's (n_pages, 16, n_kv, d) paged views
        (arena.py:857-859): strided views of the MI355X pools, so element
        [p, s, h, d] is the same value the reference's view holds."""
        return (layout.k_paged_view(self.k[layer]), layout.v_paged_view(self.v[layer]))

    def block_table(self, keys, pad_to=None):
        """Block table and token counts of the keys (arena.py:861-872)."""
        table = self.block_table_rows([self.accounting.table_pages(k) for k in keys],
                                      pad_to=pad_to)
        used = self.torch.tensor([int(self.accounting._info(k)[0]) for k in keys],
                                 dtype=self.torch.int32)
        return table, used

    @staticmethod
    def block_table_np(pages, pad_to=None):
        """int32 [len(pages), width] table, zero-padded (arena.py:874-887)."""
        width = max((len(p) for p in pages), default=0)
        if pad_to:
            width = max(width, pad_to)
        table = np.zeros((len(pages), width), dtype=np.int32)
        for row, p in enumerate(pages):
            table[row, :len(p)] = p
        return table

    def block_table_rows(self, pages, pad_to=None):
        return self.torch.from_numpy(self.block_table_np(pages, pad_to))
