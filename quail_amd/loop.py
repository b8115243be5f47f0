"""Chunk packing and the overlapped filter and join loops.

Admission, page activation and the chunk's integer arrays are built by
libquail_host.so (quail_amd/host); this module moves them to the GPU and
drives the forward passes. The arrays are bit-exact with the reference's
pack_chunk (quail/backends/quail/executor/loop.py:219-577) and the loops
make the reference's decisions in the reference's order (loop.py:609-976,
:1195-1559): the previous chunk's answers are read while the current one
runs, pages are freed on a FALSE or after the last stage, and a filter's
held survivors can stream into a join as resident anchors.

Every array of a chunk reaches the GPU in one pinned H2D copy (Stager).
"""

import logging
import time

import numpy as np

from quail_amd import _host
from quail_amd._host import ArenaFullError
from quail_amd.pack import FilterAdmission, JoinAdmission, partner_pages
from quail_amd.tokens import token_array, token_parts

logger = logging.getLogger(__name__)

ATTENTION_PATHS = ("unified", "tree")

# the chunk builder's arrays, in its id order (include/quail_host.h)
ARRAY_NAMES = ("input_ids", "positions", "finals", "cu_a", "a_len", "a_read", "kv_src",
               "kv_dst", "reads_rows", "reads_cu_q", "reads_used", "reads_table",
               "reads_source", "unified_src", "unified_dst", "unified_used", "unified_table",
               "unified_cu_q", "tail_src", "tail_dst", "unified_row_dst")
_WIDE = {"input_ids", "positions", "finals", "kv_src", "kv_dst", "reads_rows", "unified_src",
         "unified_dst", "tail_src", "tail_dst", "unified_row_dst"}
_TABLES = {"reads_table", "unified_table"}

__all__ = ["ArenaFullError", "Chunk", "FilterStream", "pack_chunk", "run_filter", "run_join",
           "attention_path", "Stager", "TokenTable", "ChunkBuilder"]


class Chunk:
    """One packed forward pass (attention.py:45-72)."""

    __slots__ = ("input_ids", "positions", "final_indices", "meta",
                 "attention_mode", "tokens", "layout", "temporary_keys",
                 "fresh_keys", "host")

    def __init__(self, input_ids, positions, final_indices, meta, attention_mode,
                 tokens, layout, temporary_keys=(), fresh_keys=(), host=None):
        self.input_ids = input_ids
        self.positions = positions
        self.final_indices = final_indices
        self.meta = meta
        self.attention_mode = attention_mode
        self.tokens = tokens
        self.layout = layout
        self.temporary_keys = temporary_keys
        self.fresh_keys = fresh_keys
        self.host = host   # numpy copies of every staged array, by name


class _Clock:
    """Host seconds per phase of the loop, into a caller's dict."""

    def __init__(self, timing):
        self.timing = timing
        self.t = time.perf_counter() if timing is not None else 0.0

    def lap(self, key):
        if self.timing is None:
            return
        now = time.perf_counter()
        self.timing[key] = self.timing.get(key, 0.0) + now - self.t
        self.t = now


class TokenTable:
    """Token sequences the native packer reads in place (numpy arrays,
    memory-mapped Arrow views, chains of them); one entry per sequence."""

    def __init__(self, sequences=()):
        self._native = _host.Handle(_host.fn("qp_tokens_new")(), "qp_tokens_delete")
        self._keep = []
        self._lengths = []
        self.extend(sequences)

    def extend(self, sequences):
        """Add many sequences at once over one flat buffer: the one a source
        with flat_tokens() (RowPrompts, TokenStore) already holds, else one
        int64 copy."""
        if hasattr(sequences, "flat_tokens"):
            flat, offsets = sequences.flat_tokens()
            if flat.dtype not in (np.int32, np.int64) or not flat.flags.c_contiguous:
                flat = np.ascontiguousarray(flat, dtype=np.int64)
            offsets = np.ascontiguousarray(offsets, dtype=np.int64)
            lengths = np.diff(offsets)
        else:
            arrays = [token_array(seq) for seq in sequences]
            lengths = np.fromiter((a.size for a in arrays), dtype=np.int64, count=len(arrays))
            flat = np.concatenate(arrays).astype(np.int64, copy=False) if lengths.sum() else \
                np.zeros(1, dtype=np.int64)
            offsets = np.zeros(len(arrays) + 1, dtype=np.int64)
            np.cumsum(lengths, out=offsets[1:])
        if not lengths.size:
            return
        if not flat.size:
            flat = np.zeros(1, dtype=flat.dtype)
        self._keep.append((flat, offsets))
        _host.call("qp_tokens_add_flat", self._native.ptr, flat.ctypes.data, flat.itemsize,
                   lengths.size, offsets.ctypes.data)
        self._lengths.extend(lengths.tolist())

    @property
    def native(self):
        return self._native.ptr

    def __len__(self):
        return len(self._lengths)

    def length(self, entry):
        return self._lengths[entry]

    def add(self, seq):
        parts = []
        for part in token_parts(seq):
            if part.dtype not in (np.int32, np.int64) or not part.flags.c_contiguous:
                part = np.ascontiguousarray(part, dtype=np.int64)
            parts.append(part)
        self._keep.append(parts)
        ptrs = np.array([p.ctypes.data for p in parts], dtype=np.uint64)
        lens = np.array([p.size for p in parts], dtype=np.int64)
        elem = np.array([p.itemsize for p in parts], dtype=np.int32)
        entry = _host.call("qp_tokens_add", self._native.ptr, _host.ptr(ptrs), _host.ptr(lens),
                           _host.ptr(elem), len(parts))
        self._lengths.append(int(lens.sum()))
        return entry


class ChunkBuilder:
    """The native chunk builder (pack_chunk's arrays, loop.py:219-577)."""

    def __init__(self):
        self._native = _host.Handle(_host.fn("qp_chunk_new")(), "qp_chunk_delete")
        self._summary = np.empty(16, dtype=np.int64)
        self._arrays = np.empty(4 * _host.CHUNK_ARRAYS, dtype=np.int64)
        self._offsets = np.empty(_host.CHUNK_ARRAYS, dtype=np.int64)

    @property
    def native(self):
        return self._native.ptr

    def reset(self):
        _host.call("qp_chunk_reset", self._native.ptr)

    def add_group(self, key, fresh, start, f, write_suffix_tokens, prefix, suffixes,
                  read_key=None):
        """prefix: (table, entry, skip) or None; suffixes: (table, entries)."""
        table, entries = suffixes
        idx = _host.i32(entries)
        p_table, p_entry, p_skip = prefix if prefix is not None else (None, 0, 0)
        _host.call("qp_chunk_add_group", self._native.ptr, int(key),
                   0 if read_key is None else int(read_key), int(read_key is not None),
                   int(bool(fresh)), int(start), int(f), int(write_suffix_tokens),
                   None if p_table is None else p_table.native, int(p_entry), int(p_skip),
                   table.native if table is not None else None, _host.ptr(idx), int(idx.size))

    def build(self, arena, tree_path):
        _host.call("qp_chunk_build", self._native.ptr, arena.native, int(bool(tree_path)))

    def summary(self):
        _host.call("qp_chunk_summary", self._native.ptr, self._summary.ctypes.data)
        return self._summary

    def handles(self, name):
        f = _host.fn(name)
        n = _host.check(name, f(self._native.ptr, None, 0))
        out = np.empty(n, dtype=np.int64)
        if n:
            _host.check(name, f(self._native.ptr, out.ctypes.data, n))
        return out

    def host_arrays(self):
        """Every built array, copied out of the chunk builder: {name: ndarray}, and
        the one buffer they all live in (16-byte aligned slots)."""
        _host.call("qp_chunk_arrays", self._native.ptr, self._arrays.ctypes.data)
        total = _host.call("qp_chunk_emit", self._native.ptr, None, 0,
                           self._offsets.ctypes.data)
        buf = np.empty(max(total, 16), dtype=np.uint8)
        _host.call("qp_chunk_emit", self._native.ptr, buf.ctypes.data, buf.size,
                   self._offsets.ctypes.data)
        arrays, layout = {}, {}
        for i, name in enumerate(ARRAY_NAMES):
            present, count, rows, cols = (int(v) for v in self._arrays[4 * i:4 * i + 4])
            if not present:
                continue
            dtype = np.int64 if name in _WIDE else np.int32
            off = int(self._offsets[i])
            a = buf[off:off + count * np.dtype(dtype).itemsize].view(dtype)
            shape = (rows, cols) if name in _TABLES else (count,)
            arrays[name] = a.reshape(shape)
            layout[name] = (off, dtype, shape)
        return arrays, layout, buf


class Stager:
    """Moves a chunk's host buffer to the GPU in one copy.

    Two pinned host buffers alternate; before one is rewritten, the copy
    that last read it is waited on (the reference's InputStaging guard,
    loop.py:74-86). The device buffer is reused in stream order. On a CPU
    device the arrays become CPU tensors over the host buffer itself.
    """

    def __init__(self, torch, device):
        self.torch = torch
        self.device = torch.device(device)
        self.cuda = self.device.type == "cuda"
        self._pinned = [None, None]
        self._events = [None, None]
        self._dev = None
        self._turn = 0

    def stage(self, buf, layout):
        """{name: (offset, dtype, shape)} over buf -> {name: tensor on the device}."""
        torch = self.torch
        if not self.cuda:
            t = torch.from_numpy(buf)
            return {name: t[off:off + int(np.prod(shape)) * np.dtype(dt).itemsize]
                    .view(_TORCH[np.dtype(dt)]).view(*shape)
                    for name, (off, dt, shape) in layout.items()}
        total = buf.size
        slot = self._turn
        self._turn ^= 1
        if self._events[slot] is not None:
            self._events[slot].synchronize()
        host = self._pinned[slot]
        if host is None or host.numel() < total:
            host = torch.empty(max(total, 1 << 20), dtype=torch.uint8, pin_memory=True)
            self._pinned[slot] = host
        host.numpy()[:total] = buf
        if self._dev is None or self._dev.numel() < total:
            self._dev = torch.empty(max(total, 1 << 20), dtype=torch.uint8, device=self.device)
        dev = self._dev
        dev[:total].copy_(host[:total], non_blocking=True)
        event = torch.cuda.Event()
        event.record()
        self._events[slot] = event
        return {name: dev[off:off + int(np.prod(shape)) * np.dtype(dt).itemsize]
                .view(_TORCH[np.dtype(dt)]).view(*shape)
                for name, (off, dt, shape) in layout.items()}


_TORCH = {}


def _torch_dtypes():
    if not _TORCH:
        import torch
        _TORCH.update({np.dtype(np.int64): torch.int64, np.dtype(np.int32): torch.int32})


def _chunk(torch, arena, builder, mode, staging, layout_groups, device=None):
    """The built arrays staged to the device, as a Chunk with the reference's
    meta schema (loop.py:392-408, :507-512) plus a_read and work counts."""
    _torch_dtypes()
    s = builder.summary()
    (tokens, max_a, has_reads, r_max_q, r_max_used, r_rows, has_uni, u_max_q, u_max_used,
     own_pairs, uni_pairs, uni_kv, read_pairs, read_kv, n_temp, n_fresh) = (int(v) for v in s)
    host, layout, buf = builder.host_arrays()
    if staging is None:
        staging = Stager(torch, device if device is not None else arena.device)
    dev = staging.stage(buf, layout)
    temporaries = tuple(arena.key_of(h) for h in builder.handles("qp_chunk_temporaries"))
    fresh = tuple(arena.key_of(h) for h in builder.handles("qp_chunk_fresh_keys"))
    reads = None
    if has_reads:
        reads = dict(rows=dev["reads_rows"], cu_q=dev["reads_cu_q"], used=dev["reads_used"],
                     table=dev["reads_table"], source=dev["reads_source"], max_q=r_max_q,
                     max_used=r_max_used, n_rows=r_rows)
    unified = None
    if has_uni:
        unified = dict(src=dev["unified_src"], dst=dev["unified_dst"],
                       row_dst=dev.get("unified_row_dst"), tail_src=dev.get("tail_src"),
                       tail_dst=dev.get("tail_dst"), used=dev["unified_used"],
                       table=dev["unified_table"], cu_q=dev["unified_cu_q"],
                       max_used=u_max_used, max_q=u_max_q)
    work = {"own_pairs": own_pairs}
    if has_uni:
        work.update(unified_pairs=uni_pairs, unified_kv_rows=uni_kv)
    if has_reads:
        work.update(read_pairs=read_pairs, read_kv_rows=read_kv)
    meta = dict(layer=0, kv_src=dev.get("kv_src"), kv_dst=dev.get("kv_dst"),
                a_read=dev.get("a_read"), work=work, reads=reads, unified=unified,
                canvas=None, cu_a=dev["cu_a"], a_len=dev["a_len"], max_a=max_a)
    return Chunk(input_ids=dev["input_ids"], positions=dev["positions"],
                 final_indices=dev["finals"], meta=meta, attention_mode=mode, tokens=tokens,
                 layout=layout_groups, temporary_keys=temporaries, fresh_keys=fresh, host=host)


def pack_chunk(torch, arena, groups, timing=None, pinned=True, *, attention_mode,
               staging=None, canvas=(), answer_row=0, device=None):
    """Build one chunk's tensors from groups in chunk order (loop.py:219-577).

    Each group is a dict: key, prefix (fresh token ids or None), start
    (logical position of the first fresh token; pages before it are
    borrowed), read_key (tree path: the parent the fresh rows read),
    f (kept-context length; suffix positions start there), suffixes (token
    id lists), write_suffix_tokens (leading rows of the first suffix kept in
    the key's pages after the prefix).
    """
    if attention_mode not in ATTENTION_PATHS:
        raise ValueError(f"attention_mode must be one of {ATTENTION_PATHS}, "
                         f"got {attention_mode!r}")
    if tuple(canvas):
        raise ValueError("canvas rows belong to diffusion models, which quail_amd does not run")
    clock = _Clock(timing)
    tokens = TokenTable()
    builder = ChunkBuilder()
    layout = []
    for g in groups:
        fresh = g.get("prefix") is not None
        prefix = (tokens, tokens.add(g["prefix"]), 0) if fresh else None
        entries = [tokens.add(s) for s in g["suffixes"]]
        read_key = g.get("read_key")
        builder.add_group(arena.handle(g["key"]), fresh, g.get("start", 0), g["f"],
                          g.get("write_suffix_tokens", 0), prefix, (tokens, entries),
                          read_key=None if read_key is None else arena.handle(read_key))
        layout.append((g["key"], len(g["suffixes"])))
    clock.lap("pack_py")
    builder.build(arena, attention_mode == "tree")
    clock.lap("pack_build")
    chunk = _chunk(torch, arena, builder, attention_mode, staging, layout, device)
    clock.lap("pack_h2d")
    return chunk


def attention_path(pipeline, requested, default="unified") -> str:
    """The path a filter runs: the plan's request where the model has it (loop.py:580-590)."""
    requested = default if requested is None else requested
    return "tree" if requested == "tree" and pipeline.tree_attention else "unified"


def _forward(pipeline, arena, chunk):
    """Run the forward pass, then free the chunk's temporary pages (loop.py:593-604)."""
    try:
        return pipeline.forward_chunk(chunk)
    finally:
        keys, chunk.temporary_keys = chunk.temporary_keys, ()
        for key in keys:
            arena.free_key(key)


def shared_preamble(question_ids):
    """Tokens every stage's question starts with (loop.py:1157-1165); 0 for one stage."""
    if len(question_ids) < 2:
        return 0
    n = min(len(q) for q in question_ids)
    first = np.asarray(question_ids[0][:n])
    same = np.ones(n, dtype=bool)
    for q in question_ids[1:]:
        same &= np.asarray(q[:n]) == first
    mismatch = np.flatnonzero(~same)
    return int(mismatch[0]) if mismatch.size else n


class FilterStream:
    """The filter chain, one chunk per next() call (loop.py:1195-1532).

    Continuous admission with survivor priority; pages freed on FALSE or
    after the last stage. The previous chunk's answers are read while the
    current chunk runs. Admission, page activation and packing happen in
    one native call per chunk.
    """

    def __init__(self, torch, arena, pipeline, async_ans, doc_ids, question_ids,
                 budget, timing=None, pinned=True, limit=None, *, arena_writes,
                 arena_keys=None, retain_survivors=(), hold_survivors=False,
                 hold_extra_tokens=0, attention_mode=None, document_done=None,
                 prefix_tree=None, spans=None):
        keys = list(range(len(doc_ids))) if arena_keys is None else list(arena_keys)
        if len(keys) != len(doc_ids):
            raise ValueError("arena_keys must match doc_ids")
        self.retain_all = retain_survivors is True
        self.retain = set() if self.retain_all else set(retain_survivors)
        if hold_survivors and (self.retain_all or self.retain):
            raise ValueError("held survivors are pinned, not retained")
        arena_writes = bool(arena_writes or getattr(pipeline, "needs_pages", False))
        # stage 0 asks its whole question; later stages continue after the
        # preamble all questions share, kept in the document's pages
        p = shared_preamble(question_ids)
        self.tails = [list(question_ids[0])] + [list(q[p:]) for q in question_ids[1:]]
        for i, tail in enumerate(self.tails):
            if not tail:
                raise ValueError(f"stage {i} question has no tokens beyond the "
                                 f"shared preamble ({p} tokens)")
        if not arena_writes and (len(question_ids) > 1 or self.retain_all or self.retain
                                 or hold_survivors):
            raise ValueError("arena_writes=False needs a single stage")
        self.attention_mode = attention_path(pipeline, attention_mode)
        unified = self.attention_mode == "unified"
        if prefix_tree is not None and not prefix_tree.shared_tokens:
            prefix_tree = None
        if prefix_tree is not None and not arena_writes:
            raise ValueError("a prefix tree needs arena writes")
        # pages a document keeps: the preamble, and on the unified path room
        # for the longest later question's rows
        extra = p + (max(0, *(len(q) - p for q in question_ids)) if unified and arena_writes
                     else 0)
        if hold_survivors:
            extra = max(extra, hold_extra_tokens)
        if arena.retention_cap_pages is None:
            arena.retention_cap_pages = max(0, arena.n_pages - arena.pages_needed(2 * budget))
        self.docs = TokenTable(doc_ids)
        self.tail_table = TokenTable(self.tails)
        self.sched = FilterAdmission(
            [self.docs.length(i) for i in range(len(doc_ids))],
            [len(t) for t in self.tails], budget,
            arena_pages=arena.n_pages if arena_writes else None,
            page_tokens=arena.page_tokens, kept_extra_tokens=extra, limit=limit,
            tree=prefix_tree)
        self.sched.bind_arena(arena, keys)
        self.builder = ChunkBuilder()
        borrowers = self.sched.borrowing.borrowers()
        self._parents = [keys[d] for d, n in enumerate(borrowers) if n]
        self.torch, self.arena, self.pipeline = torch, arena, pipeline
        self.async_ans = async_ans
        self.doc_ids, self.keys = doc_ids, keys
        self.timing, self.pinned = timing, pinned
        self.arena_writes = arena_writes
        self.hold = hold_survivors
        self.preamble = p
        self.capacity_extra = extra
        self.tree = prefix_tree
        self.spans = [] if spans is None else spans
        self.tokens = 0
        self.chunks = 0
        self.done = False
        self.outstanding = []
        self.document_done = document_done
        self.staging = None
        self.reserve_pages = 0
        self.packed_groups = []   # per chunk, the groups it ran (for checkers)

    @property
    def answers(self):
        return self.sched.answers

    def set_reserve(self, pages):
        """Keep `pages` free for a join consumer's partner rows (loop.py:1361-1374)."""
        for doc in range(len(self.doc_ids)):
            need = self.arena.page_cost(self.docs.length(doc) + self.capacity_extra)
            if need + pages > self.arena.n_pages:
                raise ValueError(f"document {doc} needs more pages than the arena holds "
                                 f"beside the join's {pages} pages of partner rows")
        self.reserve_pages = pages

    def _report(self, entry, items):
        clock = _Clock(self.timing)
        groups, handle = entry
        bits = self.async_ans.result(handle)
        clock.lap("report_wait")
        last_stage = len(self.tails) - 1
        if not (self.retain_all or self.retain or self.hold):
            # nothing kept past its answer: one native call reports the chunk
            # and frees each finished document's pages in order
            self._report_chunk(groups, bits, last_stage)
            clock.lap("report_rest")
            return
        finished = []
        arena, sched = self.arena, self.sched
        for (doc, stage, _), bit in zip(groups, bits):
            passed = bool(bit)
            survivor = passed and stage == last_stage
            keep = survivor and (self.retain_all or doc in self.retain)
            hold = survivor and self.hold
            for d in sched.report(doc, stage, passed, release=not (keep or hold)):
                arena.free_key(self.keys[d])
            if keep:
                arena.retain(self.keys[doc], self.docs.length(doc))
            if hold:
                items.append((self.keys[doc], self.doc_ids[doc]))
            if not passed or stage == last_stage:
                finished.append((doc, stage, passed))
        if finished and self.document_done is not None:
            self.document_done(finished)
        clock.lap("report_rest")

    def _report_chunk(self, groups, bits, last_stage):
        n = len(groups)
        docs = np.fromiter((g[0] for g in groups), dtype=np.int32, count=n)
        stages = np.fromiter((g[1] for g in groups), dtype=np.int32, count=n)
        passed = (np.asarray(bits[:n]) != 0).astype(np.uint8)
        _host.call("qp_filter_report_chunk", self.sched.native,
                   self.arena.native if self.arena_writes else None, n, docs.ctypes.data,
                   stages.ctypes.data, passed.ctypes.data)
        answers = self.sched.answers
        for doc, ok in zip(docs.tolist(), passed.tolist()):
            answers.setdefault(doc, []).append(ok)
        if self.document_done is not None:
            done = (passed == 0) | (stages == last_stage)
            finished = [(int(d), int(st), bool(ok)) for d, st, ok, f
                        in zip(docs, stages, passed, done) if f]
            if finished:
                self.document_done(finished)

    def _finish(self, items):
        while self.outstanding:
            self._report(self.outstanding.pop(0), items)
        for doc in self.sched.drain_ready():
            self.arena.free_key(self.keys[doc])
        self.arena.drop_holds(self._parents)
        self.arena.forget(self.keys)
        self.done = True

    def _admit(self, items, evict_retained):
        """Groups of the next chunk, reading answers in flight or freeing pages
        until one fits; (None, blocked) when the stream ended or must wait for
        its held survivors to be consumed."""
        sched, arena = self.sched, self.arena
        while True:
            if sched.done():
                self._finish(items)
                return None, False
            free = (max(0, arena.free_pages - self.reserve_pages) if self.arena_writes
                    else None)
            clock = _Clock(self.timing)
            groups = sched.next_chunk(free)
            clock.lap("next_chunk")
            if groups:
                return groups, False
            if self.outstanding:
                self._report(self.outstanding.pop(0), items)
                continue
            short = sched.blocked_pages
            if short and (evict_retained or not self.hold) and arena.evict_retained(short):
                continue
            if self.hold and short and not evict_retained:
                return None, True
            # parents kept for queued children: let the children pack whole
            if arena.drop_holds(self._parents):
                continue
            if self.hold and short:
                return None, True
            raise AssertionError("nothing buildable and nothing in flight")

    def next(self, evict_retained=False):
        """Run one chunk; returns (held (key, prefix) pairs, blocked)."""
        items = []
        if self.done:
            return items, False
        groups, blocked = self._admit(items, evict_retained)
        if groups is None:
            return items, blocked
        clock = _Clock(self.timing)
        arena = self.arena
        sibling_order = self.tree is not None and self.attention_mode != "unified"
        _host.call("qp_filter_stage_chunk", self.sched.native, arena.native,
                   self.builder.native, self.docs.native, self.tail_table.native,
                   self.preamble, self.capacity_extra, int(self.attention_mode == "tree"),
                   int(sibling_order), int(self.arena_writes))
        arena.drain_evictions()
        groups = self.sched.chunk_groups()
        clock.lap("stage")
        if self.staging is None and str(getattr(arena, "device", "cpu")).startswith("cuda"):
            self.staging = Stager(self.torch, arena.device)
        layout = [(self.keys[doc], 1) for doc, _, _ in groups]
        chunk = _chunk(self.torch, arena, self.builder, self.attention_mode, self.staging,
                       layout)
        self.packed_groups.append(groups)
        clock.lap("h2d")
        self.tokens += chunk.tokens
        normed = _forward(self.pipeline, arena, chunk)
        clock.lap("forward_launch")
        self.outstanding.append((groups, self.async_ans.submit(normed)))
        self.chunks += 1
        clock.lap("submit")
        if self.timing is not None:
            self.timing["n_chunks"] = self.timing.get("n_chunks", 0) + 1
        while len(self.outstanding) > 1:
            self._report(self.outstanding.pop(0), items)
        return items, bool(self.hold and self.sched.blocked_pages)


def run_filter(torch, arena, pipeline, async_ans, doc_ids, question_ids, budget,
               timing=None, pinned=True, limit=None, *, arena_writes, arena_keys=None,
               retain_survivors=(), attention_mode=None, document_done=None,
               prefix_tree=None, stats=None):
    """The filter chain run to the end (loop.py:1535-1559).

    Returns (answers, spans, tokens): answers[d] is the 0/1 list up to the
    first FALSE.
    """
    stream = FilterStream(torch, arena, pipeline, async_ans, doc_ids, question_ids,
                          budget, timing=timing, pinned=pinned, limit=limit,
                          arena_writes=arena_writes, arena_keys=arena_keys,
                          retain_survivors=retain_survivors,
                          attention_mode=attention_mode, document_done=document_done,
                          prefix_tree=prefix_tree)
    while not stream.done:
        stream.next()
    if stats is not None:
        stats["borrowed_tokens"] = stream.sched.borrowing.borrowed_tokens
        stats["chunks"] = stream.chunks
    return stream.answers, stream.spans, stream.tokens


# ------------------------------------------------------------------ the join


class _Join:
    """One run_join call: the native join plan, the anchors' arena keys and
    token tables, and the chunks in flight (loop.py:609-956)."""

    def __init__(self, torch, arena, pipeline, async_ans, prefixes, keys, stage_suffixes,
                 budget, frames, anchor_done, source, anchor_partners, anchor_batch, staging,
                 mode, tree):
        self.torch, self.arena, self.pipeline = torch, arena, pipeline
        self.async_ans = async_ans
        self.prefixes, self.keys = prefixes, keys
        self.budget = budget
        self.frames = frames
        self.anchor_done = anchor_done
        self.source = source
        self.anchor_partners = anchor_partners
        self.anchor_batch = anchor_batch
        self.staging = staging
        self.mode = mode
        self.n_stages = len(stage_suffixes)
        # a frame entry's rows land in the anchor's pages after its document
        self.frame_max = max(len(f) for f in frames)
        self.spans, self.tokens = [], 0
        self.outstanding, self.packed_groups = [], []
        self.anchors = TokenTable(prefixes)
        self.frame_table = TokenTable(frames)
        self.partner_tables = [TokenTable(s) for s in stage_suffixes]
        self.builder = ChunkBuilder()
        resident = {a: self.held_pages(keys[a], self.anchors.length(a))
                    for a in range(len(keys)) if arena.is_resident(keys[a])}
        for a in resident:   # resident anchors stay for the whole join
            arena.pin(keys[a])
        self.sched = JoinAdmission(
            [self.anchors.length(a) for a in range(len(keys))],
            [[len(s) for s in sufs] for sufs in stage_suffixes], budget, arena.n_pages,
            arena.page_tokens, frame_tokens=[len(f) for f in frames], resident=resident,
            anchor_partners={a: self.partners_of(keys[a]) for a in range(len(keys))},
            temporary_suffix_pages=mode == "unified", answer_dtype=async_ans.dtype,
            tree=tree)
        self.sched.bind_arena(arena, keys)
        # counted after resident anchors detach: they borrow nothing
        self.borrowers = self.sched.borrowing.borrowers()
        self.tree_parent = self.sched.borrowing.tree_parent
        self.held = [keys[a] for a, n in enumerate(self.borrowers) if n]

    def partners_of(self, key):
        return None if self.anchor_partners is None else self.anchor_partners(key)

    def held_pages(self, key, prefix_tokens):
        """Pages a resident anchor already covers of what admission prices."""
        capacity = prefix_tokens + self.frame_max
        return self.arena.page_cost(capacity) - self.arena.growth_cost(key, capacity)

    # ---- streamed anchors ------------------------------------------------

    def take(self, items):
        """Anchors a source stream hands over, as (key, prefix) pairs with
        their KV already resident: those the batch filter keeps join the
        plan; the others' pages are freed at once."""
        if self.anchor_batch is not None and items:
            wanted = set(self.anchor_batch([key for key, _ in items]))
            dropped = [key for key, _ in items if key not in wanted]
            for key in dropped:
                if self.arena.is_resident(key):
                    self.arena.free_key(key)
            items = [item for item in items if item[0] in wanted]
        for key, prefix in items:
            self.register(key, prefix)

    def register(self, key, prefix):
        """One streamed anchor into the plan: pinned for the whole join, its
        held pages priced, its partner lists looked up by key."""
        if not self.arena.is_resident(key):
            raise ValueError(f"streamed anchor {key!r} has no KV in the arena")
        self.arena.pin(key)
        self.keys.append(key)
        self.prefixes.append(prefix)
        index = self.anchors.add(prefix)
        tokens = self.anchors.length(index)
        planned = self.sched.admit(tokens, self.held_pages(key, tokens),
                                   partners=self.partners_of(key))
        assert planned == index, "anchor index out of step with its token table"
        self.sched.set_key(index, self.arena.handle(key))

    def source_active(self):
        return self.source is not None and not self.source.done

    def feed(self, may_evict=False, at_least_once=False):
        """Let the anchor source run its chunks until the plan holds a full
        join chunk of work or the source has to wait; with at_least_once
        the source runs once even if the plan is full. Returns whether the
        source launched a chunk or handed over an anchor."""
        progressed = False
        first = at_least_once
        while self.source_active():
            if not first and self.sched.buildable_tokens() >= self.budget:
                break
            first = False
            launched = self.source.chunks
            items, waiting = self.source.next(evict_retained=may_evict)
            self.take(items)
            progressed = progressed or bool(items) or self.source.chunks != launched
            if waiting:
                break
        return progressed

    # ---- chunks ------------------------------------------------------------

    def entry_rows(self, a, j, start, end, carried):
        rows = self.anchors.length(a) if carried else 0
        rows += sum(self.partner_tables[j].length(i)
                    for i in self.sched.partner_indices(a, j, start, end))
        if self.frames[j] and start == 0:
            rows += len(self.frames[j])
        return rows

    def stage(self, groups):
        """Activate fresh anchors' pages and add every group's rows to the chunk builder."""
        arena, sched, b = self.arena, self.sched, self.builder
        borrowing = sched.borrowing
        b.reset()
        layout = []
        for a, j, start, end, carried in groups:
            key = self.keys[a]
            f = self.anchors.length(a)
            parent, shared = ((borrowing.parent(a), borrowing.shared(a)) if carried
                              else (None, 0))
            fresh = not arena.is_resident(key)
            got = arena.activate(key, f, capacity_tokens=f + self.frame_max, base_tokens=f,
                                 borrow=(self.keys[parent], shared) if shared else None)
            assert got is not None, "scheduler admitted an anchor the arena cannot hold"
            if fresh and a < len(self.borrowers) and self.borrowers[a]:
                arena.hold(key, self.borrowers[a])
            # a borrowing anchor's fresh rows read its borrowed pages through
            # its own key: join groups name no read key
            handle = arena.handle(key)
            prefix = (self.anchors, a, shared) if carried else None
            partners = (self.partner_tables[j], sched.partner_indices(a, j, start, end))
            frame = len(self.frames[j])
            if frame and start == 0:
                # frame entry: the frame is written into the anchor's KV after
                # its document (its answer row is read and discarded); the
                # partners then read document + frame
                b.add_group(handle, carried, shared, f, frame, prefix, (self.frame_table, [j]))
                b.add_group(handle, False, 0, f + frame, 0, None, partners)
                layout += [(key, 1), (key, len(partners[1]))]
            else:
                b.add_group(handle, carried, shared, f + frame, 0, prefix, partners)
                layout.append((key, len(partners[1])))
        return layout

    def launch(self, groups):
        """Run one admitted chunk. Admission prices the temporary pages of a
        chunk's partner rows, but the packer claims them a page at a time,
        so a chunk can still meet a full arena: then retained KV the size of
        the chunk's rows is evicted and the chunk tried again, or, with
        nothing left to evict, the chunk is split in two and the halves run
        in order (each may split again)."""
        stack = [list(groups)]
        while stack:
            part = stack.pop()
            try:
                self.run_one(part)
            except ArenaFullError as error:
                rows = sum(self.entry_rows(*g) for g in part)
                if self.arena.evict_retained(self.arena.page_cost(rows)):
                    logger.info("arena full for a join chunk of %d groups: retained KV "
                                "evicted, chunk retried", len(part))
                    stack.append(part)
                elif len(part) > 1:
                    logger.info("arena full for a join chunk of %d groups (%s): split "
                                "in two", len(part), error)
                    mid = len(part) // 2
                    stack.extend((part[mid:], part[:mid]))
                else:
                    raise

    def run_one(self, part):
        torch, arena = self.torch, self.arena
        if self.staging is None and str(getattr(arena, "device", "cpu")).startswith("cuda"):
            self.staging = Stager(torch, arena.device)
        layout = self.stage(part)
        self.builder.build(arena, self.mode == "tree")
        chunk = _chunk(torch, arena, self.builder, self.mode, self.staging, layout)
        self.packed_groups.append(list(part))
        self.tokens += chunk.tokens
        events = None
        if torch.cuda.is_available() and str(getattr(arena, "device", "")).startswith("cuda"):
            events = (torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
            events[0].record()
        normed = _forward(self.pipeline, arena, chunk)
        if events is not None:
            events[1].record()
        self.spans.append((part[0][1],) + (events or (None, None)))
        self.outstanding.append((part, self.async_ans.submit(normed)))
        # read the previous chunk's answers while this one runs
        while len(self.outstanding) > 1:
            self.report(self.outstanding.pop(0))

    # ---- answers -------------------------------------------------------------

    def event(self, kind, anchor):
        key = self.keys[anchor]
        if kind == "finished" and self.anchor_done is not None:
            self.anchor_done(anchor, self.sched.answers[self.n_stages - 1].get(anchor, []))
        elif self.arena.is_resident(key):
            self.arena.free_key(key)

    def report(self, entry):
        """Hand a finished chunk's answer rows to the plan, group by group. A
        frame entry (the first group of an anchor's stage) leads with the
        frame's own answer row, which answers nothing and is skipped."""
        groups, handle = entry
        bits = self.async_ans.result(handle)
        first = 0
        for a, j, start, end, _ in groups:
            if start == 0 and self.frames[j]:
                first += 1
            last = first + (end - start)
            for kind, anchor in self.sched.report(a, j, start, end, bits[first:last]):
                self.event(kind, anchor)
            first = last

    def run(self):
        """Launch chunks until the plan and the anchor source are both done."""
        while True:
            if self.source_active():
                self.feed()
            # anchors with no partner at a stage settle without a chunk
            for kind, anchor in self.sched.take_settled():
                self.event(kind, anchor)
            if self.sched.done() and not self.source_active():
                break
            groups = self.next_groups()
            if groups:
                self.launch(groups)
                self.release_parents(groups)
            elif not self.unstick():
                raise AssertionError("no join chunk can be built and none is in flight")
        while self.outstanding:
            self.report(self.outstanding.pop(0))
        self.arena.drop_holds(self.held)
        self.arena.forget(self.keys)

    def next_groups(self):
        """The next chunk's groups; a fresh anchor short of pages first has
        retained KV (which no anchor here reads) evicted for it."""
        if self.sched.blocked_pages:
            self.arena.evict_retained(self.sched.blocked_pages)
        return self.sched.next_chunk(self.arena.free_pages)

    def release_parents(self, groups):
        """A child packed whole of its borrowed pages now holds them itself,
        so its parent's hold for it ends."""
        parents = self.tree_parent
        for a, _, start, _, carried in groups:
            parent = parents[a] if a < len(parents) else None
            if carried and start == 0 and parent is not None:
                self.arena.release(self.keys[parent])

    def unstick(self):
        """No chunk could be built: free something, in this order, and say
        whether anything moved - read the oldest chunk in flight, let the
        source run (evicting retained KV for its documents), evict retained
        KV for the blocked anchor, or end the holds of parents kept for
        children that then pack their whole prefixes."""
        if self.outstanding:
            self.report(self.outstanding.pop(0))
            return True
        if self.source_active() and self.feed(may_evict=True, at_least_once=True):
            return True
        short = self.sched.blocked_pages
        if short and self.arena.evict_retained(short):
            return True
        return bool(self.arena.drop_holds(self.held))


def run_join(torch, arena, pipeline, async_ans, anchor_prefixes, stage_suffixes, budget,
             stage_frames=None, anchor_keys=None, anchor_done=None, anchor_source=None,
             anchor_partners=None, anchor_batch=None, staging=None, attention_mode=None,
             prefix_tree=None, stats=None):
    """The join driver: stream every anchor's partners, gating between stages
    (loop.py:609-976).

    Args follow the reference: anchor_prefixes[a] is anchor a's prefix ids
    (document, with any shared instruction); stage_suffixes[j] the partner
    suffix id lists of stage j; stage_frames[j] the framing ids written into
    the anchor's KV after its document; anchor_keys stable arena keys;
    anchor_done(a, row) owns a finished anchor's pages; anchor_source a
    stream (a FilterStream holding its survivors) that hands over resident
    anchors while the join runs; anchor_partners(key) per-stage partner
    index lists; anchor_batch(keys) filters streamed anchors; attention_mode
    "tree" (the default for joins) or "unified"; prefix_tree a PrefixTree
    over the anchors, so children borrow their parent's pages.

    Returns (answers, spans, tokens): answers[j][a] is anchor a's 0/1 row
    over its stage-j partners; spans (stage, start event, end event) per
    forward pass; tokens the fresh tokens packed.
    """
    k = len(stage_suffixes)
    if anchor_source is not None:
        if anchor_prefixes or anchor_keys:
            raise ValueError("anchor_source fills anchor_prefixes and anchor_keys")
        prefixes, keys = anchor_prefixes, anchor_keys
        if prefixes is None:
            prefixes = []
        if keys is None:
            keys = []
    else:
        prefixes = list(anchor_prefixes)
        keys = list(range(len(prefixes))) if anchor_keys is None else list(anchor_keys)
    if len(keys) != len(prefixes):
        raise ValueError("anchor_keys must match anchor_prefixes")
    if tuple(getattr(pipeline, "canvas_ids", ())):
        raise ValueError("canvas rows belong to diffusion models, which quail_amd does not run")
    frames = stage_frames or [[] for _ in range(k)]
    if k == 0:
        return [], [], 0
    # a join's partners read their anchor: tree unless the plan says otherwise
    mode = attention_path(pipeline, attention_mode, default="tree")
    if anchor_source is not None and mode == "unified":
        # leave room for one partner's temporary rows beside held anchors
        longest = [max((len(s) for s in sufs), default=0) for sufs in stage_suffixes]
        anchor_source.set_reserve(max(
            (partner_pages(arena.page_cost, arena.page_tokens, len(doc), len(frame), rows)
             for doc in anchor_source.doc_ids for frame, rows in zip(frames, longest)),
            default=0))
    if prefix_tree is not None and not prefix_tree.shared_tokens:
        prefix_tree = None
    join = _Join(torch, arena, pipeline, async_ans, prefixes, keys, stage_suffixes, budget,
                 frames, anchor_done, anchor_source, anchor_partners, anchor_batch, staging,
                 mode, prefix_tree)
    join.run()
    if stats is not None:
        stats["borrowed_tokens"] = join.sched.borrowing.borrowed_tokens
        stats["chunks"] = len(join.packed_groups)
    return join.sched.answers, join.spans, join.tokens
