"""Chunk packing and the overlapped filter loop.

pack_chunk turns admitted groups into one forward pass: token ids,
positions, answer rows and the attention bookkeeping (scatter maps, block
tables, sequence bounds). Its outputs are bit-exact restatements of the
reference's (quail/backends/quail/executor/loop.py:219-577), since the
kernels read KV through them; all integer work is numpy on the host, and
every array of a chunk reaches the GPU in one pinned H2D copy.

FilterStream / run_filter drive the filter: admit, activate pages, pack,
launch the forward pass, and read the previous chunk's answers while the
current one runs (loop.py:1195-1559). run_join drives a join the same way
over JoinAdmission's groups (loop.py:609-976).
"""

import logging
import time

import numpy as np

from quail_amd.pack import FilterAdmission, JoinAdmission, partner_pages

logger = logging.getLogger(__name__)

ATTENTION_PATHS = ("unified", "tree")


class ArenaFullError(RuntimeError):
    """A chunk's suffix pages do not fit the free KV arena (loop.py:30-31)."""


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


def _tick(timing, key, t0):
    if timing is not None:
        timing[key] = timing.get(key, 0.0) + time.perf_counter() - t0
    return time.perf_counter()


class Stager:
    """Packs a chunk's host arrays into one pinned buffer and one H2D copy.

    Two pinned host buffers alternate; before one is rewritten, the copy
    that last read it is waited on (the reference's InputStaging guard,
    loop.py:74-86). The device buffer is reused in stream order. On a CPU
    device the arrays become CPU tensors directly.
    """

    ALIGN = 16

    def __init__(self, torch, device):
        self.torch = torch
        self.device = torch.device(device)
        self.cuda = self.device.type == "cuda"
        self._host = [None, None]
        self._events = [None, None]
        self._dev = None
        self._turn = 0

    def stage(self, arrays):
        """{name: np.ndarray} -> {name: tensor on the device}."""
        torch = self.torch
        if not self.cuda:
            return {k: torch.from_numpy(np.ascontiguousarray(v)) for k, v in arrays.items()}
        offsets, total = {}, 0
        for name, arr in arrays.items():
            offsets[name] = total
            total += -(-arr.nbytes // self.ALIGN) * self.ALIGN
        total = max(total, self.ALIGN)
        slot = self._turn
        self._turn ^= 1
        host = self._host[slot]
        if self._events[slot] is not None:
            self._events[slot].synchronize()
        if host is None or host.numel() < total:
            host = torch.empty(max(total, 1 << 20), dtype=torch.uint8, pin_memory=True)
            self._host[slot] = host
        hnp = host.numpy()
        for name, arr in arrays.items():
            off = offsets[name]
            hnp[off:off + arr.nbytes] = np.ascontiguousarray(arr).view(np.uint8).reshape(-1)
        if self._dev is None or self._dev.numel() < total:
            self._dev = torch.empty(max(total, 1 << 20), dtype=torch.uint8, device=self.device)
            # a fresh device buffer: nothing queued reads the old one after this
        dev = self._dev
        dev[:total].copy_(host[:total], non_blocking=True)
        event = torch.cuda.Event()
        event.record()
        self._events[slot] = event
        out = {}
        for name, arr in arrays.items():
            off = offsets[name]
            dtype = _TORCH_DTYPE[arr.dtype.str]
            view = dev[off:off + arr.nbytes].view(dtype)
            out[name] = view.view(arr.shape) if arr.ndim != 1 else view
        return out


_TORCH_DTYPE = {}


def _init_dtypes():
    import torch
    _TORCH_DTYPE.update({np.dtype(np.int64).str: torch.int64,
                         np.dtype(np.int32).str: torch.int32})


def _cat(parts, dtype=np.int64):
    return np.concatenate(parts).astype(dtype, copy=False) if parts else np.empty(0, dtype)


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
        raise ValueError("canvas rows belong to diffusion models, not this build")
    if not _TORCH_DTYPE:
        _init_dtypes()
    t = time.perf_counter() if timing is not None else 0.0
    tree_path = attention_mode == "tree"
    page = arena.page_tokens
    id_parts, pos_parts = [], []
    token_count = 0
    cu_a, finals = [0], []
    reader_parts = []            # ranges of rows reading resident KV (call B)
    kv_writes, layout = [], []
    fresh_keys = []
    read_keys, read_used, cu_q = [], [], [0]
    max_q = 0
    unified_groups = []
    for g in groups:
        fresh = g.get("prefix") is not None
        f = g["f"]
        key = g["key"]
        start = g.get("start", 0)
        suffixes = g["suffixes"]
        paged = arena.is_resident(key)
        row0 = token_count
        borrowing = bool(fresh and start and tree_path)
        stacked = borrowing and len(suffixes) == 1 and g.get("read_key") is not None
        n_prefix = 0
        if fresh:
            if not paged and len(suffixes) > 1:
                raise ValueError(
                    f"group {key!r}: an unpaged fresh group packs [prefix | suffix] "
                    f"as one causal segment, which only one suffix may join")
            if start and not paged:
                raise ValueError(f"group {key!r}: a borrowed prefix needs arena pages")
            prefix = np.asarray(g["prefix"], dtype=np.int64)
            n_prefix = prefix.size
            id_parts.append(prefix)
            token_count += n_prefix
            pos_parts.append(np.arange(start, start + n_prefix, dtype=np.int64))
            if (paged or not suffixes) and not stacked:
                cu_a.append(token_count)
            if borrowing and not stacked:
                reader_parts.append((row0, token_count))
                cu_q.append(cu_q[-1] + token_count - row0)
                read_keys.append(key)
                read_used.append(start)
                max_q = max(max_q, token_count - row0)
            if paged and tree_path:
                kv_writes.append((key, row0, row0 + n_prefix, start))
                fresh_keys.append(key)
        prefix_end = token_count
        s_row0 = token_count
        suffix_spans = []
        for si, suf in enumerate(suffixes):
            srow = token_count
            suf = np.asarray(suf, dtype=np.int64)
            id_parts.append(suf)
            token_count += suf.size
            pos_parts.append(np.arange(f, f + suf.size, dtype=np.int64))
            finals.append(token_count - 1)
            suffix_spans.append((srow, token_count))
            cu_a.append(token_count)
            wst = g.get("write_suffix_tokens", 0)
            if si == 0 and wst and paged and tree_path:
                dest = start + n_prefix if fresh else f
                kv_writes.append((key, srow, srow + wst, dest))
        s_count = token_count - s_row0
        layout.append((key, len(suffixes)))
        if stacked:
            count = token_count - row0
            reader_parts.append((row0, token_count))
            read_key = g["read_key"]
            if read_keys and read_keys[-1] == read_key and read_used[-1] == start:
                cu_q[-1] += count
                max_q = max(max_q, cu_q[-1] - cu_q[-2])
            else:
                cu_q.append(cu_q[-1] + count)
                read_keys.append(read_key)
                read_used.append(start)
                max_q = max(max_q, count)
        elif s_count and f and paged and tree_path:
            reader_parts.append((s_row0, token_count))
            cu_q.append(cu_q[-1] + s_count)
            read_keys.append(key)
            read_used.append(f)
            max_q = max(max_q, s_count)
        if attention_mode == "unified":
            if paged:
                unified_groups.append((key, fresh, f, row0, start, prefix_end,
                                       token_count, suffix_spans))
            elif not fresh:
                raise ValueError("unified attention requires pages for a kept group")
    t = _tick(timing, "pack_py", t)

    arrays = {}
    host_ints = {}
    reads = None
    if read_keys:
        table = arena.block_table_np([arena.owned_pages(k) for k in read_keys])
        rows = _cat([np.arange(a, b, dtype=np.int64) for a, b in reader_parts])
        source = np.full(token_count, -1, dtype=np.int32)
        source[rows] = np.arange(rows.size, dtype=np.int32)
        arrays.update(reads_rows=rows, reads_cu_q=np.asarray(cu_q, dtype=np.int32),
                      reads_used=np.asarray(read_used, dtype=np.int32),
                      reads_table=table, reads_source=source)
        host_ints["reads"] = dict(max_q=max_q, max_used=max(read_used),
                                  n_rows=int(rows.size))
    if tree_path:
        # per causal segment, the read sequence all of its rows attend (or
        # -1): what lets one fused kernel run call A, call B and the merge
        arrays["a_read"] = _segment_reads(np.asarray(cu_a, dtype=np.int64), arrays)
    t = _tick(timing, "pack_reads", t)

    temporary_keys = []
    unified_host = None
    if attention_mode == "unified" and unified_groups:
        if len(unified_groups) != len(layout):
            raise ValueError("a unified chunk cannot mix paged and unpaged groups")
        src, dst, tail_src, tail_dst = [], [], [], []
        page_rows, lengths = [], []
        ucu = [0]
        try:
            for (key, fresh, f, r0, start, prefix_end, r1, spans) in unified_groups:
                logical_start = start if fresh else f
                if fresh:
                    fresh_keys.append(key)
                count = r1 - r0
                rows_np = arena.capacity_rows_np(key)
                pages = arena.owned_pages(key)
                direct = len(spans) == 1 and logical_start + count <= rows_np.size
                suffix_total = sum(e - s for s, e in spans)
                if direct:
                    src.append(np.arange(r0, r1, dtype=np.int64))
                    dst.append(rows_np[logical_start:logical_start + count])
                    page_rows.append(pages)
                    lengths.append(f + suffix_total)
                    ucu.append(ucu[-1] + count)
                    continue
                prefix_count = prefix_end - r0
                if prefix_count:
                    src.append(np.arange(r0, prefix_end, dtype=np.int64))
                    dst.append(rows_np[start:start + prefix_count])
                    page_rows.append(pages[:arena.pages_needed(f)])
                    lengths.append(f)
                    ucu.append(ucu[-1] + prefix_count)
                for s0, s1 in spans:
                    n_suffix = s1 - s0
                    remainder = f % page
                    got = arena.alloc_temporary(remainder + n_suffix)
                    if got is None:
                        raise ArenaFullError(
                            f"unified suffix pages exceed the free KV arena; split the "
                            f"chunk (asked {remainder + n_suffix} rows; free pages "
                            f"{arena.free_pages}; groups {len(groups)})")
                    temp_key, _ = got
                    temporary_keys.append(temp_key)
                    temp_rows = arena.capacity_rows_np(temp_key)
                    temp_pages = arena.owned_pages(temp_key)
                    src.append(np.arange(s0, s1, dtype=np.int64))
                    dst.append(temp_rows[remainder:remainder + n_suffix])
                    if remainder:
                        anchor = pages[f // page] * page
                        tail_src.append(np.arange(anchor, anchor + remainder, dtype=np.int64))
                        tail_dst.append(temp_rows[:remainder])
                    page_rows.append(pages[:f // page] + temp_pages)
                    lengths.append(f + n_suffix)
                    ucu.append(ucu[-1] + n_suffix)
        except Exception:
            for key in temporary_keys:
                arena.free_key(key)
            raise
        usrc, udst = _cat(src), _cat(dst)
        arrays.update(unified_src=usrc, unified_dst=udst,
                      unified_used=np.asarray(lengths, dtype=np.int32),
                      unified_table=arena.block_table_np(page_rows),
                      unified_cu_q=np.asarray(ucu, dtype=np.int32))
        if tail_src:
            arrays.update(tail_src=_cat(tail_src), tail_dst=_cat(tail_dst))
        # the arena row of every chunk row, when the scatter writes each row
        # exactly once (it does: every group's rows are emitted once): lets
        # the q/k norm + RoPE kernel write k and v into the arena itself
        if usrc.size == token_count:
            row_dst = np.full(token_count, -1, dtype=np.int64)
            row_dst[usrc] = udst
            if (row_dst >= 0).all():
                arrays["unified_row_dst"] = row_dst
        unified_host = dict(max_used=max(lengths),
                            max_q=max(b - a for a, b in zip(ucu, ucu[1:])))

    kv_src = kv_dst = None
    if kv_writes:
        srcs, dsts = [], []
        for key, r0, r1, dest in kv_writes:
            srcs.append(np.arange(r0, r1, dtype=np.int64))
            rows_np = arena.capacity_rows_np(key)[dest:dest + (r1 - r0)]
            if rows_np.size != r1 - r0:
                raise AssertionError("KV write exceeds reserved rows")
            dsts.append(rows_np)
        arrays.update(kv_src=_cat(srcs), kv_dst=_cat(dsts))
    t = _tick(timing, "pack_kv", t)

    arrays.update(input_ids=_cat(id_parts), positions=_cat(pos_parts),
                  finals=np.asarray(finals, dtype=np.int64),
                  cu_a=np.asarray(cu_a, dtype=np.int32),
                  a_len=np.diff(np.asarray(cu_a, dtype=np.int32)))
    dev = device if device is not None else arena.device
    if staging is None:
        staging = Stager(torch, dev)
    staged = staging.stage(arrays)

    if reads is None and "reads_rows" in staged:
        reads = dict(rows=staged["reads_rows"], cu_q=staged["reads_cu_q"],
                     used=staged["reads_used"], table=staged["reads_table"],
                     source=staged["reads_source"], **host_ints["reads"])
    unified = None
    if unified_host is not None:
        unified = dict(src=staged["unified_src"], dst=staged["unified_dst"],
                       row_dst=staged.get("unified_row_dst"),
                       tail_src=staged.get("tail_src"), tail_dst=staged.get("tail_dst"),
                       used=staged["unified_used"], table=staged["unified_table"],
                       cu_q=staged["unified_cu_q"], **unified_host)
    # attention work per layer, for throughput accounting: (query, key) pairs
    # attended and KV rows gathered, per call
    a_len = np.diff(np.asarray(cu_a, dtype=np.int64))
    work = {"own_pairs": int((a_len * (a_len + 1) // 2).sum())}
    if unified_host is not None:
        c = np.diff(arrays["unified_cu_q"].astype(np.int64))
        used = arrays["unified_used"].astype(np.int64)
        work["unified_pairs"] = int((c * (used - c) + c * (c + 1) // 2).sum())
        work["unified_kv_rows"] = int(used.sum())
    if "reads_rows" in arrays:
        c = np.diff(arrays["reads_cu_q"].astype(np.int64))
        used = arrays["reads_used"].astype(np.int64)
        work["read_pairs"] = int((c * used).sum())
        work["read_kv_rows"] = int(used.sum())
    meta = dict(layer=0, kv_src=staged.get("kv_src"), kv_dst=staged.get("kv_dst"),
                a_read=staged.get("a_read"),
                work=work,
                reads=reads, unified=unified, canvas=None, cu_a=staged["cu_a"],
                a_len=staged["a_len"],
                max_a=max(cu_a[i + 1] - cu_a[i] for i in range(len(cu_a) - 1)))
    chunk = Chunk(input_ids=staged["input_ids"], positions=staged["positions"],
                  final_indices=staged["finals"], meta=meta,
                  attention_mode=attention_mode, tokens=token_count, layout=layout,
                  temporary_keys=tuple(temporary_keys), fresh_keys=tuple(fresh_keys),
                  host=arrays)
    _tick(timing, "pack_h2d", t)
    return chunk


def _segment_reads(cu_a, arrays):
    """Read sequence of each causal segment, -1 for none.

    Every reader range pack_chunk lays out covers whole segments (a stacked
    group is one segment; a borrowing prefix is one; a group's suffixes all
    read its key), so a segment's first row names the read of every row in
    it; the check below holds that invariant.
    """
    n_seg = cu_a.size - 1
    out = np.full(n_seg, -1, dtype=np.int32)
    if "reads_source" not in arrays or n_seg == 0:
        return out
    source = arrays["reads_source"].astype(np.int64)
    cu_q = arrays["reads_cu_q"].astype(np.int64)
    row_read = np.where(source >= 0, np.searchsorted(cu_q, source, side="right") - 1, -1)
    lens = np.diff(cu_a)
    starts = cu_a[:-1]
    nonempty = lens > 0
    out[nonempty] = row_read[starts[nonempty]]
    if row_read.size and not np.array_equal(row_read, np.repeat(out, lens)):
        raise AssertionError("a causal segment mixes rows with different reads")
    return out


def attention_path(pipeline, requested, default="unified") -> str:
    """The path a filter runs: the plan's request where the model has it (loop.py:580-590)."""
    if requested is None:
        requested = default
    if requested == "tree" and pipeline.tree_attention:
        return "tree"
    return "unified"


def _forward(pipeline, arena, chunk):
    """Run the forward pass, then free the chunk's temporary pages (loop.py:593-604)."""
    try:
        return pipeline.forward_chunk(chunk)
    finally:
        keys, chunk.temporary_keys = chunk.temporary_keys, ()
        for key in keys:
            arena.free_key(key)


def _shared_preamble_tokens(question_ids):
    """Longest common token prefix of the stage questions (loop.py:1157-1165)."""
    if len(question_ids) < 2:
        return 0
    p = 0
    while all(len(q) > p and q[p] == question_ids[0][p] for q in question_ids):
        p += 1
    return p


def borrow_check(arena, keys, borrowing):
    """can_borrow for Borrowing: whether the arena can serve a borrow (loop.py:1168-1182)."""
    def can_borrow(doc, parent, same_chunk):
        shared = borrowing.tree_shared[doc]
        if not same_chunk or arena.is_resident(keys[parent]):
            return arena.can_borrow(keys[parent], shared)
        return arena.origin(borrowing.shared(parent)) <= arena.origin(shared)
    return can_borrow


def lowest_borrows(borrowing):
    lowest = {}
    for doc, parent in enumerate(borrowing.tree_parent):
        if parent is not None:
            shared = borrowing.tree_shared[doc]
            lowest[parent] = min(lowest.get(parent, shared), shared)
    return lowest


class _Progress:
    def __init__(self, *a, **k):
        pass

    def update(self, n):
        pass

    def finish(self, *a):
        pass


class FilterStream:
    """The filter chain, one chunk per next() call (loop.py:1195-1532).

    Continuous admission with survivor priority; pages freed on FALSE or
    after the last stage. The previous chunk's answers are read while the
    current chunk runs.
    """

    def __init__(self, torch, arena, pipeline, async_ans, doc_ids, question_ids,
                 budget, timing=None, pinned=True, limit=None, *, arena_writes,
                 arena_keys=None, retain_survivors=(), hold_survivors=False,
                 hold_extra_tokens=0, attention_mode=None, document_done=None,
                 prefix_tree=None, spans=None):
        p = _shared_preamble_tokens(question_ids)
        keys = range(len(doc_ids)) if arena_keys is None else arena_keys
        if len(keys) != len(doc_ids):
            raise ValueError("arena_keys must match doc_ids")
        retain_all = retain_survivors is True
        retain = set() if retain_all else set(retain_survivors)
        if hold_survivors and (retain_all or retain):
            raise ValueError("held survivors are pinned, not retained")
        arena_writes = arena_writes or getattr(pipeline, "needs_pages", False)
        stage_tokens = [len(question_ids[0])] + [len(q) - p for q in question_ids[1:]]
        tails = [list(question_ids[0])] + [list(q[p:]) for q in question_ids[1:]]
        for i, tail in enumerate(tails):
            if not tail:
                raise ValueError(f"stage {i} question has no tokens beyond the "
                                 f"shared preamble ({p} tokens)")
        if not arena_writes and (len(question_ids) > 1 or retain_all or retain
                                 or hold_survivors):
            raise ValueError("arena_writes=False needs a single stage")
        self.attention_mode = attention_path(pipeline, attention_mode)
        unified = self.attention_mode == "unified"
        if prefix_tree is not None and prefix_tree.shared_tokens:
            if not arena_writes:
                raise ValueError("a prefix tree needs arena writes")
        else:
            prefix_tree = None
        temp_tail = (max(0, *(len(q) - p for q in question_ids))
                     if unified and arena_writes else 0)
        capacity_extra = p + temp_tail
        if hold_survivors:
            capacity_extra = max(capacity_extra, hold_extra_tokens)
        if arena.retention_cap_pages is None:
            arena.retention_cap_pages = max(0, arena.n_pages - arena.pages_needed(2 * budget))
        self.sched = FilterAdmission(
            [len(d) for d in doc_ids], stage_tokens, budget,
            arena_pages=arena.n_pages if arena_writes else None,
            page_tokens=arena.page_tokens, kept_extra_tokens=capacity_extra,
            limit=limit, page_cost=arena.page_cost, tree=prefix_tree)
        borrowing = self.sched.borrowing
        borrowing.can_borrow = borrow_check(arena, keys, borrowing)
        self.tree = prefix_tree
        self.tree_position = ({doc: i for i, doc in enumerate(prefix_tree.order)}
                              if prefix_tree is not None else {})
        self.borrowers = borrowing.borrowers()
        self.lowest_borrow = lowest_borrows(borrowing)
        self.reserve_pages = 0
        self.torch = torch
        self.arena = arena
        self.pipeline = pipeline
        self.async_ans = async_ans
        self.doc_ids = doc_ids
        self.keys = keys
        self.timing = timing
        self.pinned = pinned
        self.arena_writes = arena_writes
        self.retain_all = retain_all
        self.retain = retain
        self.hold = hold_survivors
        self.preamble = p
        self.capacity_extra = capacity_extra
        self.tails = tails
        self.spans = [] if spans is None else spans
        self.tokens = 0
        self.chunks = 0
        self.done = False
        self.outstanding = []
        self.progress = _Progress()
        self._finished = 0
        self.document_done = document_done
        self.staging = None
        self.packed_groups = []   # per chunk, the groups it ran (for checkers)

    @property
    def answers(self):
        return self.sched.answers

    def _spec(self, doc, stage, fresh):
        if fresh:
            borrowing = self.sched.borrowing
            shared = borrowing.shared(doc)
            prefix = self.doc_ids[doc]
            read_key = None
            if shared:
                prefix = prefix[shared:]
                read_key = self.keys[borrowing.parent(doc)]
            return dict(key=self.keys[doc], prefix=prefix, start=shared,
                        read_key=read_key, f=len(self.doc_ids[doc]),
                        suffixes=[self.tails[0]], write_suffix_tokens=self.preamble)
        return dict(key=self.keys[doc], prefix=None,
                    f=len(self.doc_ids[doc]) + self.preamble,
                    suffixes=[self.tails[stage]])

    def set_reserve(self, pages):
        """Keep `pages` free for a join consumer's partner rows (loop.py:1361-1374)."""
        for doc, ids in enumerate(self.doc_ids):
            if self.arena.page_cost(len(ids) + self.capacity_extra) + pages > self.arena.n_pages:
                raise ValueError(f"document {doc} needs more pages than the arena holds "
                                 f"beside the join's {pages} pages of partner rows")
        self.reserve_pages = pages

    def _activate(self, doc):
        borrowing = self.sched.borrowing
        key = self.keys[doc]
        shared = borrowing.shared(doc)
        got = self.arena.activate(
            key, len(self.doc_ids[doc]) + self.preamble,
            capacity_tokens=len(self.doc_ids[doc]) + self.capacity_extra,
            base_tokens=len(self.doc_ids[doc]),
            borrow=(self.keys[borrowing.parent(doc)], shared) if shared else None)
        assert got is not None, "scheduler admitted a doc the arena cannot hold"
        if self.borrowers[doc]:
            self.arena.hold(key, self.borrowers[doc])
            self.arena.keep_window(key, self.lowest_borrow[doc])

    def _report(self, entry, items):
        timing = self.timing
        t = time.perf_counter() if timing is not None else 0.0
        groups, handle = entry
        bits = self.async_ans.result(handle)
        t = _tick(timing, "report_wait", t)
        last_stage = len(self.tails) - 1
        finished = []
        for (doc, stage, _fresh), bit in zip(groups, bits):
            passed = bool(bit)
            last = stage == last_stage
            keep = passed and last and (self.retain_all or doc in self.retain)
            hold = passed and last and self.hold
            for d in self.sched.report(doc, stage, passed, release=not (keep or hold)):
                self.arena.free_key(self.keys[d])
            if keep:
                self.arena.retain(self.keys[doc], len(self.doc_ids[doc]))
            if hold:
                items.append((self.keys[doc], self.doc_ids[doc]))
            if not passed or last:
                self._finished += 1
                finished.append((doc, stage, passed))
        if finished and self.document_done is not None:
            self.document_done(finished)
        _tick(timing, "report_rest", t)

    def _finish(self, items):
        while self.outstanding:
            self._report(self.outstanding.pop(0), items)
        for doc in self.sched.drain_ready():
            self.arena.free_key(self.keys[doc])
        self.arena.drop_holds([self.keys[doc] for doc, n in enumerate(self.borrowers) if n])
        self.done = True

    def next(self, evict_retained=False):
        """Run one chunk; returns (held (key, prefix) pairs, blocked)."""
        items = []
        if self.done:
            return items, False
        sched = self.sched
        arena = self.arena
        timing = self.timing
        while True:
            if sched.done():
                self._finish(items)
                return items, False
            free = max(0, arena.free_pages - self.reserve_pages) if self.arena_writes else None
            t = time.perf_counter() if timing is not None else 0.0
            groups = sched.next_chunk(free)
            t = _tick(timing, "next_chunk", t)
            if groups:
                break
            if self.outstanding:
                self._report(self.outstanding.pop(0), items)
                continue
            if sched.blocked_pages and (evict_retained or not self.hold):
                if arena.evict_retained(sched.blocked_pages):
                    continue
            if self.hold and sched.blocked_pages and not evict_retained:
                return items, True
            if arena.drop_holds([self.keys[doc] for doc, n in enumerate(self.borrowers) if n]):
                continue
            if self.hold and sched.blocked_pages:
                return items, True
            raise AssertionError("nothing buildable and nothing in flight")
        if self.tree is not None and self.attention_mode != "unified":
            # siblings back to back read their parent's pages once; a parent
            # sorts under its own parent's place, so before them
            def borrow_order(group):
                doc, _, fresh = group
                if not fresh:
                    return (False, -1, 0)
                parent = sched.borrowing.parent(doc)
                return (True, self.tree_position[doc if parent is None else parent],
                        sched.borrowing.shared(doc))
            groups.sort(key=borrow_order)
        fresh_docs = [doc for doc, _, fresh in groups if fresh]
        if self.arena_writes:
            for doc in fresh_docs:
                self._activate(doc)
        t = _tick(timing, "alloc", t)
        if self.staging is None and str(getattr(arena, "device", "cpu")).startswith("cuda"):
            self.staging = Stager(self.torch, arena.device)
        chunk = pack_chunk(self.torch, arena, [self._spec(*g) for g in groups],
                           timing=timing, pinned=self.pinned,
                           attention_mode=self.attention_mode, staging=self.staging)
        for doc in fresh_docs:
            parent = sched.borrowing.tree_parent[doc]
            if parent is not None:
                arena.release(self.keys[parent])
        self.packed_groups.append(list(groups))
        t = _tick(timing, "pack", t)
        self.tokens += chunk.tokens
        normed = _forward(self.pipeline, arena, chunk)
        t = _tick(timing, "forward_launch", t)
        self.outstanding.append((groups, self.async_ans.submit(normed)))
        self.chunks += 1
        t = _tick(timing, "submit", t)
        if timing is not None:
            timing["n_chunks"] = timing.get("n_chunks", 0) + 1
        while len(self.outstanding) > 1:
            self._report(self.outstanding.pop(0), items)
        return items, bool(self.hold and sched.blocked_pages)


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


class _JoinDriver:
    """State of one run_join call: the scheduler, the arena keys, launches in flight."""

    def __init__(self, torch, arena, pipeline, async_ans, prefixes, keys, stage_suffixes,
                 budget, frames, anchor_done, anchor_source, anchor_partners, anchor_batch,
                 staging, mode, prefix_tree):
        self.torch, self.arena, self.pipeline = torch, arena, pipeline
        self.async_ans = async_ans
        self.prefixes, self.keys = prefixes, keys
        self.stage_suffixes = stage_suffixes
        self.budget = budget
        self.frames = frames
        self.anchor_done = anchor_done
        self.source = anchor_source
        self.anchor_partners = anchor_partners
        self.anchor_batch = anchor_batch
        self.staging = staging
        self.mode = mode
        self.n_stages = len(stage_suffixes)
        # a frame entry's rows land in the anchor's pages after its document
        self.frame_max = max(len(f) for f in frames)
        self.spans = []
        self.tokens = 0
        self.outstanding = []          # (groups, readout handle), launch order
        self.packed_groups = []
        resident = {a: self.held_pages(keys[a], len(prefixes[a]))
                    for a in range(len(keys)) if arena.is_resident(keys[a])}
        # resident anchors stay for the whole join
        for a in resident:
            arena.pin(keys[a])
        self.sched = JoinAdmission(
            [len(p) for p in prefixes], [[len(s) for s in sufs] for sufs in stage_suffixes],
            budget, arena.n_pages, arena.page_tokens,
            frame_tokens=[len(f) for f in frames], resident=resident,
            anchor_partners={a: self.partners_of(keys[a]) for a in range(len(keys))},
            temporary_suffix_pages=mode == "unified",
            answer_dtype=async_ans.dtype, page_cost=arena.page_cost, tree=prefix_tree)
        borrowing = self.sched.borrowing
        borrowing.can_borrow = borrow_check(arena, keys, borrowing)
        # counted after resident anchors detach: they borrow nothing
        self.borrowers = borrowing.borrowers()
        self.lowest_borrow = lowest_borrows(borrowing)
        self.held = [keys[a] for a, n in enumerate(self.borrowers) if n]

    def partners_of(self, key):
        return None if self.anchor_partners is None else self.anchor_partners(key)

    def held_pages(self, key, prefix_tokens):
        """Pages a resident anchor already covers of what the scheduler prices."""
        capacity = prefix_tokens + self.frame_max
        return self.arena.page_cost(capacity) - self.arena.growth_cost(key, capacity)

    # ---- streamed anchors ------------------------------------------------

    def admit(self, items):
        arena = self.arena
        if self.anchor_batch is not None and items:
            kept = set(self.anchor_batch([key for key, _ in items]))
            for key, _ in items:
                if key not in kept and arena.is_resident(key):
                    arena.free_key(key)
            items = [(key, prefix) for key, prefix in items if key in kept]
        for key, prefix in items:
            if not arena.is_resident(key):
                raise ValueError(f"streamed anchor {key!r} has no KV in the arena")
            arena.pin(key)
            self.keys.append(key)
            self.prefixes.append(prefix)
            self.sched.admit(len(prefix), self.held_pages(key, len(prefix)),
                             partners=self.partners_of(key))

    def pull(self, evict_retained=False, force=False):
        """Run source chunks until a join chunk can fill or the source blocks."""
        moved = False
        source = self.source
        while not source.done and (force or self.sched.buildable_tokens() < self.budget):
            force = False
            before = source.chunks
            items, blocked = source.next(evict_retained=evict_retained)
            self.admit(items)
            moved = moved or bool(items) or source.chunks > before
            if blocked:
                break
        return moved

    # ---- chunks ------------------------------------------------------------

    def entry_rows(self, a, j, start, end, carried):
        rows = len(self.prefixes[a]) if carried else 0
        rows += sum(len(self.stage_suffixes[j][i])
                    for i in self.sched.partner_indices(a, j, start, end))
        if self.frames[j] and start == 0:
            rows += len(self.frames[j])
        return rows

    def specs(self, groups):
        """pack_chunk groups for one chunk; activates fresh anchors' pages."""
        arena, sched = self.arena, self.sched
        borrowing = sched.borrowing
        out = []
        for a, j, start, end, carried in groups:
            key = self.keys[a]
            f = len(self.prefixes[a])
            frame = self.frames[j]
            parent, shared = ((borrowing.parent(a), borrowing.shared(a))
                              if carried else (None, 0))
            fresh = not arena.is_resident(key)
            got = arena.activate(key, f, capacity_tokens=f + self.frame_max, base_tokens=f,
                                 borrow=(self.keys[parent], shared) if shared else None)
            assert got is not None, "scheduler admitted an anchor the arena cannot hold"
            if fresh and a < len(self.borrowers) and self.borrowers[a]:
                arena.hold(key, self.borrowers[a])
                arena.keep_window(key, self.lowest_borrow[a])
            prefix = None
            if carried:
                prefix = self.prefixes[a][shared:] if shared else self.prefixes[a]
            suffixes = [self.stage_suffixes[j][i]
                        for i in sched.partner_indices(a, j, start, end)]
            if frame and start == 0:
                # frame entry: the frame is written into the anchor's KV after
                # the document (its answer row is read and discarded); the
                # partners then read document + frame
                out.append(dict(key=key, prefix=prefix, start=shared, f=f,
                                suffixes=[frame], write_suffix_tokens=len(frame)))
                out.append(dict(key=key, prefix=None, f=f + len(frame), suffixes=suffixes))
            else:
                out.append(dict(key=key, prefix=prefix, start=shared, f=f + len(frame),
                                suffixes=suffixes))
        return out

    def run_part(self, part):
        """Run one chunk of groups; halve it when its temporary pages do not fit."""
        try:
            self.run_one(part)
        except ArenaFullError as error:
            need = self.arena.page_cost(sum(self.entry_rows(*g) for g in part))
            if self.arena.evict_retained(need):
                logger.info("join chunk of %d groups retried after evicting retained KV",
                            len(part))
                self.run_part(part)
                return
            if len(part) < 2:
                raise
            logger.info("join chunk of %d groups split: %s", len(part), error)
            half = len(part) // 2
            self.run_part(part[:half])
            self.run_part(part[half:])

    def run_one(self, part):
        torch = self.torch
        if self.staging is None and str(getattr(self.arena, "device", "cpu")).startswith("cuda"):
            self.staging = Stager(torch, self.arena.device)
        chunk = pack_chunk(torch, self.arena, self.specs(part), attention_mode=self.mode,
                           staging=self.staging)
        self.packed_groups.append(list(part))
        self.tokens += chunk.tokens
        events = None
        if torch.cuda.is_available() and str(getattr(self.arena, "device", "")).startswith("cuda"):
            events = (torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
            events[0].record()
        normed = _forward(self.pipeline, self.arena, chunk)
        if events is not None:
            events[1].record()
        for key in chunk.fresh_keys:
            self.arena.trim_window(key)
        self.spans.append((part[0][1],) + (events or (None, None)))
        self.outstanding.append((part, self.async_ans.submit(normed)))
        # read the previous chunk's answers while this one runs
        while len(self.outstanding) > 1:
            self.report(self.outstanding.pop(0))

    # ---- answers -------------------------------------------------------------

    def settle(self, anchor):
        if self.anchor_done is None:
            if self.arena.is_resident(self.keys[anchor]):
                self.arena.free_key(self.keys[anchor])
        else:
            self.anchor_done(anchor, self.sched.answers[self.n_stages - 1].get(anchor, []))

    def event(self, kind, anchor):
        if kind == "finished":
            self.settle(anchor)
        elif self.arena.is_resident(self.keys[anchor]):
            self.arena.free_key(self.keys[anchor])

    def report(self, entry):
        groups, handle = entry
        bits = self.async_ans.result(handle)
        pos = 0
        for a, j, start, end, _ in groups:
            if self.frames[j] and start == 0:
                pos += 1          # the frame entry's answer row means nothing
            count = end - start
            for kind, anchor in self.sched.report(a, j, start, end, bits[pos:pos + count]):
                self.event(kind, anchor)
            pos += count

    # ---- the loop ------------------------------------------------------------

    def run(self):
        sched, arena, source = self.sched, self.arena, self.source
        while True:
            if source is not None and not source.done:
                self.pull()
            for kind, anchor in sched.take_settled():
                self.event(kind, anchor)
            if sched.done() and (source is None or source.done):
                break
            if sched.blocked_pages:
                arena.evict_retained(sched.blocked_pages)
            groups = sched.next_chunk(arena.free_pages)
            if not groups:
                if self.outstanding:
                    self.report(self.outstanding.pop(0))
                    continue
                if source is not None and not source.done:
                    if self.pull(evict_retained=True, force=True):
                        continue
                if sched.blocked_pages and arena.evict_retained(sched.blocked_pages):
                    continue
                # parents held for queued children: the children pack whole
                if arena.drop_holds(self.held):
                    continue
                raise AssertionError("nothing buildable and nothing in flight")
            self.run_part(groups)
            # packed children hold their parents' pages now
            tree_parent = sched.borrowing.tree_parent
            for a, _, start, _, carried in groups:
                parent = tree_parent[a] if a < len(tree_parent) else None
                if carried and start == 0 and parent is not None:
                    arena.release(self.keys[parent])
        while self.outstanding:
            self.report(self.outstanding.pop(0))
        arena.drop_holds(self.held)


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
    else:
        prefixes = list(anchor_prefixes)
        keys = list(range(len(prefixes))) if anchor_keys is None else list(anchor_keys)
    if len(keys) != len(prefixes):
        raise ValueError("anchor_keys must match anchor_prefixes")
    if tuple(getattr(pipeline, "canvas_ids", ())):
        raise ValueError("canvas rows belong to diffusion models, not this build")
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
    driver = _JoinDriver(torch, arena, pipeline, async_ans, prefixes, keys, stage_suffixes,
                         budget, frames, anchor_done, anchor_source, anchor_partners,
                         anchor_batch, staging, mode, prefix_tree)
    driver.run()
    if stats is not None:
        stats["borrowed_tokens"] = driver.sched.borrowing.borrowed_tokens
        stats["chunks"] = len(driver.packed_groups)
    return driver.sched.answers, driver.spans, driver.tokens
