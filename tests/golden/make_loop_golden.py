"""Writes the golden chunk fixtures from the reference's own host code.

Loads the reference's arena.py, pack.py, attention.py (the Chunk type),
loop.py, tokens.py and progress.py by file path under empty package
shells (the reference's quail/__init__.py pulls in the SQL frontend, which
this path does not use), runs its run_filter / run_join on a tensor-free
CPU arena with a stand-in model that answers from each final row's token
and position (scenarios.answer_bit), and records every chunk pack_chunk
built: token ids, positions, final rows, causal segments, scatter maps,
block tables, temporaries and reads. Also records prefix_tree on tie-heavy
corpora. The fixtures are plain .npz arrays + JSON; the reference itself
never leaves this container.

Run from the repository root: python tests/golden/make_loop_golden.py
"""

import importlib.util
import json
import os
import sys
import types

import numpy as np
import torch

REF = "/root/reference"
HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, HERE)
import scenarios  # noqa: E402


def _shell(name):
    mod = types.ModuleType(name)
    mod.__path__ = []
    sys.modules[name] = mod
    return mod


def _load(name, rel):
    spec = importlib.util.spec_from_file_location(name, os.path.join(REF, rel))
    mod = importlib.util.module_from_spec(spec)
    sys.modules[name] = mod
    spec.loader.exec_module(mod)
    return mod


def load_reference():
    for pkg in ("quail", "quail.backends", "quail.backends.quail",
                "quail.backends.quail.executor", "quail.execution"):
        _shell(pkg)
    _load("quail.progress", "quail/progress.py")
    arena = _load("quail.backends.quail.executor.arena", "quail/backends/quail/executor/arena.py")
    _load("quail.backends.quail.executor.pack", "quail/backends/quail/executor/pack.py")
    _load("quail.backends.quail.executor.attention", "quail/backends/quail/executor/attention.py")
    loop = _load("quail.backends.quail.executor.loop", "quail/backends/quail/executor/loop.py")
    tokens = _load("quail.execution.tokens", "quail/execution/tokens.py")

    # chunk tensors stay on the CPU (the loop stages them to the GPU)
    def staged(torch_, data, dtype, pinned=True):
        if isinstance(data, np.ndarray) or torch.is_tensor(data):
            return torch.as_tensor(data, dtype=dtype)
        return torch.tensor(data, dtype=dtype)

    def staged_token_parts(torch_, sequences, total, pinned=True, staging=None):
        ids = [int(t) for seq in sequences for part in loop._token_parts(seq) for t in part]
        assert len(ids) == total
        return torch.tensor(ids, dtype=torch.int64)

    loop._staged = staged
    loop._staged_token_parts = staged_token_parts
    return arena, loop, tokens


def _np(t):
    return None if t is None else np.asarray(t.detach().cpu().numpy() if torch.is_tensor(t) else t)


def chunk_arrays(chunk):
    """The chunk's integer arrays under quail_amd's Chunk.host names."""
    m = chunk.meta
    out = {"input_ids": _np(chunk.input_ids), "positions": _np(chunk.positions),
           "finals": _np(chunk.final_indices), "cu_a": _np(m["cu_a"])}
    if m.get("kv_src") is not None:
        out.update(kv_src=_np(m["kv_src"]), kv_dst=_np(m["kv_dst"]))
    r = m.get("reads")
    if r is not None:
        out.update(reads_rows=_np(r["rows"]), reads_cu_q=_np(r["cu_q"]),
                   reads_used=_np(r["used"]), reads_table=_np(r["table"]),
                   reads_source=_np(r["source"]))
    u = m.get("unified")
    if u is not None:
        out.update(unified_src=_np(u["src"]), unified_dst=_np(u["dst"]),
                   unified_used=_np(u["used"]), unified_table=_np(u["table"]),
                   unified_cu_q=_np(u["cu_q"]))
        if u.get("tail_src") is not None:
            out.update(tail_src=_np(u["tail_src"]), tail_dst=_np(u["tail_dst"]))
    return {k: v for k, v in out.items() if v is not None}


class Recorder:
    canvas_ids = ()
    canvas_answer_row = 0
    needs_pages = False
    tree_attention = True

    def __init__(self):
        self.chunks = []

    def forward_chunk(self, chunk):
        arrays = chunk_arrays(chunk)
        self.chunks.append((arrays, chunk.attention_mode, chunk.tokens,
                            int(chunk.meta["max_a"])))
        ids, pos = arrays["input_ids"], arrays["positions"]
        return [scenarios.answer_bit(ids[f], pos[f]) for f in arrays["finals"]]


class _Event:
    def __init__(self, **kw):
        pass

    def record(self, *a):
        pass

    def elapsed_time(self, other):
        return 0.0

    def synchronize(self):
        pass


class CPUTorch:
    """torch as the loop sees it on a CPU-only host: its CUDA events and
    synchronisation are no-ops; everything else is torch."""

    cuda = types.SimpleNamespace(Event=_Event, synchronize=lambda: None,
                                 is_available=lambda: False)

    def __getattr__(self, name):
        return getattr(torch, name)


class Passthrough:
    dtype = None

    def submit(self, v):
        return v

    def result(self, v):
        return v


def cpu_arena(arena_mod, pages):
    return arena_mod.KVArena(n_layers=1, n_pages=pages, page_tokens=16, n_kv=1, d_head=1,
                             dtype=torch.float32, device="cpu")


def save(name, rec, extra):
    arrays, meta = {}, []
    for i, (a, mode, tokens, max_a) in enumerate(rec.chunks):
        for k, v in a.items():
            arrays[f"c{i}_{k}"] = v
        meta.append(dict(mode=mode, tokens=tokens, max_a=max_a, keys=sorted(a)))
    np.savez_compressed(os.path.join(HERE, f"{name}.npz"), **arrays)
    with open(os.path.join(HERE, f"{name}.json"), "w") as f:
        json.dump(dict(chunks=meta, **extra), f, indent=1, sort_keys=True)


def main():
    arena_mod, loop, tokens = load_reference()
    for sc in scenarios.FILTERS:
        docs, questions, budget, pages = scenarios.filter_inputs(sc["seed"])
        arena = cpu_arena(arena_mod, pages)
        rec = Recorder()
        stats = {}
        answers, _, total = loop.run_filter(
            CPUTorch(), arena, rec, Passthrough(), docs, questions, budget, arena_writes=True,
            arena_keys=[("d", i) for i in range(len(docs))], attention_mode=sc["path"],
            prefix_tree=tokens.prefix_tree(docs, 16), stats=stats)
        save(sc["name"], rec, dict(answers={str(k): v for k, v in answers.items()},
                                   tokens=total, borrowed=stats["borrowed_tokens"]))
        print(sc["name"], len(rec.chunks), "chunks", total, "tokens")
    for sc in scenarios.JOINS:
        anchors, frames, suffixes, budget, pages = scenarios.join_inputs(sc["seed"])
        arena = cpu_arena(arena_mod, pages)
        rec = Recorder()
        stats = {}
        keys = [("a", i) for i in range(len(anchors))]
        answers, _, total = loop.run_join(
            CPUTorch(), arena, rec, Passthrough(), anchors, suffixes, budget, stage_frames=frames,
            anchor_keys=keys, attention_mode=sc["path"],
            prefix_tree=tokens.prefix_tree(anchors, 16), stats=stats)
        save(sc["name"], rec, dict(answers=[{str(k): v for k, v in s.items()} for s in answers],
                                   tokens=total, borrowed=stats["borrowed_tokens"]))
        print(sc["name"], len(rec.chunks), "chunks", total, "tokens")
    trees = {}
    for sc in scenarios.TREES:
        docs = scenarios.tree_inputs(sc["seed"])
        t = tokens.prefix_tree(docs, 16)
        trees[sc["name"]] = dict(order=list(t.order), parent=list(t.parent),
                                 shared=list(t.shared))
    with open(os.path.join(HERE, "prefix_trees.json"), "w") as f:
        json.dump(trees, f, indent=1, sort_keys=True)
    print("prefix trees", len(trees))


if __name__ == "__main__":
    main()
