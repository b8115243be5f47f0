"""End-to-end support: run the AI.IF filter on the GPU and replay it on the oracle.

The GPU run records every chunk it executed (the staged host arrays, the
attention path, the final-normed rows and the readout margins); the
oracle then replays the same chunks in order over its own logical arena,
so both sides see identical packing, page tables and KV placement.
"""

import numpy as np
import torch

from oracle import forward as oracle_forward
from quail_amd import budgets, loop
from quail_amd.aiif import RowPrompts
from quail_amd.model import build_random_qwen3
from quail_amd.qwen3 import Qwen3Pipeline
from quail_amd.readout import AnswerRows, AsyncAnswers
from quail_amd.specs import ModelSpec
from quail_amd.tokens import prefix_tree
from quail_amd.arena import KVArena

TINY = ModelSpec(name="qwen3-tiny", params=0.03e9, layers=2, hidden=1024, n_q=8, n_kv=2,
                 d_head=128, ffn_width=3072, vocab=4096, tied_head=True)
TINY_TRUE = (11, 500, 1201, 3333)
TINY_FALSE = (12, 777, 2048, 4000)


class Recorder:
    """Wraps a pipeline; keeps (host arrays, path, normed rows) per chunk."""

    def __init__(self, pipeline):
        self.pipeline = pipeline
        self.tree_attention = pipeline.tree_attention
        self.canvas_ids = ()
        self.needs_pages = False
        self.records = []

    def forward_chunk(self, chunk):
        normed = self.pipeline.forward_chunk(chunk)
        self.records.append((chunk.host, chunk.attention_mode, normed.cpu()))
        return normed


def gpu_filter(model, spec, docs, tail, *, path, pages, budget, true_ids, false_ids,
               ue8m0=False, **engine_options):
    arena = KVArena(len(model.model.layers), pages, 16, spec.n_kv, spec.d_head,
                    dtype=torch.bfloat16, device="cuda")
    pipe = Recorder(Qwen3Pipeline(model, arena, spec=spec, ue8m0=ue8m0, **engine_options))
    rows = AnswerRows(torch, model, true_ids, false_ids)
    ans = AsyncAnswers(torch, rows, keep_margins=True)
    stream = loop.FilterStream(torch, arena, pipe, ans, docs, [list(tail)], budget,
                               arena_writes=True, attention_mode=path,
                               prefix_tree=prefix_tree(docs, 16))
    while not stream.done:
        stream.next()
    torch.cuda.synchronize()
    assert not arena.accounting.owned
    # margins per document, in the order chunks answered
    margins = {}
    for groups, m in zip(stream.packed_groups, ans.margins):
        for (doc, _, _), v in zip(groups, m):
            margins[doc] = float(v)
    answers = {d: stream.answers[d][0] for d in range(len(docs))}
    return answers, margins, pipe.records, stream


def oracle_replay(model, spec, records, pages, true_ids, false_ids, gemm=None):
    w = oracle_forward.cpu_weights(model)
    arena = oracle_forward.OracleArena(len(w["layers"]), pages, spec.n_kv, spec.d_head)
    gemm = gemm or oracle_forward.exact_gemm
    outs = []
    for host, path, _ in records:
        normed = oracle_forward.forward_chunk(w, host, path, arena, gemm=gemm)
        bits, margin = oracle_forward.readout(w, normed, true_ids, false_ids)
        outs.append((normed, bits, margin))
    return outs


def tiny_workload(seed, n_rows, prefix=40, max_doc=150, tail_len=9, vocab=4096):
    rng = np.random.default_rng(seed)
    instruction = rng.integers(0, vocab, size=prefix)
    documents = [rng.integers(0, vocab, size=int(rng.integers(1, max_doc)))
                 for _ in range(n_rows)]
    tail = rng.integers(0, vocab, size=tail_len)
    return RowPrompts(instruction, documents), tail


def tiny_model(seed=0):
    return build_random_qwen3(TINY, seed=seed, device="cuda", max_pos=2048,
                              answer_token_ids=TINY_TRUE + TINY_FALSE)


def gpu_join(model, spec, anchors, frame, partners, *, path, pages, budget, true_ids,
             false_ids, stages=1):
    """Run a join on the GPU; returns (answers, per-chunk margins of every
    final row, records, stats)."""
    arena = KVArena(len(model.model.layers), pages, 16, spec.n_kv, spec.d_head,
                    dtype=torch.bfloat16, device="cuda")
    pipe = Recorder(Qwen3Pipeline(model, arena, spec=spec))
    rows = AnswerRows(torch, model, true_ids, false_ids)
    ans = AsyncAnswers(torch, rows, keep_margins=True)
    stats = {}
    answers, _, _ = loop.run_join(
        torch, arena, pipe, ans, [list(a) for a in anchors],
        [[list(p) for p in partners]] * stages, budget, stage_frames=[list(frame)] * stages,
        attention_mode=path, prefix_tree=prefix_tree(anchors, 16), stats=stats)
    torch.cuda.synchronize()
    assert not arena.accounting.owned
    return answers, ans.margins, pipe.records, stats


def tiny_join(seed, n_anchors, n_partners, root=40, max_doc=60, frame_len=5, vocab=4096):
    rng = np.random.default_rng(seed)
    head = rng.integers(0, vocab, size=root)
    anchors = [np.concatenate([head, rng.integers(0, vocab, size=int(rng.integers(1, max_doc)))])
               for _ in range(n_anchors)]
    frame = rng.integers(0, vocab, size=frame_len)
    partners = [rng.integers(0, vocab, size=int(rng.integers(2, 30))) for _ in range(n_partners)]
    return anchors, frame, partners


def decision_stats(gpu, ref, alt):
    """Decision parity of a GPU run against the oracle, measured against the
    oracle's own floor. Each argument is (bits, margins), dicts or lists by
    row; ref is the fp64 oracle, alt the fp32 oracle.

    The oracle pair's margin shift |alt - ref| is the noise any change of
    accumulation order makes on this model. Its 99th percentile is the
    band: a row whose fp64 margin lies beyond it is decided by the
    algorithm, not by rounding, to 99 % confidence per row; beyond twice
    the band, by a wide margin. Returns a dict of counts and shifts."""
    n = len(ref[0])
    rows = range(n)
    rb, rm = [ref[0][d] for d in rows], np.array([ref[1][d] for d in rows])
    ab, am = [alt[0][d] for d in rows], np.array([alt[1][d] for d in rows])
    gb, gm = [gpu[0][d] for d in rows], np.array([gpu[1][d] for d in rows])
    oracle_shift = np.abs(am - rm)
    gpu_shift = np.abs(gm - rm)
    band = float(np.quantile(oracle_shift, 0.99))
    out = {"rows": n, "band": band,
           "gpu_agree": sum(g == r for g, r in zip(gb, rb)),
           "floor": sum(a == r for a, r in zip(ab, rb)),
           "median_margin": float(np.median(np.abs(rm))),
           "oracle_shift_median": float(np.median(oracle_shift)),
           "gpu_shift_median": float(np.median(gpu_shift)),
           "oracle_shift_p90": float(np.quantile(oracle_shift, 0.9)),
           "gpu_shift_p90": float(np.quantile(gpu_shift, 0.9))}
    for name, width in (("band", band), ("wide", 2 * band)):
        clear = [d for d in rows if abs(rm[d]) > width]
        out[f"outside_{name}"] = len(clear)
        out[f"gpu_agree_{name}"] = sum(gb[d] == rb[d] for d in clear)
        out[f"floor_{name}"] = sum(ab[d] == rb[d] for d in clear)
    out["disagree_margins"] = sorted(round(float(rm[d]), 4) for d in rows if gb[d] != rb[d])
    return out


def describe(stats):
    s = stats
    return (f"{s['rows']} rows: GPU-vs-fp64 {s['gpu_agree']}, fp32-vs-fp64 {s['floor']}; "
            f"band (p99 of the oracle pair's margin shift) {s['band']:.4f}: outside it "
            f"{s['outside_band']} rows, GPU agrees on {s['gpu_agree_band']}, fp32 on "
            f"{s['floor_band']}; outside twice it {s['outside_wide']} rows, GPU agrees on "
            f"{s['gpu_agree_wide']}; margin shift median / p90 GPU {s['gpu_shift_median']:.4f}"
            f" / {s['gpu_shift_p90']:.4f}, oracle pair {s['oracle_shift_median']:.4f} / "
            f"{s['oracle_shift_p90']:.4f}; median |margin| {s['median_margin']:.4f}")
