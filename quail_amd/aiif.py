"""AI.IF filter over rows on one GPU: synthetic workloads and the runner.

The runner wires what the reference's LoadedGpu + execute_single_graph do
for one filter node (quail/backends/quail/worker.py:46-148; backend.py:
107-161): build the arena (sized by the budget formulas), the Qwen3
pipeline and the answer readout, then run loop.run_filter over
`DocumentPrefixes(instruction, documents)` with the prefix tree deciding
page borrowing. Rows are synthetic (no dataset or tokenizer offline).
"""

import time

import numpy as np

from quail_amd import budgets, loop
from quail_amd.arena import KVArena
from quail_amd.model import SYNTHETIC_FALSE_IDS, SYNTHETIC_TRUE_IDS
from quail_amd.qwen3 import Qwen3Pipeline
from quail_amd.readout import AnswerRows, AsyncAnswers
from quail_amd.specs import MI355X
from quail_amd.tokens import _Rows, chain_tokens, flat_tokens, prefix_tree


def lognormal_lengths(n, median, mean, cap, rng):
    """Rounded lognormal lengths with the given median and mean, in [1, cap]."""
    mu = np.log(median)
    sigma = np.sqrt(2.0 * np.log(mean / median))
    lens = np.rint(rng.lognormal(mu, sigma, size=n)).astype(np.int64)
    return np.clip(lens, 1, cap)


def synthetic_filter_workload(n_rows, *, prefix_tokens=64, median=180, mean=230,
                              cap=1024, tail_tokens=24, vocab=151_936, seed=0,
                              uniform_lengths=None):
    """Rows of an AI.IF over a Qwen3-sized vocabulary.

    Every row is a shared `prefix_tokens`-token instruction, then a
    document of uniform random ids whose length is lognormal (median, mean,
    capped) or, with uniform_lengths=(lo, hi), uniform in [lo, hi]; one
    question tail of `tail_tokens` ids follows each row.
    Returns (instruction ids, documents, question tail).
    """
    rng = np.random.default_rng(seed)
    instruction = rng.integers(0, vocab, size=prefix_tokens, dtype=np.int64)
    if uniform_lengths is None:
        lens = lognormal_lengths(n_rows, median, mean, cap, rng)
    else:
        lens = rng.integers(uniform_lengths[0], uniform_lengths[1] + 1, size=n_rows)
    documents = [rng.integers(0, vocab, size=int(L), dtype=np.int64) for L in lens]
    tail = rng.integers(0, vocab, size=tail_tokens, dtype=np.int64)
    return instruction, documents, tail


class RowPrompts(_Rows):
    """Row i = instruction + document i (tokens.DocumentPrefixes).

    Rows read from a token store are chains of the instruction and a view of
    the mapped file, built on access; other rows are views of one buffer of
    every row's ids, built once. flat_tokens() hands that buffer (for a
    store, built on first call) to the prefix tree and the packer's token
    table, which read all rows at once.
    """

    def __init__(self, instruction, documents):
        self.instruction = np.asarray(instruction, dtype=np.int64).reshape(-1)
        self.documents = documents
        self._stored = len(documents) > 0 and hasattr(documents[0], "token_parts")
        self._flat = None if self._stored else flat_tokens(documents, self.instruction)

    def __len__(self):
        return len(self.documents)

    def row(self, i):
        if self._stored:
            return chain_tokens(self.instruction, self.documents[i])
        ids, offsets = self._flat
        return ids[offsets[i]:offsets[i + 1]]

    @property
    def rows(self):
        return [self[i] for i in range(len(self))]

    def lengths(self):
        """Every row's token count (int64 array)."""
        if self._flat is not None:
            return np.diff(self._flat[1])
        if hasattr(self.documents, "lengths"):
            return self.documents.lengths.numpy() + self.instruction.size
        return np.fromiter((len(d) for d in self.documents), dtype=np.int64,
                           count=len(self.documents)) + self.instruction.size

    def flat_tokens(self):
        if self._flat is None:
            self._flat = flat_tokens(self.documents, self.instruction)
        return self._flat


class FilterRunner:
    """One GPU's AI.IF executor: model, arena, pipeline, readout.

    Args:
        model: a quail_amd.model model (weights on the GPU).
        spec: its ModelSpec.
        n_pages: arena pages; None sizes the arena with budgets.arena_pages
            for `device_spec` (the reference's formula).
        budget: chunk tokens; None uses budgets.chunk_budget.
        attention_mode: "unified", "tree" or None (unified).
        gemm_hook: passed to the engine (GEMM timing in bench.py).
        tree_kernel: the tree path's attention kernel, "fused" (node pages
            streamed per q-tile), "resident" (a node's K/V held in LDS for
            the q-tiles that read it) or "two_pass" (the reference's three
            launches).
    """

    def __init__(self, model, spec, *, device_spec=MI355X, n_pages=None, budget=None,
                 attention_mode=None, ue8m0=False, gemm_hook=None, attention_hook=None,
                 keep_margins=True, tree_kernel="fused",
                 true_ids=SYNTHETIC_TRUE_IDS, false_ids=SYNTHETIC_FALSE_IDS):
        import torch
        self.torch = torch
        self.spec = spec
        n_layers = len(model.model.layers)
        self.budget = budget or budgets.chunk_budget(spec, device_spec)
        if n_pages is None:
            n_pages, _ = budgets.arena_pages(spec, device_spec, self.budget)
        self.arena = KVArena(n_layers, n_pages, budgets.PAGE_TOKENS, spec.n_kv,
                             spec.d_head, dtype=torch.bfloat16, device="cuda")
        self.pipeline = Qwen3Pipeline(model, self.arena, spec=spec, ue8m0=ue8m0,
                                      gemm_hook=gemm_hook, attention_hook=attention_hook,
                                      tree_kernel=tree_kernel)
        self.rows = AnswerRows(torch, model, true_ids, false_ids)
        self.answers = AsyncAnswers(torch, self.rows, keep_margins=keep_margins)
        self.attention_mode = attention_mode
        self.last = {}

    def run(self, instruction, documents, tail, *, timing=None, document_done=None):
        """Run the filter; returns (answers per row, stats). document_done,
        if given, is called after each chunk's report with the documents it
        finished, as [(doc, stage, passed)]."""
        torch = self.torch
        docs = RowPrompts(instruction, documents)
        tree = prefix_tree(docs, budgets.PAGE_TOKENS)
        self.answers.margins = []
        stats = {}
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        answers, _, tokens = loop.run_filter(
            torch, self.arena, self.pipeline, self.answers, docs, [list(tail)],
            self.budget, timing=timing, arena_writes=True,
            attention_mode=self.attention_mode, prefix_tree=tree, stats=stats,
            document_done=document_done)
        torch.cuda.synchronize()
        wall = time.perf_counter() - t0
        if self.arena.accounting.owned:
            raise AssertionError("the filter left pages resident")
        input_tokens = int(docs.lengths().sum()) + len(tail) * len(docs)
        stats.update(wall_s=wall, fresh_tokens=tokens, input_tokens=input_tokens,
                     rows=len(docs), shared_tokens=tree.shared_tokens)
        self.last = stats
        return [answers[i][0] for i in range(len(docs))], stats


def synthetic_join_workload(n_left, n_right, *, root_tokens=48, left_median=120,
                            right_median=120, spread=230 / 180, left_cap=1024,
                            right_cap=512, frame_tokens=8, label_tokens=4, tail_tokens=16,
                            vocab=151_936, seed=0):
    """Rows of an AI join over a Qwen3-sized vocabulary.

    Anchor a = a shared `root_tokens`-token instruction + left document a
    (written into the arena once; the prefix tree lets every anchor borrow
    the root's whole pages). Each anchor's frame (`frame_tokens` ids, the
    join framing the reference writes into the anchor's KV ahead of its
    partners) follows it. Every partner suffix = a `label_tokens`-id
    partner label + right document + a `tail_tokens`-id question tail, so
    a pair's prompt is root + left doc + frame + label + right doc + tail
    (the reference's render_join_prompt_ids layout, prompts.py). Document
    lengths are rounded lognormals with the given medians and mean/median
    ratio `spread`, capped. Returns (anchor prefixes, frame, partner suffixes).
    """
    rng = np.random.default_rng(seed)
    root = rng.integers(0, vocab, size=root_tokens, dtype=np.int64)
    left = lognormal_lengths(n_left, left_median, left_median * spread, left_cap, rng)
    right = lognormal_lengths(n_right, right_median, right_median * spread, right_cap, rng)
    anchors = [np.concatenate([root, rng.integers(0, vocab, size=int(n), dtype=np.int64)])
               for n in left]
    frame = rng.integers(0, vocab, size=frame_tokens, dtype=np.int64)
    label = rng.integers(0, vocab, size=label_tokens, dtype=np.int64)
    tail = rng.integers(0, vocab, size=tail_tokens, dtype=np.int64)
    partners = [np.concatenate([label, rng.integers(0, vocab, size=int(n), dtype=np.int64),
                                tail]) for n in right]
    return anchors, frame, partners


class JoinRunner(FilterRunner):
    """One GPU's AI join executor (the join branch of backend.py:162-279):
    the same model, arena, pipeline and readout as FilterRunner, driven by
    loop.run_join over anchors with a prefix tree."""

    def run_join(self, anchors, frame, partners, *, stages=1):
        """Run the join; returns (answers[j][a] rows, stats)."""
        torch = self.torch
        tree = prefix_tree(anchors, budgets.PAGE_TOKENS)
        self.answers.margins = []
        stats = {}
        frames = [list(frame)] * stages
        suffixes = [[list(p) for p in partners]] * stages
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        answers, _, tokens = loop.run_join(
            torch, self.arena, self.pipeline, self.answers, [list(a) for a in anchors],
            suffixes, self.budget, stage_frames=frames,
            attention_mode=self.attention_mode or "tree", prefix_tree=tree, stats=stats)
        torch.cuda.synchronize()
        wall = time.perf_counter() - t0
        if self.arena.accounting.owned:
            raise AssertionError("the join left pages resident")
        pairs = sum(len(row) for row in answers[-1].values())
        input_tokens = sum((len(a) + len(frame)) * len(partners) + sum(map(len, partners))
                           for a in anchors)
        stats.update(wall_s=wall, fresh_tokens=tokens, input_tokens=input_tokens,
                     rows=pairs, anchors=len(anchors), shared_tokens=tree.shared_tokens)
        self.last = stats
        return answers, stats
