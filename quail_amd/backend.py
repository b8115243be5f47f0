"""The model-backend side of the drop-in boundary (quail/backends/base.py:40-75).

QuailBackend is what the reference's planner and runner see of a model
backend: a name, a support check (its device allow-list is the first
CUDA-specific gate of the reference, backend.py:333-344; this one admits
MI355X), and start(), which boots one GPU's executor and returns a
ModelExecution. QuailModelExecution.execute runs one AI.IF / AI_FILTER or
AI join node over the loaded state, through loop.run_filter / run_join
(backend.py:76-279).

Plan nodes are read by attribute, so the reference's AiFilter / AiJoin
(quail/physical/nodes.py:571, :687) work unchanged; FilterNode and JoinNode
below carry the same fields for callers without the planner.
"""

from dataclasses import dataclass, field
from typing import Any, Mapping, Optional

from quail_amd import budgets, loop
from quail_amd.specs import DEVICES, ModelSpec, DeviceSpec
from quail_amd.tokens import prefix_tree

SUPPORTED_ARCHS = frozenset({"qwen3"})


@dataclass(frozen=True)
class SupportResult:
    """Result of one support check (quail/planner/physical_optimizer.py:13-25)."""

    supported: bool
    reason: Optional[str] = None

    @classmethod
    def accept(cls) -> "SupportResult":
        return cls(True)

    @classmethod
    def reject(cls, reason: str) -> "SupportResult":
        return cls(False, reason)


@dataclass(frozen=True)
class GpuContext:
    """Configuration of one GPU executor (quail/backends/base.py:18-26)."""

    gpu_index: int
    gpu_count: int
    model: ModelSpec
    device: DeviceSpec
    query_settings: Mapping[str, Any] = field(default_factory=dict)


@dataclass(frozen=True)
class FilterNode:
    """The AiFilter fields the executor reads (quail/physical/nodes.py:571-649)."""

    alias: str
    question_token_ids: tuple
    attention: Optional[str] = None      # "unified" | "tree" | None (unified)
    share_prefixes: bool = False
    arena_writes: bool = True
    pin_survivors: bool = False
    hold_tokens: int = 0


@dataclass(frozen=True)
class JoinStage:
    written_pos: int
    partners: tuple = ()
    semantics: str = "semi"
    selectivity: Optional[float] = None


@dataclass(frozen=True)
class JoinNode:
    """The AiJoin fields the executor reads (quail/physical/nodes.py:687)."""

    anchor: str
    stages: tuple
    attention: Optional[str] = None      # None: tree, a join's default
    share_prefixes: bool = False


@dataclass
class NodeResult:
    """What one node hands back to the graph runner (quail/execution/runner.py)."""

    outputs: dict
    metrics: dict = field(default_factory=dict)
    finalize: Any = None


class DocumentKeys:
    """Arena keys of a node's documents: (alias, document id) per row, the
    form retained KV is matched by across operators."""

    def __init__(self, alias, document_ids):
        self.alias = alias
        self.document_ids = list(document_ids)

    def __len__(self):
        return len(self.document_ids)

    def __getitem__(self, i):
        return (self.alias, self.document_ids[i])

    def __iter__(self):
        return ((self.alias, d) for d in self.document_ids)


def _is_filter(node):
    return hasattr(node, "question_token_ids")


def _is_join(node):
    return hasattr(node, "stages") and hasattr(node, "anchor")


class QuailModelExecution:
    """Shared model state for one query on one GPU (backend.py:50-279)."""

    def __init__(self, context, *, model=None, arena=None, pipeline=None):
        self.context = context
        self._state = {}
        if model is not None:
            self._state["model"] = model
        if arena is not None:
            self._state["arena"] = arena
        if pipeline is not None:
            self._state["pipeline"] = pipeline

    @property
    def arena(self):
        return self._state.get("arena")

    @property
    def pipeline(self):
        return self._state.get("pipeline")

    def bind_query(self, *, torch, async_answers, answer_rows, chunk_tokens: int) -> None:
        """Attach the state valid for the current query (backend.py:62-74)."""
        self._state.update(torch=torch, async_answers=async_answers,
                           answer_rows=answer_rows, chunk_tokens=chunk_tokens)

    def execute(self, node, inputs: Mapping[str, Any]) -> NodeResult:
        if _is_filter(node):
            return self._filter(node, inputs)
        if _is_join(node):
            return self._join(node, inputs)
        raise TypeError(f"Quail cannot execute physical node {type(node).__name__!r}")

    def _require(self):
        missing = {"torch", "async_answers", "chunk_tokens", "arena", "pipeline"} \
            - set(self._state)
        if missing:
            raise RuntimeError(f"Quail model execution is missing state {sorted(missing)}")
        s = self._state
        return s["torch"], s["arena"], s["pipeline"], s["async_answers"], s["chunk_tokens"]

    def _tree(self, node, documents, arena):
        if not getattr(node, "share_prefixes", False):
            return None
        return prefix_tree(documents, arena.page_tokens)

    def _filter(self, node, inputs):
        torch, arena, pipeline, answers_out, budget = self._require()
        if getattr(node, "pin_survivors", False):
            raise ValueError("a filter whose survivors feed a join runs inside that join "
                             "(inputs['anchor_stream'])")
        document_ids = list(inputs["document_ids"])
        retain = inputs.get("retain_survivors", ())
        if retain is False:
            retain = ()
        limit = inputs.get("limit")
        # sorted admission would change which rows a limit keeps
        tree = None if limit is not None else self._tree(node, inputs["documents"], arena)
        stats = {}
        answers, spans, tokens = loop.run_filter(
            torch, arena, pipeline, answers_out, inputs["documents"],
            [list(q) for q in node.question_token_ids], budget, limit=limit,
            arena_writes=node.arena_writes,
            arena_keys=DocumentKeys(node.alias, document_ids), retain_survivors=retain,
            document_done=inputs.get("document_done"), prefix_tree=tree,
            attention_mode=node.attention or None, stats=stats)
        n_stages = len(node.question_token_ids)
        survivors = [document_ids[d] for d, row in sorted(answers.items())
                     if len(row) == n_stages and all(row)]
        return NodeResult(
            outputs={f"ids:{node.alias}": survivors,
                     f"filter_answers:{node.alias}": {document_ids[d]: row
                                                      for d, row in answers.items()}},
            metrics={"input_rows": len(document_ids), "output_rows": len(survivors),
                     "fresh_tokens": tokens, "chunks": stats.get("chunks", 0),
                     "borrowed_prefix_tokens": stats.get("borrowed_tokens", 0)})

    def _join(self, node, inputs):
        torch, arena, pipeline, answers_out, budget = self._require()
        lists_for = inputs.get("anchor_partners")
        anchor_ids = list(inputs["anchor_ids"])
        stats = {}
        answers, spans, tokens = loop.run_join(
            torch, arena, pipeline, answers_out, inputs["prefixes"],
            inputs["stage_suffixes"], budget, stage_frames=inputs.get("stage_frames"),
            anchor_keys=inputs.get("anchor_keys"), anchor_done=inputs.get("anchor_done"),
            anchor_partners=(None if lists_for is None
                             else lambda key: lists_for(key[1] if isinstance(key, tuple)
                                                        else key)),
            anchor_batch=inputs.get("anchor_batch"), attention_mode=node.attention or None,
            prefix_tree=self._tree(node, inputs["prefixes"], arena), stats=stats)
        last = answers[-1] if answers else {}
        matched = {anchor_ids[int(a)] for a, row in last.items() if any(row)}
        anti = node.stages[-1].semantics == "anti"
        survivors = [d for d in anchor_ids if (d in matched) != anti]
        outputs = {f"ids:{node.anchor}": survivors}
        partner_index = inputs.get("partner_indices", {})
        for stage, rows in zip(node.stages, answers):
            outputs[f"join_answers:{stage.written_pos}"] = {
                "rows": rows, "anchor_index": anchor_ids,
                "partner_index": partner_index.get(stage.written_pos),
                "anchor": node.anchor, "partners": list(stage.partners),
                "semantics": stage.semantics, "selectivity": stage.selectivity,
                "written_pos": stage.written_pos}
        return NodeResult(outputs=outputs, metrics={
            "input_rows": len(anchor_ids), "output_rows": len(survivors),
            "evaluated_document_pairs": sum(sum(len(r) for r in st.values())
                                            for st in answers),
            "fresh_tokens": tokens, "chunks": stats.get("chunks", 0),
            "borrowed_prefix_tokens": stats.get("borrowed_tokens", 0)})


class QuailBackend:
    """Plan-side face of the executor (backend.py:327-472): support and start."""

    name = "quail"
    runtime_package = "quail_amd (libquail_hip.so, gfx950)"
    devices = frozenset({"mi355x"})

    def supports(self, model, device, gpu_count: int) -> SupportResult:
        """The device allow-list admits MI355X, the only target of this
        build's kernels; one executor drives one GPU."""
        if device.name not in self.devices:
            return SupportResult.reject(
                f"Quail-on-MI355X does not support device {device.name!r}")
        if model.arch not in SUPPORTED_ARCHS:
            return SupportResult.reject(
                f"Quail does not support model {model.name!r}: "
                f"no forward pass for architecture {model.arch!r}")
        if gpu_count != 1:
            return SupportResult.reject(
                "this executor drives one GPU per process; run one executor per GPU")
        return SupportResult.accept()

    def start(self, context: GpuContext) -> QuailModelExecution:
        """Boot one GPU: model, arena sized by the reference's formula, pipeline
        (worker.py:46-106). query_settings may carry a loaded `model`
        (weights on the GPU); otherwise a random-init model of the spec's
        geometry is built (no checkpoint is reachable offline), from `seed`.
        """
        import torch

        from quail_amd.arena import KVArena
        from quail_amd.model import build_random_qwen3
        from quail_amd.qwen3 import build_pipeline

        verdict = self.supports(context.model, context.device, context.gpu_count)
        if not verdict.supported:
            raise ValueError(verdict.reason)
        settings = dict(context.query_settings or {})
        spec = context.model
        model = settings.get("model")
        if model is None:
            model = build_random_qwen3(spec, seed=int(settings.get("seed", 0)),
                                       device="cuda", layers=settings.get("layers"))
        chunk = int(settings.get("chunk_tokens") or budgets.chunk_budget(spec, context.device))
        n_pages = settings.get("n_pages")
        if n_pages is None:
            n_pages, _ = budgets.arena_pages(spec, context.device, chunk)
        arena = KVArena(len(model.model.layers), int(n_pages), budgets.PAGE_TOKENS,
                        spec.n_kv, spec.d_head, dtype=torch.bfloat16, device="cuda")
        pipeline = build_pipeline(spec, model, arena, **settings.get("engine_options", {}))
        execution = QuailModelExecution(context, model=model, arena=arena, pipeline=pipeline)
        execution._state["chunk_tokens"] = chunk
        return execution


    def plan(self, region, context):
        """ModelBackend.plan (base.py:62-67; backend.py:346-400). Planning -
        filter ordering, join search, prefix-sharing and tree-attention
        rules - is the reference's planner (quail/planner), which quail_amd
        does not carry; it executes the physical nodes that
        planner produces. Raises NotImplementedError."""
        raise NotImplementedError(
            "QuailBackend.plan: quail_amd carries the executor, not the planner "
            "(quail/planner); plan with the reference's QuailBackend.plan and run its "
            "AiFilter/AiJoin nodes through QuailBackend().start(GpuContext).execute(node, inputs)")

    def prepare_request(self, context) -> None:
        """Boot ahead of a request (backend.py:466-468): part of the request
        runner, which quail_amd does not carry. Raises NotImplementedError."""
        raise NotImplementedError(
            "QuailBackend.prepare_request: the request runner (worker.py) is not part of "
            "quail_amd; start(GpuContext) boots the GPU")

    def execute_request(self, context):
        """ModelBackend.execute_request (base.py:69-75; backend.py:470-472):
        the compute-process request runner (worker.py, graph.py) around the
        executor, which quail_amd does not carry. Raises
        NotImplementedError."""
        raise NotImplementedError(
            "QuailBackend.execute_request: the request runner (worker.py, graph.py) is not "
            "part of quail_amd; run each node with "
            "QuailBackend().start(GpuContext).execute(node, inputs)")


def device_spec(name: str) -> DeviceSpec:
    try:
        return DEVICES[name]
    except KeyError:
        raise ValueError(f"unknown device {name!r}; known: {sorted(DEVICES)}") from None
