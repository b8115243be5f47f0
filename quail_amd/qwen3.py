"""The Qwen3 forward pass over the engine (quail/backends/quail/executor/models/).

ModelPipeline is the contract between the chunk loop and a model family
(models/base.py:11-47); Qwen3Pipeline is the Qwen3 layer loop
(models/qwen3.py:46-77): input RMSNorm + fp8 quant, QKV GEMM, per-head Q/K
RMSNorm + rotary, attention, O GEMM, post-attention RMSNorm + quant (adds
the residual), gate_up GEMM + SiLU gate + quant (one fused kernel), down
GEMM; after the last layer the answer rows are gathered and final-normed.
In the last layer the answer rows are gathered right after attention
instead: from o_proj on every op is row-wise and only those rows are read.
"""

from quail_amd import kernels
from quail_amd.engine import Engine


class ModelPipeline:
    engine = None
    max_chunk_tokens = None
    canvas_ids = ()
    canvas_answer_row = 0
    needs_pages = False
    tree_attention = True
    gemm_warmup = True

    def forward_chunk(self, chunk):
        raise NotImplementedError

    def linears(self):
        raise NotImplementedError


class Qwen3Pipeline(ModelPipeline):
    """Forward passes for a Qwen3-architecture fp8 model."""

    def __init__(self, model, arena, *, spec=None, kernels="quail",
                 engine_class=Engine, **engine_options):
        """The reference's constructor (models/qwen3.py:21-38); engine_options
        (ue8m0, gemm_hook, attention_hook, tree_kernel, fuse_kv_write,
        fuse_qkv_epilogue) go to quail_amd's Engine."""
        import torch
        self.layers = model.model.layers
        self.embed = model.model.embed_tokens
        self.final_norm = model.model.norm
        attn = self.layers[0].self_attn
        fp8 = attn.qkv_proj.weight.dtype == torch.float8_e4m3fn
        self.engine = engine_class(arena, n_q=attn.num_heads, n_kv=attn.num_kv_heads,
                                   head_dim=attn.head_dim, rotary=attn.rotary_emb,
                                   fp8=fp8, kernels=kernels, **engine_options)
        self.tree_attention = fp8
        widest = max(max(layer.self_attn.qkv_proj.weight.shape[0],
                         layer.mlp.gate_up_proj.weight.shape[0]) for layer in self.layers)
        self.max_chunk_tokens = (2**31 - 1) // widest

    def linears(self):
        layer = self.layers[0]
        return (layer.self_attn.qkv_proj, layer.self_attn.o_proj,
                layer.mlp.gate_up_proj, layer.mlp.down_proj)

    trace = None   # optional callable(layer, hidden, residual) at each layer's input
    # The last layer's o_proj, post-attention norm and MLP on the answer rows
    # only (its attention still writes every row's K/V). Off while a trace
    # is attached, which reads every row of every layer.
    prune_last_layer = True

    def forward_chunk(self, chunk):
        """The final-normed hidden state of chunk.final_indices, [R, hidden] bf16."""
        engine = self.engine
        trace = self.trace
        meta = chunk.meta
        meta["layer"] = 0
        positions = chunk.positions
        hidden = kernels.gather_rows(self.embed.weight, chunk.input_ids)
        residual = None
        prune_at = -1
        if self.prune_last_layer and trace is None and chunk.final_indices.numel() > 0:
            prune_at = len(self.layers) - 1
        for index, layer in enumerate(self.layers):
            if trace is not None:
                trace(index, hidden, residual)
            attn = layer.self_attn
            if residual is None:
                residual = hidden
                q_in, q_scale = engine.norm_quant(hidden, layer.input_layernorm)
            else:
                q_in, q_scale = engine.norm_quant(hidden, layer.input_layernorm, residual)
            # qkv GEMM, q/k norm + RoPE, KV write and attention
            # (models/qwen3.py:60-65); the norm and rotary in the GEMM's epilogue
            o_in, o_scale = engine.qkv_project_attention(q_in, q_scale, attn, positions, chunk)
            if index == prune_at:
                o_in, o_scale, residual = engine.select_rows(o_in, o_scale, residual,
                                                             chunk.final_indices)
            hidden = engine.gemm(o_in, o_scale, attn.o_proj, "o")
            g_in, g_scale = engine.norm_quant(hidden, layer.post_attention_layernorm,
                                              residual)
            # gate_up GEMM + SiLU gate + quant (models/qwen3.py:113-116), fused
            d_in, d_scale = engine.gemm_silu_quant(g_in, g_scale, layer.mlp.gate_up_proj)
            hidden = engine.gemm(d_in, d_scale, layer.mlp.down_proj, "down")
        if trace is not None:
            trace(len(self.layers), hidden, residual)
        if prune_at >= 0:
            normed, _ = engine.fused_add_rms_norm(hidden, residual, self.final_norm)
            return normed
        return engine.fused_add_rms_norm_rows(hidden, residual, chunk.final_indices,
                                              self.final_norm)


PIPELINES = {"qwen3": Qwen3Pipeline}


def build_pipeline(spec, model, arena, **kwargs):
    try:
        cls = PIPELINES[spec.arch]
    except KeyError:
        raise ValueError(f"no forward pass for architecture {spec.arch!r}; "
                         f"known: {sorted(PIPELINES)}") from None
    return cls(model, arena, spec=spec, **kwargs)
