"""The reference's forward loop drives quail_amd's Engine (MI355X only).

reference_call_sequence() issues the Engine calls the reference's
Qwen3Pipeline.forward_chunk makes (quail/backends/quail/executor/models/
qwen3.py:46-77), in its order and with its arguments: embedding, norm_quant,
gemm, qk_norm_rope -> (q, k), v as a strided view of the qkv output,
attention(q, k, v, chunk), gemm, norm_quant with the residual, gemm of
gate_up, activation_quant, gemm of down, index_select of the final rows and
fused_add_rms_norm. quail_amd's own pipeline fuses several of those steps
(q/k norm + RoPE writing the arena, gate_up + SiLU + quant, gather + final
norm); every fusion is bit-identical to its parts, so the two loops must
produce identical final rows, on both attention paths.
"""

import pytest
import torch

from e2e_support import TINY, TINY_FALSE, TINY_TRUE, tiny_model, tiny_workload
from quail_amd import loop
from quail_amd.arena import KVArena
from quail_amd.qwen3 import Qwen3Pipeline
from quail_amd.readout import AnswerRows, AsyncAnswers
from quail_amd.tokens import prefix_tree

pytestmark = pytest.mark.gpu


def reference_call_sequence(pipe, chunk):
    engine = pipe.engine
    meta = chunk.meta
    meta["layer"] = 0
    positions = chunk.positions
    hidden = torch.nn.functional.embedding(chunk.input_ids, pipe.embed.weight)
    residual = None
    for layer in pipe.layers:
        attn = layer.self_attn
        if residual is None:
            residual = hidden
            q_in, q_scale = engine.norm_quant(hidden, layer.input_layernorm)
        else:
            q_in, q_scale = engine.norm_quant(hidden, layer.input_layernorm, residual)
        qkv = engine.gemm(q_in, q_scale, attn.qkv_proj)
        q, k = engine.qk_norm_rope(qkv, positions, attn)
        v = qkv[:, (engine.num_q_heads + engine.num_kv_heads) * engine.head_dim:]
        o_in, o_scale = engine.attention(q, k, v, chunk)
        hidden = engine.gemm(o_in, o_scale, attn.o_proj)
        g_in, g_scale = engine.norm_quant(hidden, layer.post_attention_layernorm, residual)
        gate_up = engine.gemm(g_in, g_scale, layer.mlp.gate_up_proj)
        d_in, d_scale = engine.activation_quant(gate_up)
        hidden = engine.gemm(d_in, d_scale, layer.mlp.down_proj)
    final = chunk.final_indices
    last_hidden = hidden.index_select(0, final)
    last_residual = residual.index_select(0, final)
    normed, _ = engine.fused_add_rms_norm(last_hidden, last_residual, pipe.final_norm)
    return normed


@pytest.mark.parametrize("path", ["unified", "tree"])
def test_reference_call_sequence_matches_the_fused_pipeline(path):
    model = tiny_model(seed=5)
    # a checkpoint-style linear: block scales under weight_scale_inv only
    for layer in model.model.layers:
        for lin in (layer.self_attn.qkv_proj, layer.self_attn.o_proj,
                    layer.mlp.gate_up_proj, layer.mlp.down_proj):
            del lin.weight_scale
    docs, tail = tiny_workload(seed=6, n_rows=24)
    arena = KVArena(TINY.layers, 200, 16, TINY.n_kv, TINY.d_head, device="cuda")
    pipe = Qwen3Pipeline(model, arena, spec=TINY, kernels="quail")
    compared = []

    class Both:
        tree_attention, canvas_ids, needs_pages = True, (), False

        def forward_chunk(self, chunk):
            ours = pipe.forward_chunk(chunk)
            theirs = reference_call_sequence(pipe, chunk)
            compared.append((chunk.attention_mode, ours.cpu(), theirs.cpu()))
            if chunk.attention_mode == "unified" and chunk.meta["unified"] is not None:
                # attention_unified is the bf16 call; quant of it is attention()
                n = chunk.input_ids.numel()
                layer0 = pipe.layers[0].self_attn
                q_in, q_s = pipe.engine.norm_quant(
                    pipe.embed.weight.index_select(0, chunk.input_ids),
                    pipe.layers[0].input_layernorm)
                qkv = pipe.engine.gemm(q_in, q_s, layer0.qkv_proj)
                q, k, v = pipe.engine.qkv_norm_rope(qkv, chunk.positions, layer0)
                H, KH, D = TINY.n_q, TINY.n_kv, TINY.d_head
                chunk.meta["layer"] = 0
                bf = pipe.engine.attention_unified(q.view(n, H, D), k.view(n, KH, D),
                                                   v.view(n, KH, D), chunk.meta)
                assert bf.dtype == torch.bfloat16 and bf.shape == (n, H * D)
                chunk.meta["layer"] = 0
                q8, s8 = pipe.engine.attention(q, k, v, chunk)
                r8, rs = pipe.engine.quant(bf)
                assert torch.equal(q8.view(torch.uint8), r8.view(torch.uint8))
                assert torch.equal(s8, rs)
            return ours

    ans = AsyncAnswers(torch, AnswerRows(torch, model, TINY_TRUE, TINY_FALSE))
    stream = loop.FilterStream(torch, arena, Both(), ans, docs, [list(tail)], 900,
                               arena_writes=True, attention_mode=path,
                               prefix_tree=prefix_tree(docs, 16))
    while not stream.done:
        stream.next()
    torch.cuda.synchronize()
    assert len(compared) >= 2 and all(mode == path for mode, _, _ in compared)
    for _, ours, theirs in compared:
        assert torch.equal(ours.view(torch.int16), theirs.view(torch.int16))
