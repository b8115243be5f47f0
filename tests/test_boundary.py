"""The drop-in boundary on the CPU: the reference's callers construct and
call quail_amd's Engine, pipeline and backend without changes.

- Engine is built exactly the way the reference's Qwen3Pipeline builds it
  (quail/backends/quail/executor/models/qwen3.py:26-29: positional arena,
  keyword geometry, fp8=, kernels=);
- weight_scale reads weight_scale, else weight_scale_inv (attention.py:121-127),
  the name vLLM's block-fp8 linears carry;
- QuailBackend.supports admits mi355x (the reference's allow-list,
  backend.py:333-344, is the gate this replaces);
- KVArena.paged_kv gives the reference's (pages, 16, n_kv, d) views of the
  MI355X pools, and layer_kv row-indexed pools over the reference's flat
  row numbering (reads and writes).
"""

from types import SimpleNamespace

import pytest
import torch

from quail_amd import budgets, layout
from quail_amd.arena import KVArena
from quail_amd.backend import (FilterNode, GpuContext, JoinNode, JoinStage, QuailBackend,
                               QuailModelExecution, SupportResult)
from quail_amd.engine import Engine
from quail_amd.qwen3 import Qwen3Pipeline
from quail_amd.specs import H100_SXM, MI355X, QWEN3_4B_FP8, ModelSpec


def _linear(n_out, n_in, scale_name):
    w = torch.zeros(n_out, n_in, dtype=torch.float8_e4m3fn)
    s = torch.full((n_out // 128, n_in // 128), 0.5)
    return SimpleNamespace(weight=w, **{scale_name: s})


def _tiny_model(scale_name="weight_scale_inv"):
    norm = SimpleNamespace(weight=torch.ones(128, dtype=torch.bfloat16), variance_epsilon=1e-6)
    rotary = SimpleNamespace(cos_sin_cache=torch.zeros(64, 128, dtype=torch.bfloat16))
    attn = SimpleNamespace(qkv_proj=_linear(768, 256, scale_name),
                           o_proj=_linear(256, 512, scale_name), q_norm=norm, k_norm=norm,
                           num_heads=4, num_kv_heads=1, head_dim=128, rotary_emb=rotary)
    mlp = SimpleNamespace(gate_up_proj=_linear(1024, 256, scale_name),
                          down_proj=_linear(256, 512, scale_name))
    layer = SimpleNamespace(self_attn=attn, mlp=mlp, input_layernorm=norm,
                            post_attention_layernorm=norm)
    inner = SimpleNamespace(layers=[layer], embed_tokens=SimpleNamespace(
        weight=torch.zeros(32, 256, dtype=torch.bfloat16)), norm=norm)
    return SimpleNamespace(model=inner)


def test_engine_builds_the_way_the_reference_pipeline_builds_it():
    arena = KVArena(1, 8, 16, 1, 128, device="cpu", allocate=False)
    attn = _tiny_model().model.layers[0].self_attn
    # models/qwen3.py:26-29, argument for argument
    engine = Engine(arena, n_q=attn.num_heads, n_kv=attn.num_kv_heads,
                    head_dim=attn.head_dim, rotary=attn.rotary_emb, fp8=True, kernels="quail")
    assert engine.kernels == "quail" and engine.is_fp8
    assert (engine.num_q_heads, engine.num_kv_heads, engine.head_dim) == (4, 1, 128)
    assert engine.softmax_scale == pytest.approx(128 ** -0.5)
    with pytest.raises(ValueError, match="vLLM kernel set"):
        Engine(arena, n_q=4, n_kv=1, head_dim=128, rotary=attn.rotary_emb, fp8=True,
               kernels="vllm")
    with pytest.raises(ValueError, match="kernels must be"):
        Engine(arena, n_q=4, n_kv=1, head_dim=128, rotary=attn.rotary_emb, fp8=True,
               kernels="triton")
    with pytest.raises(ValueError, match="fp8"):
        Engine(arena, n_q=4, n_kv=1, head_dim=128, rotary=attn.rotary_emb, fp8=False)


def test_pipeline_takes_the_reference_constructor():
    arena = KVArena(1, 8, 16, 1, 128, device="cpu", allocate=False)
    model = _tiny_model()
    pipe = Qwen3Pipeline(model, arena, spec=None, kernels="quail", engine_class=Engine)
    assert pipe.tree_attention
    assert pipe.max_chunk_tokens == (2 ** 31 - 1) // 1024
    assert isinstance(pipe.engine, Engine)


@pytest.mark.parametrize("name", ["weight_scale", "weight_scale_inv"])
def test_weight_scale_reads_either_vllm_name(name):
    lin = _linear(256, 256, name)
    assert Engine.weight_scale(lin) is getattr(lin, name)


def test_weight_scale_prefers_weight_scale_and_raises_on_neither():
    a, b = torch.ones(1, 1), torch.zeros(1, 1)
    assert Engine.weight_scale(SimpleNamespace(weight_scale=a, weight_scale_inv=b)) is a
    with pytest.raises(AttributeError, match="no weight scale"):
        Engine.weight_scale(SimpleNamespace(weight=None))


def test_ue8m0_scale_check_reads_weight_scale_inv():
    arena = KVArena(1, 8, 16, 1, 128, device="cpu", allocate=False)
    attn = _tiny_model().model.layers[0].self_attn
    engine = Engine(arena, n_q=4, n_kv=1, head_dim=128, rotary=attn.rotary_emb, fp8=True,
                    ue8m0=True)
    lin = _linear(256, 256, "weight_scale_inv")
    assert engine.hw_scales(lin)            # 0.5 is a power of two
    lin2 = _linear(256, 256, "weight_scale_inv")
    lin2.weight_scale_inv = torch.full((2, 2), 0.3)
    assert not engine.hw_scales(lin2)


def test_backend_admits_mi355x():
    backend = QuailBackend()
    assert backend.name == "quail"
    assert backend.supports(QWEN3_4B_FP8, MI355X, 1) == SupportResult.accept()
    rejected = backend.supports(QWEN3_4B_FP8, H100_SXM, 1)
    assert not rejected.supported and "h100-sxm" in rejected.reason
    other = ModelSpec(name="gemma", params=1e9, layers=2, hidden=256, n_q=2, n_kv=1,
                      d_head=128, ffn_width=1024, arch="diffusion_gemma")
    assert "diffusion_gemma" in backend.supports(other, MI355X, 1).reason
    assert not backend.supports(QWEN3_4B_FP8, MI355X, 8).supported
    with pytest.raises(ValueError, match="h100"):
        backend.start(GpuContext(0, 1, QWEN3_4B_FP8, H100_SXM, {}))


def test_execution_reports_missing_state_and_unknown_nodes():
    ctx = GpuContext(0, 1, QWEN3_4B_FP8, MI355X, {})
    ex = QuailModelExecution(ctx)
    with pytest.raises(RuntimeError, match="missing state"):
        ex.execute(FilterNode("docs", ((1, 2),)), {"document_ids": [0], "documents": [[5]]})
    with pytest.raises(TypeError, match="cannot execute"):
        ex.execute(SimpleNamespace(type_name="AiScore"), {})
    join = JoinNode("a", (JoinStage(0),))
    with pytest.raises(RuntimeError, match="missing state"):
        ex.execute(join, {"anchor_ids": [], "prefixes": [], "stage_suffixes": [[]]})


def test_backend_plan_and_request_runner_raise_clearly():
    backend = QuailBackend()
    for call in (lambda: backend.plan(None, None), lambda: backend.prepare_request(None),
                 lambda: backend.execute_request(None)):
        with pytest.raises(NotImplementedError, match="start\\(GpuContext\\)"):
            call()


def test_paged_kv_views_match_the_reference_row_numbering():
    arena = KVArena(1, 6, 16, 2, 128, device="cpu")
    kp, vp = arena.page_pools(0)
    kp.copy_(torch.randn(kp.shape).to(torch.bfloat16))
    vp.copy_(torch.randn(vp.shape).to(torch.bfloat16))
    kv, vv = arena.paged_kv(0)
    assert kv.shape == (6, 16, 2, 128) and vv.shape == (6, 16, 2, 128)
    # the reference's flat row r = page * 16 + slot holds [n_kv, d]
    k_rows, v_rows = layout.k_rows(kp), layout.v_rows(vp)
    for page, slot in ((0, 0), (3, 7), (5, 15)):
        assert torch.equal(kv[page, slot], k_rows[page * 16 + slot])
        assert torch.equal(vv[page, slot], v_rows[page * 16 + slot])
    # layer_kv: the reference's flat rows, read and written through the pages
    kf, vf = arena.layer_kv(0)
    assert kf.shape == (96, 2, 128) and vf.shape == (96, 2, 128) and len(kf) == 96
    rows = torch.tensor([5, 17, 95, 40])
    assert torch.equal(kf[rows], k_rows[rows]) and torch.equal(vf[rows], v_rows[rows])
    assert torch.equal(kf[33], k_rows[33]) and torch.equal(vf[-1], v_rows[95])
    assert torch.equal(vf[16:20], v_rows[16:20])
    new_k = torch.randn(4, 2, 128).to(torch.bfloat16)
    new_v = torch.randn(4, 2, 128).to(torch.bfloat16)
    kf[rows] = new_k
    vf[rows] = new_v
    want_k, want_v = k_rows.clone(), v_rows.clone()
    want_k[rows], want_v[rows] = new_k, new_v
    assert torch.equal(layout.k_rows(kp), want_k) and torch.equal(layout.v_rows(vp), want_v)
    with pytest.raises(IndexError):
        kf[torch.tensor([96])]


def test_backend_sizes_the_arena_with_the_reference_formula():
    chunk = budgets.chunk_budget(QWEN3_4B_FP8, MI355X)
    pages, _ = budgets.arena_pages(QWEN3_4B_FP8, MI355X, chunk)
    assert (chunk, pages) == (110_376, 106_394)
