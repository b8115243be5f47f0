"""End-to-end AI.IF on the GPU against the oracle (MI355X only).

A random-init Qwen3-architecture fp8 model filters rows sharing a 40-token
instruction, with a chunk budget small enough that page borrowing crosses
chunks; the oracle replays the exact chunks the GPU ran.

Dynamic 1x128 fp8 activation scales make a random model's forward chaotic
at the percent level: a one-ulp change in a group's largest value
re-quantizes the whole group. Two equally valid CPU restatements (fp64
block sums vs dequantize-then-fp32 GEMM) already differ by ~0.7% per layer
and disagree on ~1-2% of decisions, all within ~0.2 of a tie; the GPU adds
FlashAttention's bf16 P and bf16 output rounding (~0.1% per attention
output). The bars, written in the tests:
  - per stage, each kernel given the GPU's own input of that stage:
    within 1e-3 relative L2 of the oracle (2e-3 for attention's bf16 out);
  - teacher-forced per layer (the oracle layer gets the GPU's layer input,
    so drift cannot cascade across layers): down-projection output within
    8% relative L2 (worst row 20%), residual stream within 2%;
  - decisions, against the noise of the two oracle forms measured in the
    same test: every row whose margin lies beyond twice the 99th
    percentile of the oracles' margin shift is decided as the oracle
    decides it, the GPU's median margin shift is at most 2.5 times the
    oracle pair's, and it disagrees on at most about twice as many rows as
    the oracles do.
"""

from dataclasses import replace

import numpy as np
import pytest
import torch

from e2e_support import (TINY, TINY_FALSE, TINY_TRUE, decision_stats, describe, gpu_filter,
                         tiny_workload)
from oracle import forward as oforward
from quail_amd import loop
from quail_amd.arena import KVArena
from quail_amd.model import build_random_qwen3
from quail_amd.qwen3 import Qwen3Pipeline
from quail_amd.readout import AnswerRows, AsyncAnswers
from quail_amd.tokens import prefix_tree

pytestmark = pytest.mark.gpu


def _rel(x, y):
    x, y = x.float().cpu(), y.float().cpu()
    return ((x - y).norm() / y.norm()).item()


@pytest.mark.parametrize("path", ["unified", "tree"])
def test_every_layer_matches_the_oracle_teacher_forced(path):
    spec = replace(TINY, layers=4)
    model = build_random_qwen3(spec, seed=3, device="cuda", max_pos=2048,
                               answer_token_ids=TINY_TRUE + TINY_FALSE)
    docs, tail = tiny_workload(seed=4, n_rows=40)
    pages = 240
    arena = KVArena(spec.layers, pages, 16, spec.n_kv, spec.d_head, device="cuda")
    pipe = Qwen3Pipeline(model, arena, spec=spec)
    traces, hosts = [], []

    def trace(layer, hidden, residual):
        traces[-1].append((hidden.float().cpu(),
                           None if residual is None else residual.float().cpu()))

    class Rec:
        tree_attention, canvas_ids, needs_pages = True, (), False

        def forward_chunk(self, chunk):
            traces.append([])
            hosts.append((chunk.host, chunk.attention_mode))
            return pipe.forward_chunk(chunk)

    pipe.trace = trace
    ans = AsyncAnswers(torch, AnswerRows(torch, model, TINY_TRUE, TINY_FALSE))
    stream = loop.FilterStream(torch, arena, Rec(), ans, docs, [list(tail)], 1100,
                               arena_writes=True, attention_mode=path,
                               prefix_tree=prefix_tree(docs, 16))
    while not stream.done:
        stream.next()
    assert stream.chunks >= 3 and stream.sched.borrowing.borrowed_tokens > 0
    w = oforward.cpu_weights(model)
    oarena = oforward.OracleArena(spec.layers, pages, spec.n_kv, spec.d_head)
    report = []
    for (host, mode), layers in zip(hosts, traces):
        for li, L in enumerate(w["layers"]):
            h_in, r_in = layers[li]
            h_in = h_in.to(torch.bfloat16)
            r_in = None if r_in is None else r_in.to(torch.bfloat16)
            h_ref, r_ref = oforward.layer_step(L, li, h_in, r_in, host, mode, oarena)
            h_gpu, r_gpu = layers[li + 1]
            worst = ((h_gpu - h_ref.float()).norm(dim=1)
                     / h_ref.float().norm(dim=1).clamp(min=1e-6)).max().item()
            rec = (li, _rel(h_gpu, h_ref), worst, _rel(r_gpu, r_ref))
            report.append(rec)
            assert rec[1] < 0.08 and rec[2] < 0.20 and rec[3] < 0.02, f"layer {rec}"
    print("teacher-forced (layer, hidden rel, worst row, residual rel):",
          [tuple(round(x, 5) for x in r) for r in report[:6]])


@pytest.mark.parametrize("path", ["unified", "tree"])
def test_qwen3_32b_geometry_layers_match_the_oracle(path):
    """The Qwen3-32B layer geometry (hidden 5120, 64 query / 8 KV heads = GQA
    8:1, FFN 25,600: GEMMs (10240|5120|51200|5120) x (5120|8192|5120|25600))
    through two layers, teacher-forced against the oracle with the same bars."""
    from quail_amd.specs import QWEN3_32B_FP8
    spec = replace(QWEN3_32B_FP8, layers=2, vocab=4096, tied_head=True)
    model = build_random_qwen3(spec, seed=5, device="cuda", max_pos=2048,
                               answer_token_ids=TINY_TRUE + TINY_FALSE)
    docs, tail = tiny_workload(seed=6, n_rows=10, max_doc=80)
    pages = 120
    arena = KVArena(spec.layers, pages, 16, spec.n_kv, spec.d_head, device="cuda")
    pipe = Qwen3Pipeline(model, arena, spec=spec)
    traces, hosts = [], []

    def trace(layer, hidden, residual):
        traces[-1].append((hidden.float().cpu(),
                           None if residual is None else residual.float().cpu()))

    class Rec:
        tree_attention, canvas_ids, needs_pages = True, (), False

        def forward_chunk(self, chunk):
            traces.append([])
            hosts.append((chunk.host, chunk.attention_mode))
            return pipe.forward_chunk(chunk)

    pipe.trace = trace
    ans = AsyncAnswers(torch, AnswerRows(torch, model, TINY_TRUE, TINY_FALSE))
    stream = loop.FilterStream(torch, arena, Rec(), ans, docs, [list(tail)], 400,
                               arena_writes=True, attention_mode=path,
                               prefix_tree=prefix_tree(docs, 16))
    while not stream.done:
        stream.next()
    assert stream.chunks >= 2 and stream.sched.borrowing.borrowed_tokens > 0
    w = oforward.cpu_weights(model)
    oarena = oforward.OracleArena(spec.layers, pages, spec.n_kv, spec.d_head)
    for (host, mode), layers in zip(hosts, traces):
        for li, L in enumerate(w["layers"]):
            h_in, r_in = layers[li]
            h_in = h_in.to(torch.bfloat16)
            r_in = None if r_in is None else r_in.to(torch.bfloat16)
            h_ref, r_ref = oforward.layer_step(L, li, h_in, r_in, host, mode, oarena)
            h_gpu, r_gpu = layers[li + 1]
            worst = ((h_gpu - h_ref.float()).norm(dim=1)
                     / h_ref.float().norm(dim=1).clamp(min=1e-6)).max().item()
            rec = (li, _rel(h_gpu, h_ref), worst, _rel(r_gpu, r_ref))
            assert rec[1] < 0.08 and rec[2] < 0.20 and rec[3] < 0.02, f"layer {rec}"


@pytest.mark.parametrize("path", ["unified", "tree"])
def test_decisions_agree_outside_the_noise_band(path):
    model = build_random_qwen3(TINY, seed=3, device="cuda", max_pos=2048,
                               answer_token_ids=TINY_TRUE + TINY_FALSE)
    docs, tail = tiny_workload(seed=4, n_rows=400)
    pages = 400 * 14 + 64
    answers, margins, records, stream = gpu_filter(
        model, TINY, docs, tail, path=path, pages=pages, budget=2000,
        true_ids=TINY_TRUE, false_ids=TINY_FALSE)
    w = oforward.cpu_weights(model)
    a1 = oforward.OracleArena(TINY.layers, pages, TINY.n_kv, TINY.d_head)
    a2 = oforward.OracleArena(TINY.layers, pages, TINY.n_kv, TINY.d_head)
    dequant = oforward.DequantGemm()
    ref_bits, ref_margin, alt_bits, alt_margin = {}, {}, {}, {}
    for (host, mode, _), groups in zip(records, stream.packed_groups):
        n1 = oforward.forward_chunk(w, host, mode, a1)
        n2 = oforward.forward_chunk(w, host, mode, a2, gemm=dequant)
        b1, m1 = oforward.readout(w, n1, TINY_TRUE, TINY_FALSE)
        b2, m2 = oforward.readout(w, n2, TINY_TRUE, TINY_FALSE)
        for (doc, _, _), x1, y1, x2, y2 in zip(groups, b1.tolist(), m1.tolist(),
                                               b2.tolist(), m2.tolist()):
            ref_bits[doc], ref_margin[doc], alt_bits[doc], alt_margin[doc] = x1, y1, x2, y2
    n = len(docs)
    stats = decision_stats((answers, margins), (ref_bits, ref_margin), (alt_bits, alt_margin))
    print(f"{path}: {describe(stats)}; oracle margins of the rows decided differently "
          f"{stats['disagree_margins']}", flush=True)
    # the bars are the oracle pair's own noise, measured here: every row whose
    # fp64 margin lies beyond twice the 99th-percentile oracle shift is
    # decided as the oracle decides it; the GPU's margins move at most 2.5
    # times as far as the oracle pair's (median; measured 1.8-1.85: the GPU
    # differs from the fp64 oracle in GEMM block sums, attention's bf16
    # roundings and norm summation orders, the fp32 oracle in GEMM order
    # only, and taking any one of the three from the oracle leaves the
    # shift within 0.035-0.049 against the GPU's 0.039); and it disagrees
    # with the fp64 oracle on at most twice as many rows as the fp32 oracle
    # does, plus three Poisson standard deviations of that count
    assert stats["gpu_agree_wide"] == stats["outside_wide"], stats
    assert stats["gpu_shift_median"] <= 2.5 * stats["oracle_shift_median"] + 1e-3, stats
    pair = n - stats["floor"]
    assert n - stats["gpu_agree"] <= 2 * pair + 3.0 * max(1.0, (2 * pair) ** 0.5), stats


def test_ue8m0_mode_runs_the_mfma_scaled_gemms_and_agrees_with_the_oracle():
    """UE8M0 mode end to end: power-of-two weight block scales and UE8M0
    activation quantization, so every GEMM runs with the MFMA applying the
    scales (qh_fp8_gemm_nt_ue8m0, qh_fp8_gemm_silu_quant_ue8m0). The oracle
    replays the chunks in UE8M0 mode; decisions agree outside the noise band
    as in fp32-scale mode."""
    model = build_random_qwen3(TINY, seed=5, device="cuda", max_pos=2048,
                               answer_token_ids=TINY_TRUE + TINY_FALSE, ue8m0=True)
    docs, tail = tiny_workload(seed=6, n_rows=64)
    pages = 300
    answers, margins, records, stream = gpu_filter(
        model, TINY, docs, tail, path="unified", pages=pages, budget=2000,
        true_ids=TINY_TRUE, false_ids=TINY_FALSE, ue8m0=True)
    layer = model.model.layers[0]
    for lin in (layer.self_attn.qkv_proj, layer.self_attn.o_proj, layer.mlp.gate_up_proj,
                layer.mlp.down_proj):
        assert getattr(lin, "quail_ue8m0_scales", False) is True
    w = oforward.cpu_weights(model)
    arena = oforward.OracleArena(TINY.layers, pages, TINY.n_kv, TINY.d_head)
    ref_bits, ref_m = {}, {}
    for (host, mode, _), groups in zip(records, stream.packed_groups):
        normed = oforward.forward_chunk(w, host, mode, arena, ue8m0=True)
        b, m = oforward.readout(w, normed, TINY_TRUE, TINY_FALSE)
        for (doc, _, _), x, y in zip(groups, b.tolist(), m.tolist()):
            ref_bits[doc], ref_m[doc] = x, y
    n = len(docs)
    agree = sum(answers[d] == ref_bits[d] for d in range(n))
    for d in range(n):
        if answers[d] != ref_bits[d]:
            assert abs(ref_m[d]) <= 0.25, f"row {d}: decision differs at margin {ref_m[d]:.4f}"
    assert agree >= 0.95 * n, f"GPU agrees on {agree}/{n}"
    print(f"ue8m0: GPU-vs-oracle {agree}/{n}")


def test_each_layer_stage_matches_the_oracle_on_identical_inputs():
    import math
    from oracle import ops
    from quail_amd import kernels as K, layout
    from e2e_support import tiny_model
    model = tiny_model(seed=3)
    docs, tail = tiny_workload(seed=4, n_rows=6)
    arena = KVArena(2, 200, 16, TINY.n_kv, TINY.d_head, device="cuda")
    groups = []
    for i in range(6):
        arena.activate(("d", i), len(docs[i]), capacity_tokens=len(docs[i]) + 9)
        groups.append(dict(key=("d", i), prefix=docs[i], f=len(docs[i]), suffixes=[list(tail)]))
    chunk = loop.pack_chunk(torch, arena, groups, attention_mode="unified")
    h = chunk.host
    L = model.model.layers[0]
    a = L.self_attn
    cpu = lambda t: t.cpu()
    emb = K.gather_rows(model.model.embed_tokens.weight, chunk.input_ids)
    assert torch.equal(cpu(emb), model.model.embed_tokens.weight.cpu()[torch.from_numpy(h["input_ids"])])
    qi, qs = K.add_rmsnorm_quant(emb, L.input_layernorm.weight, 1e-6)
    qr, sr = ops.norm_quant_plain(cpu(emb), cpu(L.input_layernorm.weight), 1e-6)
    assert _rel(ops.dequant_rows(cpu(qi), cpu(qs)), ops.dequant_rows(qr, sr)) < 1e-3
    gemm_ref = lambda x, s, lin: ops.fp8_gemm(cpu(x), cpu(s).contiguous(), cpu(lin.weight),
                                              cpu(lin.weight_scale))
    qkv = K.fp8_gemm_nt(qi, qs, a.qkv_proj.weight, a.qkv_proj.weight_scale)
    assert _rel(qkv, gemm_ref(qi, qs, a.qkv_proj)) < 1e-3
    cs = model.rotary.cos_sin_cache
    q, k, v = K.qk_norm_rope(qkv, chunk.positions, cs, a.q_norm.weight, a.k_norm.weight,
                             1e-6, 8, 2, 128)
    q2, k2, v2 = ops.qk_norm_rope(cpu(qkv), torch.from_numpy(h["positions"]), cpu(cs),
                                  cpu(a.q_norm.weight), cpu(a.k_norm.weight), 1e-6, 8, 2, 128)
    assert _rel(q, q2) < 1e-3 and _rel(k, k2) < 1e-3 and torch.equal(cpu(v), v2)
    T = q.shape[0]
    u = chunk.meta["unified"]
    kp, vp = arena.page_pools(0)
    K.kv_row_scatter(k.view(T, 2, 128), v.view(T, 2, 128), kp, vp, u["src"], u["dst"])
    out, _ = K.attention(q.view(T, 8, 128), u["cu_q"], u["used"], n_queries=T,
                         max_q=u["max_q"], softmax_scale=1 / math.sqrt(128), causal=True,
                         k_pool=kp, v_pool=vp, table=u["table"], n_kv=2)
    out_ref, _ = ops.paged_attention(cpu(q).view(T, 8, 128), layout.k_rows(cpu(kp)),
                                     layout.v_rows(cpu(vp)),
                                     torch.from_numpy(h["unified_cu_q"]),
                                     torch.from_numpy(h["unified_used"]),
                                     torch.from_numpy(h["unified_table"]),
                                     1 / math.sqrt(128), True)
    assert _rel(out, out_ref) < 2e-3
    oq, os_ = K.group_quant(out.view(T, -1))
    hid = K.fp8_gemm_nt(oq, os_, a.o_proj.weight, a.o_proj.weight_scale)
    assert _rel(hid, gemm_ref(oq, os_, a.o_proj)) < 1e-3
    res = emb.clone()
    gq, gs = K.add_rmsnorm_quant(hid, L.post_attention_layernorm.weight, 1e-6, residual=res)
    gqr, gsr, resr = ops.add_rms_norm_quant(cpu(hid), cpu(emb), cpu(L.post_attention_layernorm.weight), 1e-6)
    assert torch.equal(cpu(res), resr)
    assert _rel(ops.dequant_rows(cpu(gq), cpu(gs)), ops.dequant_rows(gqr, gsr)) < 1e-3
    gu = K.fp8_gemm_nt(gq, gs, L.mlp.gate_up_proj.weight, L.mlp.gate_up_proj.weight_scale)
    assert _rel(gu, gemm_ref(gq, gs, L.mlp.gate_up_proj)) < 1e-3
    dq, ds = K.silu_mul_quant(gu)
    dqr, dsr = ops.silu_mul_quant(cpu(gu))
    assert _rel(ops.dequant_rows(cpu(dq), cpu(ds)), ops.dequant_rows(dqr, dsr)) < 1e-3
    dn = K.fp8_gemm_nt(dq, ds, L.mlp.down_proj.weight, L.mlp.down_proj.weight_scale)
    assert _rel(dn, gemm_ref(dq, ds, L.mlp.down_proj)) < 1e-3


def test_unified_and_tree_paths_agree_on_the_gpu():
    model = build_random_qwen3(TINY, seed=5, device="cuda", max_pos=2048,
                               answer_token_ids=TINY_TRUE + TINY_FALSE)
    docs, tail = tiny_workload(seed=6, n_rows=32)
    a, ma, _, _ = gpu_filter(model, TINY, docs, tail, path="unified", pages=160,
                             budget=900, true_ids=TINY_TRUE, false_ids=TINY_FALSE)
    b, mb, _, _ = gpu_filter(model, TINY, docs, tail, path="tree", pages=160,
                             budget=900, true_ids=TINY_TRUE, false_ids=TINY_FALSE)
    for d in range(len(docs)):
        if a[d] != b[d]:
            assert abs(ma[d]) <= 0.25 and abs(mb[d]) <= 0.25, f"row {d}"


def test_node_resident_tree_kernel_gives_the_same_answers():
    """The tree path with tree_kernel="resident" (each node's K/V held in
    LDS; every read table of this workload fits 16 pages) against the
    streaming kernel: the same answers and margins, bit for bit."""
    model = build_random_qwen3(TINY, seed=5, device="cuda", max_pos=2048,
                               answer_token_ids=TINY_TRUE + TINY_FALSE)
    docs, tail = tiny_workload(seed=7, n_rows=32)
    runs = [gpu_filter(model, TINY, docs, tail, path="tree", pages=160, budget=900,
                       true_ids=TINY_TRUE, false_ids=TINY_FALSE, tree_kernel=kind)
            for kind in ("fused", "resident")]
    (a, ma, _, _), (b, mb, _, _) = runs
    assert a == b
    assert ma == mb


def test_fused_kv_write_gives_the_same_answers():
    """The unified path with q/k norm + RoPE writing k and v into the arena
    itself answers every row with the same margins, bit for bit, as with the
    separate k/v rows and scatter."""
    model = build_random_qwen3(TINY, seed=9, device="cuda", max_pos=2048,
                               answer_token_ids=TINY_TRUE + TINY_FALSE)
    docs, tail = tiny_workload(seed=10, n_rows=24)
    runs = []
    for fuse in (False, True):
        arena = KVArena(len(model.model.layers), 160, 16, TINY.n_kv, TINY.d_head,
                        dtype=torch.bfloat16, device="cuda")
        pipe = Qwen3Pipeline(model, arena, spec=TINY, fuse_kv_write=fuse)
        rows = AnswerRows(torch, model, TINY_TRUE, TINY_FALSE)
        ans = AsyncAnswers(torch, rows, keep_margins=True)
        stream = loop.FilterStream(torch, arena, pipe, ans, docs, [list(tail)], 900,
                                   arena_writes=True, attention_mode="unified",
                                   prefix_tree=prefix_tree(docs, 16))
        while not stream.done:
            stream.next()
        torch.cuda.synchronize()
        runs.append(([stream.answers[d][0] for d in range(len(docs))],
                     [float(m) for ms in ans.margins for m in ms]))
    assert runs[0] == runs[1]


@pytest.mark.gpu
def test_filter_from_a_token_store_matches_in_memory_documents(tmp_path):
    """The same rows read from a memory-mapped Arrow token store (int32 ids,
    several record batches) pack the same chunks and give the same answers
    and margins, bit for bit."""
    from quail_amd.tokens import TokenStore
    model = build_random_qwen3(TINY, seed=7, device="cuda", max_pos=2048,
                               answer_token_ids=TINY_TRUE + TINY_FALSE)
    docs, tail = tiny_workload(seed=8, n_rows=24)
    store = TokenStore.from_documents(str(tmp_path / "rows.arrow"), docs, batch_rows=5)
    a, ma, ra, _ = gpu_filter(model, TINY, docs, tail, path="tree", pages=160,
                              budget=900, true_ids=TINY_TRUE, false_ids=TINY_FALSE)
    b, mb, rb, _ = gpu_filter(model, TINY, store, tail, path="tree", pages=160,
                              budget=900, true_ids=TINY_TRUE, false_ids=TINY_FALSE)
    assert a == b and ma == mb
    assert len(ra) == len(rb)
    for (ha, _, _), (hb, _, _) in zip(ra, rb):
        assert np.array_equal(ha["input_ids"], hb["input_ids"])
        assert np.array_equal(ha["positions"], hb["positions"])


@pytest.mark.parametrize("path", ["unified", "tree"])
def test_join_layers_match_the_oracle_teacher_forced(path):
    """An AI join (anchors sharing a 40-token root, a frame entry, partner
    streams cut across chunks; unified temporaries with kept-tail copies or
    tree reads of the anchor) through 3 layers, teacher-forced against the
    oracle replaying the same chunks, with the filter's bars."""
    from e2e_support import tiny_join
    spec = replace(TINY, layers=3)
    model = build_random_qwen3(spec, seed=8, device="cuda", max_pos=2048,
                               answer_token_ids=TINY_TRUE + TINY_FALSE)
    anchors, frame, partners = tiny_join(seed=9, n_anchors=6, n_partners=13)
    pages = 200
    arena = KVArena(spec.layers, pages, 16, spec.n_kv, spec.d_head, device="cuda")
    pipe = Qwen3Pipeline(model, arena, spec=spec)
    traces, hosts = [], []

    def trace(layer, hidden, residual):
        traces[-1].append((hidden.float().cpu(),
                           None if residual is None else residual.float().cpu()))

    class Rec:
        tree_attention, canvas_ids, needs_pages = True, (), False

        def forward_chunk(self, chunk):
            traces.append([])
            hosts.append((chunk.host, chunk.attention_mode))
            return pipe.forward_chunk(chunk)

    pipe.trace = trace
    ans = AsyncAnswers(torch, AnswerRows(torch, model, TINY_TRUE, TINY_FALSE))
    stats = {}
    out, _, _ = loop.run_join(torch, arena, Rec(), ans, [list(a) for a in anchors],
                              [[list(p) for p in partners]], 300, stage_frames=[list(frame)],
                              attention_mode=path, prefix_tree=prefix_tree(anchors, 16),
                              stats=stats)
    assert stats["chunks"] >= 3 and stats["borrowed_tokens"] > 0
    assert sorted(out[0]) == list(range(len(anchors)))
    assert all(len(row) == len(partners) for row in out[0].values())
    if path == "unified":
        assert any("tail_src" in host for host, _ in hosts)
    else:
        assert any("reads_rows" in host for host, _ in hosts)
    w = oforward.cpu_weights(model)
    oarena = oforward.OracleArena(spec.layers, pages, spec.n_kv, spec.d_head)
    for (host, mode), layers in zip(hosts, traces):
        for li, L in enumerate(w["layers"]):
            h_in, r_in = layers[li]
            h_in = h_in.to(torch.bfloat16)
            r_in = None if r_in is None else r_in.to(torch.bfloat16)
            h_ref, r_ref = oforward.layer_step(L, li, h_in, r_in, host, mode, oarena)
            h_gpu, r_gpu = layers[li + 1]
            worst = ((h_gpu - h_ref.float()).norm(dim=1)
                     / h_ref.float().norm(dim=1).clamp(min=1e-6)).max().item()
            rec = (li, _rel(h_gpu, h_ref), worst, _rel(r_gpu, r_ref))
            assert rec[1] < 0.08 and rec[2] < 0.20 and rec[3] < 0.02, f"layer {rec}"


def _join_decision_stats(records, margins, replays):
    """decision_stats over every final row of every chunk of a join, in chunk
    order: the GPU's margins (bit = margin > 0, the strict readout) against
    the fp64 and the fp32 oracle replays [(bits, margins) per chunk]."""
    gm = [float(v) for m in margins for v in m.tolist()]
    runs = []
    for replay in replays:
        bits = [int(x) for _, chunk_bits, _ in replay for x in chunk_bits.tolist()]
        marg = [float(x) for _, _, chunk_margins in replay for x in chunk_margins.tolist()]
        runs.append((bits, marg))
    assert len(gm) == len(runs[0][0]) == len(runs[1][0])
    return decision_stats(([int(v > 0) for v in gm], gm), runs[0], runs[1])


@pytest.mark.parametrize("path", ["unified", "tree"])
def test_join_decisions_agree_outside_the_noise_band(path):
    """Every final row of every chunk of a 2-stage join (frame entries
    included): GPU decisions against the oracle's two replays (fp64 block
    sums, dequantize-then-fp32 GEMMs), with the filter's bars measured
    against the pair's own noise: every row beyond twice the band (the p99
    of the pair's margin shift) decided as the fp64 oracle decides it, and
    at most twice the pair's disagreements plus three Poisson deviations."""
    from e2e_support import gpu_join, oracle_replay, tiny_join
    model = build_random_qwen3(TINY, seed=10, device="cuda", max_pos=2048,
                               answer_token_ids=TINY_TRUE + TINY_FALSE)
    anchors, frame, partners = tiny_join(seed=11, n_anchors=8, n_partners=12)
    pages = 300
    _, margins, records, stats = gpu_join(model, TINY, anchors, frame, partners, path=path,
                                          pages=pages, budget=400, true_ids=TINY_TRUE,
                                          false_ids=TINY_FALSE, stages=2)
    assert stats["chunks"] >= 3
    ref = oracle_replay(model, TINY, records, pages, TINY_TRUE, TINY_FALSE)
    alt = oracle_replay(model, TINY, records, pages, TINY_TRUE, TINY_FALSE,
                        gemm=oforward.DequantGemm())
    st = _join_decision_stats(records, margins, (ref, alt))
    print(f"join {path}: {describe(st)}", flush=True)
    n = st["rows"]
    assert n >= 8 * 12
    assert st["gpu_agree_wide"] == st["outside_wide"], st
    pair = n - st["floor"]
    assert n - st["gpu_agree"] <= 2 * pair + 3.0 * max(1.0, (2 * pair) ** 0.5), st


@pytest.mark.parametrize("path", ["tree", "unified"])
def test_qwen3_4b_join_decisions_at_full_depth_agree_within_the_oracle_floor(path):
    """The AI join at Qwen3-4B geometry, 36 layers: the first 6 anchors of
    the seeded join workload (48-token root + left document) x its first 32
    partners, budget 4,096 (several chunks, anchors borrowed across them);
    every final row against both oracle forms replayed on the GPU. Bars as
    for the filter at full depth: every row beyond twice the band agrees,
    and the GPU's agreement is within three binomial standard deviations of
    the oracle pair's."""
    from e2e_support import gpu_join
    from quail_amd.aiif import synthetic_join_workload
    from quail_amd.model import SYNTHETIC_FALSE_IDS, SYNTHETIC_TRUE_IDS
    from quail_amd.specs import QWEN3_4B_FP8

    spec = QWEN3_4B_FP8
    model = build_random_qwen3(spec, seed=0, device="cuda", max_pos=2048)
    anchors, frame, partners = synthetic_join_workload(256, 256, seed=0, vocab=spec.vocab)
    anchors, partners = anchors[:6], partners[:32]
    pages = 4000
    _, margins, records, stats = gpu_join(model, spec, anchors, frame, partners, path=path,
                                          pages=pages, budget=4096,
                                          true_ids=SYNTHETIC_TRUE_IDS,
                                          false_ids=SYNTHETIC_FALSE_IDS)
    assert stats["chunks"] >= 3 and all(mode == path for _, mode, _ in records)
    torch.backends.cuda.matmul.allow_tf32 = False
    w = oforward.oracle_weights(model, "cuda")
    replays = []
    for gemm in (oforward.exact_gemm, oforward.DequantGemm()):
        arena = oforward.OracleArena(spec.layers, pages, spec.n_kv, spec.d_head, device="cuda")
        out = []
        with torch.no_grad():
            for host, mode, _ in records:
                normed = oforward.forward_chunk(w, host, mode, arena, gemm=gemm)
                bits, margin = oforward.readout(w, normed, SYNTHETIC_TRUE_IDS,
                                                SYNTHETIC_FALSE_IDS)
                out.append((None, bits.cpu(), margin.cpu()))
        replays.append(out)
        del arena
        torch.cuda.empty_cache()
    st = _join_decision_stats(records, margins, replays)
    print(f"join 4B {path}: {stats['chunks']} chunks; {describe(st)}; oracle margins of the "
          f"rows decided differently {st['disagree_margins']}", flush=True)
    n = st["rows"]
    assert st["gpu_agree_wide"] == st["outside_wide"], st
    q = 1.0 - st["floor"] / n
    slack = 3.0 * (2.0 * n * q * (1.0 - q)) ** 0.5
    assert st["gpu_agree"] >= st["floor"] - slack, st


@pytest.mark.parametrize("path", ["unified", "tree"])
def test_qwen3_4b_decisions_agree_with_the_oracle_within_its_noise(path):
    """Full Qwen3-4B geometry (36 layers, random init) over the first 192
    rows of the seeded 4096-row filter workload, four chunks, on each
    attention path (the oracle replays the chunks on the path they ran).
    The oracle replays every chunk on the GPU (the same torch functions the
    CPU runs, on device tensors) twice: with fp64 block sums and with
    dequantize-then-fp32 GEMMs. The two are equally valid restatements, so
    their disagreement measures how well posed the decisions are.

    They are not well posed: 36 layers of dynamic 1x128 fp8 re-quantization
    amplify a one-ulp difference until the two oracles disagree on about
    one row in ten, with margin shifts as large as the median margin
    (scaling the layers' residual writes down by 10x does not change
    that). The band is the 99th percentile of the oracle pair's margin
    shift. Bars: every row whose fp64 margin lies beyond twice the band is
    decided as the fp64 oracle decides it, and the GPU agrees with that
    oracle as often as the other oracle does, within three binomial
    standard deviations of the two counts."""
    from quail_amd.aiif import synthetic_filter_workload
    from quail_amd.model import SYNTHETIC_FALSE_IDS, SYNTHETIC_TRUE_IDS
    from quail_amd.specs import QWEN3_4B_FP8

    spec = QWEN3_4B_FP8
    n = 192
    model = build_random_qwen3(spec, seed=0, device="cuda", max_pos=2048)
    instruction, documents, tail = synthetic_filter_workload(4096, seed=0, vocab=spec.vocab)
    docs = [np.concatenate([instruction, d]) for d in documents[:n]]
    pages = sum(-(-(len(d) + len(tail)) // 16) for d in docs) + 64
    answers, margins, records, stream = gpu_filter(
        model, spec, docs, tail, path=path, pages=pages, budget=16384,
        true_ids=SYNTHETIC_TRUE_IDS, false_ids=SYNTHETIC_FALSE_IDS)
    assert len(records) >= 3 and all(mode == path for _, mode, _ in records)
    print(f"{path}: {len(records)} chunks, "
          f"{sum(len(r[0]['positions']) for r in records)} tokens", flush=True)

    torch.backends.cuda.matmul.allow_tf32 = False
    w = oforward.oracle_weights(model, "cuda")
    runs = {}
    for name, gemm in (("fp64", oforward.exact_gemm), ("fp32", oforward.DequantGemm())):
        arena = oforward.OracleArena(spec.layers, pages, spec.n_kv, spec.d_head, device="cuda")
        bits, marg = {}, {}
        with torch.no_grad():
            for (host, mode, _), groups in zip(records, stream.packed_groups):
                normed = oforward.forward_chunk(w, host, mode, arena, gemm=gemm)
                b, m = oforward.readout(w, normed, SYNTHETIC_TRUE_IDS, SYNTHETIC_FALSE_IDS)
                for (doc, _, _), x, y in zip(groups, b.tolist(), m.tolist()):
                    bits[doc], marg[doc] = x, y
        runs[name] = (bits, marg)
        del arena
        torch.cuda.empty_cache()
    stats = decision_stats((answers, margins), runs["fp64"], runs["fp32"])
    print(f"{describe(stats)}; oracle margins of the rows decided differently "
          f"{stats['disagree_margins']}", flush=True)
    assert stats["gpu_agree_wide"] == stats["outside_wide"], stats
    floor, agree = stats["floor"], stats["gpu_agree"]
    q = 1.0 - floor / n
    slack = 3.0 * (2.0 * n * q * (1.0 - q)) ** 0.5
    assert agree >= floor - slack, f"GPU agrees on {agree}/{n}, the oracles on {floor}/{n}"


@pytest.mark.parametrize("path", ["unified", "tree"])
def test_last_layer_on_the_answer_rows_gives_the_same_rows(path):
    """The last layer's o_proj, post-attention norm and MLP run on the answer
    rows only (gathered after attention): every chunk's final-normed rows
    equal, bit for bit, those of the full last layer followed by the
    reference's index_select of the final rows, and so do the answers and
    margins."""
    model = build_random_qwen3(TINY, seed=11, device="cuda", max_pos=2048,
                               answer_token_ids=TINY_TRUE + TINY_FALSE)
    docs, tail = tiny_workload(seed=12, n_rows=28)
    runs = []
    for prune in (False, True):
        arena = KVArena(len(model.model.layers), 160, 16, TINY.n_kv, TINY.d_head,
                        dtype=torch.bfloat16, device="cuda")
        pipe = Qwen3Pipeline(model, arena, spec=TINY)
        pipe.prune_last_layer = prune
        normed = []

        class Rec:
            tree_attention, canvas_ids, needs_pages = True, (), False

            def forward_chunk(self, chunk):
                out = pipe.forward_chunk(chunk)
                normed.append(out.clone())
                return out

        rows = AnswerRows(torch, model, TINY_TRUE, TINY_FALSE)
        ans = AsyncAnswers(torch, rows, keep_margins=True)
        stream = loop.FilterStream(torch, arena, Rec(), ans, docs, [list(tail)], 900,
                                   arena_writes=True, attention_mode=path,
                                   prefix_tree=prefix_tree(docs, 16))
        while not stream.done:
            stream.next()
        torch.cuda.synchronize()
        assert stream.chunks >= 3
        runs.append((normed, [stream.answers[d][0] for d in range(len(docs))],
                     [float(m) for ms in ans.margins for m in ms]))
    (full, a_full, m_full), (pruned, a_pruned, m_pruned) = runs
    assert len(full) == len(pruned)
    for x, y in zip(full, pruned):
        assert x.shape == y.shape and torch.equal(x.view(torch.int16), y.view(torch.int16))
    assert a_full == a_pruned and m_full == m_pruned
