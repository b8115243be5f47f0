"""Pins of the CPU oracle: each function against a library routine, a closed
form, an invariant or the reference's own literal cases, chosen so that a
dropped term, a wrong sign/index or a transposed operand fails one of them.
"""

import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import forward as oforward
from oracle import ops


def gen(seed):
    return torch.Generator().manual_seed(seed)


# ---------------------------------------------------------------- fp8 quant

def test_group_quant_maps_amax_to_448_and_round_trips_within_half_a_step():
    x = torch.randn(16, 512, generator=gen(0)) * 5
    q, s = ops.group_quant(x)
    g = q.float().view(16, 4, 128)
    assert torch.equal(g.abs().amax(dim=2), torch.full((16, 4), 448.0))
    back = ops.dequant_rows(q, s)
    # e4m3 has 3 mantissa bits: relative half-step 2^-4, absolute floor at
    # the subnormal step 2^-9 * scale
    err = (back - x).abs()
    bound = x.abs() * 2 ** -4 + s.repeat_interleave(128, dim=1) * 2 ** -10
    assert (err <= bound + 1e-12).all()


def test_group_quant_ue8m0_scales_are_the_least_power_of_two_covering_amax():
    x = torch.randn(8, 256, generator=gen(1)) * 3
    _, s = ops.group_quant(x, ue8m0=True)
    amax = x.view(8, 2, 128).abs().amax(dim=2)
    e = torch.log2(s)
    assert torch.equal(e, torch.round(e))
    assert (s >= amax / 448).all() and (s / 2 < amax / 448).all()


def test_weight_block_quant_round_trip():
    w = torch.randn(256, 384, generator=gen(2)) * 0.02
    q, s = ops.quantize_weight_blocks(w)
    assert s.shape == (2, 3)
    back = ops.dequant_weight(q, s)
    assert (back - w).abs().max() <= s.max() * 448 * 2 ** -4


# ---------------------------------------------------------------- norms / rope / silu

def test_rms_norms_match_torch_rms_norm():
    x = torch.randn(7, 2560, generator=gen(3)).to(torch.bfloat16)
    r = torch.randn(7, 2560, generator=gen(4)).to(torch.bfloat16)
    w = (1 + 0.1 * torch.randn(2560, generator=gen(5))).to(torch.bfloat16)
    lib = F.rms_norm(x.float(), (2560,), w.float(), eps=1e-6)
    ours = ops.rms_norm_bf16(x, w, 1e-6).float()
    assert torch.allclose(ours, lib, rtol=2 ** -7, atol=1e-6)
    out, z = ops.fused_add_rms_norm(x, r, w, 1e-6)
    assert torch.equal(z, (x.float() + r.float()).to(torch.bfloat16))
    lib = F.rms_norm(z.float(), (2560,), w.float(), eps=1e-6)
    assert torch.allclose(out.float(), lib, rtol=2 ** -6, atol=1e-6)
    # the fused add+norm+quant normalizes the fp32 sum (not its bf16 rounding)
    q, s, new_r = ops.add_rms_norm_quant(x, r, w, 1e-6)
    lib = F.rms_norm(x.float() + r.float(), (2560,), w.float(), eps=1e-6)
    assert torch.allclose(ops.dequant_rows(q, s), lib, rtol=2 ** -4, atol=1e-3)
    assert torch.equal(new_r, z)


def test_qk_norm_rope_identity_at_zero_norm_preserving_and_complex_rotation():
    T, nq, nkv, d = 6, 4, 2, 128
    qkv = torch.randn(T, (nq + 2 * nkv) * d, generator=gen(6)).to(torch.bfloat16)
    qw = torch.ones(d, dtype=torch.bfloat16)
    cs = ops.rope_cache(64, d, 1e6, dtype=torch.float32)
    pos = torch.tensor([0, 1, 5, 17, 33, 63])
    q, k, v = ops.qk_norm_rope(qkv, pos, cs, qw, qw, 1e-6, nq, nkv, d)
    assert torch.equal(v, qkv[:, (nq + nkv) * d:])
    normed = F.rms_norm(qkv[:, :nq * d].float().view(T, nq, d), (d,), eps=1e-6)
    got = q.float().view(T, nq, d)
    # position 0: rotation is the identity
    assert torch.allclose(got[0], normed[0], atol=2e-2)
    # the rotation preserves each (a_i, b_i) pair's norm
    pair = lambda t: t[..., :64] ** 2 + t[..., 64:] ** 2
    assert torch.allclose(pair(got), pair(normed), rtol=3e-2, atol=3e-2)
    # and equals multiplication by e^{i pos theta_i} on a + i b (NeoX halves)
    inv = 1.0 / (1e6 ** (torch.arange(0, d, 2).float() / d))
    ang = pos[:, None].float() * inv[None]
    z = torch.complex(normed[..., :64], normed[..., 64:]) * torch.polar(
        torch.ones_like(ang), ang)[:, None, :]
    want = torch.cat([z.real, z.imag], dim=-1)
    assert torch.allclose(got, want, atol=3e-2)


def test_silu_mul_matches_torch_silu():
    gu = torch.randn(5, 2 * 256, generator=gen(7)).to(torch.bfloat16)
    want = F.silu(gu[:, :256].float()) * gu[:, 256:].float()
    assert torch.allclose(ops.silu_mul(gu), want, rtol=1e-6, atol=1e-6)


# ---------------------------------------------------------------- GEMM

def test_fp8_gemm_exact_on_small_integers_and_block_linear():
    g = gen(8)
    a = torch.randint(-8, 9, (5, 256), generator=g).float()
    w = torch.randint(-8, 9, (256, 256), generator=g).float()
    aq, wq = a.to(torch.float8_e4m3fn), w.to(torch.float8_e4m3fn)
    ones_a = torch.ones(5, 2)
    ones_w = torch.ones(2, 2)
    out = ops.fp8_gemm(aq, ones_a, wq, ones_w, out_dtype=torch.float64)
    assert torch.equal(out, (a.double() @ w.double().T))
    # scaling activation block 1 of row 2 by 4 scales only that block's share
    sa = ones_a.clone()
    sa[2, 1] = 4.0
    out2 = ops.fp8_gemm(aq, sa, wq, ones_w, out_dtype=torch.float64)
    share = a[2, 128:].double() @ w[:, 128:].double().T
    assert torch.equal(out2[2] - out[2], 3 * share)
    assert torch.equal(out2[[0, 1, 3, 4]], out[[0, 1, 3, 4]])
    # weight block (n-block 1, k-block 0) scaled by 0.5
    sw = ones_w.clone()
    sw[1, 0] = 0.5
    out3 = ops.fp8_gemm(aq, ones_a, wq, sw, out_dtype=torch.float64)
    share = a[:, :128].double() @ w[128:, :128].double().T
    assert torch.equal(out3[:, 128:] - out[:, 128:], -0.5 * share)


# ---------------------------------------------------------------- attention

def _dense(T, H, KH, d, seed):
    g = gen(seed)
    q = torch.randn(T, H, d, generator=g)
    k = torch.randn(T, KH, d, generator=g)
    v = torch.randn(T, KH, d, generator=g)
    return q, k, v


@pytest.mark.parametrize("causal", [True, False])
def test_attention_matches_sdpa(causal):
    T, H, KH, d = 37, 8, 2, 64
    q, k, v = _dense(T, H, KH, d, 9)
    scale = 1 / math.sqrt(d)
    cu = torch.tensor([0, T])
    out, lse = ops.varlen_attention(q, k, v, cu, scale, causal=causal)
    rep = H // KH
    want = F.scaled_dot_product_attention(
        q.transpose(0, 1)[None], k.repeat_interleave(rep, 1).transpose(0, 1)[None],
        v.repeat_interleave(rep, 1).transpose(0, 1)[None], is_causal=causal, scale=scale)
    assert torch.allclose(out, want[0].transpose(0, 1), atol=1e-5)
    s = torch.einsum("thd,uhd->htu", q, k.repeat_interleave(rep, 1)) * scale
    if causal:
        s = s.masked_fill(~torch.ones(T, T, dtype=torch.bool).tril(), float("-inf"))
    assert torch.allclose(lse, torch.logsumexp(s, dim=-1), atol=1e-5)


def test_paged_attention_is_invariant_to_the_physical_pages_and_bottom_right():
    g = gen(10)
    H, KH, d, page = 4, 1, 32, 16
    used, c = 70, 9                     # 9 queries over 70 keys
    keys = torch.randn(used, KH, d, generator=g)
    vals = torch.randn(used, KH, d, generator=g)
    q = torch.randn(c, H, d, generator=g)
    scale = 0.3
    pages = -(-used // page)
    for perm_seed in range(3):
        n_pages = pages + 5
        phys = torch.randperm(n_pages, generator=gen(100 + perm_seed))[:pages]
        kp = torch.zeros(n_pages * page, KH, d)
        vp = torch.zeros(n_pages * page, KH, d)
        rows = (phys[torch.arange(used) // page] * page + torch.arange(used) % page)
        kp[rows], vp[rows] = keys, vals
        table = torch.zeros(1, pages + 2, dtype=torch.int32)
        table[0, :pages] = phys.int()
        out, lse = ops.paged_attention(q, kp, vp, [0, c], [used], table, scale, True)
        # brute force: query i sees keys 0 .. used - c + i (kv_checker's alignment)
        for i in range(c):
            visible = used - c + i + 1
            s = (q[i].unsqueeze(1) * keys[:visible].transpose(0, 1)).sum(-1) * scale
            p = torch.softmax(s, dim=-1)
            want = (p.unsqueeze(-1) * vals[:visible].transpose(0, 1)).sum(1)
            assert torch.allclose(out[i], want, atol=1e-5)
            assert torch.allclose(lse[:, i], torch.logsumexp(s, -1), atol=1e-5)


def test_merge_of_a_split_key_set_equals_attention_over_all_keys():
    g = gen(11)
    H, KH, d = 4, 1, 128
    c, n_node = 5, 40
    q = torch.randn(c, H, d, generator=g) * 0.3
    node_k, node_v = torch.randn(n_node, KH, d, generator=g), torch.randn(n_node, KH, d, generator=g)
    own_k, own_v = torch.randn(c, KH, d, generator=g), torch.randn(c, KH, d, generator=g)
    scale = 1 / math.sqrt(d)
    out_a, lse_a = ops.varlen_attention(q, own_k, own_v, [0, c], scale, causal=True)
    out_b, lse_b = ops.attend(q, node_k, node_v, scale, torch.ones(c, n_node, dtype=torch.bool))
    merged = ops.merge_attn(out_a.to(torch.bfloat16), lse_a, out_b.to(torch.bfloat16), lse_b,
                            torch.arange(c, dtype=torch.int32))
    allk, allv = torch.cat([node_k, own_k]), torch.cat([node_v, own_v])
    vis = torch.cat([torch.ones(c, n_node, dtype=torch.bool),
                     torch.ones(c, c, dtype=torch.bool).tril()], dim=1)
    want, _ = ops.attend(q, allk, allv, scale, vis)
    assert (merged - want).abs().max() < 2e-2
    # source -1 passes out_a through
    passed = ops.merge_attn(out_a.to(torch.bfloat16), lse_a, out_b.to(torch.bfloat16), lse_b,
                            torch.full((c,), -1, dtype=torch.int32))
    assert torch.equal(passed, out_a.to(torch.bfloat16).float())


def test_tree_attention_equals_sdpa_per_segment_and_the_exact_lse_merge():
    # segments with and without a read, a partial last node page, permuted
    # physical pages; pinned against torch's scaled_dot_product_attention
    # over [node keys | own keys] with the node fully visible and the own
    # part causal, and against the LSE combination of call A and call B in
    # fp32 (sigmoid weights, no bf16 rounding)
    g = gen(13)
    H, KH, d, page = 8, 2, 128, 16
    n_pages = 12
    k_pool = torch.randn(n_pages * page, KH, d, generator=g).to(torch.bfloat16)
    v_pool = torch.randn(n_pages * page, KH, d, generator=g).to(torch.bfloat16)
    perm = torch.randperm(n_pages, generator=g).to(torch.int32)
    table = torch.stack([perm[:4], perm[4:8]])
    used = torch.tensor([37, 64], dtype=torch.int32)
    cu_a = [0, 5, 9, 30, 31]
    seg_read = torch.tensor([0, -1, 1, 0], dtype=torch.int32)
    T = cu_a[-1]
    q = (torch.randn(T, H, d, generator=g) * 0.3).to(torch.bfloat16)
    k3 = torch.randn(T, KH, d, generator=g).to(torch.bfloat16)
    v3 = torch.randn(T, KH, d, generator=g).to(torch.bfloat16)
    scale = 1 / math.sqrt(d)
    got = ops.tree_attention(q, k3, v3, cu_a, seg_read, k_pool, v_pool, table, used, scale)
    out_a, lse_a = ops.varlen_attention(q, k3, v3, cu_a, scale, causal=True)
    for s in range(len(cu_a) - 1):
        a, b = cu_a[s], cu_a[s + 1]
        r = int(seg_read[s])
        qs = q[a:b].float().transpose(0, 1)                       # [H, c, d]
        own_k = k3[a:b].float().repeat_interleave(H // KH, 1).transpose(0, 1)
        own_v = v3[a:b].float().repeat_interleave(H // KH, 1).transpose(0, 1)
        mask = torch.ones(b - a, b - a, dtype=torch.bool).tril()
        if r >= 0:
            n = int(used[r])
            rows = table[r][torch.arange(n) // page].long() * page + torch.arange(n) % page
            nk = k_pool[rows].float().repeat_interleave(H // KH, 1).transpose(0, 1)
            nv = v_pool[rows].float().repeat_interleave(H // KH, 1).transpose(0, 1)
            own_k, own_v = torch.cat([nk, own_k], 1), torch.cat([nv, own_v], 1)
            mask = torch.cat([torch.ones(b - a, n, dtype=torch.bool), mask], 1)
            # call B alone, merged with call A by the exact LSE rule
            out_b, lse_b = ops.attend(q[a:b], k_pool[rows], v_pool[rows], scale,
                                      torch.ones(b - a, n, dtype=torch.bool))
            w = torch.sigmoid(lse_b - lse_a[:, a:b]).T[..., None]
            merged = out_a[a:b] + (out_b - out_a[a:b]) * w
            assert (got[a:b] - merged).abs().max() < 1e-5
        want = torch.nn.functional.scaled_dot_product_attention(
            qs, own_k, own_v, attn_mask=mask, scale=scale).transpose(0, 1)
        assert (got[a:b] - want).abs().max() < 1e-5, f"segment {s}"


# ---------------------------------------------------------------- readout

def test_answer_bits_reference_literal_case_and_strict_ties():
    # the reference's tests/test_model.py:64-81: hidden rows against an
    # output head of 8 rows, TRUE = ids {1, 3}, FALSE = {5}
    head = torch.nn.Linear(4, 8, bias=False, dtype=torch.bfloat16)
    torch.nn.init.normal_(head.weight, generator=gen(12))
    hidden = torch.tensor([[1, 2, -1, 0], [0, 1, 3, -2]], dtype=torch.bfloat16)
    full = F.linear(hidden, head.weight)
    expected = (full[:, [1, 3]].amax(1) > full[:, 5]).to(torch.uint8)
    retained = head.weight.detach()[[1, 3, 5]]
    bits, _ = ops.answer_bits(hidden, retained, [0, 1], [2])
    assert torch.equal(bits, expected)
    # a tie reads FALSE
    same = torch.ones(2, 4, dtype=torch.bfloat16)
    bits, margin = ops.answer_bits(torch.ones(1, 4, dtype=torch.bfloat16), same, [0], [1])
    assert bits.tolist() == [0] and margin.tolist() == [0.0]


# ---------------------------------------------------------------- forward

def test_forward_matches_transformers_qwen3_without_activation_quant():
    transformers = pytest.importorskip("transformers")
    from quail_amd import loop
    from quail_amd.arena import KVArena
    from quail_amd.model import build_random_qwen3
    from e2e_support import TINY

    model = build_random_qwen3(TINY, seed=1, device="cpu", max_pos=512,
                               answer_token_ids=(1, 2, 3, 4))
    w = oforward.cpu_weights(model)
    rng = np.random.default_rng(0)
    ids = rng.integers(0, TINY.vocab, size=50)
    arena = KVArena(1, 16, 16, 1, 1, device="cpu", allocate=False)
    arena.activate("doc", 50, capacity_tokens=50)
    chunk = loop.pack_chunk(torch, arena, [dict(key="doc", prefix=ids[:45], f=45,
                                                suffixes=[ids[45:]])],
                            attention_mode="unified")
    oarena = oforward.OracleArena(TINY.layers, 16, TINY.n_kv, TINY.d_head)
    ours = oforward.forward_chunk(w, chunk.host, "unified", oarena, quantize=False)

    cfg = transformers.Qwen3Config(
        vocab_size=TINY.vocab, hidden_size=TINY.hidden,
        intermediate_size=TINY.intermediate, num_hidden_layers=TINY.layers,
        num_attention_heads=TINY.n_q, num_key_value_heads=TINY.n_kv, head_dim=TINY.d_head,
        rms_norm_eps=TINY.rms_eps, rope_theta=TINY.rope_theta, max_position_embeddings=512,
        tie_word_embeddings=True, attention_bias=False)
    hf = transformers.Qwen3ForCausalLM(cfg).float().eval()
    sd = {"model.embed_tokens.weight": w["embed"].float(), "model.norm.weight": w["final_norm"].float()}
    qw, kw = TINY.n_q * TINY.d_head, TINY.n_kv * TINY.d_head
    inter = TINY.intermediate
    for i, L in enumerate(w["layers"]):
        p = f"model.layers.{i}."
        qkv = ops.dequant_weight(*L["qkv"])
        gu = ops.dequant_weight(*L["gate_up"])
        sd.update({
            p + "self_attn.q_proj.weight": qkv[:qw], p + "self_attn.k_proj.weight": qkv[qw:qw + kw],
            p + "self_attn.v_proj.weight": qkv[qw + kw:],
            p + "self_attn.o_proj.weight": ops.dequant_weight(*L["o"]),
            p + "self_attn.q_norm.weight": L["q_norm"].float(),
            p + "self_attn.k_norm.weight": L["k_norm"].float(),
            p + "mlp.gate_proj.weight": gu[:inter], p + "mlp.up_proj.weight": gu[inter:],
            p + "mlp.down_proj.weight": ops.dequant_weight(*L["down"]),
            p + "input_layernorm.weight": L["in_norm"].float(),
            p + "post_attention_layernorm.weight": L["post_norm"].float()})
    missing, _ = hf.load_state_dict(sd, strict=False)
    assert [m for m in missing if "lm_head" not in m] == []
    with torch.no_grad():
        hidden = hf.model(torch.from_numpy(ids)[None]).last_hidden_state[0, -1]
    rel = (ours[0].float() - hidden).norm() / hidden.norm()
    assert rel < 0.03, f"relative L2 {rel:.4f}"
