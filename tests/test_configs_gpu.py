"""The workload configurations' own shapes against the oracle (MI355X only).

- fp8 block-scaled GEMM sweep at the Qwen3-4B shapes, M = 16,384 tokens:
  (N, K) in {(6144, 2560) qkv, (2560, 4096) o, (19456, 2560) gate_up,
  (2560, 9728) down}; weights N(0, 0.02) with fp32 128x128 block scales,
  activations N(0, 1) with fp32 1x128 scales. 256 sampled rows per shape
  against the oracle's fp64 block sums (the same bar as the small-shape
  GEMM test: |err| <= 2^-8 |want| + 1e-3 max|want|); gate_up's fused
  SiLU + fp8 quant epilogue is bit-identical to the GEMM then
  silu_mul_quant, which is within one e4m3 step of the oracle's on the
  same bf16 input (on at most 0.1 % of the codes).
- paged attention at the Qwen3-32B geometry (64 query / 8 KV heads) over
  rows of 1-4 k tokens, keys up to 4,224: bottom-right causal max-abs
  <= 2e-3 against the fp32 oracle on the last 64 rows of every sequence
  (those that attend the most keys), and the fused tree kernel over a
  3,072-key node with 1,024-row own segments against the fp32 oracle run
  on the GPU.
- the prefix-shared attention layer at its own shape (64 rows x 256-token
  prefix, 32/8 heads): unified, tree and two-pass paths against the fp32
  oracle.
- one chunk packed at the full Qwen3-4B filter budget (110,376 tokens)
  through every stage of one layer, each stage against the oracle on the
  GPU's own input to it.
- the AI join at Qwen3-4B geometry, four layers, both attention paths:
  every layer's attention against the oracle on the same q, k, v and
  pages, and each layer teacher-forced against the oracle.
- yes/no decisions at full depth (36 layers) over 1,024 rows of the
  4096-row filter workload, against the oracle's two restatements and the
  floor of their own disagreement.
"""

import math

import pytest
import torch

from oracle import ops as ref
from quail_amd import kernels as K
from quail_amd import layout

pytestmark = pytest.mark.gpu
DEV = "cuda"
M = 16384
C2_SHAPES = [("qkv", 6144, 2560), ("o", 2560, 4096), ("gate_up", 19456, 2560),
             ("down", 2560, 9728)]


def _e4m3_steps(a, b):
    def key(q):
        u = q.view(torch.uint8).to(torch.int32)
        mag = u & 0x7F
        return torch.where(u >= 0x80, -mag, mag)
    return (key(a) - key(b)).abs()


def _c2_inputs(seed, N, Kd):
    g = torch.Generator(device=DEV).manual_seed(seed)
    w = torch.randn(N, Kd, generator=g, device=DEV) * 0.02
    wq, ws = ref.quantize_weight_blocks(w)
    del w
    x = torch.randn(M, Kd, generator=g, device=DEV)
    xq, xs = ref.group_quant(x)
    del x
    xs_dev = K.col_major_scales(M, Kd, DEV)
    xs_dev.copy_(xs)
    return xq, xs, xs_dev, wq.contiguous(), ws.contiguous()


@pytest.mark.parametrize("name,N,Kd", C2_SHAPES, ids=[s[0] for s in C2_SHAPES])
def test_qwen3_4b_gemm_shapes_at_16384_tokens(name, N, Kd):
    xq, xs, xs_dev, wq, ws = _c2_inputs(100 + N + Kd, N, Kd)
    got = K.fp8_gemm_nt(xq, xs_dev, wq, ws)
    rows = torch.randperm(M, generator=torch.Generator().manual_seed(N))[:256].sort().values
    want = ref.fp8_gemm(xq[rows.to(DEV)].cpu(), xs[rows.to(DEV)].cpu(), wq.cpu(), ws.cpu(),
                        out_dtype=torch.float64)
    g = got[rows.to(DEV)].cpu().double()
    err = (g - want).abs()
    tol = want.abs() * 2 ** -8 + 1e-3 * want.abs().max()
    bad = (err > tol).sum().item()
    print(f"{name}: M={M} N={N} K={Kd}, 256 rows, max err {err.max().item():.3e} "
          f"(scale {want.abs().max().item():.3e}), rel L2 "
          f"{((g - want).norm() / want.norm()).item():.2e}", flush=True)
    assert bad == 0, f"{bad} outputs outside the bar"
    if name == "gate_up":
        # the fused epilogue is the GEMM's bf16 output through silu_mul_quant,
        # bit for bit over all 16,384 rows; silu_mul_quant is the oracle's on
        # that same bf16 input (within one e4m3 step: the oracle's sigmoid and
        # the kernel's exp2/reciprocal round differently near midpoints)
        q, s = K.fp8_gemm_silu_quant(xq, xs_dev, wq, ws)
        pq, ps = K.silu_mul_quant(got)
        assert torch.equal(q.view(torch.uint8), pq.view(torch.uint8)) and torch.equal(s, ps)
        q_ref, s_ref = ref.silu_mul_quant(got[rows.to(DEV)].cpu())
        q_got, s_got = q[rows.to(DEV)].cpu(), s[rows.to(DEV)].cpu()
        assert torch.allclose(s_got, s_ref, rtol=1e-6, atol=0)
        steps = _e4m3_steps(q_got, q_ref)
        frac = (steps > 0).float().mean().item()
        print(f"gate_up + SiLU + quant: fused == pair on {M} rows; {frac:.2e} of codes one "
              f"step from the oracle", flush=True)
        assert steps.max().item() <= 1 and frac <= 1e-3


def _long_paged_case(seed, lengths, prefix, n_q=64, n_kv=8, d=128):
    """Sequences over a shared `prefix`-token node plus own pages, physical
    pages permuted; query rows are each sequence's own tokens."""
    g = torch.Generator().manual_seed(seed)
    page = 16
    node = -(-prefix // page)
    own = [-(-(prefix + n) // page) - prefix // page for n in lengths]
    n_pages = node + sum(own) + 4
    perm = torch.randperm(n_pages, generator=g).tolist()
    shared, cursor = perm[:node], node
    tables, used = [], []
    for n, extra in zip(lengths, own):
        tables.append(shared[:prefix // page] + perm[cursor:cursor + extra])
        cursor += extra
        used.append(prefix + n)
    width = max(map(len, tables))
    table = torch.zeros(len(lengths), width, dtype=torch.int32)
    for i, p in enumerate(tables):
        table[i, :len(p)] = torch.tensor(p, dtype=torch.int32)
    cu_q = torch.zeros(len(lengths) + 1, dtype=torch.int32)
    cu_q[1:] = torch.cumsum(torch.tensor(lengths), 0)
    T = int(cu_q[-1])
    q = (torch.randn(T, n_q, d, generator=g) / math.sqrt(d)).to(torch.bfloat16)
    k_rows = (torch.randn(n_pages * page, n_kv, d, generator=g) / math.sqrt(d)).to(torch.bfloat16)
    v_rows = (torch.randn(n_pages * page, n_kv, d, generator=g) / math.sqrt(d)).to(torch.bfloat16)
    return dict(q=q, k_rows=k_rows, v_rows=v_rows, table=table,
                used=torch.tensor(used, dtype=torch.int32), cu_q=cu_q, lengths=lengths,
                n_kv=n_kv)


def test_paged_attention_over_4k_keys_at_32b_geometry():
    case = _long_paged_case(41, lengths=[4096, 1100, 2900], prefix=128)
    assert max(case["used"].tolist()) >= 4096 + 128
    scale = 1 / math.sqrt(128)
    kp = layout.k_pool_from_rows(case["k_rows"]).to(DEV)
    vp = layout.v_pool_from_rows(case["v_rows"]).to(DEV)
    T = int(case["cu_q"][-1])
    out, lse = K.attention(case["q"].to(DEV), case["cu_q"].to(DEV), case["used"].to(DEV),
                           n_queries=T, max_q=max(case["lengths"]), softmax_scale=scale,
                           causal=True, k_pool=kp, v_pool=vp, table=case["table"].to(DEV),
                           n_kv=case["n_kv"], want_lse=True)
    out, lse = out.cpu().float(), lse.cpu()
    # the oracle on the last 64 rows of each sequence: bottom-right alignment
    # lets a shorter query run stand for the tail of the full one
    tail = 64
    ends = case["cu_q"][1:].tolist()
    rows = torch.cat([torch.arange(e - tail, e) for e in ends])
    cu = torch.arange(0, tail * (len(ends) + 1), tail, dtype=torch.int32)
    want, want_lse = ref.paged_attention(case["q"], case["k_rows"], case["v_rows"], cu,
                                         case["used"], case["table"], scale, True,
                                         q_rows=rows)
    err = (out[rows] - want).abs().max().item()
    lse_err = (lse[:, rows] - want_lse).abs().max().item()
    print(f"paged 32B geometry, keys up to {max(case['used'].tolist())}: max-abs {err:.2e}, "
          f"lse {lse_err:.2e}", flush=True)
    assert err <= 2e-3 and lse_err <= 2e-3
    # fp8 epilogue on the same call is the bf16 output quantized
    q8, s8 = K.attention_fp8(case["q"].to(DEV), case["cu_q"].to(DEV), case["used"].to(DEV),
                             n_queries=T, max_q=max(case["lengths"]), softmax_scale=scale,
                             causal=True, k_pool=kp, v_pool=vp, table=case["table"].to(DEV),
                             n_kv=case["n_kv"])
    bf = K.attention(case["q"].to(DEV), case["cu_q"].to(DEV), case["used"].to(DEV),
                     n_queries=T, max_q=max(case["lengths"]), softmax_scale=scale,
                     causal=True, k_pool=kp, v_pool=vp, table=case["table"].to(DEV),
                     n_kv=case["n_kv"])[0]
    rq, rs = K.group_quant(bf.view(T, -1))
    assert torch.equal(q8.view(torch.uint8), rq.view(torch.uint8)) and torch.equal(s8, rs)


def test_tree_attention_over_a_3072_key_node_at_32b_geometry():
    """Two 1,024-row causal segments reading one 3,072-key node (a long
    shared document prefix, as in the Qwen3-32B rows), GQA 8:1, against
    the fp32 oracle run on the GPU (its own rows causal, the node in full)."""
    g = torch.Generator().manual_seed(43)
    n_q, n_kv, d, page = 64, 8, 128, 16
    node, segs = 3072, [1024, 1000]
    n_pages = node // page + 8
    perm = torch.randperm(n_pages, generator=g)
    table = perm[:node // page].to(torch.int32)[None, :].contiguous()
    T = sum(segs)
    q = (torch.randn(T, n_q, d, generator=g) / math.sqrt(d)).to(torch.bfloat16)
    k3 = (torch.randn(T, n_kv, d, generator=g) / math.sqrt(d)).to(torch.bfloat16)
    v3 = (torch.randn(T, n_kv, d, generator=g) / math.sqrt(d)).to(torch.bfloat16)
    k_rows = (torch.randn(n_pages * page, n_kv, d, generator=g) / math.sqrt(d)).to(torch.bfloat16)
    v_rows = (torch.randn(n_pages * page, n_kv, d, generator=g) / math.sqrt(d)).to(torch.bfloat16)
    cu = torch.tensor([0, segs[0], T], dtype=torch.int32)
    seg_read = torch.zeros(2, dtype=torch.int32)
    used = torch.tensor([node], dtype=torch.int32)
    scale = 1 / math.sqrt(d)
    kp = layout.k_pool_from_rows(k_rows).to(DEV)
    vp = layout.v_pool_from_rows(v_rows).to(DEV)
    got = K.tree_attention(q.to(DEV), k3.to(DEV), v3.to(DEV), cu.to(DEV), seg_read.to(DEV),
                           softmax_scale=scale, k_pool=kp, v_pool=vp, table=table.to(DEV),
                           used=used.to(DEV), fp8=False).float()
    with torch.no_grad():
        want = ref.tree_attention(q.to(DEV), k3.to(DEV), v3.to(DEV), cu, seg_read,
                                  k_rows.to(DEV), v_rows.to(DEV), table, used, scale)
    err = (got - want.to(got.device)).abs().max().item()
    print(f"tree 32B geometry, node {node} keys + own up to {max(segs)}: max-abs {err:.2e}",
          flush=True)
    assert err <= 2e-3


def _prefix_shared_layer(seed, rows=64, prefix=256, n_q=32, n_kv=8, d=128, page=16):
    """One prefix-shared attention layer: `rows` sequences share a
    `prefix`-token node, each adds U[32, 256] own tokens; all pages are a
    seeded permutation of the arena. The node's K/V are in the arena; the
    rows' own K/V are chunk rows, scattered into their pages by the unified
    path. Returns host tensors (the arena as rows, before the scatter)."""
    g = torch.Generator().manual_seed(seed)
    suf = torch.randint(32, 257, (rows,), generator=g)
    own = [-(-int(n) // page) for n in suf]
    n_pages = prefix // page + sum(own) + 8
    perm = torch.randperm(n_pages, generator=g).to(torch.int32)
    node_pages = perm[:prefix // page]
    table = torch.zeros(rows, (prefix + 256) // page, dtype=torch.int32)
    dst, at = [], prefix // page
    for r, n in enumerate(suf.tolist()):
        mine = perm[at:at + own[r]]
        at += own[r]
        table[r, :prefix // page] = node_pages
        table[r, prefix // page:prefix // page + own[r]] = mine
        j = torch.arange(n)
        dst.append(mine[j // page].long() * page + j % page)
    T = int(suf.sum())
    sd = 1 / math.sqrt(d)
    q = (torch.randn(T, n_q, d, generator=g) * sd).to(torch.bfloat16)
    k3 = (torch.randn(T, n_kv, d, generator=g) * sd).to(torch.bfloat16)
    v3 = (torch.randn(T, n_kv, d, generator=g) * sd).to(torch.bfloat16)
    # arena rows no sequence reads hold NaN: nothing may read them
    k_rows = torch.full((n_pages * page, n_kv, d), float("nan"), dtype=torch.bfloat16)
    v_rows = torch.full((n_pages * page, n_kv, d), float("nan"), dtype=torch.bfloat16)
    node_rows = node_pages[torch.arange(prefix) // page].long() * page + torch.arange(prefix) % page
    k_rows[node_rows] = (torch.randn(prefix, n_kv, d, generator=g) * sd).to(torch.bfloat16)
    v_rows[node_rows] = (torch.randn(prefix, n_kv, d, generator=g) * sd).to(torch.bfloat16)
    cu = torch.zeros(rows + 1, dtype=torch.int32)
    cu[1:] = torch.cumsum(suf, 0)
    return dict(q=q, k3=k3, v3=v3, k_rows=k_rows, v_rows=v_rows, table=table,
                node_table=node_pages[None, :].contiguous(), dst=torch.cat(dst), cu=cu,
                used=(prefix + suf).to(torch.int32), prefix=prefix, max_q=int(suf.max()),
                n_kv=n_kv, scale=sd)


def test_prefix_shared_layer_at_64_rows_every_path_matches_the_oracle():
    """The attention layer the prefix-shared attention bench times (64 rows
    x 256-token prefix, suffixes U[32, 256], 32/8 heads, permuted pages),
    each path against the fp32 oracle on the GPU:
      unified   scatter of the rows' K/V into their pages, then paged causal
                attention over prefix + own pages (bf16 out and lse; its
                fp8 epilogue is that output quantized, bit for bit);
      tree      the fused kernel (node in full + own rows causal), bf16 out;
      two_pass  call A (own rows, causal) and call B (node, stacked), each
                against its oracle, and their merge against the oracle's
                merge of the kernels' own outputs (scales within 1e-6
                relative, at most 0.1 % of codes differing, by at most
                an eighth of their group's largest value)."""
    c = _prefix_shared_layer(61)
    T, rows = int(c["cu"][-1]), c["cu"].numel() - 1
    scale, n_kv = c["scale"], c["n_kv"]
    kp = layout.k_pool_from_rows(c["k_rows"]).to(DEV)
    vp = layout.v_pool_from_rows(c["v_rows"]).to(DEV)
    qd, kd, vd, cu_d = c["q"].to(DEV), c["k3"].to(DEV), c["v3"].to(DEV), c["cu"].to(DEV)
    node_tab, node_used = c["node_table"].to(DEV), torch.tensor([c["prefix"]],
                                                                dtype=torch.int32, device=DEV)
    seg_read = torch.zeros(rows, dtype=torch.int32, device=DEV)
    with torch.no_grad():
        want_tree = ref.tree_attention(qd, kd, vd, c["cu"], seg_read.cpu(), c["k_rows"].to(DEV),
                                       c["v_rows"].to(DEV), c["node_table"],
                                       torch.tensor([c["prefix"]], dtype=torch.int32), scale)
    # tree: the fused kernel
    got = K.tree_attention(qd, kd, vd, cu_d, seg_read, softmax_scale=scale, k_pool=kp,
                           v_pool=vp, table=node_tab, used=node_used, fp8=False).float()
    err_tree = (got - want_tree).abs().max().item()
    # two-pass: call A over the rows' own K/V, call B over the node
    a_len = (cu_d[1:] - cu_d[:-1]).to(torch.int32)
    out_a, lse_a = K.attention(qd, cu_d, a_len, n_queries=T, max_q=c["max_q"],
                               softmax_scale=scale, causal=True, k_rows=kd, v_rows=vd,
                               cu_k=cu_d, n_kv=n_kv, want_lse=True)
    cu_b = torch.tensor([0, T], dtype=torch.int32, device=DEV)
    all_rows = torch.arange(T, dtype=torch.int64, device=DEV)
    out_b, lse_b = K.attention(qd, cu_b, node_used, n_queries=T, max_q=T, softmax_scale=scale,
                               causal=False, k_pool=kp, v_pool=vp, table=node_tab,
                               q_rows=all_rows, n_kv=n_kv, want_lse=True)
    with torch.no_grad():
        want_a, want_la = ref.varlen_attention(qd, kd, vd, c["cu"], scale, causal=True)
        want_b, want_lb = ref.paged_attention(qd, c["k_rows"].to(DEV), c["v_rows"].to(DEV),
                                              torch.tensor([0, T], dtype=torch.int32),
                                              torch.tensor([c["prefix"]], dtype=torch.int32),
                                              c["node_table"], scale, False)
    err_a = (out_a.float() - want_a).abs().max().item()
    err_b = (out_b.float() - want_b).abs().max().item()
    lse_ab = max((lse_a - want_la).abs().max().item(), (lse_b - want_lb).abs().max().item())
    source = torch.arange(T, dtype=torch.int32, device=DEV)
    q2, s2 = K.merge_attn_quant(out_a, lse_a, out_b, lse_b, source)
    q2_ref, s2_ref = ref.merge_attn_quant(out_a.cpu(), lse_a.cpu(), out_b.cpu(), lse_b.cpu(),
                                          source.cpu())
    # unified: the rows' K/V into their own pages, then one paged call
    K.kv_row_scatter(kd, vd, kp, vp, torch.arange(T, dtype=torch.int64, device=DEV),
                     c["dst"].to(DEV))
    k_after, v_after = c["k_rows"].clone(), c["v_rows"].clone()
    k_after[c["dst"]], v_after[c["dst"]] = c["k3"], c["v3"]
    args = dict(n_queries=T, max_q=c["max_q"], softmax_scale=scale, causal=True, k_pool=kp,
                v_pool=vp, table=c["table"].to(DEV), n_kv=n_kv)
    out_u, lse_u = K.attention(qd, cu_d, c["used"].to(DEV), want_lse=True, **args)
    with torch.no_grad():
        want_u, want_lu = ref.paged_attention(qd, k_after.to(DEV), v_after.to(DEV), c["cu"],
                                              c["used"], c["table"], scale, True)
    err_u = (out_u.float() - want_u).abs().max().item()
    lse_u_err = (lse_u - want_lu).abs().max().item()
    q8, s8 = K.attention_fp8(qd, cu_d, c["used"].to(DEV), **args)
    rq, rs = K.group_quant(out_u.view(T, -1))
    # unified and tree compute one function: the oracles agree
    oracles = (want_u - want_tree).abs().max().item()
    print(f"prefix-shared layer, {rows} rows / {T} query rows: unified {err_u:.2e} "
          f"(lse {lse_u_err:.2e}), tree {err_tree:.2e}, call A {err_a:.2e}, call B "
          f"{err_b:.2e} (lse {lse_ab:.2e}); oracles apart {oracles:.2e}", flush=True)
    assert oracles <= 1e-5
    assert err_u <= 2e-3 and lse_u_err <= 2e-3
    assert torch.equal(q8.view(torch.uint8), rq.view(torch.uint8)) and torch.equal(s8, rs)
    assert err_tree <= 2e-3
    assert err_a <= 2e-3 and err_b <= 2e-3 and lse_ab <= 2e-3
    # the merge kernel's weight (hardware exp) and its fused a + (b - a) w may
    # round a bf16 step apart from torch's; where a and b nearly cancel that
    # moves a small value's e4m3 code by several steps of its own scale, so
    # the bar is one step at the top of the group: |dequantized difference|
    # <= amax / 8 per (row, head) group, and differing codes rare
    assert torch.allclose(s2.cpu(), s2_ref, rtol=1e-6, atol=0)
    s2c = s2.cpu()
    steps = _e4m3_steps(q2.cpu(), q2_ref)
    deq = q2.cpu().float().view(T, -1, 128) * s2c[:, :, None]
    deq_ref = q2_ref.float().view(T, -1, 128) * s2_ref[:, :, None]
    top = ((deq - deq_ref).abs().amax(-1) / (448 * s2_ref)).max().item()
    frac = (steps > 0).float().mean().item()
    print(f"two-pass merge + quant against the oracle's merge of the same outputs: "
          f"{frac:.2e} of codes differ, at most {steps.max().item()} steps, largest "
          f"difference {top:.3f} of the group's amax", flush=True)
    assert frac <= 1e-3 and top <= 0.125


# ---------------------------------------------------------------------------
# one chunk at the full Qwen3-4B chunk budget (110,376 tokens): the budget is
# the int32 element cap of the widest projection, (2^31 - 1) // 19,456, so
# gate_up's last element offsets sit just under 2^31

def _rows_sample(T, n, seed):
    """n random rows and the last n rows of a T-row chunk (the highest offsets)."""
    g = torch.Generator().manual_seed(seed)
    pick = torch.randperm(T - n, generator=g)[:n]
    return torch.cat([pick, torch.arange(T - n, T)]).sort().values


def test_one_chunk_at_the_full_qwen3_4b_budget_matches_the_oracle_per_stage():
    from oracle import forward as oforward
    from quail_amd import budgets, loop
    from quail_amd.aiif import RowPrompts, synthetic_filter_workload
    from quail_amd.arena import KVArena
    from quail_amd.model import build_random_qwen3
    from quail_amd.pack import FilterAdmission
    from quail_amd.specs import MI355X, QWEN3_4B_FP8

    spec = QWEN3_4B_FP8
    budget = budgets.chunk_budget(spec, MI355X)
    assert budget == 110_376 and budget * spec.ffn_width < 2 ** 31
    instruction, documents, tail = synthetic_filter_workload(600, seed=0, vocab=spec.vocab)
    docs = RowPrompts(instruction, documents)
    # the first chunk of the filter: admission fills the budget in queue order
    sched = FilterAdmission([len(d) for d in docs], [len(tail)], budget, arena_pages=1 << 20,
                            page_tokens=16)
    groups = sched.next_chunk(1 << 20)
    n_rows = len(groups)
    tokens = sum(len(docs[d]) + len(tail) for d, _, _ in groups)
    taken = {d for d, _, _ in groups}
    left = [len(docs[d]) + len(tail) for d in range(len(docs)) if d not in taken]
    assert left and min(left) > budget - tokens, "a waiting row fits the unused room"
    pages = sum(-(-(len(docs[d]) + len(tail)) // 16) for d, _, _ in groups) + 16
    model = build_random_qwen3(spec, seed=0, device="cuda", layers=1, max_pos=2048)
    arena = KVArena(1, pages, 16, spec.n_kv, spec.d_head, device="cuda")
    specs = []
    for d, _, _ in groups:
        arena.activate(("d", d), len(docs[d]), capacity_tokens=len(docs[d]) + len(tail))
        specs.append(dict(key=("d", d), prefix=docs[d], f=len(docs[d]), suffixes=[list(tail)]))
    chunk = loop.pack_chunk(torch, arena, specs, attention_mode="unified")
    T = chunk.tokens
    assert T == tokens and T > 0.99 * budget
    print(f"full-budget chunk: {n_rows} rows, {T} tokens of {budget}", flush=True)
    h = chunk.host
    w = oforward.oracle_weights(model, "cuda")
    L = w["layers"][0]
    lin = model.model.layers[0]
    rows = _rows_sample(T, 128, 5).to(DEV)

    def gemm_check(name, x_q, x_s, linear):
        got = K.fp8_gemm_nt(x_q, x_s, linear.weight, linear.weight_scale)
        want = ref.fp8_gemm(x_q[rows], x_s[rows].contiguous(), linear.weight, linear.weight_scale)
        rel = ((got[rows].double() - want.double()).norm() / want.double().norm()).item()
        print(f"  {name}: rel L2 {rel:.2e} on 256 rows", flush=True)
        assert rel < 1e-3
        return got

    emb = K.gather_rows(w["embed"], chunk.input_ids)
    qi, qs = K.add_rmsnorm_quant(emb, L["in_norm"], L["eps"])
    qkv = gemm_check("qkv", qi, qs, lin.self_attn.qkv_proj)
    attn = lin.self_attn
    q, k, v = K.qk_norm_rope(qkv, chunk.positions, w["cos_sin"], L["q_norm"], L["k_norm"],
                             L["eps"], spec.n_q, spec.n_kv, spec.d_head)
    u = chunk.meta["unified"]
    kp, vp = arena.page_pools(0)
    K.kv_row_scatter(k.view(T, spec.n_kv, 128), v.view(T, spec.n_kv, 128), kp, vp, u["src"],
                     u["dst"])
    out, _ = K.attention(q.view(T, spec.n_q, 128), u["cu_q"], u["used"], n_queries=T,
                         max_q=u["max_q"], softmax_scale=1 / math.sqrt(128), causal=True,
                         k_pool=kp, v_pool=vp, table=u["table"], n_kv=spec.n_kv)
    # the fp32 oracle over 8 sequences, the last one included
    cu = h["unified_cu_q"]
    n_seq = len(cu) - 1
    seqs = sorted(set(torch.randperm(n_seq, generator=torch.Generator().manual_seed(6))[:7]
                      .tolist()) | {n_seq - 1})
    k_rows, v_rows = layout.k_rows(kp), layout.v_rows(vp)
    worst = 0.0
    for s in seqs:
        a, b = int(cu[s]), int(cu[s + 1])
        want, _ = ref.paged_attention(q.view(T, spec.n_q, 128)[a:b], k_rows, v_rows,
                                      torch.tensor([0, b - a]),
                                      torch.tensor([int(h["unified_used"][s])]),
                                      torch.from_numpy(h["unified_table"][s:s + 1]),
                                      1 / math.sqrt(128), True)
        # q, k and v come from the model here (v has unit RMS, outputs are
        # O(1), where one bf16 step is 2^-8..2^-7): the bar is one bf16 step
        # of each value plus a quarter step of the largest. In L2, the kernel
        # rounds twice to bf16 (the probabilities before the PV product, as
        # FlashAttention does, and the output), each at most 2^-7/sqrt(12)
        # relative RMS: sqrt(2) * 2^-7 / sqrt(12) = 3.19e-3.
        got_s = out[a:b].float()
        err = (got_s - want).abs()
        bound = want.abs() * 2 ** -7 + want.abs().max() * 2 ** -9
        rel = ((got_s - want).norm() / want.norm()).item()
        worst = max(worst, rel)
        assert (err <= bound).all() and rel <= 3.19e-3, \
            f"sequence {s}: max-abs {err.max().item():.3e}, rel L2 {rel:.2e}"
    print(f"  attention: 8 sequences, worst rel L2 {worst:.2e}", flush=True)
    oq, os_ = K.group_quant(out.view(T, -1))
    hid = gemm_check("o", oq, os_, attn.o_proj)
    res = emb.clone()
    gq, gs = K.add_rmsnorm_quant(hid, L["post_norm"], L["eps"], residual=res)
    want_res = (hid[rows].float() + emb[rows].float()).to(torch.bfloat16)
    assert torch.equal(res[rows], want_res), "residual write-back"
    gu = gemm_check("gate_up", gq, gs, lin.mlp.gate_up_proj)
    dq, ds = K.fp8_gemm_silu_quant(gq, gs, lin.mlp.gate_up_proj.weight,
                                   lin.mlp.gate_up_proj.weight_scale)
    pq, ps = K.silu_mul_quant(gu)
    assert torch.equal(dq[rows].view(torch.uint8), pq[rows].view(torch.uint8))
    assert torch.equal(ds[rows], ps[rows])
    gemm_check("down", dq, ds, lin.mlp.down_proj)


# ---------------------------------------------------------------------------
# the AI join at Qwen3-4B geometry: a slice of the seeded 256 x 256 workload,
# four layers, teacher-forced against the oracle on the GPU

def _checked_engine(records):
    """An Engine that checks each layer's attention as it runs: the kernel's
    bf16 form against the oracle's exact attention on the same q, k, v and
    arena pages, and the fp8 result the pipeline uses against group_quant
    of that bf16 output, bit for bit. The kernel rounds the probabilities
    and the output to bf16 (unit roundoff u = 2^-8), so elementwise
    |got - want| <= u |want| + u (1 + u) sum_j p_j |v_j|, the second term
    being the oracle's attention over |V|; the bar takes 2^-8 |want| +
    2^-7 of that mass. In L2 the two roundings are independent, each at
    most 2^-7 / sqrt(12) relative RMS: sqrt(2) * 2^-7 / sqrt(12) = 3.19e-3."""
    from quail_amd.engine import Engine

    def check(kind, got_q, bf, want, mass):
        bf, want, mass = bf.float(), want.float().view(bf.shape), mass.float().view(bf.shape)
        err = (bf - want).abs()
        bound = want.abs() * 2 ** -8 + mass * 2 ** -7
        rel = ((bf - want).norm() / want.norm()).item()
        T = bf.shape[0]
        q8, s8 = K.group_quant(bf.to(torch.bfloat16).view(T, -1))
        same = (torch.equal(got_q[0].view(torch.uint8), q8.view(torch.uint8))
                and torch.equal(got_q[1], s8))
        records.append(dict(kind=kind, excess=(err - bound).max().item(), rel=rel, same=same,
                            rows=T))

    class CheckedEngine(Engine):
        def attention_tree(self, q3, k3, v3, meta):
            layer = meta["layer"]
            got = super().attention_tree(q3, k3, v3, meta)
            reads = meta["reads"]
            kp, vp = self.arena.page_pools(layer)
            kw = {}
            if reads is not None:
                kw = dict(k_pool=kp, v_pool=vp, table=reads["table"], used=reads["used"])
            bf = K.tree_attention(q3, k3, v3, meta["cu_a"], meta["a_read"],
                                  softmax_scale=self.softmax_scale, fp8=False, **kw)
            k_rows, v_rows = layout.k_rows(kp), layout.v_rows(vp)
            want, mass = (ref.tree_attention(
                q3, k3, vv, meta["cu_a"].cpu(), meta["a_read"].cpu(), k_rows, pool,
                None if reads is None else reads["table"].cpu(),
                None if reads is None else reads["used"].cpu(), self.softmax_scale)
                for vv, pool in ((v3, v_rows), (v3.abs(), v_rows.abs())))
            check("tree", got, bf, want, mass)
            return got

        def _unified_fp8(self, q3, k3, v3, meta):
            layer, u = meta["layer"], meta["unified"]
            got = super()._unified_fp8(q3, k3, v3, meta)
            if u is None:
                return got
            kp, vp = self.arena.page_pools(layer)
            n = q3.shape[0]
            bf, _ = K.attention(q3, u["cu_q"], u["used"], n_queries=n, max_q=u["max_q"],
                                softmax_scale=self.softmax_scale, causal=True, k_pool=kp,
                                v_pool=vp, table=u["table"], n_kv=self.num_kv_heads)
            k_rows, v_rows = layout.k_rows(kp), layout.v_rows(vp)
            want, mass = (ref.paged_attention(q3, k_rows, pool, u["cu_q"].cpu(), u["used"].cpu(),
                                              u["table"].cpu(), self.softmax_scale, True)[0]
                          for pool in (v_rows, v_rows.abs()))
            check("unified", got, bf, want, mass)
            return got

    return CheckedEngine


def _teacher_forced(model, spec, hosts, traces, pages):
    """Replay every recorded chunk's layers on the oracle, each layer from
    the GPU's input to it, over the oracle's own arena on the GPU; returns
    the worst (hidden rel L2, row rel L2, residual rel L2). Four GEMM inputs
    per layer are quantized to e4m3 (2^-3 steps), so wherever the GPU's and
    the oracle's bf16 values straddle a rounding boundary a code moves one
    step; the callers' bars cover that."""
    from oracle import forward as oforward

    w = oforward.oracle_weights(model, "cuda")
    oarena = oforward.OracleArena(spec.layers, pages, spec.n_kv, spec.d_head, device="cuda")
    worst = [0.0, 0.0, 0.0]
    with torch.no_grad():
        for (host, mode), layers in zip(hosts, traces):
            for li, L in enumerate(w["layers"]):
                h_in, r_in = layers[li]
                h_ref, r_ref = oforward.layer_step(L, li, h_in, r_in, host, mode, oarena)
                h_gpu, r_gpu = layers[li + 1]
                rel = ((h_gpu.float() - h_ref.float()).norm() / h_ref.float().norm()).item()
                row = ((h_gpu.float() - h_ref.float()).norm(dim=1)
                       / h_ref.float().norm(dim=1).clamp(min=1e-6)).max().item()
                res = ((r_gpu.float() - r_ref.float()).norm() / r_ref.float().norm()).item()
                worst = [max(worst[0], rel), max(worst[1], row), max(worst[2], res)]
                del h_ref, r_ref
    return worst


@pytest.mark.parametrize("path", ["tree", "unified"])
def test_qwen3_4b_join_layers_match_the_oracle_teacher_forced(path):
    from dataclasses import replace

    from quail_amd import loop
    from quail_amd.aiif import synthetic_join_workload
    from quail_amd.arena import KVArena
    from quail_amd.model import SYNTHETIC_FALSE_IDS, SYNTHETIC_TRUE_IDS, build_random_qwen3
    from quail_amd.qwen3 import Qwen3Pipeline
    from quail_amd.readout import AnswerRows, AsyncAnswers
    from quail_amd.specs import QWEN3_4B_FP8
    from quail_amd.tokens import prefix_tree

    spec = replace(QWEN3_4B_FP8, layers=4)
    anchors, frame, partners = synthetic_join_workload(256, 256, seed=0, vocab=spec.vocab)
    anchors, partners = anchors[:4], partners[:24]
    model = build_random_qwen3(spec, seed=1, device="cuda", max_pos=4096)
    pages = 4000
    arena = KVArena(spec.layers, pages, 16, spec.n_kv, spec.d_head, device="cuda")
    checks = []
    pipe = Qwen3Pipeline(model, arena, spec=spec, engine_class=_checked_engine(checks))
    traces, hosts = [], []

    def trace(layer, hidden, residual):
        traces[-1].append((hidden.clone(), None if residual is None else residual.clone()))

    class Rec:
        tree_attention, canvas_ids, needs_pages = True, (), False

        def forward_chunk(self, chunk):
            traces.append([])
            hosts.append((chunk.host, chunk.attention_mode))
            return pipe.forward_chunk(chunk)

    pipe.trace = trace
    ans = AsyncAnswers(torch, AnswerRows(torch, model, SYNTHETIC_TRUE_IDS, SYNTHETIC_FALSE_IDS))
    stats = {}
    loop.run_join(torch, arena, Rec(), ans, [list(a) for a in anchors],
                  [[list(p) for p in partners]], 2048, stage_frames=[list(frame)],
                  attention_mode=path, prefix_tree=prefix_tree(anchors, 16), stats=stats)
    torch.cuda.synchronize()
    assert stats["chunks"] >= 3 and stats["borrowed_tokens"] > 0
    kinds = {c["kind"] for c in checks}
    assert len(checks) == stats["chunks"] * spec.layers and kinds == {path}, (len(checks), kinds)
    print(f"join {path}: {len(checks)} attention calls, worst rel L2 "
          f"{max(c['rel'] for c in checks):.2e}, worst excess over the bar "
          f"{max(c['excess'] for c in checks):.2e}", flush=True)
    for i, c in enumerate(checks):
        assert c["excess"] <= 0 and c["rel"] <= 3.19e-3 and c["same"], (i, c)
    worst = _teacher_forced(model, spec, hosts, traces, pages)
    print(f"join {path}: {stats['chunks']} chunks x {spec.layers} layers teacher-forced, worst "
          f"hidden rel {worst[0]:.4f}, worst row {worst[1]:.4f}, residual {worst[2]:.4f}",
          flush=True)
    assert worst[0] < 0.08 and worst[1] < 0.20 and worst[2] < 0.04, worst


# ---------------------------------------------------------------------------
# Qwen3-32B at its own lengths: rows of a 128-token instruction and a
# document of 1,024-4,096 tokens (the 32B filter workload's seeded
# generator), packed at the Qwen3-32B chunk budget of 41,943 tokens, two
# layers of the 32B geometry

@pytest.mark.parametrize("path", ["unified", "tree"])
def test_qwen3_32b_rows_at_their_chunk_budget_match_the_oracle(path):
    """The first 24 rows of the 32B workload (two chunks, the first filled
    to the budget; every row borrows the instruction's 8 pages through the
    prefix tree, across the chunk boundary too) through two layers of the
    Qwen3-32B geometry (hidden 5120, 64 query / 8 KV heads, FFN 25,600).
    Every attention call is checked as it runs against the oracle's exact
    attention on the same q, k, v and pages, with the kernel-rounding bound
    of the join test; every layer is teacher-forced against the oracle on
    the GPU with the join test's bars."""
    from dataclasses import replace

    from quail_amd import budgets, loop
    from quail_amd.aiif import RowPrompts, synthetic_filter_workload
    from quail_amd.arena import KVArena
    from quail_amd.model import SYNTHETIC_FALSE_IDS, SYNTHETIC_TRUE_IDS, build_random_qwen3
    from quail_amd.qwen3 import Qwen3Pipeline
    from quail_amd.readout import AnswerRows, AsyncAnswers
    from quail_amd.specs import MI355X, QWEN3_32B_FP8
    from quail_amd.tokens import prefix_tree

    budget = budgets.chunk_budget(QWEN3_32B_FP8, MI355X)
    assert budget == 41_943 and budget * QWEN3_32B_FP8.ffn_width < 2 ** 31
    spec = replace(QWEN3_32B_FP8, layers=2)
    instruction, documents, tail = synthetic_filter_workload(
        24, prefix_tokens=128, uniform_lengths=(1024, 4096), seed=0, vocab=spec.vocab)
    docs = RowPrompts(instruction, documents)
    assert min(len(d) for d in documents) >= 1024 and max(len(d) for d in documents) <= 4096
    model = build_random_qwen3(spec, seed=0, device="cuda", max_pos=8192)
    pages = sum(-(-(len(docs[d]) + len(tail)) // 16) for d in range(len(docs))) + 64
    arena = KVArena(spec.layers, pages, 16, spec.n_kv, spec.d_head, device="cuda")
    checks = []
    pipe = Qwen3Pipeline(model, arena, spec=spec, engine_class=_checked_engine(checks))
    traces, hosts = [], []

    def trace(layer, hidden, residual):
        traces[-1].append((hidden.clone(), None if residual is None else residual.clone()))

    class Rec:
        tree_attention, canvas_ids, needs_pages = True, (), False

        def forward_chunk(self, chunk):
            traces.append([])
            hosts.append((chunk.host, chunk.attention_mode))
            return pipe.forward_chunk(chunk)

    pipe.trace = trace
    ans = AsyncAnswers(torch, AnswerRows(torch, model, SYNTHETIC_TRUE_IDS, SYNTHETIC_FALSE_IDS))
    stream = loop.FilterStream(torch, arena, Rec(), ans, docs, [list(tail)], budget,
                               arena_writes=True, attention_mode=path,
                               prefix_tree=prefix_tree(docs, 16))
    while not stream.done:
        stream.next()
    torch.cuda.synchronize()
    sizes = [len(h["positions"]) for h, _ in hosts]
    rows = [len(g) for g in stream.packed_groups]
    print(f"32B {path}: {len(hosts)} chunks of {sizes} tokens, {rows} rows, budget {budget}, "
          f"borrowed {stream.sched.borrowing.borrowed_tokens} tokens", flush=True)
    assert len(hosts) >= 2 and sizes[0] > 0.9 * budget and max(sizes) <= budget
    assert stream.sched.borrowing.borrowed_tokens == 128 * (len(docs) - 1)
    assert len(stream.answers) == len(docs)
    kinds = {c["kind"] for c in checks}
    assert len(checks) == len(hosts) * spec.layers and kinds == {path}, (len(checks), kinds)
    print(f"32B {path}: {len(checks)} attention calls, worst rel L2 "
          f"{max(c['rel'] for c in checks):.2e}, worst excess over the bar "
          f"{max(c['excess'] for c in checks):.2e}", flush=True)
    for i, c in enumerate(checks):
        assert c["excess"] <= 0 and c["rel"] <= 3.19e-3 and c["same"], (i, c)
    worst = _teacher_forced(model, spec, hosts, traces, pages)
    print(f"32B {path}: {len(hosts)} chunks x {spec.layers} layers teacher-forced, worst "
          f"hidden rel {worst[0]:.4f}, worst row {worst[1]:.4f}, residual {worst[2]:.4f}",
          flush=True)
    assert worst[0] < 0.08 and worst[1] < 0.20 and worst[2] < 0.04, worst


# ---------------------------------------------------------------------------
# One stage family from the oracle: the GPU pipeline with its GEMMs, its
# attention or its norm/quant stages computed by the oracle's functions (on
# the GPU) and every other stage by the kernels. Measuring each variant's
# decisions against the fp64 oracle shows which stage's rounding moves the
# GPU's margins.

ORACLE_STAGES = ("gemm", "attention", "norm")


def _col_major(scales):
    T, G = scales.shape
    out = K.col_major_scales(T, G * 128, scales.device)
    out.copy_(scales)
    return out


def _oracle_stage_engine(stage):
    """An Engine whose `stage` family runs the oracle's arithmetic:
    gemm      the four projections as exact fp64 block sums rounded to bf16
              (ops.fp8_gemm), the q/k norm, rotary and SiLU quant on the
              kernels that follow the plain GEMM;
    attention the unified path's paged causal attention in fp32
              (ops.paged_attention) over the arena's pages (read through
              KVArena.layer_kv), or the tree path's call A + call B + bf16
              LSE merge (ops.varlen_attention, paged_attention,
              merge_attn); the bf16 output quantized by the group-quant
              kernel (the oracle quantizes the same bf16 values);
    norm      the input / post-attention RMSNorm + quant, the q/k norm +
              rotary, the SiLU + quant and the final norm as the oracle's
              torch functions (ops.norm_quant_plain, add_rms_norm_quant,
              qk_norm_rope, silu_mul_quant, fused_add_rms_norm)."""
    from quail_amd.engine import Engine

    assert stage in ORACLE_STAGES

    class OracleStage(Engine):
        def __init__(self, arena, **kw):
            if stage in ("gemm", "norm"):
                kw["fuse_qkv_epilogue"] = False
            if stage == "norm":
                kw["fuse_kv_write"] = False
            super().__init__(arena, **kw)

        def gemm(self, q_input, input_scale, linear, name="gemm"):
            if stage != "gemm":
                return super().gemm(q_input, input_scale, linear, name)
            return ref.fp8_gemm(q_input, input_scale, linear.weight, self.weight_scale(linear))

        def gemm_silu_quant(self, q_input, input_scale, linear, name="gate_up"):
            if stage == "gemm":
                return K.silu_mul_quant(self.gemm(q_input, input_scale, linear))
            if stage == "norm":
                gu = K.fp8_gemm_nt(q_input, input_scale, linear.weight,
                                   self.weight_scale(linear))
                q, s = ref.silu_mul_quant(gu)
                return q, _col_major(s)
            return super().gemm_silu_quant(q_input, input_scale, linear, name)

        def norm_quant(self, hidden, norm, residual=None):
            if stage != "norm":
                return super().norm_quant(hidden, norm, residual)
            eps = norm.variance_epsilon
            if residual is None:
                q, s = ref.norm_quant_plain(hidden, norm.weight, eps)
            else:
                q, s, new_res = ref.add_rms_norm_quant(hidden, residual, norm.weight, eps)
                residual.copy_(new_res)
            return q, _col_major(s)

        def qkv_norm_rope(self, qkv, positions, attn):
            if stage != "norm":
                return super().qkv_norm_rope(qkv, positions, attn)
            return ref.qk_norm_rope(qkv, positions, self.rotary.cos_sin_cache,
                                    attn.q_norm.weight, attn.k_norm.weight,
                                    attn.q_norm.variance_epsilon, self.num_q_heads,
                                    self.num_kv_heads, self.head_dim)

        def fused_add_rms_norm(self, hidden, residual, norm):
            if stage != "norm":
                return super().fused_add_rms_norm(hidden, residual, norm)
            out, z = ref.fused_add_rms_norm(hidden, residual, norm.weight,
                                            norm.variance_epsilon)
            residual.copy_(z)
            return out, residual

        def fused_add_rms_norm_rows(self, hidden, residual, rows, norm):
            if stage != "norm":
                return super().fused_add_rms_norm_rows(hidden, residual, rows, norm)
            out, _ = ref.fused_add_rms_norm(hidden[rows], residual[rows], norm.weight,
                                            norm.variance_epsilon)
            return out

        def attention_tree(self, q3, k3, v3, meta):
            if stage != "attention":
                return super().attention_tree(q3, k3, v3, meta)
            # call A over the chunk's own segments, call B over the reads,
            # the bf16 LSE merge (the oracle's tree layer step)
            layer, reads = meta["layer"], meta["reads"]
            n = q3.shape[0]
            k_pool, v_pool = self.arena.page_pools(layer)
            if meta["kv_src"] is not None:
                K.kv_row_scatter(k3, v3, k_pool, v_pool, meta["kv_src"], meta["kv_dst"])
            out_a, lse_a = ref.varlen_attention(q3, k3, v3, meta["cu_a"].cpu(),
                                                self.softmax_scale, causal=True)
            out = out_a.to(torch.bfloat16)
            if reads is not None:
                k_rows, v_rows = self.arena.layer_kv(layer)
                out_b, lse_b = ref.paged_attention(
                    q3, k_rows, v_rows, reads["cu_q"].cpu(), reads["used"].cpu(),
                    reads["table"].cpu(), self.softmax_scale, False, q_rows=reads["rows"].cpu())
                out = ref.merge_attn(out, lse_a, out_b.to(torch.bfloat16), lse_b,
                                     reads["source"]).to(torch.bfloat16)
            meta["layer"] += 1
            return K.group_quant(out.reshape(n, -1), self.use_ue8m0)

        def _unified_fp8(self, q3, k3, v3, meta):
            if stage != "attention" or meta["unified"] is None:
                return super()._unified_fp8(q3, k3, v3, meta)
            layer, u = meta["layer"], meta["unified"]
            n = q3.shape[0]
            self._write_unified_kv(k3, v3, u, layer)
            k_rows, v_rows = self.arena.layer_kv(layer)
            out, _ = ref.paged_attention(q3, k_rows, v_rows, u["cu_q"].cpu(), u["used"].cpu(),
                                         u["table"].cpu(), self.softmax_scale, True)
            meta["layer"] += 1
            return K.group_quant(out.to(torch.bfloat16).view(n, -1), self.use_ue8m0)

    return OracleStage


# ---------------------------------------------------------------------------
# yes/no decisions at full depth over 1,024 rows of the 4096-row AI.IF
# workload: the GPU against the oracle's two restatements (fp64 block sums;
# dequantize-then-fp32 GEMMs). The oracle replays every chunk the GPU ran,
# in order, over its own arena on the GPU; the replay is split into parts so
# that no single test runs long. The last test aggregates.

DECIDE_ROWS = 1024
DECIDE_PARTS = {"fp64": 4, "fp32": 2}
_DECIDE = {}


def _decision_gpu_run():
    if "records" in _DECIDE:
        return _DECIDE
    import numpy as np

    from e2e_support import gpu_filter
    from quail_amd.aiif import synthetic_filter_workload
    from quail_amd.model import SYNTHETIC_FALSE_IDS, SYNTHETIC_TRUE_IDS, build_random_qwen3
    from quail_amd.specs import QWEN3_4B_FP8

    spec = QWEN3_4B_FP8
    model = build_random_qwen3(spec, seed=0, device="cuda", max_pos=2048)
    instruction, documents, tail = synthetic_filter_workload(4096, seed=0, vocab=spec.vocab)
    docs = [np.concatenate([instruction, d]) for d in documents[:DECIDE_ROWS]]
    pages = sum(-(-(len(d) + len(tail)) // 16) for d in docs) + 64
    answers, margins, records, stream = gpu_filter(
        model, spec, docs, tail, path="unified", pages=pages, budget=16384,
        true_ids=SYNTHETIC_TRUE_IDS, false_ids=SYNTHETIC_FALSE_IDS)
    torch.cuda.empty_cache()
    _DECIDE.update(model=model, spec=spec, pages=pages, answers=answers, margins=margins,
                   records=[(h, m) for h, m, _ in records], groups=stream.packed_groups,
                   runs={})
    print(f"GPU filter: {len(docs)} rows, {len(records)} chunks, "
          f"{sum(len(r[0]['positions']) for r in records)} tokens", flush=True)
    return _DECIDE


@pytest.mark.parametrize("form,part", [(f, p) for f, n in DECIDE_PARTS.items()
                                       for p in range(n)])
def test_qwen3_4b_decisions_oracle_replay(form, part):
    from oracle import forward as oforward
    from quail_amd.model import SYNTHETIC_FALSE_IDS, SYNTHETIC_TRUE_IDS

    st = _decision_gpu_run()
    spec, records, groups = st["spec"], st["records"], st["groups"]
    torch.backends.cuda.matmul.allow_tf32 = False
    if st.get("form") != form:
        # a fresh oracle arena for this restatement; replays run in chunk order
        st.pop("arena", None)
        torch.cuda.empty_cache()
        st["form"] = form
        st["arena"] = oforward.OracleArena(spec.layers, st["pages"], spec.n_kv, spec.d_head,
                                           device="cuda")
        st["w"] = st.get("w") or oforward.oracle_weights(st["model"], "cuda")
        st["gemm"] = oforward.exact_gemm if form == "fp64" else oforward.DequantGemm()
        st["runs"][form] = ({}, {})
    n_parts = DECIDE_PARTS[form]
    lo = part * len(records) // n_parts
    hi = (part + 1) * len(records) // n_parts
    bits, marg = st["runs"][form]
    with torch.no_grad():
        for i in range(lo, hi):
            host, mode = records[i]
            normed = oforward.forward_chunk(st["w"], host, mode, st["arena"], gemm=st["gemm"])
            b, m = oforward.readout(st["w"], normed, SYNTHETIC_TRUE_IDS, SYNTHETIC_FALSE_IDS)
            for (doc, _, _), x, y in zip(groups[i], b.tolist(), m.tolist()):
                bits[doc], marg[doc] = x, y
    print(f"oracle {form}: chunks {lo}..{hi - 1} of {len(records)}, {len(bits)} rows decided",
          flush=True)
    if part == n_parts - 1:
        assert len(bits) == DECIDE_ROWS
        st.pop("arena", None)
        torch.cuda.empty_cache()


def test_qwen3_4b_decisions_over_1024_rows_agree_within_the_oracle_floor():
    """The two oracle forms are equally valid restatements of the reference's
    arithmetic; their margin shift |fp32 - fp64| measures the noise any
    change of accumulation order makes on this random-init model (36
    layers of dynamic 1x128 fp8 re-quantization). The band is that shift's
    99th percentile. Bars: beyond twice the band the GPU decides every row
    as the fp64 oracle does; beyond the band it agrees on at least 98 % of
    rows; its median margin shift is at most 1.5 times the oracle pair's
    (the GPU has three families of rounding differences - GEMM block sums,
    attention's bf16 P and output, norm summation orders - where the pair
    has one); and its overall agreement is within three binomial standard
    deviations of the pair's. Taking any one of those families from the
    oracle instead leaves the agreement within a few rows of the GPU's
    (a separate run of the same rows: GEMMs 913, attention 919, norms 920 against the GPU's
    915 of 1,024), so no single stage dominates."""
    from e2e_support import decision_stats, describe

    st = _decision_gpu_run()
    assert set(st["runs"]) == set(DECIDE_PARTS), "run the replay parts first"
    n = DECIDE_ROWS
    gpu = (st["answers"], st["margins"])
    stats = decision_stats(gpu, st["runs"]["fp64"], st["runs"]["fp32"])
    print(describe(stats), flush=True)
    assert stats["gpu_agree_wide"] == stats["outside_wide"], stats["disagree_margins"]
    assert stats["gpu_agree_band"] >= 0.98 * stats["outside_band"], stats
    assert stats["gpu_shift_median"] <= 1.5 * stats["oracle_shift_median"], stats
    q = 1.0 - stats["floor"] / n
    slack = 3.0 * (2.0 * n * q * (1.0 - q)) ** 0.5
    assert stats["gpu_agree"] >= stats["floor"] - slack, stats
