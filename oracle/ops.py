"""Closed forms of the hot-path kernels on the CPU (oracle; tests only).

Every function takes and returns CPU torch tensors and states the reference
code it restates. Floating point follows the reference's op order; where
the reference rounds to bf16 between ops, so does this code.
"""

import math

import torch

GROUP = 128
FP8_MAX = 448.0
SCALE_FLOOR = 1e-10
PAGE = 16


# ---------------------------------------------------------------- fp8 quant

def group_scales(amax, ue8m0):
    """max(amax, 1e-10) / 448, rounded up to a power of two in UE8M0 mode.

    attention.py:313-316 (silu_mul_quant), :349-351, :466-468; vLLM
    per_token_group_quant_fp8 uses the same rule.
    """
    scale = torch.clamp(amax, min=SCALE_FLOOR) / FP8_MAX
    if ue8m0:
        scale = torch.exp2(torch.ceil(torch.log2(scale)))
    return scale


def group_quant(y, ue8m0=False, group=GROUP):
    """Per-row 1 x group fp8 quantization of fp32 values.

    Returns (q float8_e4m3fn [T, W], scales fp32 [T, W/group]):
    q = e4m3(clamp(y / scale, -448, 448)) (attention.py:317-321, :352-356).
    """
    y = y.float()
    T, W = y.shape
    g = y.view(T, W // group, group)
    scale = group_scales(g.abs().amax(dim=2), ue8m0)
    q = torch.clamp(g / scale[:, :, None], -FP8_MAX, FP8_MAX)
    return q.reshape(T, W).to(torch.float8_e4m3fn), scale


def dequant_rows(q, scales, group=GROUP):
    """q [T, W] e4m3 with [T, W/group] scales back to fp32."""
    T, W = q.shape
    return (q.float().view(T, W // group, group) * scales[:, :, None]).view(T, W)


def quantize_weight_blocks(w, ue8m0=False, block=GROUP):
    """Weight [N, K] fp32 -> e4m3 with one fp32 scale per 128 x 128 block.

    scale = max(amax, 1e-10) / 448 over the block, the layout vLLM keeps as
    weight_scale_inv and DeepGEMM reads (attention.py:121-141).
    """
    N, K = w.shape
    b = w.float().view(N // block, block, K // block, block)
    amax = b.abs().amax(dim=(1, 3))
    scale = group_scales(amax, ue8m0)
    q = torch.clamp(b / scale[:, None, :, None], -FP8_MAX, FP8_MAX)
    return q.reshape(N, K).to(torch.float8_e4m3fn), scale.contiguous()


def dequant_weight(q, scales, block=GROUP):
    N, K = q.shape
    b = q.float().view(N // block, block, K // block, block)
    return (b * scales[:, None, :, None]).reshape(N, K)


# ---------------------------------------------------------------- norms

def add_rms_norm_quant(x, residual, weight, eps, ue8m0=False):
    """Triton add_rms_norm_quant (attention.py:325-359).

    s = x + residual in fp32; residual <- bf16(s); y = s * rstd * w with
    rstd = 1 / sqrt(sum(s^2) / H + eps). Returns (q, scales, new_residual).
    """
    s = x.float() + residual.float()
    new_res = s.to(torch.bfloat16)
    H = s.shape[-1]
    ms = (s * s).sum(dim=-1, keepdim=True) / H
    rstd = 1.0 / torch.sqrt(ms + eps)
    y = s * rstd * weight.float()
    q, scales = group_quant(y, ue8m0)
    return q, scales, new_res


def rms_norm_bf16(x, weight, eps):
    """vLLM rms_norm as Engine.rms_norm calls it (attention.py:158-175).

    bf16(bf16(x * rstd) * w), variance over fp32 x.
    """
    xf = x.float()
    H = xf.shape[-1]
    ms = (xf * xf).sum(dim=-1, keepdim=True) / H
    rstd = 1.0 / torch.sqrt(ms + eps)
    normed = (xf * rstd).to(torch.bfloat16).float()
    return (normed * weight.float()).to(torch.bfloat16)


def norm_quant_plain(x, weight, eps, ue8m0=False):
    """Layer-0 norm_quant: quant(rms_norm(x)) (attention.py:763-766)."""
    return group_quant(rms_norm_bf16(x, weight, eps).float(), ue8m0)


def fused_add_rms_norm(hidden, residual, weight, eps):
    """vLLM fused_add_rms_norm (attention.py:177-181).

    z = bf16(h + r) (the residual written back); out = bf16(bf16(z * rstd) * w).
    Returns (out, z).
    """
    z = (hidden.float() + residual.float()).to(torch.bfloat16)
    return rms_norm_bf16(z, weight, eps), z


# ---------------------------------------------------------------- q/k norm + rope

def rope_cache(max_pos, head_dim, theta, dtype=torch.bfloat16):
    """cos | sin per position, NeoX layout, as vLLM's rotary cache holds it.

    inv_freq = theta^(-2i/d); angles = pos * inv_freq in fp32; the cache is
    stored in the model dtype (bf16).
    """
    inv_freq = 1.0 / (theta ** (torch.arange(0, head_dim, 2, dtype=torch.float32)
                                / head_dim))
    t = torch.arange(max_pos, dtype=torch.float32)
    freqs = torch.outer(t, inv_freq)
    return torch.cat([freqs.cos(), freqs.sin()], dim=-1).to(dtype)


def qk_norm_rope(qkv, positions, cos_sin, q_weight, k_weight, eps, n_q, n_kv,
                 head_dim):
    """Triton qk_norm_rope (attention.py:361-409) plus contiguous v.

    Per head: ms = (sum(a^2) + sum(b^2)) / d over the halves a, b;
    a, b <- a * rstd * w_a, b * rstd * w_b; a' = a cos - b sin,
    b' = b cos + a sin. Returns bf16 (q [T, n_q*d], k [T, n_kv*d], v).
    """
    T = qkv.shape[0]
    half = head_dim // 2
    cs = cos_sin[positions].float()
    cos, sin = cs[:, None, :half], cs[:, None, half:]

    def heads(x, w, n):
        x = x.float().view(T, n, head_dim)
        a, b = x[..., :half], x[..., half:]
        ms = ((a * a).sum(-1, keepdim=True) + (b * b).sum(-1, keepdim=True)) / head_dim
        rstd = 1.0 / torch.sqrt(ms + eps)
        wf = w.float()
        a = a * rstd * wf[:half]
        b = b * rstd * wf[half:]
        out_a = a * cos - b * sin
        out_b = b * cos + a * sin
        return torch.cat([out_a, out_b], dim=-1).reshape(T, n * head_dim).to(torch.bfloat16)

    qw = n_q * head_dim
    kw = n_kv * head_dim
    q = heads(qkv[:, :qw], q_weight, n_q)
    k = heads(qkv[:, qw:qw + kw], k_weight, n_kv)
    v = qkv[:, qw + kw:qw + 2 * kw].contiguous()
    return q, k, v


# ---------------------------------------------------------------- MLP gate

def silu_mul(gate_up):
    """gate * sigmoid(gate) * up in fp32 (attention.py:309-311)."""
    inter = gate_up.shape[1] // 2
    g = gate_up[:, :inter].float()
    u = gate_up[:, inter:].float()
    return g * torch.sigmoid(g) * u


def silu_mul_quant(gate_up, ue8m0=False):
    """Triton silu_mul_quant (attention.py:300-323)."""
    return group_quant(silu_mul(gate_up), ue8m0)


# ---------------------------------------------------------------- GEMM

def fp8_gemm(a_q, a_scales, w_q, w_scales, out_dtype=torch.bfloat16):
    """DeepGEMM fp8_gemm_nt semantics (attention.py:129-141).

    out[m, n] = sum_kb a_scales[m, kb] * w_scales[n / 128, kb] *
    sum_{k in kb} A[m, k] W[n, k], products and block sums in fp64.
    """
    M, K = a_q.shape
    N = w_q.shape[0]
    kb_n = K // GROUP
    a = a_q.double().view(M, kb_n, GROUP)
    w = w_q.double().view(N, kb_n, GROUP)
    sb = w_scales.double().repeat_interleave(GROUP, dim=0)  # [N, kb]
    out = torch.zeros(M, N, dtype=torch.float64, device=a_q.device)
    for kb in range(kb_n):
        part = a[:, kb, :] @ w[:, kb, :].T
        out += part * a_scales[:, kb].double()[:, None] * sb[:, kb][None, :]
    return out.to(out_dtype)


# ---------------------------------------------------------------- attention

def attend(q, k, v, scale, visible):
    """Softmax attention of one sequence, all heads, in fp32.

    q [c, H, d], k/v [L, KH, d]; visible [c, L] bool. GQA: head h reads KV
    head h // (H / KH). Returns (out [c, H, d] fp32, lse [H, c] fp32, natural
    log); a row with no visible key gets out 0 and lse -inf.
    """
    c, H, d = q.shape
    KH = k.shape[1]
    rep = H // KH
    kk = k.float().repeat_interleave(rep, dim=1)   # [L, H, d]
    vv = v.float().repeat_interleave(rep, dim=1)
    s = torch.einsum("chd,lhd->hcl", q.float(), kk) * scale
    s = s.masked_fill(~visible[None], float("-inf"))
    lse = torch.logsumexp(s, dim=-1)                # [H, c]
    p = torch.exp(s - lse[..., None])
    p = torch.nan_to_num(p, nan=0.0)
    out = torch.einsum("hcl,lhd->chd", p, vv)
    return out, lse


def causal_visible(c, kv_len, device="cpu"):
    """Bottom-right aligned causal mask: query i of c sees keys 0..kv_len-c+i.

    The alignment tests/kv_checker.py:132-139 asserts for the paged call.
    """
    i = torch.arange(c, device=device)[:, None]
    j = torch.arange(kv_len, device=device)[None, :]
    return j <= (kv_len - c + i)


def gather_pages(pool, table_row, kv_len, page=PAGE):
    """Logical keys 0..kv_len-1 of one sequence from a row-indexed pool.

    pool [n_pages * page, n_kv, d]; key j is arena row
    table_row[j // page] * page + j % page (arena.py:519-523, :874-887).
    """
    j = torch.arange(kv_len)
    rows = table_row.cpu()[j // page].long() * page + j % page
    return pool[rows.to(pool.device)]


def paged_attention(q3, k_pool, v_pool, cu_q, used, table, scale, causal,
                    q_rows=None, page=PAGE):
    """FlashAttention varlen over paged KV (attention.py:820-833, :939-943, :858-864).

    q3 [rows, H, d]; pools [n_rows, KH, d]; cu_q/used/table int. q_rows
    gathers the query rows (call B's reads["rows"]). Returns (out fp32
    [n_queries, H, d], lse fp32 [H, n_queries]).
    """
    cu_q = [int(x) for x in cu_q]
    used = [int(x) for x in used]
    n_queries = cu_q[-1]
    H, d = q3.shape[1], q3.shape[2]
    dev = q3.device
    out = torch.zeros(n_queries, H, d, device=dev)
    lse = torch.full((H, n_queries), float("-inf"), device=dev)
    for s in range(len(used)):
        a, b = cu_q[s], cu_q[s + 1]
        c = b - a
        if c == 0:
            continue
        rows = torch.arange(a, b) if q_rows is None else q_rows[a:b].long()
        q = q3[rows.to(dev)]
        k = gather_pages(k_pool, table[s], used[s], page)
        v = gather_pages(v_pool, table[s], used[s], page)
        vis = (causal_visible(c, used[s], dev) if causal
               else torch.ones(c, used[s], dtype=torch.bool, device=dev))
        o, l = attend(q, k, v, scale, vis)
        out[a:b] = o
        lse[:, a:b] = l
    return out, lse


def varlen_attention(q3, k3, v3, cu, scale, causal=True):
    """FlashAttention varlen over contiguous segments (attention.py:850-852).

    Segment s is rows cu[s]..cu[s+1]-1 for queries and keys alike.
    """
    cu = [int(x) for x in cu]
    T, H, d = q3.shape
    dev = q3.device
    out = torch.zeros(T, H, d, device=dev)
    lse = torch.full((H, T), float("-inf"), device=dev)
    for s in range(len(cu) - 1):
        a, b = cu[s], cu[s + 1]
        c = b - a
        if c == 0:
            continue
        vis = (causal_visible(c, c, dev) if causal
               else torch.ones(c, c, dtype=torch.bool, device=dev))
        o, l = attend(q3[a:b], k3[a:b], v3[a:b], scale, vis)
        out[a:b] = o
        lse[:, a:b] = l
    return out, lse


def tree_attention(q3, k3, v3, cu_a, seg_read, k_pool, v_pool, table, used, scale,
                   page=PAGE):
    """The tree path's attention in exact arithmetic (attention.py:835-870).

    Segment s of cu_a (rows a..b of the chunk) attends the used[r] keys of
    page-table row r = seg_read[s] (when r >= 0) in full, and its own rows
    k3/v3[a..b] causally; one softmax over both key sets. Call A (own
    segments), call B (the read) and the LSE merge compute this same value
    up to their intermediate bf16 roundings. Returns out fp32 [T, H, d].
    """
    cu = [int(x) for x in cu_a]
    T, H, d = q3.shape
    dev = q3.device
    out = torch.zeros(T, H, d, device=dev)
    for s in range(len(cu) - 1):
        a, b = cu[s], cu[s + 1]
        c = b - a
        if c == 0:
            continue
        r = int(seg_read[s])
        own_vis = causal_visible(c, c, dev)
        if r >= 0:
            n = int(used[r])
            k = torch.cat([gather_pages(k_pool, table[r], n, page).float(), k3[a:b].float()])
            v = torch.cat([gather_pages(v_pool, table[r], n, page).float(), v3[a:b].float()])
            vis = torch.cat([torch.ones(c, n, dtype=torch.bool, device=dev), own_vis], dim=1)
        else:
            k, v, vis = k3[a:b], v3[a:b], own_vis
        out[a:b], _ = attend(q3[a:b], k, v, scale, vis)
    return out


def merge_attn(out_a, lse_a, out_b, lse_b, source):
    """The LSE merge of merge_attn_quant before its quant (attention.py:440-464).

    w = bf16(sigmoid(lse_b - lse_a)); y = bf16(a + (b - a) w) where
    source[t] >= 0, else a. out_a/out_b bf16 [rows, H, d]; lse [H, rows].
    Returns fp32 values of the bf16 result.
    """
    a = out_a.float()
    src = source.long().to(a.device)
    has_b = src >= 0
    safe = src.clamp(min=0)
    b = out_b.float()[safe]
    la = lse_a.T                                     # [rows, H]
    lb = lse_b.T[safe]
    w = torch.sigmoid(lb - la).to(torch.bfloat16).float()
    merged = (a + (b - a) * w[..., None]).to(torch.bfloat16).float()
    return torch.where(has_b[:, None, None], merged, a)


def merge_attn_quant(out_a, lse_a, out_b, lse_b, source, ue8m0=False):
    y = merge_attn(out_a, lse_a, out_b, lse_b, source)
    T, H, d = y.shape
    return group_quant(y.reshape(T, H * d), ue8m0)


# ---------------------------------------------------------------- KV + readout

def kv_row_scatter(k_pool, v_pool, k_rows, v_rows, src, dst):
    """pool[dst[i]] = rows[src[i]] for K and V (attention.py:415-427), in place."""
    src, dst = src.long().to(k_pool.device), dst.long().to(k_pool.device)
    k_pool[dst] = k_rows[src]
    v_pool[dst] = v_rows[src]


def answer_bits(normed, w_ans, true_cols, false_cols):
    """AnswerRows.logits + AsyncAnswers.submit (readout.py:45-49, :70-79).

    scores = bf16(normed @ W^T); bit = max(true) > max(false), strict.
    Returns (bits uint8 [R], margin fp32 [R]).
    """
    scores = (normed.float() @ w_ans.float().T).to(torch.bfloat16).float()
    t = scores[:, true_cols].amax(dim=1)
    f = scores[:, false_cols].amax(dim=1)
    return (t > f).to(torch.uint8), t - f


def softmax_scale(head_dim):
    return 1.0 / math.sqrt(head_dim)
