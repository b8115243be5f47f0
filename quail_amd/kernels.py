"""Torch-facing wrappers of the gfx950 kernels (libquail_hip.so).

Each wrapper checks dtypes and layouts, allocates its outputs with torch on
the input's device (kernels never allocate), and launches on the current
torch stream. Activation scales come back the way the reference hands them
to its GEMM: a (T, G) fp32 view of column-major (G, T) storage
(attention.py:153-156).
"""

import torch

from quail_amd import _hip

GROUP = 128        # fp8 quant group, one MFMA K block (attention.py:30)
PAGE_TOKENS = 16   # tokens per arena page (quail/cost/budgets.py:10)


def _ptr(t):
    return None if t is None else t.data_ptr()


def _stream():
    return torch.cuda.current_stream().cuda_stream


def _check(t, dtype, name, *, dim=None, contiguous_rows=True):
    if not t.is_cuda:
        raise ValueError(f"{name} must be a GPU tensor")
    if t.dtype != dtype:
        raise ValueError(f"{name} must be {dtype}, got {t.dtype}")
    if dim is not None and t.dim() != dim:
        raise ValueError(f"{name} must have {dim} dims, got {tuple(t.shape)}")
    if contiguous_rows and t.stride(-1) != 1:
        raise ValueError(f"{name} rows must be contiguous")


def col_major_scales(n_tokens, width, device):
    """fp32 scales stored (width/128, T), viewed (T, width/128)."""
    return torch.empty((width // GROUP, n_tokens), dtype=torch.float32,
                       device=device).t()


def add_rmsnorm_quant(x, weight, eps, residual=None, ue8m0=False):
    """RMS-normed, fp8-quantized rows; adds the residual (in place) first.

    The Triton add_rms_norm_quant (attention.py:325-359) with a residual,
    the layer-0 rms_norm + quant (attention.py:158-175) without one.
    """
    _check(x, torch.bfloat16, "x", dim=2)
    _check(weight, torch.bfloat16, "weight", dim=1)
    T, H = x.shape
    if residual is not None:
        _check(residual, torch.bfloat16, "residual", dim=2)
        if residual.shape != x.shape:
            raise ValueError("residual shape differs from x")
    q = torch.empty((T, H), dtype=torch.float8_e4m3fn, device=x.device)
    scales = col_major_scales(T, H, x.device)
    _hip.call("qh_add_rmsnorm_quant", _ptr(x), x.stride(0), _ptr(residual),
              residual.stride(0) if residual is not None else 0, _ptr(weight),
              float(eps), T, H, _ptr(q), _ptr(scales), int(bool(ue8m0)),
              _stream())
    return q, scales


def group_quant(x, ue8m0=False):
    """vLLM per_token_group_quant_fp8 with column-major scales (attention.py:143-151)."""
    _check(x, torch.bfloat16, "x", dim=2)
    T, W = x.shape
    q = torch.empty((T, W), dtype=torch.float8_e4m3fn, device=x.device)
    scales = col_major_scales(T, W, x.device)
    _hip.call("qh_group_quant", _ptr(x), x.stride(0), T, W, _ptr(q),
              _ptr(scales), int(bool(ue8m0)), _stream())
    return q, scales


def _check_gemm(a, a_scales, w, w_scales):
    _check(a, torch.float8_e4m3fn, "a", dim=2)
    _check(w, torch.float8_e4m3fn, "w", dim=2)
    M, K = a.shape
    N = w.shape[0]
    if w.shape[1] != K:
        raise ValueError(f"K mismatch: a {tuple(a.shape)} w {tuple(w.shape)}")
    if a_scales.dtype != torch.float32 or tuple(a_scales.shape) != (M, K // GROUP) \
            or (M > 1 and a_scales.stride(0) != 1) or (M > 0 and a_scales.stride(1) != M):
        raise ValueError("a_scales must be a (M, K/128) view of column-major fp32")
    if w_scales.dtype != torch.float32 or tuple(w_scales.shape) != (N // GROUP, K // GROUP) \
            or not w_scales.is_contiguous():
        raise ValueError("w_scales must be contiguous fp32 (N/128, K/128)")
    return M, N, K


def fp8_gemm_nt(a, a_scales, w, w_scales, out=None, ue8m0_scales=False):
    """out = (a * a_scales) (w * w_scales)^T in bf16 (DeepGEMM fp8_gemm_nt semantics).

    a [M, K] e4m3 with (M, K/128) column-major fp32 scales; w [N, K] e4m3
    with (N/128, K/128) fp32 block scales. ue8m0_scales: every scale of both
    operands is a power of two, and the MFMA applies them itself
    (qh_fp8_gemm_nt_ue8m0).
    """
    M, N, K = _check_gemm(a, a_scales, w, w_scales)
    if out is None:
        out = torch.empty((M, N), dtype=torch.bfloat16, device=a.device)
    _hip.call("qh_fp8_gemm_nt_ue8m0" if ue8m0_scales else "qh_fp8_gemm_nt", _ptr(a),
              a.stride(0), _ptr(a_scales), _ptr(w), w.stride(0), _ptr(w_scales), _ptr(out),
              out.stride(0), M, N, K, _stream())
    return out


def fp8_gemm_silu_quant(a, a_scales, w, w_scales, ue8m0=False, ue8m0_scales=False):
    """silu_mul_quant(fp8_gemm_nt(a, w)) in one kernel, bit-identical to the pair.

    w is the merged gate_up weight [2I, K] (gate rows, then up rows) with
    (2I/128, K/128) block scales. Returns the e4m3 [M, I] activation and its
    (M, I/128) column-major scales (attention.py:300-323 semantics).
    ue8m0_scales: the input scales are powers of two, applied by the MFMA,
    and the output scales are UE8M0 too (qh_fp8_gemm_silu_quant_ue8m0).
    """
    M, N, K = _check_gemm(a, a_scales, w, w_scales)
    if N % (2 * GROUP):
        raise ValueError(f"gate_up rows {N} must be a multiple of 256")
    if ue8m0_scales and not ue8m0:
        raise ValueError("ue8m0_scales=True writes UE8M0 output scales: pass ue8m0=True")
    inter = N // 2
    q = torch.empty((M, inter), dtype=torch.float8_e4m3fn, device=a.device)
    scales = col_major_scales(M, inter, a.device)
    if ue8m0_scales:
        _hip.call("qh_fp8_gemm_silu_quant_ue8m0", _ptr(a), a.stride(0), _ptr(a_scales),
                  _ptr(w), w.stride(0), _ptr(w_scales), M, inter, K, _ptr(q), q.stride(0),
                  _ptr(scales), _stream())
    else:
        _hip.call("qh_fp8_gemm_silu_quant", _ptr(a), a.stride(0), _ptr(a_scales), _ptr(w),
                  w.stride(0), _ptr(w_scales), M, inter, K, _ptr(q), q.stride(0),
                  _ptr(scales), int(bool(ue8m0)), _stream())
    return q, scales


def fp8_gemm_qkv_rope(a, a_scales, w, w_scales, positions, cos_sin, q_weight, k_weight, eps,
                      n_q, n_kv, *, k_pool=None, v_pool=None, row_dst=None,
                      ue8m0_scales=False):
    """The qkv projection with the per-head q/k RMSNorm + NeoX rotary in its
    epilogue: fp8_gemm_nt then qk_norm_rope, bit for bit, without the qkv
    rows. Returns (q, k, v); with row_dst, k and v go to arena rows
    row_dst[m] of k_pool / v_pool instead and only q is returned."""
    _check_gemm(a, a_scales, w, w_scales)
    _check(cos_sin, torch.bfloat16, "cos_sin", dim=2)
    M, K = a.shape
    if w.shape[0] != (n_q + 2 * n_kv) * 128 or cos_sin.shape[1] != 128:
        raise ValueError("qkv weight rows must be (n_q + 2 n_kv) * 128 with head_dim 128")
    if positions.dtype != torch.int64 or positions.numel() != M or not positions.is_contiguous():
        raise ValueError("positions must be contiguous int64, one per row")
    dev = a.device
    q = torch.empty((M, n_q * 128), dtype=torch.bfloat16, device=dev)
    hw = int(bool(ue8m0_scales))
    if row_dst is None:
        k = torch.empty((M, n_kv * 128), dtype=torch.bfloat16, device=dev)
        v = torch.empty((M, n_kv * 128), dtype=torch.bfloat16, device=dev)
        _hip.call("qh_fp8_gemm_qkv_rope", _ptr(a), a.stride(0), _ptr(a_scales), _ptr(w),
                  w.stride(0), _ptr(w_scales), M, K, n_q, n_kv, _ptr(positions),
                  _ptr(cos_sin), cos_sin.shape[0], _ptr(q_weight), _ptr(k_weight),
                  float(eps), _ptr(q), q.stride(0), _ptr(k), _ptr(v), k.stride(0), hw,
                  _stream())
        return q, k, v
    if row_dst.dtype != torch.int64 or row_dst.numel() != M or not row_dst.is_contiguous():
        raise ValueError("row_dst must be contiguous int64, one arena row per row")
    _hip.call("qh_fp8_gemm_qkv_rope_kv", _ptr(a), a.stride(0), _ptr(a_scales), _ptr(w),
              w.stride(0), _ptr(w_scales), M, K, n_q, n_kv, _ptr(positions), _ptr(cos_sin),
              cos_sin.shape[0], _ptr(q_weight), _ptr(k_weight), float(eps), _ptr(q),
              q.stride(0), _ptr(k_pool), _ptr(v_pool), _ptr(row_dst), PAGE_TOKENS, hw,
              _stream())
    return q


def qk_norm_rope(qkv, positions, cos_sin, q_weight, k_weight, eps, n_q, n_kv,
                 head_dim):
    """Per-head RMSNorm + NeoX rotary of q and k, and contiguous v.

    The Triton qk_norm_rope (attention.py:361-409) plus the v copy of
    Engine.attention (attention.py:793).
    """
    _check(qkv, torch.bfloat16, "qkv", dim=2)
    _check(cos_sin, torch.bfloat16, "cos_sin", dim=2)
    if positions.dtype != torch.int64 or not positions.is_contiguous():
        raise ValueError("positions must be contiguous int64")
    T = qkv.shape[0]
    dev = qkv.device
    q = torch.empty((T, n_q * head_dim), dtype=torch.bfloat16, device=dev)
    k = torch.empty((T, n_kv * head_dim), dtype=torch.bfloat16, device=dev)
    v = torch.empty((T, n_kv * head_dim), dtype=torch.bfloat16, device=dev)
    _hip.call("qh_qk_norm_rope", _ptr(qkv), qkv.stride(0), _ptr(positions),
              _ptr(cos_sin), cos_sin.shape[0], _ptr(q_weight), _ptr(k_weight),
              float(eps), T, n_q, n_kv, head_dim, _ptr(q), _ptr(k), _ptr(v),
              _stream())
    return q, k, v


def qk_norm_rope_kv(qkv, positions, cos_sin, q_weight, k_weight, eps, n_q, n_kv,
                    head_dim, k_pool, v_pool, row_dst, page_tokens=PAGE_TOKENS):
    """qk_norm_rope with row t's k and v written to arena row row_dst[t]
    (the Triton qk_norm_rope, attention.py:361-409, then the unified call's
    kv_row_scatter, :411-427, in one pass). Returns q."""
    _check(qkv, torch.bfloat16, "qkv", dim=2)
    _check(cos_sin, torch.bfloat16, "cos_sin", dim=2)
    if positions.dtype != torch.int64 or not positions.is_contiguous():
        raise ValueError("positions must be contiguous int64")
    T = qkv.shape[0]
    if row_dst.dtype != torch.int64 or row_dst.numel() != T or not row_dst.is_contiguous():
        raise ValueError("row_dst must be contiguous int64, one arena row per chunk row")
    q = torch.empty((T, n_q * head_dim), dtype=torch.bfloat16, device=qkv.device)
    _hip.call("qh_qk_norm_rope_kv", _ptr(qkv), qkv.stride(0), _ptr(positions),
              _ptr(cos_sin), cos_sin.shape[0], _ptr(q_weight), _ptr(k_weight),
              float(eps), T, n_q, n_kv, head_dim, _ptr(q), _ptr(k_pool), _ptr(v_pool),
              _ptr(row_dst), page_tokens, _stream())
    return q


def kv_row_scatter(k_rows, v_rows, k_pool, v_pool, src, dst,
                   page_tokens=PAGE_TOKENS):
    """Arena rows dst[i] <- chunk rows src[i] (attention.py:411-427)."""
    n = src.numel()
    if n == 0:
        return
    if src.dtype != torch.int64 or dst.dtype != torch.int64 or dst.numel() != n:
        raise ValueError("src/dst must be int64 of equal length")
    n_kv, d = k_pool.shape[1], k_pool.shape[-1]
    _hip.call("qh_kv_row_scatter", _ptr(k_rows), _ptr(v_rows), _ptr(k_pool),
              _ptr(v_pool), _ptr(src), _ptr(dst), n, n_kv, d, page_tokens,
              _stream())


def kv_row_copy(k_pool, v_pool, src, dst, page_tokens=PAGE_TOKENS):
    """Arena rows dst[i] <- arena rows src[i] (the unified path's tail copy)."""
    n = src.numel()
    if n == 0:
        return
    n_kv, d = k_pool.shape[1], k_pool.shape[-1]
    _hip.call("qh_kv_row_copy", _ptr(k_pool), _ptr(v_pool), _ptr(src),
              _ptr(dst), n, n_kv, d, page_tokens, _stream())


def attention(q3, cu_q, kv_len, *, n_queries, max_q, softmax_scale, causal,
              k_pool=None, v_pool=None, table=None, k_rows=None, v_rows=None,
              cu_k=None, q_rows=None, n_kv, want_lse=False, out=None):
    """Varlen attention over paged arena KV (table) or chunk rows (cu_k).

    q3 [rows, n_q, d] bf16. Returns (out [n_queries, n_q, d] bf16, lse
    [n_q, n_queries] fp32 or None). The three FlashAttention calls of
    attention.py:850-864 and :939-943.
    """
    _check(q3, torch.bfloat16, "q", dim=3)
    rows, n_q, d = q3.shape
    n_seqs = cu_q.numel() - 1
    dev = q3.device
    if out is None:
        out = torch.empty((n_queries, n_q, d), dtype=torch.bfloat16, device=dev)
    lse = (torch.empty((n_q, n_queries), dtype=torch.float32, device=dev)
           if want_lse else None)
    ws = torch.empty(_hip.workspace_bytes(n_seqs), dtype=torch.uint8, device=dev)
    if table is not None:
        pool_pages = k_pool.shape[0]
        table_width = table.shape[1]
        args_kv = (_ptr(k_pool), _ptr(v_pool), pool_pages, _ptr(table),
                   table_width, PAGE_TOKENS, None, None, 0, None)
    else:
        args_kv = (None, None, 0, None, 0, PAGE_TOKENS, _ptr(k_rows),
                   _ptr(v_rows), k_rows.shape[0], _ptr(cu_k))
    _hip.call("qh_attention", _ptr(q3), q3.stride(0), rows, _ptr(q_rows),
              *args_kv, _ptr(cu_q), _ptr(kv_len), n_seqs, int(n_queries),
              int(max_q), n_q, n_kv, d, float(softmax_scale), int(bool(causal)),
              _ptr(out), out.stride(0), _ptr(lse),
              lse.stride(0) if lse is not None else 0, _ptr(ws), ws.numel(),
              _stream())
    return out, lse


def attention_fp8(q3, cu_q, kv_len, *, n_queries, max_q, softmax_scale, causal,
                  k_pool, v_pool, table, n_kv, q_rows=None, ue8m0=False):
    """Paged attention whose output is fp8-quantized per (row, head) in the
    kernel: (e4m3 [n_queries, n_q*d], scales (n_queries, n_q) column-major),
    bit-identical to group_quant(attention(...)) (attention.py:939-943, :798)."""
    _check(q3, torch.bfloat16, "q", dim=3)
    rows, n_q, d = q3.shape
    if d != GROUP:
        raise ValueError("one quant group per head needs head_dim 128")
    n_seqs = cu_q.numel() - 1
    dev = q3.device
    q = torch.empty((n_queries, n_q * d), dtype=torch.float8_e4m3fn, device=dev)
    scales = col_major_scales(n_queries, n_q * d, dev)
    ws = torch.empty(_hip.workspace_bytes(n_seqs), dtype=torch.uint8, device=dev)
    _hip.call("qh_attention_fp8", _ptr(q3), q3.stride(0), rows, _ptr(q_rows),
              _ptr(k_pool), _ptr(v_pool), k_pool.shape[0], _ptr(table), table.shape[1],
              PAGE_TOKENS, _ptr(cu_q), _ptr(kv_len), n_seqs, int(n_queries), int(max_q),
              n_q, n_kv, d, float(softmax_scale), int(bool(causal)), _ptr(q), q.stride(0),
              _ptr(scales), int(bool(ue8m0)), _ptr(ws), ws.numel(), _stream())
    return q, scales


def tree_attention(q3, k_rows, v_rows, cu_a, seg_read, *, softmax_scale, k_pool=None,
                   v_pool=None, table=None, used=None, fp8=True, ue8m0=False,
                   resident=False):
    """The tree path's attention in one kernel: each causal segment of cu_a
    attends its read sequence seg_read[s] (page-table row of `table`, used
    keys) in full and its own rows causally, under one softmax (the exact
    result of attention.py:835-870's call A + call B + merge).

    resident=True runs the node-resident kernel (each node's K/V held in LDS
    for all the q-tiles a workgroup takes that read it; page-table rows of at
    most 16 pages), which gives the same bits.

    Returns (e4m3 [T, n_q*d], scales (T, n_q) column-major) with fp8, else
    bf16 [T, n_q, d].
    """
    _check(q3, torch.bfloat16, "q", dim=3)
    _check(k_rows, torch.bfloat16, "k_rows", dim=3)
    _check(v_rows, torch.bfloat16, "v_rows", dim=3)
    T, n_q, d = q3.shape
    n_kv = k_rows.shape[1]
    if k_rows.shape[0] != T or v_rows.shape != k_rows.shape or k_rows.stride(0) != v_rows.stride(0):
        raise ValueError("k_rows / v_rows must be [T, n_kv, d] with one row stride")
    if k_rows.stride(1) != d or q3.stride(1) != d:
        raise ValueError("heads of q / k_rows / v_rows must be contiguous")
    n_seg = cu_a.numel() - 1
    if seg_read.dtype != torch.int32 or seg_read.numel() != n_seg:
        raise ValueError("seg_read must be int32 with one entry per segment")
    dev = q3.device
    n_reads = 0 if table is None else table.shape[0]
    if n_reads and (used is None or used.numel() != n_reads):
        raise ValueError("used must have one entry per page-table row")
    ws = torch.empty(_hip.workspace_bytes(n_seg), dtype=torch.uint8, device=dev)
    out = q = scales = None
    if fp8:
        if d != GROUP:
            raise ValueError("one quant group per head needs head_dim 128")
        q = torch.empty((T, n_q * d), dtype=torch.float8_e4m3fn, device=dev)
        scales = col_major_scales(T, n_q * d, dev)
    else:
        out = torch.empty((T, n_q, d), dtype=torch.bfloat16, device=dev)
    entry = "qh_tree_attention_resident" if resident else "qh_tree_attention"
    _hip.call(entry, _ptr(q3), q3.stride(0), T, _ptr(k_rows), _ptr(v_rows),
              k_rows.stride(0), _ptr(cu_a), _ptr(seg_read), n_seg,
              _ptr(k_pool), _ptr(v_pool), 0 if k_pool is None else k_pool.shape[0],
              _ptr(table), 0 if table is None else table.shape[1], _ptr(used), n_reads,
              PAGE_TOKENS, n_q, n_kv, d, float(softmax_scale), _ptr(out),
              0 if out is None else out.stride(0), _ptr(q), 0 if q is None else q.stride(0),
              _ptr(scales), int(bool(ue8m0)), _ptr(ws), ws.numel(), _stream())
    return (q, scales) if fp8 else out


def merge_attn_quant(out_a, lse_a, out_b, lse_b, source, ue8m0=False):
    """LSE merge of the tree path + per-head fp8 quant (attention.py:429-473).

    lse_a/lse_b are [heads, rows] fp32 (FlashAttention's layout).
    """
    T, n_h, d = out_a.shape
    if d != GROUP:
        raise ValueError("one quant group per head needs head_dim 128")
    q = torch.empty((T, n_h * d), dtype=torch.float8_e4m3fn, device=out_a.device)
    scales = col_major_scales(T, n_h * d, out_a.device)
    _hip.call("qh_merge_attn_quant", _ptr(out_a), _ptr(lse_a), lse_a.stride(0),
              _ptr(out_b), _ptr(lse_b), lse_b.stride(0), _ptr(source), T, n_h,
              _ptr(q), _ptr(scales), int(bool(ue8m0)), _stream())
    return q, scales


def silu_mul_quant(gate_up, ue8m0=False):
    """silu(gate) * up, fp8-quantized per 1x128 group (attention.py:300-323)."""
    _check(gate_up, torch.bfloat16, "gate_up", dim=2)
    T, doubled = gate_up.shape
    inter = doubled // 2
    q = torch.empty((T, inter), dtype=torch.float8_e4m3fn, device=gate_up.device)
    scales = col_major_scales(T, inter, gate_up.device)
    _hip.call("qh_silu_mul_quant", _ptr(gate_up), gate_up.stride(0), T, inter,
              _ptr(q), _ptr(scales), int(bool(ue8m0)), _stream())
    return q, scales


def gather_rows(table, idx, out=None):
    """out[i] = table[idx[i]] for bf16 rows (embedding lookup, index_select)."""
    _check(table, torch.bfloat16, "table", dim=2)
    if idx.dtype != torch.int64 or not idx.is_contiguous():
        raise ValueError("idx must be contiguous int64")
    n, W = idx.numel(), table.shape[1]
    if out is None:
        out = torch.empty((n, W), dtype=torch.bfloat16, device=table.device)
    _hip.call("qh_gather_rows", _ptr(table), table.stride(0), _ptr(idx), n, W,
              _ptr(out), _stream())
    return out


def gather_quant_rows(q, scales, idx):
    """Rows idx of an fp8 GEMM input and their 1x128 scales: (q[idx], scales[idx])
    with the scales in the same column-major (T, W/128) view."""
    _check(q, torch.float8_e4m3fn, "q", dim=2)
    T, W = q.shape
    if scales.dtype != torch.float32 or scales.shape != (T, W // GROUP) or (
            T > 0 and scales.stride() != (1, T)):
        raise ValueError("scales must be the column-major (T, W/128) fp32 view")
    if idx.dtype != torch.int64 or idx.dim() != 1 or not idx.is_contiguous():
        raise ValueError("idx must be a contiguous 1-d int64 tensor")
    n = idx.numel()
    out = torch.empty((n, W), dtype=torch.float8_e4m3fn, device=q.device)
    out_scales = col_major_scales(n, W, q.device)
    _hip.call("qh_gather_quant_rows", _ptr(q), q.stride(0), _ptr(scales), T, _ptr(idx), n, W,
              _ptr(out), out.stride(0), _ptr(out_scales), _stream())
    return out, out_scales


def final_norm(hidden, residual, final_idx, weight, eps):
    """vLLM fused_add_rms_norm on the gathered answer rows (models/qwen3.py:119-124)."""
    _check(hidden, torch.bfloat16, "hidden", dim=2)
    _check(residual, torch.bfloat16, "residual", dim=2)
    if not (hidden.is_contiguous() and residual.is_contiguous()):
        raise ValueError("hidden and residual must be contiguous")
    R, H = final_idx.numel(), hidden.shape[1]
    out = torch.empty((R, H), dtype=torch.bfloat16, device=hidden.device)
    _hip.call("qh_final_norm", _ptr(hidden), _ptr(residual), _ptr(final_idx), R,
              H, _ptr(weight), float(eps), _ptr(out), _stream())
    return out


def fused_add_rms_norm(hidden, residual, weight, eps):
    """vLLM fused_add_rms_norm in place (attention.py:177-181): residual <-
    hidden + residual, hidden <- RMSNorm(residual) * weight; returns both."""
    _check(hidden, torch.bfloat16, "hidden", dim=2)
    _check(residual, torch.bfloat16, "residual", dim=2)
    if not (hidden.is_contiguous() and residual.is_contiguous()):
        raise ValueError("hidden and residual must be contiguous")
    if hidden.shape != residual.shape:
        raise ValueError("hidden and residual shapes differ")
    R, H = hidden.shape
    _hip.call("qh_fused_add_rms_norm", _ptr(hidden), _ptr(residual), R, H, _ptr(weight),
              float(eps), _stream())
    return hidden, residual


def answer_bits(normed, w_ans, is_true, with_margin=True):
    """TRUE/FALSE bit per row from the retained answer rows (readout.py:45-49, :70-79)."""
    _check(normed, torch.bfloat16, "normed", dim=2)
    R, H = normed.shape
    bits = torch.empty(R, dtype=torch.uint8, device=normed.device)
    margin = (torch.empty(R, dtype=torch.float32, device=normed.device)
              if with_margin else None)
    _hip.call("qh_answer_bits", _ptr(normed), R, H, _ptr(w_ans), w_ans.shape[0],
              _ptr(is_true), _ptr(bits), _ptr(margin), _stream())
    return bits, margin


def e4m3_encode(x):
    """fp32 values -> e4m3 through the fused epilogues' encoder (no clamp)."""
    _check(x, torch.float32, "x", dim=1)
    n = x.shape[0]
    out = torch.empty(n, dtype=torch.uint8, device=x.device)
    _hip.call("qh_e4m3_encode", _ptr(x), n, _ptr(out), _stream())
    return out


def answer_logits(normed, w_ans, is_true):
    """Per row, the best bf16 score of each class (readout.py:45-49)."""
    _check(normed, torch.bfloat16, "normed", dim=2)
    R, H = normed.shape
    best_t = torch.empty(R, dtype=torch.bfloat16, device=normed.device)
    best_f = torch.empty(R, dtype=torch.bfloat16, device=normed.device)
    _hip.call("qh_answer_logits", _ptr(normed), R, H, _ptr(w_ans), w_ans.shape[0],
              _ptr(is_true), _ptr(best_t), _ptr(best_f), _stream())
    return best_t, best_f
