"""The forward-pass engine: the primitives a model loop calls, on gfx950 kernels.

Same surface as the reference's Engine (quail/backends/quail/executor/
attention.py:84-953): the constructor Qwen3Pipeline calls
(models/qwen3.py:26-29), weight_scale, gemm, quant, norm_quant,
activation_quant, qk_norm_rope, attention, attention_unified,
attention_tree, fused_add_rms_norm. Every primitive launches a kernel of
libquail_hip.so; nothing falls back to torch math. Two attention paths:

  unified  scatter the chunk's fresh K/V rows into the arena (plus the
           kept-page tail copies of suffix temporaries), then one paged
           causal call in which every row reads the KV its document needs
           (attention.py:878-953). attention() runs it with the 1x128 fp8
           quant in the kernel's epilogue; attention_unified() returns the
           bf16 output, as the reference's does.
  tree     scatter the kept rows, then one fused kernel: each causal
           segment attends its node (resident KV its rows read, non-causal)
           and its own rows (causal) under one softmax, fp8-quantized in the
           epilogue - the exact attention the reference's call A + call B +
           LSE merge compose (attention.py:835-870). tree_kernel="two_pass"
           runs that three-launch form instead (call A, call B stacked,
           merge_attn_quant), with the reference's bf16 roundings.
"""

import math

from quail_amd import kernels

GROUP = kernels.GROUP


class Engine:
    """Kernels, quantization and attention over the paged arena.

    Args (the reference's first, attention.py:98-99):
        arena: KVArena the attention paths read and write.
        n_q, n_kv, head_dim: head geometry.
        rotary: object with cos_sin_cache ([max_pos, head_dim] bf16, cos|sin).
        fp8: whether linears are fp8 block-quantized. bf16 linears (the
            reference's rerankers) are not part of quail_amd: False raises.
        kernels: "quail", the fused kernel set. The reference's "vllm"
            ablation set (attention.py:690-723) is not built here and raises.
    Options of quail_amd's engine:
        ue8m0: round activation scales up to powers of two (DeepGEMM's
            UE8M0 mode, attention.py:115); fp32 scales otherwise.
        gemm_hook: optional callable(name, M, N, K, launch) wrapping GEMM
            launches (bench.py times them with HIP events).
        attention_hook: optional callable(kind, pairs, kv_rows, n_queries,
            launch) wrapping attention launches.
        tree_kernel: "fused" (one kernel, node pages streamed per q-tile),
            "resident" (one kernel, each node's K/V held in LDS while a
            workgroup walks the q-tiles that read it; used when every
            page-table row of the chunk's reads fits 16 pages, the fused
            kernel otherwise; same bits) or "two_pass" (call A, call B,
            merge).
        fuse_kv_write: on the unified path, let the q/k norm + RoPE kernel
            write k and v into the arena (no separate scatter).
        fuse_qkv_epilogue: run the q/k norm + RoPE (and, with fuse_kv_write,
            the arena write) in the qkv GEMM's epilogue, so the qkv rows are
            never written (qkv_project_attention); bit-identical to the
            separate kernels.
    """

    def __init__(self, arena, *, n_q, n_kv, head_dim, rotary, fp8=True,
                 kernels="quail", ue8m0=False, gemm_hook=None,
                 attention_hook=None, tree_kernel="fused", fuse_kv_write=True,
                 fuse_qkv_epilogue=True):
        import torch
        if kernels not in ("quail", "vllm"):
            raise ValueError(f"kernels must be 'quail' or 'vllm', got {kernels!r}")
        if kernels == "vllm":
            raise ValueError("the unfused vLLM kernel set is not part of quail_amd; "
                             "use kernels='quail'")
        if tree_kernel not in ("fused", "resident", "two_pass"):
            raise ValueError("tree_kernel must be 'fused', 'resident' or 'two_pass', "
                             f"got {tree_kernel!r}")
        if not fp8:
            raise ValueError("quail_amd runs fp8 block-scaled linears only")
        self.kernels = kernels
        self.tree_kernel = tree_kernel
        self.fuse_kv_write = bool(fuse_kv_write)
        self.fuse_qkv_epilogue = (bool(fuse_qkv_epilogue) and head_dim == 128
                                  and n_q % 2 == 0 and n_kv % 2 == 0)
        self.torch = torch
        self.arena = arena
        self.rotary = rotary
        self.num_q_heads = n_q
        self.num_kv_heads = n_kv
        self.head_dim = head_dim
        self.use_ue8m0 = bool(ue8m0)
        self.fp8 = torch.float8_e4m3fn
        self.is_fp8 = True
        self.softmax_scale = 1.0 / math.sqrt(head_dim)
        self.gemm_hook = gemm_hook
        self.attention_hook = attention_hook

    # ---- weights and quant ------------------------------------------

    @staticmethod
    def weight_scale(linear):
        """The linear's fp32 block scales: vLLM names them weight_scale or,
        on block-fp8 linears, weight_scale_inv (attention.py:121-127)."""
        for name in ("weight_scale", "weight_scale_inv"):
            scale = getattr(linear, name, None)
            if scale is not None:
                return scale
        raise AttributeError(f"no weight scale on {type(linear).__name__}")

    def hw_scales(self, linear):
        """Whether this linear's GEMMs hand their scales to the MFMA: UE8M0
        mode, and weight block scales that are all powers of two (as vLLM
        leaves them when DeepGEMM runs with UE8M0). Decided once per linear."""
        if not self.use_ue8m0:
            return False
        flag = getattr(linear, "quail_ue8m0_scales", None)
        if flag is None:
            mant, _ = self.torch.frexp(self.weight_scale(linear))
            flag = bool((mant == 0.5).all().item())
            linear.quail_ue8m0_scales = flag
        return flag

    def gemm(self, q_input, input_scale, linear, name="gemm"):
        """bf16 (q_input * input_scale) (W * W_scale)^T (attention.py:129-141)."""
        w = linear.weight
        scale = self.weight_scale(linear)
        hw = self.hw_scales(linear)
        launch = lambda: kernels.fp8_gemm_nt(q_input, input_scale, w, scale,
                                             ue8m0_scales=hw)
        if self.gemm_hook is not None:
            return self.gemm_hook(name, q_input.shape[0], w.shape[0], w.shape[1], launch)
        return launch()

    def gemm_silu_quant(self, q_input, input_scale, linear, name="gate_up"):
        """gate_up GEMM + SiLU gate + fp8 quant in one kernel (gemm then
        activation_quant, bit-identical)."""
        w = linear.weight
        scale = self.weight_scale(linear)
        hw = self.hw_scales(linear)
        launch = lambda: kernels.fp8_gemm_silu_quant(q_input, input_scale, w, scale,
                                                     self.use_ue8m0, ue8m0_scales=hw)
        if self.gemm_hook is not None:
            return self.gemm_hook(name, q_input.shape[0], w.shape[0], w.shape[1], launch)
        return launch()

    def quant(self, x):
        """1x128 fp8 group quant with column-major scales (attention.py:143-151)."""
        return kernels.group_quant(x, self.use_ue8m0)

    def norm_quant(self, hidden, norm, residual=None):
        """RMS-normed, fp8-quantized GEMM input; adds the residual first when given."""
        return kernels.add_rmsnorm_quant(hidden, norm.weight, norm.variance_epsilon,
                                         residual=residual, ue8m0=self.use_ue8m0)

    def activation_quant(self, gate_up):
        """SiLU-gated product of the two gate_up halves, quantized."""
        return kernels.silu_mul_quant(gate_up, self.use_ue8m0)

    def qkv_norm_rope(self, qkv, positions, attn):
        """Normed, rotated q and k, and contiguous v, from the fused qkv output."""
        return kernels.qk_norm_rope(
            qkv, positions, self.rotary.cos_sin_cache, attn.q_norm.weight,
            attn.k_norm.weight, attn.q_norm.variance_epsilon, self.num_q_heads,
            self.num_kv_heads, self.head_dim)

    def qk_norm_rope(self, qkv, positions, attn):
        """Per-head normed and rotated q and k (attention.py:777-781)."""
        q, k, _ = self.qkv_norm_rope(qkv, positions, attn)
        return q, k

    def qkv_attention(self, qkv, positions, attn, chunk):
        """qk_norm_rope then attention, as one step of quail_amd's pipeline.
        On the unified path, where every chunk row is written to the arena,
        the norm/RoPE kernel writes k and v into the layer's pages itself (no
        k/v rows, no separate scatter); the result is bit-identical to the
        two-step form."""
        meta = chunk.meta
        unified = meta.get("unified")
        if (self.fuse_kv_write and chunk.attention_mode != "tree" and unified is not None
                and unified.get("row_dst") is not None):
            k_pool, v_pool = self.arena.page_pools(meta["layer"])
            q = kernels.qk_norm_rope_kv(
                qkv, positions, self.rotary.cos_sin_cache, attn.q_norm.weight,
                attn.k_norm.weight, attn.q_norm.variance_epsilon, self.num_q_heads,
                self.num_kv_heads, self.head_dim, k_pool, v_pool, unified["row_dst"])
            n = q.shape[0]
            return self._unified_fp8(q.view(n, self.num_q_heads, self.head_dim), None,
                                     None, meta)
        q, k, v = self.qkv_norm_rope(qkv, positions, attn)
        return self.attention(q, k, v, chunk)

    def qkv_project_attention(self, q_input, input_scale, attn, positions, chunk):
        """The qkv projection, q/k norm + RoPE, the KV write and attention:
        gemm(qkv_proj) then qkv_attention, with the norm, the rotary and (on
        the unified path) the arena write done in the GEMM's epilogue; the
        same bits as the separate kernels. Returns the o_proj input."""
        if not self.fuse_qkv_epilogue:
            qkv = self.gemm(q_input, input_scale, attn.qkv_proj, "qkv")
            return self.qkv_attention(qkv, positions, attn, chunk)
        lin = attn.qkv_proj
        w, scale, hw = lin.weight, self.weight_scale(lin), self.hw_scales(lin)
        H, KH, D = self.num_q_heads, self.num_kv_heads, self.head_dim
        meta = chunk.meta
        unified = meta.get("unified")
        args = (q_input, input_scale, w, scale, positions, self.rotary.cos_sin_cache,
                attn.q_norm.weight, attn.k_norm.weight, attn.q_norm.variance_epsilon, H, KH)
        if (self.fuse_kv_write and chunk.attention_mode != "tree" and unified is not None
                and unified.get("row_dst") is not None):
            k_pool, v_pool = self.arena.page_pools(meta["layer"])
            launch = lambda: kernels.fp8_gemm_qkv_rope(
                *args, k_pool=k_pool, v_pool=v_pool, row_dst=unified["row_dst"],
                ue8m0_scales=hw)
            q = self._gemm_timed("qkv", q_input.shape[0], w.shape[0], w.shape[1], launch)
            n = q.shape[0]
            return self._unified_fp8(q.view(n, H, D), None, None, meta)
        launch = lambda: kernels.fp8_gemm_qkv_rope(*args, ue8m0_scales=hw)
        q, k, v = self._gemm_timed("qkv", q_input.shape[0], w.shape[0], w.shape[1], launch)
        return self.attention(q, k, v, chunk)

    def _gemm_timed(self, name, M, N, K, launch):
        if self.gemm_hook is not None:
            return self.gemm_hook(name, M, N, K, launch)
        return launch()

    def fused_add_rms_norm(self, hidden, residual, norm):
        """vLLM fused_add_rms_norm in place (attention.py:177-181): residual +=
        hidden, hidden = RMSNorm(residual); returns (hidden, residual)."""
        return kernels.fused_add_rms_norm(hidden, residual, norm.weight,
                                          norm.variance_epsilon)

    def select_rows(self, o_in, o_scale, residual, rows):
        """The answer rows of the last layer's o_proj input and of the residual
        stream: the reference's index_select of the final rows
        (models/qwen3.py:73-74), taken before o_proj instead of after down_proj
        (every op from o_proj on is row-wise, so each kept row's values are
        the same bits)."""
        o_in, o_scale = kernels.gather_quant_rows(o_in, o_scale, rows)
        return o_in, o_scale, kernels.gather_rows(residual, rows)

    def fused_add_rms_norm_rows(self, hidden, residual, rows, norm):
        """The final norm of the answer rows in one kernel: the reference's
        index_select of hidden and residual at `rows`, then
        fused_add_rms_norm (models/qwen3.py:72-76); returns the normed rows."""
        return kernels.final_norm(hidden, residual, rows, norm.weight,
                                  norm.variance_epsilon)

    # ---- attention ----------------------------------------------------

    def attention(self, q, k, v, chunk):
        """Attention over the chunk and the arena; the quantized o_proj input.

        q, k and v are the flat per-row projections (v may be a strided view
        of the qkv output, as the reference's pipeline passes it).
        """
        n = q.shape[0]
        H, KH, D = self.num_q_heads, self.num_kv_heads, self.head_dim
        q3 = q.view(n, H, D)
        k3 = k.view(n, KH, D)
        v3 = v.contiguous().view(n, KH, D)
        if chunk.attention_mode == "tree":
            return self.attention_tree(q3, k3, v3, chunk.meta)
        # attention_unified then quant, with the quant in the kernel's epilogue
        return self._unified_fp8(q3, k3, v3, chunk.meta)

    def _timed(self, kind, pairs, kv_rows, n_queries, launch):
        if self.attention_hook is None:
            return launch()
        return self.attention_hook(kind, pairs, kv_rows, n_queries, launch)

    def _causal_own(self, q3, k3, v3, meta, want_lse):
        """Causal attention of each packed segment over its own rows (call A)."""
        n = q3.shape[0]
        work = meta.get("work", {})
        return self._timed("own", work.get("own_pairs", 0), n, n, lambda: kernels.attention(
            q3, meta["cu_a"], meta["a_len"], n_queries=n, max_q=meta["max_a"],
            softmax_scale=self.softmax_scale, causal=True, k_rows=k3, v_rows=v3,
            cu_k=meta["cu_a"], n_kv=self.num_kv_heads, want_lse=want_lse))

    def _write_unified_kv(self, k3, v3, unified, layer):
        """The unified call's KV writes: chunk rows, then the kept-page tails."""
        k_pool, v_pool = self.arena.page_pools(layer)
        if k3 is not None:  # else the norm/RoPE kernel already wrote the rows
            kernels.kv_row_scatter(k3, v3, k_pool, v_pool, unified["src"], unified["dst"])
        if unified["tail_src"] is not None:
            kernels.kv_row_copy(k_pool, v_pool, unified["tail_src"], unified["tail_dst"])
        return k_pool, v_pool

    def attention_unified(self, q3, k3, v3, meta, *, softmax_scale=None, window=None):
        """Write the chunk's KV to its arena rows, then one causal paged call
        over retained and current KV (attention.py:878-953). Returns the bf16
        output, (rows, heads * dim)."""
        if window is not None:
            raise ValueError("quail_amd has no sliding-window attention")
        scale = self.softmax_scale if softmax_scale is None else float(softmax_scale)
        n = q3.shape[0]
        layer = meta["layer"]
        unified = meta["unified"]
        if unified is None:
            out, _ = self._causal_own(q3, k3, v3, meta, want_lse=False)
            meta["layer"] += 1
            return out.view(n, -1)
        k_pool, v_pool = self._write_unified_kv(k3, v3, unified, layer)
        out, _ = kernels.attention(
            q3, unified["cu_q"], unified["used"], n_queries=n, max_q=unified["max_q"],
            softmax_scale=scale, causal=True, k_pool=k_pool, v_pool=v_pool,
            table=unified["table"], n_kv=self.num_kv_heads)
        meta["layer"] += 1
        return out.view(n, -1)

    def _unified_fp8(self, q3, k3, v3, meta):
        """attention_unified followed by quant, in one kernel: the paged causal
        call with the per-head fp8 quant in its epilogue (bit-identical to the
        pair). Returns (e4m3, scales)."""
        n = q3.shape[0]
        layer = meta["layer"]
        unified = meta["unified"]
        if unified is None:
            out, _ = self._causal_own(q3, k3, v3, meta, want_lse=False)
            meta["layer"] += 1
            return self.quant(out.view(n, -1))
        k_pool, v_pool = self._write_unified_kv(k3, v3, unified, layer)
        work = meta.get("work", {})
        q_out = self._timed(
            "unified", work.get("unified_pairs", 0), work.get("unified_kv_rows", 0), n,
            lambda: kernels.attention_fp8(
                q3, unified["cu_q"], unified["used"], n_queries=n, max_q=unified["max_q"],
                softmax_scale=self.softmax_scale, causal=True, k_pool=k_pool,
                v_pool=v_pool, table=unified["table"], n_kv=self.num_kv_heads,
                ue8m0=self.use_ue8m0))
        meta["layer"] += 1
        return q_out

    def attention_tree(self, q3, k3, v3, meta):
        """The tree path (attention.py:835-870): call A over the chunk's own
        segments, call B over resident KV, LSE merge and fp8 quant. Returns
        the (e4m3, scales) o_proj input."""
        n = q3.shape[0]
        layer = meta["layer"]
        k_pool, v_pool = self.arena.page_pools(layer)
        if meta["kv_src"] is not None:
            kernels.kv_row_scatter(k3, v3, k_pool, v_pool, meta["kv_src"], meta["kv_dst"])
        reads = meta["reads"]
        if self.tree_kernel in ("fused", "resident"):
            resident = (self.tree_kernel == "resident" and reads is not None
                        and reads["table"].shape[1] * kernels.PAGE_TOKENS <= 256)
            work = meta.get("work", {})
            pairs = work.get("own_pairs", 0) + work.get("read_pairs", 0)
            kv_rows = n + work.get("read_kv_rows", 0)
            q_out = self._timed("tree", pairs, kv_rows, n, lambda: kernels.tree_attention(
                q3, k3, v3, meta["cu_a"], meta["a_read"], softmax_scale=self.softmax_scale,
                k_pool=k_pool if reads is not None else None,
                v_pool=v_pool if reads is not None else None,
                table=reads["table"] if reads is not None else None,
                used=reads["used"] if reads is not None else None, ue8m0=self.use_ue8m0,
                resident=resident))
            meta["layer"] += 1
            return q_out
        out_a, lse_a = self._causal_own(q3, k3, v3, meta, want_lse=reads is not None)
        if reads is None:
            meta["layer"] += 1
            return self.quant(out_a.view(n, -1))
        work = meta.get("work", {})
        out_b, lse_b = self._timed(
            "read", work.get("read_pairs", 0), work.get("read_kv_rows", 0), reads["n_rows"],
            lambda: kernels.attention(
                q3, reads["cu_q"], reads["used"], n_queries=reads["n_rows"],
                max_q=reads["max_q"], softmax_scale=self.softmax_scale, causal=False,
                k_pool=k_pool, v_pool=v_pool, table=reads["table"], q_rows=reads["rows"],
                n_kv=self.num_kv_heads, want_lse=True))
        q_out, scales = kernels.merge_attn_quant(out_a, lse_a, out_b, lse_b,
                                                 reads["source"], self.use_ue8m0)
        meta["layer"] += 1
        return q_out, scales
