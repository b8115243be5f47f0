"""Qwen3 forward over a packed chunk on the CPU (oracle; tests and cpu_baseline only).

Restates Qwen3Pipeline.forward_chunk of the reference (models/qwen3.py:
46-77) with the Engine semantics of attention.py (norm_quant :763-769,
gemm :129-141, qk_norm_rope :361-409, attention_unified :878-953,
attention_tree :835-870, activation_quant :300-323, final
fused_add_rms_norm :177-181). KV lives in a logical arena: per layer, K and
V as (rows, n_kv, d) bf16 indexed by the reference's arena row numbers; the
chunk's scatter maps write it exactly as the kernels write the device pools.
"""

import torch

from oracle import ops


class OracleArena:
    """Per-layer logical K/V pools, arena rows page * 16 + slot."""

    def __init__(self, n_layers, n_pages, n_kv, head_dim, page_tokens=16, device="cpu"):
        rows = n_pages * page_tokens
        self.k = [torch.zeros(rows, n_kv, head_dim, dtype=torch.bfloat16, device=device)
                  for _ in range(n_layers)]
        self.v = [torch.zeros(rows, n_kv, head_dim, dtype=torch.bfloat16, device=device)
                  for _ in range(n_layers)]


def cpu_weights(model):
    """CPU copies of a quail_amd.model model's tensors, in a flat dict."""
    return oracle_weights(model, "cpu")


def oracle_weights(model, device):
    """A quail_amd.model model's tensors on `device`, in a flat dict. The
    oracle only reads them; on the model's own device they are the model's
    tensors themselves."""
    inner = model.model
    to = lambda x: x.to(device)
    w = {"embed": to(inner.embed_tokens.weight), "final_norm": to(inner.norm.weight),
         "final_eps": inner.norm.variance_epsilon,
         "cos_sin": to(model.rotary.cos_sin_cache),
         "answer": to(model.quail_answer_weights),
         "answer_ids": model.quail_answer_token_ids, "layers": []}
    for layer in inner.layers:
        a, m = layer.self_attn, layer.mlp
        w["layers"].append(dict(
            qkv=(to(a.qkv_proj.weight), to(a.qkv_proj.weight_scale)),
            o=(to(a.o_proj.weight), to(a.o_proj.weight_scale)),
            gate_up=(to(m.gate_up_proj.weight), to(m.gate_up_proj.weight_scale)),
            down=(to(m.down_proj.weight), to(m.down_proj.weight_scale)),
            q_norm=to(a.q_norm.weight), k_norm=to(a.k_norm.weight),
            in_norm=to(layer.input_layernorm.weight),
            post_norm=to(layer.post_attention_layernorm.weight),
            eps=layer.input_layernorm.variance_epsilon, cos_sin=w["cos_sin"],
            n_q=a.num_heads, n_kv=a.num_kv_heads, head_dim=a.head_dim))
    return w


class DequantGemm:
    """fp8 GEMM as dequantize-to-fp32 then one fp32 matmul, weights cached.

    Same sum as ops.fp8_gemm in fp32 accumulation; the CPU baseline uses it
    (dequantize with block scales, then matmul).
    """

    def __init__(self):
        self.cache = {}

    def __call__(self, a_q, a_s, w_q, w_s):
        key = w_q.data_ptr()
        w = self.cache.get(key)
        if w is None:
            w = ops.dequant_weight(w_q, w_s).T.contiguous()
            self.cache[key] = w
        a = ops.dequant_rows(a_q, a_s)
        return (a @ w).to(torch.bfloat16)


def exact_gemm(a_q, a_s, w_q, w_s):
    return ops.fp8_gemm(a_q, a_s, w_q, w_s)


class Unquantized:
    """Activation-quantization-free numerics for pinning the layer loop.

    Every quantize step passes its fp32 input through with unit scales, and
    the GEMM multiplies by the dequantized weights in fp32. Only the
    forward-vs-library test uses it.
    """

    @staticmethod
    def gemm(a, a_s, w_q, w_s):
        w = ops.dequant_weight(w_q, w_s)
        return (a.float() @ w.T).to(torch.bfloat16)

    @staticmethod
    def quant(y, ue8m0=False):
        return y.float(), None


def forward_chunk(w, host, attention_mode, arena, gemm=exact_gemm, ue8m0=False,
                  page_tokens=16, quantize=True):
    """The final-normed rows of one chunk, [R, hidden] bf16.

    host: the chunk's staged arrays as numpy (Chunk.host). arena:
    OracleArena, updated in place by the chunk's KV writes. quantize=False
    skips the fp8 activation quantization (see Unquantized).
    """
    if not quantize:
        return _forward(w, host, attention_mode, arena, Unquantized.gemm,
                        Unquantized.quant, ue8m0, page_tokens)
    return _forward(w, host, attention_mode, arena, gemm, ops.group_quant, ue8m0,
                    page_tokens)


def _forward(w, host, attention_mode, arena, gemm, quant, ue8m0, page_tokens):
    dev = w["embed"].device
    ids = torch.from_numpy(host["input_ids"]).to(dev)
    finals = torch.from_numpy(host["finals"]).to(dev)
    hidden = w["embed"][ids]
    residual = None
    for li, L in enumerate(w["layers"]):
        hidden, residual = layer_step(L, li, hidden, residual, host, attention_mode, arena,
                                      gemm, quant, ue8m0, page_tokens)
    normed, _ = ops.fused_add_rms_norm(hidden[finals], residual[finals], w["final_norm"],
                                       w["final_eps"])
    return normed


def layer_step(L, li, hidden, residual, host, attention_mode, arena, gemm=exact_gemm,
               quant=ops.group_quant, ue8m0=False, page_tokens=16):
    """One Qwen3 decoder layer (models/qwen3.py:55-71): (hidden, residual) in,
    (down-projection output, residual) out; residual None at layer 0.
    Writes the layer's KV into arena.k[li] / arena.v[li] as the chunk says."""
    t = lambda name: torch.from_numpy(host[name])   # host side; ops move what they index with
    pos = t("positions").to(hidden.device)
    T = pos.numel()
    n_q, n_kv, d, eps = L["n_q"], L["n_kv"], L["head_dim"], L["eps"]
    if residual is None:
        residual = hidden
        q_in, q_s = quant(ops.rms_norm_bf16(hidden, L["in_norm"], eps).float(), ue8m0)
    else:
        q_in, q_s, residual = _add_norm_quant(hidden, residual, L["in_norm"], eps,
                                              quant, ue8m0)
    qkv = gemm(q_in, q_s, *L["qkv"])
    q, k, v = ops.qk_norm_rope(qkv, pos, L["cos_sin"], L["q_norm"], L["k_norm"], eps,
                               n_q, n_kv, d)
    q3, k3, v3 = q.view(T, n_q, d), k.view(T, n_kv, d), v.view(T, n_kv, d)
    scale = ops.softmax_scale(d)
    kp, vp = arena.k[li], arena.v[li]
    if attention_mode == "tree":
        if "kv_src" in host:
            ops.kv_row_scatter(kp, vp, k3, v3, t("kv_src"), t("kv_dst"))
        out_a, lse_a = ops.varlen_attention(q3, k3, v3, t("cu_a"), scale, causal=True)
        out_a = out_a.to(torch.bfloat16)
        if "reads_rows" in host:
            out_b, lse_b = ops.paged_attention(
                q3, kp, vp, t("reads_cu_q"), t("reads_used"), t("reads_table"), scale,
                causal=False, q_rows=t("reads_rows"), page=page_tokens)
            merged = ops.merge_attn(out_a, lse_a, out_b.to(torch.bfloat16), lse_b,
                                    t("reads_source"))
            o_in, o_s = quant(merged.reshape(T, -1), ue8m0)
        else:
            o_in, o_s = quant(out_a.float().view(T, -1), ue8m0)
    else:
        if "unified_src" in host:
            ops.kv_row_scatter(kp, vp, k3, v3, t("unified_src"), t("unified_dst"))
            if "tail_src" in host:
                src, dst = t("tail_src").to(kp.device), t("tail_dst").to(kp.device)
                kp[dst] = kp[src]
                vp[dst] = vp[src]
            out, _ = ops.paged_attention(q3, kp, vp, t("unified_cu_q"), t("unified_used"),
                                         t("unified_table"), scale, causal=True,
                                         page=page_tokens)
        else:
            out, _ = ops.varlen_attention(q3, k3, v3, t("cu_a"), scale, causal=True)
        o_in, o_s = quant(out.to(torch.bfloat16).float().view(T, -1), ue8m0)
    hidden = gemm(o_in, o_s, *L["o"])
    g_in, g_s, residual = _add_norm_quant(hidden, residual, L["post_norm"], eps, quant, ue8m0)
    gate_up = gemm(g_in, g_s, *L["gate_up"])
    d_in, d_s = quant(ops.silu_mul(gate_up), ue8m0)
    hidden = gemm(d_in, d_s, *L["down"])
    return hidden, residual


def _add_norm_quant(x, residual, weight, eps, quant, ue8m0):
    """attention.py:325-359 with the quantizer as a parameter."""
    s = x.float() + residual.float()
    new_res = s.to(torch.bfloat16)
    ms = (s * s).sum(dim=-1, keepdim=True) / s.shape[-1]
    y = s * (1.0 / torch.sqrt(ms + eps)) * weight.float()
    q, scales = quant(y, ue8m0)
    return q, scales, new_res


def readout(w, normed, true_ids, false_ids):
    """(bits, margins) of the final-normed rows (readout.py:45-49, :70-79)."""
    allowed = list(w["answer_ids"])
    true_cols = [i for i, t in enumerate(allowed) if t in set(true_ids)]
    false_cols = [i for i, t in enumerate(allowed) if t in set(false_ids)]
    return ops.answer_bits(normed, w["answer"], true_cols, false_cols)
