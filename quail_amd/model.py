"""Qwen3-architecture fp8 model with random weights, and the answer-row head.

No checkpoint or tokenizer is reachable offline, so the model is a random
init of the Qwen3 geometry: embedding N(0, 0.02) bf16, every linear
N(0, 0.02) quantized to OCP e4m3 with one fp32 scale per 128 x 128 block
(vLLM's weight / weight_scale_inv layout that DeepGEMM reads,
attention.py:121-141), RMSNorm weights 1. The module tree mirrors the one
the reference's Qwen3 loop walks (models/qwen3.py:64-91): model.layers[i].
{self_attn.{qkv_proj, o_proj, q_norm, k_norm}, mlp.{gate_up_proj,
down_proj}, input_layernorm, post_attention_layernorm}, model.embed_tokens,
model.norm.

The TRUE/FALSE token ids are fixed synthetic sets (the reference reads the
first token of "TRUE", " TRUE", "True", " True" and the FALSE spellings from
the tokenizer, quail/logical/prompts.py:19-34).
"""

from types import SimpleNamespace

SYNTHETIC_TRUE_IDS = (2514, 3007, 4167, 24678)
SYNTHETIC_FALSE_IDS = (2469, 3557, 4195, 5183)
INIT_STD = 0.02


def _block_quant(torch, w, block=128, ue8m0=False):
    """fp32 [N, K] -> (e4m3 [N, K], fp32 [N/128, K/128]), scale = max(amax,1e-10)/448,
    rounded up to a power of two with ue8m0 (vLLM's requantization of the
    weight scales when DeepGEMM runs in UE8M0 mode)."""
    N, K = w.shape
    b = w.view(N // block, block, K // block, block)
    amax = b.abs().amax(dim=(1, 3))
    scale = amax.clamp(min=1e-10) / 448.0
    if ue8m0:
        scale = torch.exp2(torch.ceil(torch.log2(scale)))
    q = (b / scale[:, None, :, None]).clamp(-448.0, 448.0)
    return q.reshape(N, K).to(torch.float8_e4m3fn), scale.contiguous()


def _linear(torch, gen, n_out, n_in, device, ue8m0=False):
    w = torch.randn(n_out, n_in, generator=gen, device=device, dtype=torch.float32) * INIT_STD
    q, s = _block_quant(torch, w, ue8m0=ue8m0)
    return SimpleNamespace(weight=q, weight_scale=s, weight_scale_inv=s)


def _norm(torch, width, eps, device):
    return SimpleNamespace(weight=torch.ones(width, dtype=torch.bfloat16, device=device),
                           variance_epsilon=eps)


def rope_cache(torch, max_pos, head_dim, theta, device):
    """cos | sin per position in bf16, NeoX halves (vLLM's rotary cache layout)."""
    inv_freq = 1.0 / (theta ** (torch.arange(0, head_dim, 2, dtype=torch.float32) / head_dim))
    t = torch.arange(max_pos, dtype=torch.float32)
    freqs = torch.outer(t, inv_freq)
    cache = torch.cat([freqs.cos(), freqs.sin()], dim=-1).to(torch.bfloat16)
    return cache.to(device)


def build_random_qwen3(spec, *, seed=0, device="cuda", layers=None, max_pos=8192,
                       answer_token_ids=None, ue8m0=False):
    """A random-init Qwen3-architecture fp8 model of `spec`'s geometry.

    layers overrides spec.layers (tests use shallow models). The same seed
    gives the same weights on any device with the same torch RNG stream.
    ue8m0: power-of-two weight block scales (the UE8M0 mode's weights).
    """
    import torch
    n_layers = spec.layers if layers is None else layers
    gen = torch.Generator(device=device).manual_seed(seed)
    H, d = spec.hidden, spec.d_head
    eps = spec.rms_eps
    model = SimpleNamespace()
    inner = SimpleNamespace()
    embed = (torch.randn(spec.vocab, H, generator=gen, device=device,
                         dtype=torch.float32) * INIT_STD).to(torch.bfloat16)
    inner.embed_tokens = SimpleNamespace(weight=embed)
    rotary = SimpleNamespace(cos_sin_cache=rope_cache(torch, max_pos, d, spec.rope_theta,
                                                      device))
    inner.layers = []
    for _ in range(n_layers):
        attn = SimpleNamespace(
            qkv_proj=_linear(torch, gen, spec.qkv_width, H, device, ue8m0),
            o_proj=_linear(torch, gen, H, spec.n_q * d, device, ue8m0),
            q_norm=_norm(torch, d, eps, device), k_norm=_norm(torch, d, eps, device),
            num_heads=spec.n_q, num_kv_heads=spec.n_kv, head_dim=d, rotary_emb=rotary)
        mlp = SimpleNamespace(
            gate_up_proj=_linear(torch, gen, spec.ffn_width, H, device, ue8m0),
            down_proj=_linear(torch, gen, H, spec.intermediate, device, ue8m0))
        inner.layers.append(SimpleNamespace(
            self_attn=attn, mlp=mlp, input_layernorm=_norm(torch, H, eps, device),
            post_attention_layernorm=_norm(torch, H, eps, device)))
    inner.norm = _norm(torch, H, eps, device)
    model.model = inner
    model.lm_head = inner.embed_tokens if spec.tied_head else SimpleNamespace(
        weight=(torch.randn(spec.vocab, H, generator=gen, device=device) * INIT_STD)
        .to(torch.bfloat16))
    model.rotary = rotary
    ids = answer_token_ids or (SYNTHETIC_TRUE_IDS + SYNTHETIC_FALSE_IDS)
    retain_answer_head(torch, model, ids)
    return model


def retain_answer_head(torch, model, token_ids):
    """Keep the answer rows of the output head, drop the head (model.py:112-126)."""
    allowed = tuple(sorted(set(int(t) for t in token_ids)))
    if not allowed:
        raise ValueError("TRUE/FALSE token ids must not be empty")
    if getattr(model, "quail_answer_token_ids", None) is not None:
        answer_weights(model, allowed)
        return
    weight = model.lm_head.weight
    idx = torch.tensor(allowed, device=weight.device, dtype=torch.long)
    model.quail_answer_weights = weight.detach().index_select(0, idx).to(torch.bfloat16)
    model.quail_answer_token_ids = allowed
    model.lm_head = None


def answer_weights(model, token_ids):
    """The retained rows for a query's answer ids (model.py:129-134)."""
    if tuple(token_ids) != model.quail_answer_token_ids:
        raise ValueError("Query answer token ids differ from the loaded model's retained rows")
    return model.quail_answer_weights
