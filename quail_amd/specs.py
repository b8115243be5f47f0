"""Model and device geometry the sizing formulas read (quail/specs/base.py).

ModelSpec keeps the fields the hot path and its sizing use; DeviceSpec adds
MI355X beside the H100 spec the reference's budget tests are quoted on.
"""

from dataclasses import dataclass, replace

ACT_BYTES_PER_HIDDEN = 32   # peak activation bytes per token per hidden dim


@dataclass(frozen=True)
class ModelSpec:
    name: str
    params: float          # dense params used per token (2P FLOPs/token)
    layers: int
    hidden: int
    n_q: int
    n_kv: int
    d_head: int
    ffn_width: int         # gate_up output columns (2 x intermediate)
    w_bytes: float = 1.0   # fp8 weights
    kv_bytes: float = 2.0  # bf16 KV
    w_mem_bytes: float = 0.0
    vocab: int = 0
    tied_head: bool = False
    arch: str = "qwen3"
    rope_theta: float = 1e6
    rms_eps: float = 1e-6
    chunk_cap_tokens: int = 0

    @property
    def intermediate(self) -> int:
        return self.ffn_width // 2

    @property
    def qkv_width(self) -> int:
        return (self.n_q + 2 * self.n_kv) * self.d_head

    @property
    def widest_projection(self) -> int:
        return max(self.ffn_width, self.qkv_width)

    @property
    def kv_elements_per_token(self) -> int:
        return 2 * self.layers * self.n_kv * self.d_head

    @property
    def kappa(self) -> float:
        """KV bytes per cached token over all layers (base.py:94-101)."""
        return self.kv_elements_per_token * self.kv_bytes

    kappa_full = kappa

    @property
    def W_mem(self) -> float:  # noqa: N802
        return self.w_mem_bytes or self.params * self.w_bytes

    @property
    def head_mem_bytes(self) -> float:
        return 0.0 if self.tied_head else self.vocab * self.hidden * 2.0

    @property
    def W_resident(self) -> float:  # noqa: N802
        return self.W_mem - self.head_mem_bytes

    @property
    def act_per_token(self) -> float:
        return ACT_BYTES_PER_HIDDEN * self.hidden

    def gemm_flops_per_token(self) -> float:
        """2 * (QKV + O + gate_up + down) weights per layer, all layers."""
        per_layer = (self.hidden * self.qkv_width
                     + self.n_q * self.d_head * self.hidden
                     + self.hidden * self.ffn_width
                     + self.intermediate * self.hidden)
        return 2.0 * per_layer * self.layers

    def with_kv_bytes(self, kv_bytes: float) -> "ModelSpec":
        return replace(self, kv_bytes=kv_bytes)


@dataclass(frozen=True)
class DeviceSpec:
    name: str
    mem_bytes: float
    hbm_bw: float
    peak_flops: float       # dense peak at the executor's compute dtype (fp8)
    bf16_flops: float = 0.0

    @property
    def attn_flops(self) -> float:
        return self.bf16_flops or self.peak_flops / 2


QWEN3_4B_FP8 = ModelSpec(
    name="qwen3-4b-fp8", params=3.6e9, layers=36, hidden=2560, n_q=32, n_kv=8,
    d_head=128, ffn_width=19456, w_mem_bytes=4.5e9, vocab=151_936, tied_head=True)

QWEN3_32B_FP8 = ModelSpec(
    name="qwen3-32b-fp8", params=31.2e9, layers=64, hidden=5120, n_q=64, n_kv=8,
    d_head=128, ffn_width=51200, w_mem_bytes=34.37e9, vocab=151_936,
    tied_head=False)

MODELS = {m.name: m for m in (QWEN3_4B_FP8, QWEN3_32B_FP8)}

# AMD published MI355X peaks (dense, no sparsity): 256 CUs at 2.4 GHz.
MI355X = DeviceSpec(name="mi355x", mem_bytes=288e9, hbm_bw=8.0e12,
                    peak_flops=5.0332e15, bf16_flops=2.5166e15)

# The reference planner's H100 spec (quail/specs/h100_sxm.py:3-13); its
# budget tests are quoted on it.
H100_SXM = DeviceSpec(name="h100-sxm", mem_bytes=80e9, hbm_bw=3.35e12,
                      peak_flops=1.979e15, bf16_flops=0.9895e15)

DEVICES = {d.name: d for d in (MI355X, H100_SXM)}
