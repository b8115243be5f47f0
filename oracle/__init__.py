"""CPU oracle of the Quail executor hot path: TEST INFRASTRUCTURE ONLY.

This package restates, on the CPU with torch/numpy, what the reference
computes on its hot path (citations are to animysore/quail files). It is the
checker the GPU kernels are compared against and the timed CPU baseline of
bench.py. Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline
leg may import it; the product (quail_amd) never does, and has no CPU
fallback.

Modules
  ops      - per-kernel closed forms: fp8 group/block quant, RMSNorm variants,
             QK-norm + rotary, SiLU gate, fp8 block GEMM, paged/varlen
             attention with LSE, the tree LSE merge, KV row scatter, the
             answer readout.
  forward  - the Qwen3 layer loop over a packed chunk (models/qwen3.py:46-77)
             built from ops, with its own logical KV arena.

How each function is pinned (tests/test_oracle.py):
  group_quant, quantize_weight_blocks: the amax element maps to +-448
      exactly; dequantized values match inputs within half an e4m3 step;
      UE8M0 scales are the least power of two >= amax/448.
  rms_norm_*: torch.nn.functional.rms_norm (library) at fp32 precision.
  qk_norm_rope: identity at position 0; per-pair norm preserved; equals a
      complex-multiplication rotary on the normed heads.
  silu_mul: torch.nn.functional.silu (library).
  fp8_gemm: exact integer matmul on small-integer fp8 inputs with unit
      scales; block-scale linearity (scaling one block scales its share).
  attention: torch scaled_dot_product_attention (library) on dense causal and
      non-causal cases; invariance under a random page permutation; LSE
      equals torch.logsumexp of the scaled scores; bottom-right causal
      alignment equals the HashModel position rule (tests/kv_checker.py:
      132-139 of the reference) on a brute-force tiny case.
  merge: merging a split of one key set reproduces attention over the whole
      set (Milakov & Gimelshein); source = -1 passes out_a through.
  answer_bits: the reference's literal readout case (tests/test_model.py:
      31-81 of the reference) and the strict tie rule.
  forward: a dequantized, unquantized-activation variant matches
      transformers' Qwen3ForCausalLM (library) on the same weights.
"""
