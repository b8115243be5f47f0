"""MI355X-native Quail executor hot path: paged KV arena, row packer,
prefix-shared attention and FP8 block-scaled Qwen3 prefill on gfx950."""

__version__ = "0.1.0"
