"""myk_llm_amd: MI355X-native (gfx950) FlashAttention, a drop-in for the attention ops of
myk-llm (src/myk_llm/ops/__init__.py:1 re-exports the same three functions)."""

from .flash_attn import flash_attn_func, flash_attn_varlen_func, flash_attn_with_kvcache

__all__ = ["flash_attn_func", "flash_attn_varlen_func", "flash_attn_with_kvcache"]
