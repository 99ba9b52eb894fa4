"""MI355X-native (gfx950) attention path: drop-in for `flashattention_custom`.

Exports the reference's three operators (flashattention_custom/__init__.py:1-3)
backed by hand-written HIP kernels in libfa_mi355x.so, the fused decode step
(flash_attn_paged_append: append then attention in one call), and a
shared-pool paged K/V cache (the caller-side cache of engine/llama_tp.py:21-107).
"""
from .ops import (flash_attn, flash_attn_paged, flash_attn_paged_append, paged_kv_append,
                  paged_kv_scatter)
from .kv_cache import PagedKVCache, chunked_prefill_plan, chunked_prefill_schedule
from .rope import build_rope_cache

__all__ = ["flash_attn", "flash_attn_paged", "flash_attn_paged_append", "paged_kv_append",
           "paged_kv_scatter", "PagedKVCache", "build_rope_cache", "chunked_prefill_plan",
           "chunked_prefill_schedule"]
