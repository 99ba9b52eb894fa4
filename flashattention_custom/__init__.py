"""Import-compatible alias of the reference package name.

Code written against `flashattention_custom` (e.g. `from
flashattention_custom.ops import flash_attn_paged, paged_kv_append`, as in the
reference's engine/llama_tp.py:8) runs unchanged on the MI355X kernels.
"""
from hrm_flashrenderer_amd.ops import flash_attn, flash_attn_paged, paged_kv_append

__all__ = ["flash_attn", "flash_attn_paged", "paged_kv_append"]
