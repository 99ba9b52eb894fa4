"""`flashattention_custom.ops` alias: the reference's operator module path."""
from hrm_flashrenderer_amd.ops import flash_attn, flash_attn_paged, paged_kv_append

__all__ = ["flash_attn", "flash_attn_paged", "paged_kv_append"]
