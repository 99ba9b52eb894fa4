"""Rotary tables for the fused rotary embedding (`rope=(cos, sin)`).

`build_rope_cache` keeps the signature and result of the reference's
engine/rope.py:6-13: inv_freq_j = 1 / theta^(j / half) for j < half = D/2,
angles t * inv_freq_j in fp32 for t < max_seq_len, and cos / sin of them in
`dtype`, each of shape [max_seq_len, D/2]. Pass the pair to
flash_attn_paged / paged_kv_append / PagedKVCache as rope=(cos, sin); the
kernels then apply engine/rope.py:15-24 (apply_rope) themselves.
"""
from __future__ import annotations

import torch


def build_rope_cache(max_seq_len: int, head_dim: int, theta: float = 10000.0,
                     device="cuda", dtype=torch.float16):
    half = head_dim // 2
    inv_freq = 1.0 / (theta ** (torch.arange(0, half, device=device, dtype=torch.float32) / half))
    t = torch.arange(max_seq_len, device=device, dtype=torch.float32)
    freqs = t[:, None] * inv_freq[None, :]
    return torch.cos(freqs).to(dtype).contiguous(), torch.sin(freqs).to(dtype).contiguous()
