"""Decode attention over the token-major KV cache of the reference's INT8 engine.

The engine (scripts/deepseek_native_engine.sh) keeps one fp16 K and one fp16 V
cache per layer, shaped [Tmax, KVH*Dh] and written one row per token by
kv_store (:553-559). Each decode step then runs attn_decode (:562-604,
launched at :1077): query head h (fp32 q [H, Dh]) attends rows 0..t of KV head
h % KVH, and the output is fp32 [H, Dh].

`decode_token_major` runs that step on this library's split-K decode kernels
through the C entry point fa_decode_token_major (the engine's C++ host code
calls the same entry point directly). The engine computes q . k in fp32
(:573-577); the kernel splits each query row into fp16 hi and lo parts (after
a power-of-two prescale when |q| >= 2^15) and takes both through the matrix
cores, so the scores keep about 22 bits of q. Softmax and the output
accumulate in fp32.
"""
from __future__ import annotations

import math
from typing import Optional

import torch

from . import _lib
from .ops import _DeviceScope, _check, _resolve_heads_per_kv


def workspace_bytes(heads: int, kv_heads: int, head_dim: int, t_max: int,
                    heads_per_kv_bound: Optional[int] = None) -> int:
    """Workspace of one decode step at any position t <= t_max (0: unsupported).
    `heads_per_kv_bound`: the most heads a custom head map sends to one KV head
    (default: ceil(heads / kv_heads), the engine's map h % KVH)."""
    hpk = -(-heads // kv_heads) if heads_per_kv_bound is None else int(heads_per_kv_bound)
    return int(_lib.load().fa_decode_token_major_workspace_bytes(heads, kv_heads, head_dim, t_max,
                                                                 hpk))


def decode_token_major(q: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor, t: int,
                       *, scale: Optional[float] = None, head_map: Optional[torch.Tensor] = None,
                       workspace: Optional[torch.Tensor] = None,
                       heads_per_kv: Optional[int] = None) -> torch.Tensor:
    """One decode step of attn_decode (deepseek_native_engine.sh:562-604).

    q: fp32 [H, Dh]; k_cache, v_cache: fp16 [T, KVH, Dh] (the engine's
    [Tmax, KVH*Dh] buffers viewed per head), rows 0..t are attended (t < T).
    scale: default 1/sqrt(Dh), the engine's inv_sqrt_dh (:1077).
    head_map: optional int32 [H]; default h % KVH, the engine's mapping (:568).
    workspace: optional uint8 device tensor of at least workspace_bytes(...).
    heads_per_kv: with a head_map, the most heads it sends to one KV head
    when the caller knows it (otherwise the map is read back once per map).
    Returns fp32 [H, Dh].
    """
    _check(q.is_cuda and k_cache.is_cuda and v_cache.is_cuda, "q/k/v must be CUDA")
    _check(q.dtype == torch.float32, "q must be fp32")
    _check(k_cache.dtype == torch.float16 and v_cache.dtype == torch.float16, "fp16 required")
    _check(q.is_contiguous() and k_cache.is_contiguous() and v_cache.is_contiguous(),
           "contiguous required")
    _check(q.dim() == 2, "q [H, Dh] required")
    _check(k_cache.dim() == 3 and k_cache.shape == v_cache.shape,
           "k_cache/v_cache [T, KVH, Dh] required")
    _check(k_cache.device == q.device and v_cache.device == q.device, "device mismatch")
    H, Dh = q.shape
    T, KVH = k_cache.size(0), k_cache.size(1)
    _check(k_cache.size(2) == Dh, "D mismatch")
    t = int(t)
    _check(0 <= t < T, f"position t={t} outside the cache of {T} rows")
    if head_map is not None:
        _check(head_map.is_cuda and head_map.device == q.device, "head_map must be CUDA")
        _check(head_map.dtype == torch.int32, "head_map int32 required")
        _check(head_map.is_contiguous() and head_map.numel() == H, "head_map [H] required")
    sc = 1.0 / math.sqrt(Dh) if scale is None else float(scale)
    lib = _lib.load()
    hpk = -(-H // KVH) if head_map is None else _resolve_heads_per_kv(heads_per_kv, head_map, KVH)
    need = lib.fa_decode_token_major_workspace_bytes(H, KVH, Dh, t, hpk)
    if workspace is None:
        workspace = torch.empty(max(need, 1), dtype=torch.uint8, device=q.device)
    else:
        _check(workspace.is_cuda and workspace.device == q.device, "workspace must be CUDA")
        _check(workspace.dtype == torch.uint8 and workspace.is_contiguous(),
               "workspace uint8 contiguous required")
    out = torch.empty_like(q)
    with _DeviceScope(q) as stream:
        _lib.check(lib.fa_decode_token_major(
            out.data_ptr(), q.data_ptr(), k_cache.data_ptr(), v_cache.data_ptr(), t, H, KVH, Dh,
            sc, head_map.data_ptr() if head_map is not None else None, hpk,
            workspace.data_ptr(), workspace.numel(), stream))
    return out
