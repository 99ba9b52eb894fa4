"""Operator API of the MI355X attention path — drop-in for `flashattention_custom.ops`.

Public functions (same names, positional order, defaults and return
conventions as the reference, flashattention_custom/ops.py:79-99):

  flash_attn(q, k, v, causal=True, q_offset=0, k_offset=0) -> Tensor
  flash_attn_paged(q, k_pages, v_pages, seqlen, page_size, head_map,
                   causal=True, q_offset=0, k_offset=0, *, block_table=None) -> Tensor
  paged_kv_append(k_pages, v_pages, k_new, v_new, start_pos, page_size,
                  *, block_table=None) -> None

Each validates its arguments in Python with the reference extension's
messages (csrc/ext.cpp:30-89), then calls a `torch.library` custom op
(`hrm_fa::*`) whose body calls the C ABI of libfa_mi355x.so on the current
stream of the tensors' device. There is no CPU fallback: tensors must be on a
ROCm device and the library must be built, otherwise a RuntimeError is raised
(the reference's `_ext` raises the same "CUDA required" checks; the wording
refers to torch's device type, which is "cuda" on ROCm).

Additive, keyword-compatible extensions (defaults give the reference
behaviour):
  * `q_offset` / `k_offset` / `start_pos` accept an int32 device tensor [B]
    of per-sequence values besides a Python int.
  * `block_table` (int32 [B, max_blocks]): logical page p of sequence b is
    physical page phi = block_table[b, p] of the pool, i.e.
    k_pages[phi // P, :, phi % P]. With it, k_pages.size(0) need not be B.
  * `flash_attn` also accepts fp32 q/k/v (fp32 arithmetic) and GQA
    (k.size(1) dividing q.size(1); q head h reads K/V head h // (Hq // Hk)).
  * `rope=(cos, sin)` (fp16 [L, D/2] tables, engine/rope.py:6-13) on
    `flash_attn_paged` rotates each query row at its position q_offset + i
    as it is loaded, and on `paged_kv_append` rotates each key row at its
    position before it is written: engine/rope.py:15-24's apply_rope fused
    into the kernels, bit-identical to it.
"""
from __future__ import annotations

import weakref
from typing import Optional, Union

import torch

from . import _lib

IntOrTensor = Union[int, torch.Tensor]

_HEAD_DIMS = (64, 128)


def _check(cond: bool, msg: str) -> None:
    if not cond:
        raise RuntimeError(msg)


def _device_index(t: torch.Tensor) -> int:
    return t.device.index if t.device.index is not None else torch.cuda.current_device()


class _DeviceScope:
    """Makes the tensors' device current for the duration of a library call."""

    __slots__ = ("idx", "prev")

    def __init__(self, t: torch.Tensor):
        self.idx = _device_index(t)
        self.prev = None

    def __enter__(self):
        cur = torch.cuda.current_device()
        if cur != self.idx:
            self.prev = cur
            torch.cuda.set_device(self.idx)
        return torch.cuda.current_stream(self.idx).cuda_stream

    def __exit__(self, *exc):
        if self.prev is not None:
            torch.cuda.set_device(self.prev)
        return False


def _per_seq(value: IntOrTensor, B: int, name: str, device: torch.device,
             require_device: bool = True):
    """Split a scalar-or-tensor offset into (int scalar, optional int32 [B] tensor)."""
    if isinstance(value, torch.Tensor):
        if value.dim() == 0:
            return int(value.item()), None
        if require_device:
            _check(value.is_cuda, f"{name} tensor must be CUDA")
        _check(value.device == device, f"{name} tensor must be on the q device")
        _check(value.dtype == torch.int32, f"{name} int32 required")
        _check(value.is_contiguous(), "contiguous required")
        _check(value.dim() == 1 and value.numel() == B, f"{name} [B] required")
        return 0, value
    return int(value), None


def _check_block_table(block_table: Optional[torch.Tensor], B: int, device: torch.device,
                       require_device: bool = True) -> int:
    if block_table is None:
        return 0
    if require_device:
        _check(block_table.is_cuda, "CUDA required")
    _check(block_table.device == device, "tensors must be on one device")
    _check(block_table.dtype == torch.int32, "block_table int32 required")
    _check(block_table.is_contiguous(), "contiguous required")
    _check(block_table.dim() == 2 and block_table.size(0) == B, "block_table [B, max_blocks] required")
    return int(block_table.size(1))


def _check_rope(rope, D: int, device: torch.device, require_device: bool = True):
    """(cos, sin) fp16 tables [L, D/2] on the tensors' device, or None."""
    if rope is None:
        return None, None
    _check(isinstance(rope, (tuple, list)) and len(rope) == 2, "rope must be (cos, sin)")
    cos, sin = rope
    _check(isinstance(cos, torch.Tensor) and isinstance(sin, torch.Tensor), "rope must be (cos, sin)")
    if require_device:
        _check(cos.is_cuda and sin.is_cuda, "CUDA required")
    _check(cos.dtype == torch.float16 and sin.dtype == torch.float16, "rope tables fp16 required")
    _check(cos.is_contiguous() and sin.is_contiguous(), "contiguous required")
    _check(cos.dim() == 2 and cos.shape == sin.shape and cos.size(1) * 2 == D and cos.size(0) > 0,
           "rope tables cos/sin [L, D/2] required")
    _check(cos.device == device and sin.device == device, "tensors must be on one device")
    return cos, sin


def _ptr(t: Optional[torch.Tensor]) -> Optional[int]:
    return None if t is None else t.data_ptr()


# (id of a head_map tensor, Hk) -> (weak reference to it, its version counter,
# the most q heads it sends to one KV head); an entry leaves with its tensor
_HEADS_PER_KV: dict = {}


def _count_heads_per_kv(head_map: torch.Tensor, Hk: int) -> int:
    hm = head_map.detach().to("cpu", torch.int64).view(-1)
    hm = hm[(hm >= 0) & (hm < Hk)]
    n = int(torch.bincount(hm, minlength=1).max()) if hm.numel() else 0
    return max(1, n)


def heads_per_kv(head_map: torch.Tensor, Hk: int) -> int:
    """The most query heads `head_map` sends to one KV head (entries outside
    [0, Hk) are ignored), which sizes the decode workspace. The map is read
    back once per head-map tensor and remembered until the tensor changes or
    is freed; callers such as engine/llama_tp.py:145-156 build one map per
    layer and reuse it on every call.

    A tensor made under torch.inference_mode() has no version counter, so an
    in-place edit of it cannot be seen: its map is read back on every call.
    Callers that know the bound pass heads_per_kv= to the operators instead
    and skip the read-back altogether."""
    if head_map.is_inference():
        return _count_heads_per_kv(head_map, Hk)
    key = (id(head_map), int(Hk))
    ver = head_map._version
    hit = _HEADS_PER_KV.get(key)
    if hit is not None and hit[0]() is head_map and hit[1] == ver:
        return hit[2]
    n = _count_heads_per_kv(head_map, Hk)
    ref = weakref.ref(head_map, lambda _r, k=key: _HEADS_PER_KV.pop(k, None))
    _HEADS_PER_KV[key] = (ref, ver, n)
    return n


def _resolve_heads_per_kv(given: Optional[int], head_map: torch.Tensor, Hk: int) -> int:
    """The caller's stated bound (heads past it get NaN rows, as the kernels
    document), or the one read from the map."""
    if given is None:
        return heads_per_kv(head_map, Hk)
    n = int(given)
    _check(n >= 1, "heads_per_kv must be >= 1")
    return n


# --------------------------------------------------------------------------
# custom ops (bodies call the C ABI; fake impls make them traceable)
# --------------------------------------------------------------------------

@torch.library.custom_op("hrm_fa::flash_attn", mutates_args=())
def _flash_attn_op(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, causal: bool,
                   q_offset: int, k_offset: int, q_offsets: Optional[torch.Tensor],
                   k_offsets: Optional[torch.Tensor]) -> torch.Tensor:
    lib = _lib.load()
    o = torch.empty_like(q)
    B, Hq, M, D = q.shape
    Hk, N = k.size(1), k.size(2)
    dtype = _lib.FA_DTYPE_F16 if q.dtype == torch.float16 else _lib.FA_DTYPE_F32
    # few query rows per K/V head (decode over a contiguous cache) take the
    # split-K decode kernels, which need a workspace
    ws_bytes = lib.fa_flash_attn_workspace_bytes(dtype, B, Hq, Hk, M, N, D)
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=q.device) if ws_bytes else None
    with _DeviceScope(q) as stream:
        _lib.check(lib.fa_flash_attn_fwd_ws(
            q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(), dtype,
            B, Hq, Hk, M, N, D, int(causal), q_offset, k_offset,
            _ptr(q_offsets), _ptr(k_offsets), _ptr(ws), ws_bytes, stream))
    return o


@_flash_attn_op.register_fake
def _(q, k, v, causal, q_offset, k_offset, q_offsets, k_offsets):
    return torch.empty_like(q)


@torch.library.custom_op("hrm_fa::flash_attn_paged", mutates_args=())
def _flash_attn_paged_op(q: torch.Tensor, k_pages: torch.Tensor, v_pages: torch.Tensor,
                         seqlen: torch.Tensor, page_size: int, head_map: torch.Tensor,
                         causal: bool, q_offset: int, k_offset: int,
                         q_offsets: Optional[torch.Tensor], k_offsets: Optional[torch.Tensor],
                         block_table: Optional[torch.Tensor], rope_cos: Optional[torch.Tensor],
                         rope_sin: Optional[torch.Tensor],
                         q_lens: Optional[torch.Tensor] = None,
                         heads_per_kv: int = 0) -> torch.Tensor:
    lib = _lib.load()
    o = torch.empty_like(q)
    B, Hq, M, D = q.shape
    NB, Hk, P = k_pages.size(0), k_pages.size(1), k_pages.size(2)
    max_blocks = int(block_table.size(1)) if block_table is not None else 0
    cap_pages = max_blocks if block_table is not None else P
    ws_bytes = lib.fa_paged_workspace_bytes(B, Hq, M, D, Hk, cap_pages, page_size, heads_per_kv)
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=q.device) if ws_bytes else None
    with _DeviceScope(q) as stream:
        args = (q.data_ptr(), k_pages.data_ptr(), v_pages.data_ptr(), seqlen.data_ptr(),
                page_size, head_map.data_ptr(), o.data_ptr(), B, Hq, M, D, NB, Hk, P,
                int(causal), q_offset, k_offset, _ptr(q_offsets), _ptr(k_offsets),
                _ptr(q_lens), _ptr(block_table), max_blocks, heads_per_kv, _ptr(ws), ws_bytes)
        if rope_cos is None:
            _lib.check(lib.fa_flash_attn_paged_fwd(*args, stream))
        else:
            _lib.check(lib.fa_flash_attn_paged_rope_fwd(
                *args, rope_cos.data_ptr(), rope_sin.data_ptr(), rope_cos.size(0), stream))
    return o


@_flash_attn_paged_op.register_fake
def _(q, k_pages, v_pages, seqlen, page_size, head_map, causal, q_offset, k_offset, q_offsets,
      k_offsets, block_table, rope_cos, rope_sin, q_lens=None, heads_per_kv=0):
    return torch.empty_like(q)


@torch.library.custom_op("hrm_fa::paged_kv_append", mutates_args=("k_pages", "v_pages"))
def _paged_kv_append_op(k_pages: torch.Tensor, v_pages: torch.Tensor, k_new: torch.Tensor,
                        v_new: torch.Tensor, start_pos: int, start_positions: Optional[torch.Tensor],
                        page_size: int, block_table: Optional[torch.Tensor],
                        rope_cos: Optional[torch.Tensor], rope_sin: Optional[torch.Tensor]) -> None:
    lib = _lib.load()
    B, Hk, T, D = k_new.shape
    NB, P = k_pages.size(0), k_pages.size(2)
    max_blocks = int(block_table.size(1)) if block_table is not None else 0
    with _DeviceScope(k_pages) as stream:
        args = (k_pages.data_ptr(), v_pages.data_ptr(), k_new.data_ptr(), v_new.data_ptr(),
                B, Hk, T, D, NB, P, page_size, start_pos, _ptr(start_positions),
                _ptr(block_table), max_blocks)
        if rope_cos is None:
            _lib.check(lib.fa_paged_kv_append(*args, stream))
        else:
            _lib.check(lib.fa_paged_kv_append_rope(
                *args, rope_cos.data_ptr(), rope_sin.data_ptr(), rope_cos.size(0), stream))


@_paged_kv_append_op.register_fake
def _(k_pages, v_pages, k_new, v_new, start_pos, start_positions, page_size, block_table,
      rope_cos, rope_sin):
    return None


@torch.library.custom_op("hrm_fa::flash_attn_paged_append",
                         mutates_args=("k_pages", "v_pages", "seqlen"))
def _flash_attn_paged_append_op(q: torch.Tensor, k_pages: torch.Tensor, v_pages: torch.Tensor,
                                seqlen: torch.Tensor, page_size: int, head_map: torch.Tensor,
                                causal: bool, q_offset: int, q_offsets: Optional[torch.Tensor],
                                block_table: Optional[torch.Tensor], k_new: torch.Tensor,
                                v_new: torch.Tensor, advance: bool, start_pos: int,
                                start_positions: Optional[torch.Tensor],
                                rope_cos: Optional[torch.Tensor], rope_sin: Optional[torch.Tensor],
                                heads_per_kv: int = 0) -> torch.Tensor:
    lib = _lib.load()
    o = torch.empty_like(q)
    B, Hq, M, D = q.shape
    NB, Hk, P = k_pages.size(0), k_pages.size(1), k_pages.size(2)
    max_blocks = int(block_table.size(1)) if block_table is not None else 0
    cap_pages = max_blocks if block_table is not None else P
    ws_bytes = lib.fa_paged_workspace_bytes(B, Hq, M, D, Hk, cap_pages, page_size, heads_per_kv)
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=q.device) if ws_bytes else None
    with _DeviceScope(q) as stream:
        _lib.check(lib.fa_flash_attn_paged_append_fwd(
            q.data_ptr(), k_pages.data_ptr(), v_pages.data_ptr(), seqlen.data_ptr(), page_size,
            head_map.data_ptr(), o.data_ptr(), B, Hq, M, D, NB, Hk, P, int(causal), q_offset,
            _ptr(q_offsets), _ptr(block_table), max_blocks, heads_per_kv, k_new.data_ptr(),
            v_new.data_ptr(), int(advance), start_pos, _ptr(start_positions), _ptr(rope_cos),
            _ptr(rope_sin), rope_cos.size(0) if rope_cos is not None else 0, _ptr(ws), ws_bytes,
            stream))
    return o


@_flash_attn_paged_append_op.register_fake
def _(q, k_pages, v_pages, seqlen, page_size, head_map, causal, q_offset, q_offsets, block_table,
      k_new, v_new, advance, start_pos, start_positions, rope_cos, rope_sin, heads_per_kv=0):
    return torch.empty_like(q)


@torch.library.custom_op("hrm_fa::paged_kv_scatter", mutates_args=("k_pages", "v_pages"))
def _paged_kv_scatter_op(k_pages: torch.Tensor, v_pages: torch.Tensor, k_new: torch.Tensor,
                         v_new: torch.Tensor, positions: torch.Tensor, page_size: int,
                         block_table: Optional[torch.Tensor], rope_cos: Optional[torch.Tensor],
                         rope_sin: Optional[torch.Tensor]) -> None:
    lib = _lib.load()
    B, Hk, T, D = k_new.shape
    NB, P = k_pages.size(0), k_pages.size(2)
    max_blocks = int(block_table.size(1)) if block_table is not None else 0
    with _DeviceScope(k_pages) as stream:
        _lib.check(lib.fa_paged_kv_scatter(
            k_pages.data_ptr(), v_pages.data_ptr(), k_new.data_ptr(), v_new.data_ptr(),
            B, Hk, T, D, NB, P, page_size, positions.data_ptr(), _ptr(block_table), max_blocks,
            _ptr(rope_cos), _ptr(rope_sin), rope_cos.size(0) if rope_cos is not None else 0,
            stream))


@_paged_kv_scatter_op.register_fake
def _(k_pages, v_pages, k_new, v_new, positions, page_size, block_table, rope_cos, rope_sin):
    return None


# --------------------------------------------------------------------------
# public API
# --------------------------------------------------------------------------

_SHARED_POOL_HINT = ("k_pages holds one shared page pool (size(0) == 1) for {B} sequences: "
                     "pass block_table= (PagedKVCache.block_table) to map each sequence's "
                     "pages into it")


def _check_batch(q_batch: int, pool_rows: int, block_table) -> None:
    """'B mismatch' as the reference raises it (csrc/ext.cpp:58), with a hint
    when the pages are a shared pool that needs its block table."""
    if block_table is not None or q_batch == pool_rows:
        return
    if pool_rows == 1 and q_batch > 1:
        raise RuntimeError("B mismatch: " + _SHARED_POOL_HINT.format(B=q_batch))
    raise RuntimeError("B mismatch")

def validate_flash_attn(q, k, v, require_device: bool = True) -> None:
    """Argument checks of flash_attn, in the order of csrc/ext.cpp:31-38."""
    if require_device:
        _check(q.is_cuda and k.is_cuda and v.is_cuda, "q/k/v must be CUDA")
    _check((q.dtype == k.dtype == v.dtype) and q.dtype in (torch.float16, torch.float32),
           "fp16 required")
    _check(q.is_contiguous() and k.is_contiguous() and v.is_contiguous(), "contiguous required")
    _check(q.dim() == 4 and k.dim() == 4 and v.dim() == 4, "q/k/v must be 4D")
    _check(q.size(0) == k.size(0) and q.size(0) == v.size(0), "B mismatch")
    _check(k.size(1) == v.size(1) and k.size(1) > 0 and q.size(1) % k.size(1) == 0, "H mismatch")
    _check(k.size(2) == v.size(2), "N mismatch")
    _check(q.size(3) == k.size(3) and q.size(3) == v.size(3), "D mismatch")
    _check(q.device == k.device == v.device, "q/k/v must be on one device")
    _check(q.size(3) in _HEAD_DIMS, "Supported head_dim: 64 or 128")


def flash_attn(q, k, v, causal=True, q_offset=0, k_offset=0):
    """Contiguous attention O = softmax(Q K^T / sqrt(D), causal mask) V.

    Reference: flashattention_custom/ops.py:79-82 -> csrc/ext.cpp:30-40.
    q [B,Hq,M,D], k/v [B,Hk,N,D]; returns a new tensor shaped like q.
    """
    validate_flash_attn(q, k, v)
    B = q.size(0)
    qo, qo_t = _per_seq(q_offset, B, "q_offset", q.device)
    ko, ko_t = _per_seq(k_offset, B, "k_offset", q.device)
    return _flash_attn_op(q, k, v, bool(causal), qo, ko, qo_t, ko_t)


def validate_flash_attn_paged(q, k_pages, v_pages, seqlen, page_size, head_map,
                              block_table=None, require_device: bool = True) -> int:
    """Argument checks of flash_attn_paged (csrc/ext.cpp:53-66 order, then the
    extensions); returns max_blocks of the block table (0 without one)."""
    if require_device:
        _check(q.is_cuda and k_pages.is_cuda and v_pages.is_cuda, "CUDA required")
        _check(seqlen.is_cuda and head_map.is_cuda, "CUDA required")
    _check(q.dtype == torch.float16 and k_pages.dtype == torch.float16
           and v_pages.dtype == torch.float16, "fp16 required")
    _check(seqlen.dtype == torch.int32, "seqlen int32 required")
    _check(head_map.dtype == torch.int32, "head_map int32 required")
    _check(q.is_contiguous() and k_pages.is_contiguous() and v_pages.is_contiguous(),
           "contiguous required")
    _check(seqlen.is_contiguous() and head_map.is_contiguous(), "contiguous required")
    _check(q.dim() == 4, "q [B,Hq,M,D]")
    _check(k_pages.dim() == 5 and v_pages.dim() == 5, "k_pages/v_pages [B,Hk,P,PS,D]")
    _check(k_pages.shape == v_pages.shape, "k_pages/v_pages mismatch")
    B = q.size(0)
    _check_batch(B, k_pages.size(0), block_table)
    _check(head_map.dim() == 1 and q.size(1) == head_map.size(0), "Hq mismatch")
    _check(k_pages.size(3) == page_size, "page_size mismatch")
    _check(k_pages.size(4) == q.size(3), "D mismatch")
    _check(q.size(3) in _HEAD_DIMS, "Supported head_dim: 64 or 128")
    _check(seqlen.dim() == 1 and seqlen.numel() >= B, "seqlen [B] required")
    dev = q.device
    _check(k_pages.device == dev and v_pages.device == dev and seqlen.device == dev
           and head_map.device == dev, "tensors must be on one device")
    return _check_block_table(block_table, B, dev, require_device)


def flash_attn_paged(q, k_pages, v_pages, seqlen, page_size, head_map,
                     causal=True, q_offset=0, k_offset=0, *, block_table=None, rope=None,
                     q_lens=None, heads_per_kv=None):
    """Attention of q over paged K/V (prefill chunk or decode).

    Reference: flashattention_custom/ops.py:85-92 -> csrc/ext.cpp:42-68.
    q [B,Hq,M,D] fp16; k_pages/v_pages [NB,Hk,P,PS,D] fp16; seqlen int32 [B];
    head_map int32 [Hq]. Returns a new tensor shaped like q. With
    rope=(cos, sin), q is rotated in the kernel (engine/rope.py:15-24) at
    positions q_offset + i; a scalar q_offset must keep them inside the table.
    With q_lens (int32 device tensor [B]), only rows i < q_lens[b] of
    sequence b are live (a ragged chunk padded to M rows): the others are not
    computed and come out as zeros.
    heads_per_kv: the most q heads head_map sends to one KV head, when the
    caller knows it (skips reading the map back to the host; heads past a
    stated bound come out as NaN rows).
    """
    page_size = int(page_size)
    validate_flash_attn_paged(q, k_pages, v_pages, seqlen, page_size, head_map, block_table)
    B = q.size(0)
    qo, qo_t = _per_seq(q_offset, B, "q_offset", q.device)
    ko, ko_t = _per_seq(k_offset, B, "k_offset", q.device)
    cos, sin = _check_rope(rope, q.size(3), q.device)
    if cos is not None and qo_t is None and q.size(2) > 0:
        _check(qo >= 0 and qo + q.size(2) <= cos.size(0),
               f"positions {qo}..{qo + q.size(2) - 1} are outside the rotary table "
               f"of {cos.size(0)}")
    if q_lens is not None:
        _check(isinstance(q_lens, torch.Tensor), "q_lens [B] required")
        _check(q_lens.is_cuda and q_lens.device == q.device, "q_lens tensor must be CUDA")
        _check(q_lens.dtype == torch.int32, "q_lens int32 required")
        _check(q_lens.is_contiguous(), "contiguous required")
        _check(q_lens.dim() == 1 and q_lens.numel() == B, "q_lens [B] required")
    hpk = _resolve_heads_per_kv(heads_per_kv, head_map, k_pages.size(1))
    return _flash_attn_paged_op(q, k_pages, v_pages, seqlen, page_size, head_map, bool(causal),
                                qo, ko, qo_t, ko_t, block_table, cos, sin, q_lens, hpk)


def validate_paged_kv_append(k_pages, v_pages, k_new, v_new, start_pos, page_size,
                             block_table=None, require_device: bool = True,
                             check_range: bool = True):
    """Argument checks of paged_kv_append (csrc/ext.cpp:78-87 order, then the
    extensions); returns (scalar start, per-sequence start tensor or None)."""
    if require_device:
        _check(k_pages.is_cuda and v_pages.is_cuda and k_new.is_cuda and v_new.is_cuda,
               "CUDA required")
    _check(k_pages.dtype == torch.float16 and v_pages.dtype == torch.float16
           and k_new.dtype == torch.float16 and v_new.dtype == torch.float16, "fp16 required")
    _check(k_pages.is_contiguous() and v_pages.is_contiguous() and k_new.is_contiguous()
           and v_new.is_contiguous(), "contiguous required")
    _check(k_pages.dim() == 5 and k_new.dim() == 4, "shape mismatch")
    _check(k_pages.shape == v_pages.shape, "k_pages/v_pages mismatch")
    _check(k_new.shape == v_new.shape, "k_new/v_new mismatch")
    B, Hk, T, D = k_new.shape
    _check_batch(B, k_pages.size(0), block_table)
    _check(k_pages.size(1) == Hk, "Hk mismatch")
    _check(k_pages.size(3) == page_size, "page_size mismatch")
    _check(k_pages.size(4) == D, "D mismatch")
    _check(D % 8 == 0, "head_dim must be a multiple of 8")
    dev = k_pages.device
    _check(v_pages.device == dev and k_new.device == dev and v_new.device == dev,
           "tensors must be on one device")
    max_blocks = _check_block_table(block_table, B, dev, require_device)
    sp, sp_t = _per_seq(start_pos, B, "start_pos", dev, require_device)
    if check_range and sp_t is None and T > 0:
        cap = (max_blocks if block_table is not None else k_pages.size(2)) * page_size
        _check(sp >= 0 and sp + T <= cap,
               f"start_pos {sp} + T {T} exceeds the page capacity {cap}")
    return sp, sp_t


def paged_kv_append(k_pages, v_pages, k_new, v_new, start_pos, page_size, *, block_table=None,
                    rope=None):
    """Write k_new/v_new [B,Hk,T,D] at positions start_pos + t of each sequence, in place.

    Reference: flashattention_custom/ops.py:95-99 -> csrc/ext.cpp:70-89.
    A Python-int start_pos is range-checked against the page capacity and
    raises; per-sequence (tensor) starts skip out-of-range positions on the
    device, as the reference kernel does (csrc/flash_attn_sm75.cu:548).
    With rope=(cos, sin) each key row is rotated at its position before it is
    written (engine/rope.py:15-24; D a multiple of 16).
    """
    page_size = int(page_size)
    sp, sp_t = validate_paged_kv_append(k_pages, v_pages, k_new, v_new, start_pos, page_size,
                                        block_table)
    cos, sin = _check_rope(rope, k_new.size(3), k_new.device)
    if cos is not None:
        _check(k_new.size(3) % 16 == 0, "rotary append needs head_dim a multiple of 16")
        if sp_t is None and k_new.size(2) > 0:
            _check(sp + k_new.size(2) <= cos.size(0),
                   f"positions {sp}..{sp + k_new.size(2) - 1} are outside the rotary table "
                   f"of {cos.size(0)}")
    _paged_kv_append_op(k_pages, v_pages, k_new, v_new, sp, sp_t, page_size, block_table, cos, sin)


def flash_attn_paged_append(q, k_pages, v_pages, k_new, v_new, seqlen, page_size, head_map,
                            causal=False, q_offset=None, *, start_pos=None, block_table=None,
                            rope=None, heads_per_kv=None):
    """One decode step in one call: `paged_kv_append` of one new token per
    sequence, then `flash_attn_paged` over the pages that now hold it; returns
    the attention output shaped like q.

    The reference's decode step makes these two calls (cache.append,
    engine/llama_tp.py:65-78, then flash_attn_paged, :186-200). Here, with
    start_pos=None and no rope, when the attention runs on the decode kernels
    with at most 32 query rows per KV head (single-token decode at the
    benchmark shapes), the append has no launch of its own. The new token is
    every sequence's last key: the decode kernel reads it from k_new / v_new,
    and its merge kernel writes it into the pages. Other calls (rope steps
    among them, where the separate rotary append measured faster) launch the
    append kernel first. Results equal the two calls' in every case.

    k_new, v_new: fp16 [B, Hk, 1, D] (written into the pages in place).
    start_pos=None: the token of sequence b goes to position seqlen[b], the
        attention sees seqlen[b] + 1 keys, and seqlen is advanced by one on
        the device (the reference's update, llama_tp.py:77); q_offset
        defaults to seqlen (the query at the new token's position; only
        causal attention and rope read it).
    start_pos=int or int32 [B] tensor: the token goes there, and seqlen
        already counts it; q_offset defaults to 0, as in flash_attn_paged.
    rope=(cos, sin): K is rotated at its position as paged_kv_append(rope=)
        does, and q at q_offset + i as flash_attn_paged(rope=) does.
    heads_per_kv: as in flash_attn_paged.
    """
    page_size = int(page_size)
    validate_flash_attn_paged(q, k_pages, v_pages, seqlen, page_size, head_map, block_table)
    advance = start_pos is None
    sp, sp_t = validate_paged_kv_append(k_pages, v_pages, k_new, v_new, 0 if advance else start_pos,
                                        page_size, block_table)
    _check(k_new.size(0) == q.size(0), "B mismatch")
    _check(k_new.size(2) == 1, "k_new/v_new [B, Hk, 1, D]: one new token per sequence")
    _check(k_new.size(3) == q.size(3), "D mismatch")
    B = q.size(0)
    if q_offset is None:
        q_offset = seqlen if advance else 0
    qo, qo_t = _per_seq(q_offset, B, "q_offset", q.device)
    cos, sin = _check_rope(rope, q.size(3), q.device)
    if cos is not None:
        _check(q.size(3) % 16 == 0, "rotary append needs head_dim a multiple of 16")
        if not advance and sp_t is None:
            _check(0 <= sp < cos.size(0),
                   f"position {sp} is outside the rotary table of {cos.size(0)}")
        if qo_t is None and q.size(2) > 0:
            _check(qo >= 0 and qo + q.size(2) <= cos.size(0),
                   f"positions {qo}..{qo + q.size(2) - 1} are outside the rotary table "
                   f"of {cos.size(0)}")
    hpk = _resolve_heads_per_kv(heads_per_kv, head_map, k_pages.size(1))
    return _flash_attn_paged_append_op(q, k_pages, v_pages, seqlen, page_size, head_map,
                                       bool(causal), qo, qo_t, block_table, k_new, v_new,
                                       advance, sp, sp_t, cos, sin, hpk)


def paged_kv_scatter(k_pages, v_pages, k_new, v_new, positions, page_size, *, block_table=None,
                     rope=None):
    """Write token t of sequence b at positions[b, t], in place: the general
    [B, T] path of the reference's cache (engine/llama_tp.py:80-99) as one
    kernel launch instead of a Python loop of row copies.

    positions: int32 device tensor [B, T]. Negative positions, and positions
    whose page is beyond the capacity or unmapped, are skipped. Positions of
    one sequence should be distinct: the reference's loop keeps the last of
    duplicates, and here their order is unspecified (PagedKVCache.append
    removes earlier duplicates before it calls this). rope=(cos, sin) rotates
    each key at its own position. The caller updates seqlen, as the reference
    does (engine/llama_tp.py:88-91).
    """
    page_size = int(page_size)
    validate_paged_kv_append(k_pages, v_pages, k_new, v_new, 0, page_size, block_table,
                             check_range=False)
    B, T = k_new.size(0), k_new.size(2)
    _check(isinstance(positions, torch.Tensor), "positions [B, T] required")
    _check(positions.is_cuda and positions.device == k_pages.device, "positions must be CUDA")
    _check(positions.dtype == torch.int32, "positions int32 required")
    _check(positions.is_contiguous(), "contiguous required")
    _check(positions.dim() == 2 and tuple(positions.shape) == (B, T), "positions [B, T] required")
    cos, sin = _check_rope(rope, k_new.size(3), k_new.device)
    if cos is not None:
        _check(k_new.size(3) % 16 == 0, "rotary append needs head_dim a multiple of 16")
    _paged_kv_scatter_op(k_pages, v_pages, k_new, v_new, positions, page_size, block_table,
                         cos, sin)
